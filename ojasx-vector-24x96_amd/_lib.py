"""ctypes loader of the HIP C-ABI library ``libojasx_lut_hip.so``.

Mirrors the reference binding's loader
(split_manifold_lut_experiment/native/bindings/ojasx_lut_ctypes.py:16-88): the
library is located next to this package and a missing library raises
``FileNotFoundError`` at first use.  There is no CPU fallback: every entry
point runs on the GPU.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libojasx_lut_hip.so")

_lib = None

vp, ci, cf, cz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
cl = ctypes.c_long

# name -> (restype, argtypes); the set of symbols declared in include/ojasx_lut_c_api.h
SIGNATURES = {
    "ojasx_get_version": (ctypes.c_char_p, []),
    "ojasx_get_backend_name": (ctypes.c_char_p, []),
    "ojasx_get_last_error": (ctypes.c_char_p, []),
    "ojasx_kernel_timing_enable": (ci, [ci]),
    "ojasx_kernel_timing_report": (ci, [ctypes.c_char_p, ctypes.c_size_t]),
    "ojasx_create_linear": (vp, [ci, ci, ci, ci, vp, vp, vp, vp]),
    "ojasx_set_linear_outliers": (ci, [vp, ci, vp, vp, vp]),
    "ojasx_linear_forward": (ci, [vp, vp, vp, ci, ci]),
    "ojasx_get_compressed_size": (cz, [vp]),
    "ojasx_get_dense_size": (cz, [vp]),
    "ojasx_get_lut_sram_size": (cz, [vp]),
    "ojasx_get_compression_ratio": (cf, [vp]),
    "ojasx_destroy_linear": (None, [vp]),
    "ojasx_linear_forward_device": (ci, [vp, vp, vp, ci, ci, vp]),
    "ojasx_linear_device_weight_bytes": (cz, [vp]),
    "ojasx_build_lut_device": (ci, [vp, vp, ci, ci, ci, ci, vp, ci, vp]),
    "ojasx_create_kv_cache": (vp, [ci, ci, ci, ci]),
    "ojasx_kv_cache_append": (ci, [vp, ci, vp, vp]),
    "ojasx_kv_cache_attention": (ci, [vp, ci, vp, vp, cf]),
    "ojasx_kv_cache_get_memory_size": (cz, [vp]),
    "ojasx_kv_cache_get_compression_ratio": (cf, [vp]),
    "ojasx_destroy_kv_cache": (None, [vp]),
    "ojasx_kv_decode_paged_device": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci,
                                          ci, cf, vp, vp]),
    "ojasx_kv_decode_paged_device_noalloc": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci,
                                                  ci, ci, cf, vp, vp]),
    "ojasx_kv_decode_paged_device_len": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci,
                                              ci, ci, cf, ci, vp, vp]),
    "ojasx_create_moe": (vp, [ci, ci, ci, ci, ci, vp, vp, vp, vp, vp, vp]),
    "ojasx_moe_forward": (ci, [vp, vp, vp, vp, vp, ci]),
    "ojasx_moe_get_compressed_size": (cz, [vp]),
    "ojasx_moe_get_compression_ratio": (cf, [vp]),
    "ojasx_destroy_moe": (None, [vp]),
    "ojasx_moe_forward_device": (ci, [vp, vp, vp, vp, vp, ci, ci, ci, vp]),
    "ojasx_moe_route_device": (ci, [vp, ci, ci, ci, ci, vp, vp, vp]),
    "ojasx_subspace_lut_gemm_device": (ci, [vp, ci, ci, ci, vp, cz, ci, ci, ci, vp, vp, vp, vp, ci, vp]),
    "ojasx_pack_codes_device": (ci, [vp, ctypes.c_long, ci, vp, vp]),
    "ojasx_unpack_codes_device": (ci, [vp, ctypes.c_long, ci, vp, vp]),
    "ojasx_quantize_int8_device": (ci, [vp, cl, ci, ci, cl, ci, vp, cl, vp, cl, vp]),
    "ojasx_dequantize_int8_device": (ci, [vp, vp, cl, ci, ci, cl, cl, vp, ci, vp]),
    "ojasx_kv_encode_append_device": (ci, [vp, vp, ci, ci, ci, ci, vp, vp, vp, ci, ci, vp, vp, vp,
                                           vp, vp]),
    "ojasx_linear_forward_grouped_device": (ci, [vp, ci, vp, vp, vp]),
    "ojasx_create_decoder": (vp, [ci, ci, ci, ci, ci, ci, ci, ci, ci, ci, cf, cf]),
    "ojasx_destroy_decoder": (None, [vp]),
    "ojasx_decoder_set_layer": (ci, [vp, ci, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "ojasx_decoder_set_head": (ci, [vp, vp, vp, vp]),
    "ojasx_decoder_set_context": (ci, [vp, ci, vp, vp, vp, vp, ci]),
    "ojasx_decoder_reset": (ci, [vp, ci]),
    "ojasx_decoder_generate": (ci, [vp, ci, ci, ci, vp, vp]),
    "ojasx_decoder_read_kv": (ci, [vp, ci, ci, ci, vp, vp, vp, vp]),
    "ojasx_linear_forward_fused_device": (ci, [vp, vp, vp, ci, vp, cf, vp, vp]),
    "ojasx_attention_stream_init_device": (ci, [vp, vp, ci, ci, ci, vp]),
    "ojasx_attention_stream_update_device": (ci, [vp, ci, ci, ci, ci, ci, vp, ci, ci, ci,
                                                  ctypes.c_longlong, ctypes.c_longlong,
                                                  ctypes.c_double, vp]),
    "ojasx_attention_stream_finalize_device": (ci, [vp, ci, ci, vp, ci, vp, vp]),
}


class AttnTile(ctypes.Structure):
    """OjasxAttnTile: one K/V tile of a streamed attention (element strides)."""
    _fields_ = [("k", vp), ("v", vp), ("k_scale", vp), ("v_scale", vp),
                ("n_tokens", ctypes.c_longlong),
                ("batch_stride", ctypes.c_longlong), ("head_stride", ctypes.c_longlong),
                ("token_stride", ctypes.c_longlong),
                ("scale_batch_stride", ctypes.c_longlong),
                ("scale_head_stride", ctypes.c_longlong),
                ("scale_token_stride", ctypes.c_longlong)]

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F64 = 3
DTYPE_INT8 = 4


class OjasxError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def _bind_torch_runtime():
    """Load PyTorch's HIP runtime before the library.  torch ships its own
    libamdhip64 (soname libamdhip64.so.7, needed by name libamdhip64.so); if
    the system one were loaded first the process would hold two HIP runtimes
    and torch streams and allocations would not be valid in our calls.  With
    torch loaded first, the library's libamdhip64.so.7 dependency resolves to
    torch's copy: one runtime per process."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    global _lib
    if _lib is None:
        _bind_torch_runtime()
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"Native library not found at: {LIB_PATH} (build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, what):
    if rc != 0:
        msg = lib().ojasx_get_last_error().decode(errors="replace")
        raise OjasxError(f"{what} failed with code {rc}: {msg}")
    return rc


def kernel_timing_enable(on=True):
    """Start (or stop) recording per-kernel start/stop events in the library;
    starting clears earlier records."""
    check(lib().ojasx_kernel_timing_enable(1 if on else 0), "ojasx_kernel_timing_enable")


def kernel_timing_report():
    """Synchronise the device and return {kernel: {"calls": n, "avg_us": t}}
    for the launches recorded since timing was enabled (records are cleared)."""
    import json
    buf = ctypes.create_string_buffer(1 << 20)
    n = lib().ojasx_kernel_timing_report(buf, len(buf))
    if n <= 0:
        raise OjasxError("ojasx_kernel_timing_report failed: "
                         + lib().ojasx_get_last_error().decode(errors="replace"))
    return json.loads(buf.value.decode())

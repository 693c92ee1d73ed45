"""NumPy / host-array face of the engine, the same API as the reference binding
split_manifold_lut_experiment/native/bindings/ojasx_lut_ctypes.py:91-241
(``get_engine_info``, ``NativeSplitManifoldLinear``, ``NativeKVCache``,
``NativeSplitManifoldMoE``), backed by the HIP C-ABI library.

Arrays are host NumPy arrays; every call copies in, runs on the GPU and copies
out (synchronous), exactly like the reference's host-pointer C-ABI.
Differences: a non-zero status raises ``OjasxError`` with the library's
message instead of failing an ``assert``.
"""
import ctypes

import numpy as np

from ._lib import check, lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def get_engine_info():
    """ojasx_lut_ctypes.py:91-95."""
    L = lib()
    return {"version": L.ojasx_get_version().decode("utf-8"),
            "backend": L.ojasx_get_backend_name().decode("utf-8")}


class NativeSplitManifoldLinear:
    """ojasx_lut_ctypes.py:98-154."""

    def __init__(self, in_features: int, out_features: int, block_dim: int = 16,
                 codebook_size: int = 256):
        self.in_features = in_features
        self.out_features = out_features
        self.block_dim = block_dim
        self.codebook_size = codebook_size
        self._handle = None

    def initialize_weights(self, codebook, codes, scales, bias=None):
        cb = np.ascontiguousarray(codebook, np.float32)
        cd = np.ascontiguousarray(codes, np.uint8)
        sc = np.ascontiguousarray(scales, np.float32)
        bs = None if bias is None else np.ascontiguousarray(bias, np.float32)
        if self._handle:
            lib().ojasx_destroy_linear(self._handle)
        self._destroy = lib().ojasx_destroy_linear
        self._handle = lib().ojasx_create_linear(
            self.in_features, self.out_features, self.block_dim, self.codebook_size,
            _p(cb), _p(cd), _p(sc), _p(bs))
        if not self._handle:
            raise RuntimeError("ojasx_create_linear failed: "
                               + lib().ojasx_get_last_error().decode(errors="replace"))

    def set_outliers(self, row_ptrs, col_indices, values):
        assert self._handle is not None
        rp = np.ascontiguousarray(row_ptrs, np.int32)
        cl = np.ascontiguousarray(col_indices, np.int32)
        vl = np.ascontiguousarray(values, np.float32)
        check(lib().ojasx_set_linear_outliers(self._handle, len(vl), _p(rp), _p(cl), _p(vl)),
              "ojasx_set_linear_outliers")

    def forward(self, x, num_threads: int = 0):
        assert self._handle is not None
        batch = x.shape[0] if x.ndim > 1 else 1
        xf = np.ascontiguousarray(np.reshape(x, (batch, self.in_features)), np.float32)
        y = np.zeros((batch, self.out_features), np.float32)
        check(lib().ojasx_linear_forward(self._handle, _p(xf), _p(y), batch, num_threads),
              "ojasx_linear_forward")
        return y.squeeze(0) if x.ndim == 1 else y

    @property
    def compressed_bytes(self) -> int:
        return lib().ojasx_get_compressed_size(self._handle) if self._handle else 0

    @property
    def compression_ratio(self) -> float:
        return lib().ojasx_get_compression_ratio(self._handle) if self._handle else 0.0

    @property
    def handle(self):
        return self._handle

    def __del__(self):
        # the destroy entry point is bound at creation: at interpreter exit the
        # module's globals may already be gone
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_handle", None) and destroy is not None:
            destroy(self._handle)
            self._handle = None


class NativeKVCache:
    """ojasx_lut_ctypes.py:157-183."""

    def __init__(self, num_heads: int, head_dim: int = 128, max_seq_len: int = 4096,
                 block_dim: int = 16):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self._destroy = lib().ojasx_destroy_kv_cache
        self._handle = lib().ojasx_create_kv_cache(num_heads, head_dim, max_seq_len, block_dim)
        if not self._handle:
            raise RuntimeError("ojasx_create_kv_cache failed: "
                               + lib().ojasx_get_last_error().decode(errors="replace"))

    def append(self, head_idx: int, k, v):
        kc = np.ascontiguousarray(k, np.float32)
        vc = np.ascontiguousarray(v, np.float32)
        check(lib().ojasx_kv_cache_append(self._handle, head_idx, _p(kc), _p(vc)),
              "KV append")

    def attention(self, head_idx: int, q, scale_factor: float = -1.0):
        qc = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.head_dim, np.float32)
        check(lib().ojasx_kv_cache_attention(self._handle, head_idx, _p(qc), _p(out),
                                             scale_factor), "Attention")
        return out

    @property
    def total_bytes(self) -> int:
        return lib().ojasx_kv_cache_get_memory_size(self._handle)

    @property
    def compression_ratio(self) -> float:
        return lib().ojasx_kv_cache_get_compression_ratio(self._handle)

    def __del__(self):
        # the destroy entry point is bound at creation: at interpreter exit the
        # module's globals may already be gone
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_handle", None) and destroy is not None:
            destroy(self._handle)
            self._handle = None


class NativeSplitManifoldMoE:
    """ojasx_lut_ctypes.py:186-241."""

    def __init__(self, num_experts: int = 512, hidden_dim: int = 2560,
                 intermediate_dim: int = 640, top_k: int = 10, block_dim: int = 16):
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.top_k = top_k
        self.block_dim = block_dim
        self._handle = None

    def initialize_weights(self, codebook_in, codebook_down, gate_up_codes, gate_up_scales,
                           down_codes, down_scales):
        arrs = [np.ascontiguousarray(codebook_in, np.float32),
                np.ascontiguousarray(codebook_down, np.float32),
                np.ascontiguousarray(gate_up_codes, np.uint8),
                np.ascontiguousarray(gate_up_scales, np.float32),
                np.ascontiguousarray(down_codes, np.uint8),
                np.ascontiguousarray(down_scales, np.float32)]
        if self._handle:
            lib().ojasx_destroy_moe(self._handle)
        self._destroy = lib().ojasx_destroy_moe
        self._handle = lib().ojasx_create_moe(
            self.num_experts, self.hidden_dim, self.intermediate_dim, self.top_k,
            self.block_dim, *[_p(a) for a in arrs])
        assert self._handle is not None, "Failed to create Native MoE engine handle"

    def forward(self, x, top_k_indices, top_k_weights):
        assert self._handle is not None
        xc = np.ascontiguousarray(x, np.float32)
        ic = np.ascontiguousarray(top_k_indices, np.int32)
        wc = np.ascontiguousarray(top_k_weights, np.float32)
        y = np.zeros(self.hidden_dim, np.float32)
        check(lib().ojasx_moe_forward(self._handle, _p(xc), _p(ic), _p(wc), _p(y), len(ic)),
              "MoE forward")
        return y

    @property
    def compressed_bytes(self) -> int:
        return lib().ojasx_moe_get_compressed_size(self._handle) if self._handle else 0

    @property
    def compression_ratio(self) -> float:
        return lib().ojasx_moe_get_compression_ratio(self._handle) if self._handle else 0.0

    @property
    def handle(self):
        return self._handle

    def __del__(self):
        # the destroy entry point is bound at creation: at interpreter exit the
        # module's globals may already be gone
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_handle", None) and destroy is not None:
            destroy(self._handle)
            self._handle = None

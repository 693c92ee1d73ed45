"""ctypes binding of the C restatement (``oracle/liblut_oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by tests, smoke() and bench.py's
cpu_baseline leg.  Build with ``make -C oracle oracle``.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblut_oracle.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"oracle library missing: {LIB_PATH} (run `make -C oracle oracle`)")
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def _u8(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint8)


def build_lut(x, codebook):
    """LUT[g, k] for one token.  NAT/src/ojasx_lut_cpu.cpp:92-100."""
    x = _f32(x).reshape(-1)
    cb = _f32(codebook)
    kcb, d = cb.shape
    g = x.size // d
    out = np.empty((g, kcb), np.float32)
    lib().orc_build_lut(_p(x), _p(cb), g, d, kcb, _p(out))
    return out


def linear_forward(x, codebook, codes, scales=None, bias=None, row_ptrs=None,
                   cols=None, vals=None):
    """SplitManifoldLinear::forward_cpu + outliers.  NAT/src/ojasx_lut_cpu.cpp:132-206."""
    x = _f32(x)
    squeeze = x.ndim == 1
    x = x.reshape(-1, x.shape[-1])
    b, k = x.shape
    cb = _f32(codebook)
    kcb, d = cb.shape
    codes = _u8(codes)
    m = codes.shape[0]
    scales = _f32(scales)
    bias = _f32(bias)
    nnz = 0 if vals is None else int(np.asarray(vals).size)
    rp, cl, vl = _i32(row_ptrs), _i32(cols), _f32(vals)
    y = np.empty((b, m), np.float32)
    lib().orc_linear_forward(_p(x), b, k, m, d, kcb, _p(cb), _p(codes), _p(scales),
                             _p(bias), nnz, _p(rp), _p(cl), _p(vl), _p(y))
    return y[0] if squeeze else y


def moe_forward(x, cb_in, cb_down, gu_codes, gu_scales, dn_codes, dn_scales, idx, w,
                k_active=None, y_init=None):
    """SplitManifoldMoE::forward_cpu for one token.  NAT/src/ojasx_lut_cpu.cpp:213-365."""
    x = _f32(x).reshape(-1)
    cb_in, cb_down = _f32(cb_in), _f32(cb_down)
    kcb, d = cb_in.shape
    gu_codes, dn_codes = _u8(gu_codes), _u8(dn_codes)
    e = gu_codes.shape[0]
    i = gu_codes.shape[1] // 2
    h = dn_codes.shape[1]
    idx, w = _i32(idx).reshape(-1), _f32(w).reshape(-1)
    if k_active is None:
        k_active = idx.size
    y = np.zeros(h, np.float32) if y_init is None else _f32(y_init).copy()
    lib().orc_moe_forward(_p(x), e, h, i, d, kcb, _p(cb_in), _p(cb_down), _p(gu_codes),
                          _p(_f32(gu_scales)), _p(dn_codes), _p(_f32(dn_scales)),
                          _p(idx), _p(w), int(k_active), _p(y))
    return y


def kv_quantize_token(k, block_dim=16):
    """HeadKVCache::append_token quantiser.  NAT/src/ojasx_lut_kv_cache.cpp:29-46."""
    k = _f32(k).reshape(-1)
    codes = np.empty(k.size // block_dim, np.uint8)
    s = np.zeros(1, np.float32)
    lib().orc_kv_quantize_token(_p(k), k.size, block_dim, _p(codes), _p(s))
    return codes, s[0]


def kv_encode_token(k, codebook, block_dim=16):
    """Nearest-centroid codebook KV encoder for one token of one head (see
    lut_oracle.c orc_kv_encode_token)."""
    k = _f32(k).reshape(-1)
    cb = _f32(codebook)
    codes = np.empty(k.size // block_dim, np.uint8)
    s = np.zeros(1, np.float32)
    lib().orc_kv_encode_token(_p(k), k.size, block_dim, _p(cb), _p(codes), _p(s))
    return codes, s[0]


def kv_attention_ref(q, k_codes, k_scales, v_codes, v_scales, scale_factor=-1.0,
                     block_dim=16):
    """Reference scalar-codebook decode attention for one head (logits, two-pass
    softmax, context).  NAT/src/ojasx_lut_kv_cache.cpp:67-132, ojasx_lut_c_api.cpp:160-196."""
    q = _f32(q).reshape(-1)
    k_codes, v_codes = _u8(k_codes), _u8(v_codes)
    t = k_codes.shape[0]
    out = np.zeros(q.size, np.float32)
    lib().orc_kv_attention_ref(_p(q), t, q.size, block_dim, _p(k_codes), _p(_f32(k_scales)),
                               _p(v_codes), _p(_f32(v_scales)), ctypes.c_float(scale_factor),
                               _p(out))
    return out


def kv_attention_cb(q, k_cb, v_cb, k_codes, k_scales, v_codes, v_scales, scale_factor=-1.0):
    """General-codebook decode attention for one query head (see lut_oracle.c)."""
    q = _f32(q).reshape(-1)
    k_cb, v_cb = _f32(k_cb), _f32(v_cb)
    d = k_cb.shape[1]
    k_codes, v_codes = _u8(k_codes), _u8(v_codes)
    t = k_codes.shape[0]
    out = np.zeros(q.size, np.float32)
    lib().orc_kv_attention_cb(_p(q), t, q.size, d, _p(k_cb), _p(v_cb), _p(k_codes),
                              _p(_f32(k_scales)), _p(v_codes), _p(_f32(v_scales)),
                              ctypes.c_float(scale_factor), _p(out))
    return out


def router_topk(logits, k, renorm=False):
    """Router top-k + softmax weights (defined by this build; see lut_oracle.c)."""
    logits = _f32(logits)
    if logits.ndim == 1:
        logits = logits[None]
    t, e = logits.shape
    idx = np.empty((t, k), np.int32)
    w = np.empty((t, k), np.float32)
    lib().orc_router_topk(_p(logits), t, e, k, int(bool(renorm)), _p(idx), _p(w))
    return idx, w

"""ctypes binding of the reference engine compiled from its own sources.

TEST INFRASTRUCTURE ONLY.  ``oracle/_ref/libojasx_lut_ref.so`` is built by
``make -C oracle ref`` from split_manifold_lut_experiment/native/src/
{ojasx_lut_cpu,ojasx_lut_kv_cache,ojasx_lut_c_api}.cpp of the reference tree
(not copied; compiled in place).  It exports the reference C-ABI
(NAT/include/ojasx_lut_c_api.h:40-150).  Used to pin the C restatement, to write
golden fixtures, and as bench.py's CPU baseline (``kind: "reference"``).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(_HERE, "_ref")
LIB_SCALAR = os.path.join(REF_DIR, "libojasx_lut_ref.so")
LIB_AVX2 = os.path.join(REF_DIR, "libojasx_lut_ref_avx2.so")

_libs = {}


def available(path=LIB_SCALAR):
    return os.path.exists(path)


def lib(path=LIB_SCALAR):
    if path not in _libs:
        if not os.path.exists(path):
            raise FileNotFoundError(f"reference engine not built: {path}")
        L = ctypes.CDLL(path)
        vp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.ojasx_get_version.restype = ctypes.c_char_p
        L.ojasx_get_backend_name.restype = ctypes.c_char_p
        L.ojasx_create_linear.restype = vp
        L.ojasx_create_linear.argtypes = [ci, ci, ci, ci, vp, vp, vp, vp]
        L.ojasx_set_linear_outliers.restype = ci
        L.ojasx_set_linear_outliers.argtypes = [vp, ci, vp, vp, vp]
        L.ojasx_linear_forward.restype = ci
        L.ojasx_linear_forward.argtypes = [vp, vp, vp, ci, ci]
        for n in ("ojasx_get_compressed_size", "ojasx_get_dense_size", "ojasx_get_lut_sram_size",
                  "ojasx_kv_cache_get_memory_size", "ojasx_moe_get_compressed_size"):
            getattr(L, n).restype = ctypes.c_size_t
            getattr(L, n).argtypes = [vp]
        for n in ("ojasx_get_compression_ratio", "ojasx_kv_cache_get_compression_ratio",
                  "ojasx_moe_get_compression_ratio"):
            getattr(L, n).restype = cf
            getattr(L, n).argtypes = [vp]
        for n in ("ojasx_destroy_linear", "ojasx_destroy_kv_cache", "ojasx_destroy_moe"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [vp]
        L.ojasx_create_kv_cache.restype = vp
        L.ojasx_create_kv_cache.argtypes = [ci, ci, ci, ci]
        L.ojasx_kv_cache_append.restype = ci
        L.ojasx_kv_cache_append.argtypes = [vp, ci, vp, vp]
        L.ojasx_kv_cache_attention.restype = ci
        L.ojasx_kv_cache_attention.argtypes = [vp, ci, vp, vp, cf]
        L.ojasx_create_moe.restype = vp
        L.ojasx_create_moe.argtypes = [ci, ci, ci, ci, ci, vp, vp, vp, vp, vp, vp]
        L.ojasx_moe_forward.restype = ci
        L.ojasx_moe_forward.argtypes = [vp, vp, vp, vp, vp, ci]
        _libs[path] = L
    return _libs[path]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class RefLinear:
    """The reference SplitManifoldLinear behind its C-ABI."""

    def __init__(self, codebook, codes, scales=None, bias=None, csr=None, path=LIB_SCALAR):
        self.L = lib(path)
        cb = np.ascontiguousarray(codebook, np.float32)
        self.codes = np.ascontiguousarray(codes, np.uint8)
        self.M, g = self.codes.shape
        self.D = cb.shape[1]
        self.K = g * self.D
        sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
        bs = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.h = self.L.ojasx_create_linear(self.K, self.M, self.D, cb.shape[0], _p(cb),
                                            _p(self.codes), _p(sc), _p(bs))
        assert self.h
        if csr is not None:
            rp, cl, vl = (np.ascontiguousarray(csr[0], np.int32),
                          np.ascontiguousarray(csr[1], np.int32),
                          np.ascontiguousarray(csr[2], np.float32))
            assert self.L.ojasx_set_linear_outliers(self.h, vl.size, _p(rp), _p(cl), _p(vl)) == 0

    def forward(self, x, num_threads=1):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.K)
        y = np.zeros((x.shape[0], self.M), np.float32)
        rc = self.L.ojasx_linear_forward(self.h, _p(x), _p(y), x.shape[0], num_threads)
        assert rc == 0
        return y

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ojasx_destroy_linear(self.h)
            self.h = None


class RefMoE:
    def __init__(self, cb_in, cb_down, gu_codes, gu_scales, dn_codes, dn_scales, top_k=10,
                 path=LIB_SCALAR):
        self.L = lib(path)
        self.arrs = [np.ascontiguousarray(cb_in, np.float32),
                     np.ascontiguousarray(cb_down, np.float32),
                     np.ascontiguousarray(gu_codes, np.uint8),
                     np.ascontiguousarray(gu_scales, np.float32),
                     np.ascontiguousarray(dn_codes, np.uint8),
                     np.ascontiguousarray(dn_scales, np.float32)]
        e, two_i, g_in = self.arrs[2].shape
        self.H = self.arrs[4].shape[1]
        d = self.arrs[0].shape[1]
        self.h = self.L.ojasx_create_moe(e, self.H, two_i // 2, top_k, d,
                                         *[_p(a) for a in self.arrs])
        assert self.h

    def forward(self, x, idx, w, k_active=None, y_init=None):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        idx = np.ascontiguousarray(idx, np.int32).reshape(-1)
        w = np.ascontiguousarray(w, np.float32).reshape(-1)
        y = np.zeros(self.H, np.float32) if y_init is None else np.array(y_init, np.float32)
        k = idx.size if k_active is None else k_active
        assert self.L.ojasx_moe_forward(self.h, _p(x), _p(idx), _p(w), _p(y), k) == 0
        return y

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ojasx_destroy_moe(self.h)
            self.h = None


class RefKV:
    def __init__(self, num_heads, head_dim=128, max_seq_len=4096, block_dim=16, path=LIB_SCALAR):
        self.L = lib(path)
        self.head_dim = head_dim
        self.h = self.L.ojasx_create_kv_cache(num_heads, head_dim, max_seq_len, block_dim)
        assert self.h

    def append(self, head, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        return self.L.ojasx_kv_cache_append(self.h, head, _p(k), _p(v))

    def attention(self, head, q, scale_factor=-1.0, out_init=None):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.head_dim, np.float32) if out_init is None else np.array(out_init, np.float32)
        rc = self.L.ojasx_kv_cache_attention(self.h, head, _p(q), _p(out), scale_factor)
        return rc, out

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ojasx_destroy_kv_cache(self.h)
            self.h = None

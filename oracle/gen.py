"""Seeded synthetic inputs (the package's synthetic module) and the
reference tests' formula-determined known-answer setups.

TEST INFRASTRUCTURE ONLY.  The generators are the package's
``synthetic`` module, re-exported so tests and bench.py feed identical bytes
to the GPU path and to the CPU oracle.
"""
import os
import sys

import numpy as np

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import __graft_entry__  # noqa: E402

_syn = __import__(__graft_entry__.load_package().__name__ + ".synthetic", fromlist=["*"])
OUTLIER_DENSITY = _syn.OUTLIER_DENSITY
SIGMA = _syn.SIGMA
rng = _syn.rng
csr_outliers = _syn.csr_outliers
linear = _syn.linear
moe = _syn.moe
kv = _syn.kv
kv_logical = _syn.kv_logical


def reference_t2():
    """Fully formula-determined setup of the reference's linear test
    (NAT/tests/test_native_lut.cpp:30-93): 256 -> 128, D = 16."""
    in_f, out_f, D, Kcb = 256, 128, 16, 256
    G = in_f // D
    k = np.arange(Kcb, dtype=np.float32)[:, None]
    d = np.arange(D, dtype=np.float32)[None, :]
    codebook = (((k % 17) - 8) * np.float32(0.1) + d * np.float32(0.01)).astype(np.float32)
    m = np.arange(out_f)[:, None]
    g = np.arange(G)[None, :]
    codes = ((m * 3 + g * 7) % 256).astype(np.uint8)
    scales = (1.0 + 0.01 * np.arange(out_f, dtype=np.float32)).astype(np.float32)
    x = np.sin(np.arange(in_f, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    return dict(codebook=codebook, codes=codes, scales=scales, x=x)


def reference_t3():
    """CSR known answer (NAT/tests/test_native_lut.cpp:95-126): 64 -> 32, zero
    codebook, two outliers per row (+10 at col 2m mod 64, -5 at 2m+1 mod 64),
    x = 1, so y == 5 exactly."""
    in_f, out_f = 64, 32
    row_ptrs = (np.arange(out_f + 1) * 2).astype(np.int32)
    cols = np.empty(2 * out_f, np.int32)
    cols[0::2] = (np.arange(out_f) * 2) % in_f
    cols[1::2] = (np.arange(out_f) * 2 + 1) % in_f
    vals = np.tile(np.array([10.0, -5.0], np.float32), out_f)
    return dict(codebook=np.zeros((256, 16), np.float32),
                codes=np.zeros((out_f, in_f // 16), np.uint8),
                scales=np.ones(out_f, np.float32), csr=(row_ptrs, cols, vals),
                x=np.ones(in_f, np.float32))


def reference_t6():
    """MoE setup of NAT/tests/test_native_lut.cpp:186-248 (512 experts, H=256,
    I=64, top-10 with fixed indices and weights, x = 0.5)."""
    E, H, I, D = 512, 256, 64, 16
    k = np.arange(256, dtype=np.float32)[:, None]
    cb_in = np.repeat(np.float32(0.05) * ((k % 11) - 5), D, axis=1).astype(np.float32)
    cb_down = np.repeat(np.float32(0.03) * ((k % 7) - 3), D, axis=1).astype(np.float32)
    n_gu = E * 2 * I * (H // D)
    n_dn = E * H * (I // D)
    gu = (np.arange(n_gu) % 256).astype(np.uint8).reshape(E, 2 * I, H // D)
    dn = ((np.arange(n_dn, dtype=np.int64) * 3) % 256).astype(np.uint8).reshape(E, H, I // D)
    idx = np.array([4, 12, 57, 103, 199, 255, 340, 412, 480, 511], np.int32)
    w = np.array([0.25, 0.20, 0.15, 0.10, 0.08, 0.07, 0.05, 0.04, 0.03, 0.03], np.float32)
    return dict(cb_in=cb_in, cb_down=cb_down, gu_codes=gu, gu_scales=np.ones((E, 2 * I), np.float32),
                dn_codes=dn, dn_scales=np.ones((E, H), np.float32), x=np.full(H, 0.5, np.float32),
                idx=idx, w=w)

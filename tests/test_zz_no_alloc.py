"""The no-allocation KV decode (ojasx_kv_decode_paged_device_noalloc, partials
in the library's fixed per-GPU scratch) against the allocating entry point it
mirrors (ojasx_kv_decode_paged_device), through the C-ABI: bit-identical
outputs on two calls in a row, the second with a smaller context (the
scratch keeps the first call's partials), both within rel 1e-5 of the exact
fp64 attention; a request beyond the scratch is refused before any launch."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from oracle import gen, numpy_oracle as no

pytestmark = pytest.mark.gpu


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def run(pkg, fn, d, T, Hq, Hkv):
    import torch
    dev = torch.device("cuda:0")
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k])).to(dev)
         for k in ("q", "k_codes", "k_scales", "v_codes", "v_scales", "k_cb", "v_cb",
                   "block_table")}
    out = torch.full((Hq, 128), float("nan"), device=dev)
    rc = getattr(pkg.lib(), fn)(
        vp(t["q"]), vp(t["k_codes"]), vp(t["k_scales"]), vp(t["v_codes"]), vp(t["v_scales"]),
        vp(t["k_cb"]), vp(t["v_cb"]), vp(t["block_table"]), T, d["page"], Hq, Hkv, 128, 16,
        -1.0, vp(out), None)
    torch.cuda.synchronize()
    return rc, out.cpu().numpy()


def test_noalloc_matches_allocating_decode(pkg, dev):
    for T, seed in ((32768, 5), (1000, 6)):     # wide path (32 chunks), then short (16)
        print(f"no-alloc KV decode T={T} Hq=32 Hkv=8 seed={seed}", flush=True)
        d = gen.kv(H_kv=8, H_q=32, T=T, seed=seed, shuffle_pages=True)
        rc, got = run(pkg, "ojasx_kv_decode_paged_device_noalloc", d, T, 32, 8)
        assert rc == 0, pkg.lib().ojasx_get_last_error()
        rc, want = run(pkg, "ojasx_kv_decode_paged_device", d, T, 32, 8)
        assert rc == 0, pkg.lib().ojasx_get_last_error()
        assert np.array_equal(got, want), T
        for j in (0, 13, 31):
            h = j // 4
            kc, ks, vc, vs = gen.kv_logical(d, h)
            Kd = d["k_cb"][h][kc.astype(np.int64)].reshape(T, -1) * ks[:, None].astype(np.float64)
            Vd = d["v_cb"][h][vc.astype(np.int64)].reshape(T, -1) * vs[:, None].astype(np.float64)
            assert rel_err(got[j], no.full_softmax_attention(d["q"][j], Kd, Vd)) < 1e-5, (T, j)


def test_noalloc_refuses_beyond_scratch(pkg, dev):
    # 160 query heads x 64 chunks x 128 x 4 B = 5 MiB of partials > 4 MiB
    d = gen.kv(H_kv=40, H_q=160, T=4096, seed=7)
    rc, out = run(pkg, "ojasx_kv_decode_paged_device_noalloc", d, 4096, 160, 40)
    assert rc == -3
    assert b"no-allocation scratch" in pkg.lib().ojasx_get_last_error()
    assert np.isnan(out).all()

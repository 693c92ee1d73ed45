"""Writes the golden fixtures of this directory from the reference engine.

The reference's C++ engine (split_manifold_lut_experiment/native/src/
ojasx_lut_{cpu,kv_cache,c_api}.cpp) is compiled from its own sources by
``make -C oracle ref`` into ``oracle/_ref/libojasx_lut_ref.so`` and called
through its C-ABI; nothing of the reference is stored here except the
input/output vectors.  Inputs come from the repo's seeded generators
(``oracle.gen``) or from the formula-determined setups of the reference's
own tests (NAT/tests/test_native_lut.cpp T2, T3, T6), which are regenerated
from their formulas at test time, so only their outputs are stored.

Run from the repository root:  python tests/golden/make_golden.py [block_sizes]
(``block_sizes`` writes only the block-size fixtures.)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import gen, ref  # noqa: E402


def save(name, **arrs):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **{k: v for k, v in arrs.items() if v is not None})
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def linear_case(name, M, K, B, D, Kcb, seed, density, bias):
    d = gen.linear(M, K, B=B, D=D, Kcb=Kcb, seed=seed, scales="u", bias=bias, density=density)
    R = ref.RefLinear(d["codebook"], d["codes"], d["scales"], d["bias"], d["csr"])
    y = R.forward(d["x"])
    rp, cl, vl = d["csr"]
    save(name, codebook=d["codebook"], codes=d["codes"], scales=d["scales"], bias=d["bias"],
         row_ptrs=rp, cols=cl, vals=vl, x=d["x"], y=y)


def moe_case(name, E, H, I, D, seed, idx, w):
    m = gen.moe(E=E, H=H, I=I, T=1, D=D, seed=seed, scales="u")
    idx = np.array(idx, np.int32)
    w = np.array(w, np.float32)
    M = ref.RefMoE(m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"], m["dn_codes"],
                   m["dn_scales"], top_k=idx.size)
    y = M.forward(m["x"][0], idx, w)
    save(name, cb_in=m["cb_in"], cb_down=m["cb_down"], gu_codes=m["gu_codes"],
         gu_scales=m["gu_scales"], dn_codes=m["dn_codes"], dn_scales=m["dn_scales"],
         x=m["x"][0], idx=idx, w=w, y=y)


def block_size_cases():
    """Block sizes beyond the configured 16: wider than 32 and not dividing 32."""
    linear_case("linear_d64_k512_m72_b3", 72, 512, 3, 64, 256, 14, 0.02, True)
    linear_case("linear_d48_k480_m40_b2_cb100", 40, 480, 2, 48, 100, 15, 0.03, False)
    moe_case("moe_d24_e16_h96_i72", 16, 96, 72, 24, 22,
             [5, 11, 5, 0, 15, 99], [0.3, 0.2, 0.15, 0.15, 0.2, 0.5])
    moe_case("moe_d64_e8_h256_i128", 8, 256, 128, 64, 23, [7, 2, 4], [0.5, 0.3, 0.2])


def main(only=None):
    assert ref.available(), "build the reference engine first: make -C oracle ref"
    if only == "block_sizes":
        block_size_cases()
        return
    linear_case("linear_k256_m200_b3", 200, 256, 3, 16, 256, 11, 0.02, True)
    linear_case("linear_d8_k128_m96_b2_cb64", 96, 128, 2, 8, 64, 12, 0.03, False)
    linear_case("linear_k2560_m64_b1", 64, 2560, 1, 16, 256, 13, 0.0038, False)

    t2 = gen.reference_t2()
    y = ref.RefLinear(t2["codebook"], t2["codes"], t2["scales"]).forward(t2["x"])
    save("ref_t2_linear", y=y)
    t3 = gen.reference_t3()
    y = ref.RefLinear(t3["codebook"], t3["codes"], t3["scales"], csr=t3["csr"]).forward(t3["x"])
    save("ref_t3_csr", y=y)
    t6 = gen.reference_t6()
    M = ref.RefMoE(t6["cb_in"], t6["cb_down"], t6["gu_codes"], t6["gu_scales"], t6["dn_codes"],
                   t6["dn_scales"])
    save("ref_t6_moe", y=M.forward(t6["x"], t6["idx"], t6["w"]))

    m = gen.moe(E=32, H=128, I=64, T=1, seed=21, scales="u")
    idx = np.array([3, 31, 40, 7, -1, 12], np.int32)        # 40 and -1 are out of range
    w = np.array([0.3, 0.25, 0.2, 1e-9, 0.1, 0.15], np.float32)  # 1e-9 is skipped
    M = ref.RefMoE(m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"], m["dn_codes"],
                   m["dn_scales"], top_k=6)
    y = M.forward(m["x"][0], idx, w)
    save("moe_e32_h128_i64", cb_in=m["cb_in"], cb_down=m["cb_down"], gu_codes=m["gu_codes"],
         gu_scales=m["gu_scales"], dn_codes=m["dn_codes"], dn_scales=m["dn_scales"],
         x=m["x"][0], idx=idx, w=w, y=y)

    r = gen.rng(31)
    T, hd = 150, 128
    kv = ref.RefKV(2, hd, 64)                               # grows past max_seq_len
    K = r.normal(0.0, 1.0, size=(T, hd)).astype(np.float32)
    V = r.normal(0.0, 1.0, size=(T, hd)).astype(np.float32)
    K[5] = 0.0                                               # all-zero token: scale floor
    for t in range(T):
        assert kv.append(1, K[t], V[t]) == 0
    q = r.normal(0.0, 1.0, size=hd).astype(np.float32)
    rc, out = kv.attention(1, q)
    rc2, out_sf = kv.attention(1, q, 0.05)
    assert rc == 0 and rc2 == 0
    save("kv_ref_head_t150", K=K, V=V, q=q, out=out, out_sf005=out_sf)
    block_size_cases()


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else None)

"""Pins the CPU oracle (CPU only, no GPU).

Every oracle function is checked against at least one of: the golden
fixtures written by the reference engine compiled from its own sources
(tests/golden/), the reference's own known-answer setups
(NAT/tests/test_native_lut.cpp T2/T3/T6), closed forms and special cases,
float64 brute force, and -- where the reference tree was built here -- the
compiled reference itself on fresh seeded inputs.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err
from oracle import cpu, gen, numpy_oracle as no, ref


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


# ---------------------------------------------------------------- LUT build --

def test_lut_one_hot_is_codebook_column():
    """x = e_j gives LUT[g,k] = C[k, j mod D] for g = j // D and 0 elsewhere."""
    d = gen.linear(4, 64, seed=1)
    cb = d["codebook"]
    for j in (0, 5, 17, 63):
        x = np.zeros(64, np.float32)
        x[j] = 1.0
        lut = cpu.build_lut(x, cb)
        want = np.zeros_like(lut)
        want[j // 16] = cb[:, j % 16]
        assert np.array_equal(lut, want)


def test_lut_matches_fp64_dot():
    d = gen.linear(4, 2560, seed=2)
    lut = cpu.build_lut(d["x"][0], d["codebook"])
    want = no.engine_build_lut(d["x"][0], d["codebook"])
    assert rel_err(lut, want) < 1e-6


# ------------------------------------------------------------------- linear --

@pytest.mark.parametrize("name", ["linear_k256_m200_b3", "linear_d8_k128_m96_b2_cb64",
                                  "linear_k2560_m64_b1", "linear_d64_k512_m72_b3",
                                  "linear_d48_k480_m40_b2_cb100"])
def test_linear_golden_bit_exact(name):
    g = golden(name)
    y = cpu.linear_forward(g["x"], g["codebook"], g["codes"], g["scales"],
                           g["bias"] if "bias" in g else None, g["row_ptrs"], g["cols"], g["vals"])
    assert np.array_equal(y, g["y"])


def test_reference_t2_known_answer():
    """NAT/tests/test_native_lut.cpp:30-93: |y - manual unpack| < 1e-4."""
    t2 = gen.reference_t2()
    y = cpu.linear_forward(t2["x"], t2["codebook"], t2["codes"], t2["scales"])
    manual = no.linear_fp64(t2["x"], t2["codebook"], t2["codes"], t2["scales"])[0]
    assert np.abs(y - manual).max() < 1e-4
    assert np.array_equal(y, golden("ref_t2_linear")["y"][0])


def test_reference_t3_csr_exact():
    """NAT/tests/test_native_lut.cpp:95-126: zero manifold, +10 and -5 per row, x = 1."""
    t3 = gen.reference_t3()
    y = cpu.linear_forward(t3["x"], t3["codebook"], t3["codes"], t3["scales"], None, *t3["csr"])
    assert np.all(y == 5.0)
    assert np.array_equal(y, golden("ref_t3_csr")["y"][0])


def integer_case(seed, M=97, K=640, B=2):
    """Integer-valued codebook and x: every partial sum is an integer below
    2^24, so fp32 results are exact in any summation order."""
    r = gen.rng(seed)
    cb = r.integers(-8, 9, size=(256, 16)).astype(np.float32)
    codes = r.integers(0, 256, size=(M, K // 16)).astype(np.uint8)
    x = r.integers(-4, 5, size=(B, K)).astype(np.float32)
    rp, cl, vl = gen.csr_outliers(r, M, K, density=0.01)
    vl = np.round(vl * 50).astype(np.float32)               # integer outliers
    W = cb[codes.astype(np.int64)].reshape(M, K).astype(np.int64)
    rows = np.repeat(np.arange(M), np.diff(rp))
    np.add.at(W, (rows, cl), vl.astype(np.int64))
    y = x.astype(np.int64) @ W.T
    return dict(codebook=cb, codes=codes, x=x, csr=(rp, cl, vl), y=y.astype(np.float32))


def test_linear_integer_exact():
    c = integer_case(3)
    y = cpu.linear_forward(c["x"], c["codebook"], c["codes"], None, None, *c["csr"])
    assert np.array_equal(y, c["y"])


def test_linear_matches_fp64_dequantised_gemv():
    d = gen.linear(300, 2560, B=2, seed=4, scales="u", bias=True)
    y = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *d["csr"])
    y64 = no.linear_fp64(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], d["csr"])
    assert rel_err(y, y64) < 1e-5


def test_engine_forward_identity_fp64():
    """The PyTorch-engine restatement (COO outliers) equals x.W^T in fp64
    (SM/tests/test_split_manifold_lut.py:88-109 bound 1e-12)."""
    d = gen.linear(64, 512, B=4, seed=5, scales="u", bias=True, density=0.01)
    coo_i, coo_v = no.csr_to_coo(d["csr"])
    y = no.engine_forward(d["x"], d["codebook"], d["codes"], d["scales"], coo_i, coo_v, d["bias"])
    y64 = no.linear_fp64(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], d["csr"])
    assert np.abs(y - y64).max() < 1e-12


def test_checks_detect_planted_mistakes():
    """Plausible mistakes planted in a copy of the oracle's arithmetic (on the
    CPU) must each fail the comparison the GPU tests use."""
    d = gen.linear(128, 512, B=1, seed=6, scales="u", bias=True, density=0.01)
    y64 = no.linear_fp64(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], d["csr"])
    lut = no.engine_build_lut(d["x"], d["codebook"])[0]
    codes = d["codes"].astype(np.int64)
    g = np.arange(codes.shape[1])
    rp, cl, vl = d["csr"]
    rows = np.repeat(np.arange(128), np.diff(rp))
    out = np.zeros(128)
    np.add.at(out, rows, vl * d["x"][0][cl])
    good = lut[g, codes].sum(1) * d["scales"] + d["bias"] + out
    assert rel_err(good, y64) < 1e-5
    planted = {
        "dropped last group": lut[g[:-1], codes[:, :-1]].sum(1) * d["scales"] + d["bias"] + out,
        "outliers scaled": (lut[g, codes].sum(1) + out) * d["scales"] + d["bias"],
        "code off by one": lut[g, (codes + 1) % 256].sum(1) * d["scales"] + d["bias"] + out,
        "outlier sign": lut[g, codes].sum(1) * d["scales"] + d["bias"] - out,
        "transposed codebook dot": (d["x"][0].reshape(-1, 16) @ d["codebook"][:16].T)[g % 32 % 16, codes % 16].sum(1),
    }
    for what, bad in planted.items():
        assert rel_err(bad, y64) > 1e-3, what


# ---------------------------------------------------------------------- MoE --

def test_moe_reference_t6():
    t6 = gen.reference_t6()
    y = cpu.moe_forward(t6["x"], t6["cb_in"], t6["cb_down"], t6["gu_codes"], t6["gu_scales"],
                        t6["dn_codes"], t6["dn_scales"], t6["idx"], t6["w"])
    assert np.array_equal(y, golden("ref_t6_moe")["y"])
    y64 = no.moe_fp64(t6["x"], t6["cb_in"], t6["cb_down"], t6["gu_codes"], t6["gu_scales"],
                      t6["dn_codes"], t6["dn_scales"], t6["idx"], t6["w"])
    assert rel_err(y, y64) < 1e-5


def test_moe_golden_skip_rules():
    g = golden("moe_e32_h128_i64")
    y = cpu.moe_forward(g["x"], g["cb_in"], g["cb_down"], g["gu_codes"], g["gu_scales"],
                        g["dn_codes"], g["dn_scales"], g["idx"], g["w"])
    assert np.array_equal(y, g["y"])
    y64 = no.moe_fp64(g["x"], g["cb_in"], g["cb_down"], g["gu_codes"], g["gu_scales"],
                      g["dn_codes"], g["dn_scales"], g["idx"], g["w"])
    assert rel_err(y, y64) < 1e-5


@pytest.mark.parametrize("name", ["moe_d24_e16_h96_i72", "moe_d64_e8_h256_i128"])
def test_moe_golden_block_sizes(name):
    """block_dim 24 (not dividing 32) and 64, written by the compiled reference."""
    g = golden(name)
    y = cpu.moe_forward(g["x"], g["cb_in"], g["cb_down"], g["gu_codes"], g["gu_scales"],
                        g["dn_codes"], g["dn_scales"], g["idx"], g["w"])
    assert np.array_equal(y, g["y"])
    y64 = no.moe_fp64(g["x"], g["cb_in"], g["cb_down"], g["gu_codes"], g["gu_scales"],
                      g["dn_codes"], g["dn_scales"], g["idx"], g["w"])
    assert rel_err(y, y64) < 1e-5


def test_moe_k_active_zero_leaves_output():
    g = golden("moe_e32_h128_i64")
    init = np.full(128, 7.0, np.float32)
    y = cpu.moe_forward(g["x"], g["cb_in"], g["cb_down"], g["gu_codes"], g["gu_scales"],
                        g["dn_codes"], g["dn_scales"], g["idx"], g["w"], k_active=0, y_init=init)
    assert np.array_equal(y, init)


# ------------------------------------------------------------------- router --

def test_router_topk_matches_stable_argsort():
    m = gen.moe(E=512, H=16, I=16, T=16, seed=8)
    lg = m["logits"].copy()
    lg[0, 10] = lg[0, 20] = lg[0, 30] = 9.0                   # three-way tie at the top
    idx, w = cpu.router_topk(lg, 10)
    i2, w2 = no.router_topk(lg, 10)
    assert np.array_equal(idx, i2)
    assert list(idx[0, :3]) == [10, 20, 30]
    assert rel_err(w, w2) < 1e-6
    idx_r, w_r = cpu.router_topk(lg, 10, renorm=True)
    assert np.array_equal(idx_r, i2)
    assert np.allclose(w_r.sum(1), 1.0, atol=1e-6)


# ----------------------------------------------------------------------- KV --

def round_half_away(v):
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_kv_quantiser_closed_form():
    r = gen.rng(9)
    for t in range(50):
        k = r.normal(0, 2, size=128).astype(np.float32)
        if t == 0:
            k[:] = 0.0
        if t == 1:
            k[16] = 0.5 * (np.abs(k).max() / np.float32(127.0))   # an exact half step
        codes, s = cpu.kv_quantize_token(k)
        s_want = np.float32(max(np.float32(1e-8), np.abs(k).max())) / np.float32(127.0)
        assert s == s_want
        q = np.clip(round_half_away((k[::16] / s_want).astype(np.float32)), -128, 127) + 128
        assert np.array_equal(codes, q.astype(np.uint8))


def test_paged_int8_quantiser_known_answer():
    """long_context.py:234-240: scale = amax/127 kept as float16, codes rounded
    half to even (torch.round) and clamped to +-127."""
    t = np.array([[127.0, 63.5, -63.5, 0.5, 1.5, -2.5, 2.5, 0.0],
                  [1.0, -0.25, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                  [0.0] * 8], np.float32)
    q, s = no.paged_quantize_int8(t)
    assert q.dtype == np.int8 and s.dtype == np.float16
    assert q[0].tolist() == [127, 64, -64, 0, 2, -2, 2, 0]   # half away would give 1, -3, 3
    assert s[0, 0] == np.float16(1.0)
    assert s[1, 0] == np.float16(np.float32(1.0) / np.float32(127.0))
    assert q[1].tolist() == [127, -32, 0, 0, 0, 0, 0, 0]     # -31.75 -> -32
    assert not q[2].any() and s[2, 0] == np.float16(np.float32(1e-8) / np.float32(127.0))


def test_kv_golden_end_to_end():
    g = golden("kv_ref_head_t150")
    kc, ks, vc, vs = [], [], [], []
    for t in range(g["K"].shape[0]):
        c, s = cpu.kv_quantize_token(g["K"][t])
        kc.append(c)
        ks.append(s)
        c, s = cpu.kv_quantize_token(g["V"][t])
        vc.append(c)
        vs.append(s)
    kc, ks, vc, vs = map(np.array, (kc, ks, vc, vs))
    assert np.array_equal(cpu.kv_attention_ref(g["q"], kc, ks, vc, vs), g["out"])
    assert np.array_equal(cpu.kv_attention_ref(g["q"], kc, ks, vc, vs, 0.05), g["out_sf005"])
    cb = np.zeros((256, 16), np.float32)
    cb[:, 0] = np.arange(256) - 128
    assert np.array_equal(cpu.kv_attention_cb(g["q"], cb, cb, kc, ks, vc, vs), g["out"])


def test_kv_codebook_matches_fp64_full_softmax():
    d = gen.kv(H_kv=1, H_q=1, T=777, seed=10)
    kc, ks, vc, vs = gen.kv_logical(d, 0)
    out = cpu.kv_attention_cb(d["q"][0], d["k_cb"][0], d["v_cb"][0], kc, ks, vc, vs)
    Kd = d["k_cb"][0][kc.astype(np.int64)].reshape(777, -1) * ks[:, None].astype(np.float64)
    Vd = d["v_cb"][0][vc.astype(np.int64)].reshape(777, -1) * vs[:, None].astype(np.float64)
    want = no.full_softmax_attention(d["q"][0], Kd, Vd)
    assert rel_err(out, want) < 1e-5
    online = no.code_domain_kv_decode(d["q"][:1], 0, d["k_cb"][0], d["v_cb"][0], kc, ks, vc, vs)
    assert np.abs(online[0] - want).max() < 1e-12


# -------------------------------------------------------- numpy restatements --

@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_pack_unpack_roundtrip(bits):
    r = gen.rng(bits)
    codes = r.integers(0, 1 << bits, size=1001)
    packed = no.pack_codes(codes, bits)
    assert packed.size == (1001 * bits + 7) // 8
    assert np.array_equal(no.unpack_codes(packed, bits, 1001), codes)
    if bits == 2:   # little-endian: the first code sits in the low bits
        assert no.pack_codes(np.array([1, 2, 3, 0]), 2)[0] == 1 | (2 << 2) | (3 << 4)


@pytest.mark.parametrize("block,bits,stages", [(16, 8, 1), (8, 4, 2), (24, 2, 3)])
def test_subspace_lut_gemm_equals_dense(block, bits, stages):
    """math_engine.py:136-208 equals x.W^T of the summed stage codebooks
    (T/test_m10_compression_aware_math.py:244-312), with K padding."""
    r = gen.rng(block * bits + stages)
    rows, cols = 40, 100
    G = (cols + block - 1) // block
    cbs = r.normal(size=(stages, 1 << bits, block))
    codes = r.integers(0, 1 << bits, size=(stages, rows, G))
    packed = [no.pack_codes(codes[s], bits) for s in range(stages)]
    scales = r.uniform(0.5, 1.5, size=rows)
    bias = r.normal(size=rows)
    x = r.normal(size=(3, cols))
    y = no.subspace_lut_rvq_gemm(x, cbs, packed, bits, rows, cols, block, scales, bias)
    W = sum(cbs[s][codes[s]].reshape(rows, G * block) for s in range(stages))[:, :cols]
    want = x @ (W * scales[:, None]).T + bias
    assert np.abs(y - want).max() < 1e-10


def test_online_softmax_matches_full():
    r = gen.rng(12)
    q = r.normal(size=64)
    K = r.normal(size=(1000, 64))
    V = r.normal(size=(1000, 64))
    tiles = [slice(i, i + 97) for i in range(0, 1000, 97)]
    o = no.online_softmax_attention(q, [K[s] for s in tiles], [V[s] for s in tiles])
    assert np.abs(o - no.full_softmax_attention(q, K, V)).max() < 1e-12


def test_block_attention_stream_matches_masked_full():
    """The batched stream restatement against the full-matrix fp64 attention
    of the reference's M13 tests: causal GQA with a query offset, uneven
    tiles, an empty tile, and rows whose keys are all hidden (output 0)."""
    r = gen.rng(13)
    B, Hq, Hkv, Sq, D, S = 2, 8, 2, 5, 16, 300
    q = r.normal(size=(B, Hq, Sq, D))
    K = r.normal(size=(B, Hkv, S, D))
    V = r.normal(size=(B, Hkv, S, D))
    cuts = [0, 37, 37, 190, 256, 300]
    tiles = [(K[:, :, a:b], V[:, :, a:b]) for a, b in zip(cuts, cuts[1:])]
    for causal, qsp in ((True, 150), (False, 0), (True, -3)):
        o, lse, n, nt = no.block_attention_stream(q, tiles, causal, qsp)
        want = no.masked_full_attention(q, K, V, causal, qsp)
        assert np.abs(o - want).max() < 1e-12, (causal, qsp)
        assert n == S and nt == 4
    assert np.all(o[:, :, :3] == 0) and np.isinf(lse[:, :, :3]).all()   # qsp -3: rows 0..2 see nothing


def test_block_attention_stream_closed_forms():
    """Head mapping h -> h // (Hq / Hkv) (kv head j holds V = j + 1 everywhere:
    every output of query head h is h // 4 + 1), a single visible key (out =
    its V row), and n identical tiles (same output, lse + log n)."""
    r = gen.rng(14)
    B, Hq, Hkv, D = 1, 8, 2, 8
    q = r.normal(size=(B, Hq, 3, D))
    K = r.normal(size=(B, Hkv, 40, D))
    V = np.ones((B, Hkv, 40, D)) * np.arange(1, Hkv + 1).reshape(1, Hkv, 1, 1)
    o, _, _, _ = no.block_attention_stream(q, [(K, V)], causal=False)
    assert np.allclose(o, (np.arange(Hq) // 4 + 1).reshape(1, Hq, 1, 1), atol=1e-14)
    V2 = r.normal(size=(B, Hkv, 40, D))
    o, _, _, _ = no.block_attention_stream(q, [(K, V2)], causal=True, query_start_pos=0)
    assert np.array_equal(o[:, :, 0], np.repeat(V2[:, :, 0], 4, axis=1))
    o1, l1, _, _ = no.block_attention_stream(q, [(K, V2)], causal=False)
    o5, l5, n5, _ = no.block_attention_stream(q, [(K, V2)] * 5, causal=False)
    assert n5 == 200
    assert np.abs(o5 - o1).max() < 1e-13 and np.abs(l5 - (l1 + np.log(5))).max() < 1e-12


# ------------------------------------------- the compiled reference (optional) --

needs_ref = pytest.mark.skipif(not ref.available(), reason="reference engine not built here")


@needs_ref
@pytest.mark.parametrize("seed", [100, 101])
def test_oracle_equals_compiled_reference(seed):
    d = gen.linear(777, 2560, B=3, seed=seed, scales="u", bias=True)
    y = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *d["csr"])
    yr = ref.RefLinear(d["codebook"], d["codes"], d["scales"], d["bias"], d["csr"]).forward(d["x"])
    assert np.array_equal(y, yr)
    m = gen.moe(E=64, H=512, I=128, T=2, seed=seed, scales="u")
    idx, w = cpu.router_topk(m["logits"], 10)
    M = ref.RefMoE(m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"], m["dn_codes"],
                   m["dn_scales"])
    for t in range(2):
        y = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                            m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert np.array_equal(y, M.forward(m["x"][t], idx[t], w[t]))


def test_bf16_fixture_inputs_regenerate():
    """The bf16 reference-module fixture stores a digest of its inputs, not the
    inputs: the seeded generator must still produce them byte for byte."""
    import sys
    sys.path.insert(0, GOLDEN)
    from make_bf16_golden import bf16_inputs, digest
    g = np.load(os.path.join(GOLDEN, "engine_bf16_2560x6912.npz"))
    assert digest(bf16_inputs()) == str(g["inputs_sha256"])

"""GPU parity of the code-domain KV path (K5 decode, reference quantiser)
against the CPU oracle, through the C-ABI.  Bar: rel <= 1e-5 on the
attention output; quantiser codes bit-exact (checked through the reference
C-ABI's end-to-end output and directly below)."""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err
from oracle import cpu, gen, numpy_oracle as no

pytestmark = pytest.mark.gpu


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def test_host_api_golden(pkg):
    g = np.load(os.path.join(GOLDEN, "kv_ref_head_t150.npz"))
    kv = pkg.native.NativeKVCache(2, 128, 64)          # grows past 64 tokens
    for t in range(g["K"].shape[0]):
        kv.append(1, g["K"][t], g["V"][t])
    assert rel_err(kv.attention(1, g["q"]), g["out"]) < 1e-5
    assert rel_err(kv.attention(1, g["q"], 0.05), g["out_sf005"]) < 1e-5


def test_host_api_errors_and_empty(pkg):
    L = pkg.lib()
    kv = pkg.native.NativeKVCache(2, 128, 16)
    q = np.ones(128, np.float32)
    out = np.full(128, 3.0, np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert L.ojasx_kv_cache_attention(kv._handle, 0, p(q), p(out), -1.0) == 0   # empty head
    assert np.all(out == 3.0)
    assert L.ojasx_kv_cache_attention(kv._handle, 2, p(q), p(out), -1.0) == -2
    assert L.ojasx_kv_cache_append(kv._handle, -1, p(q), p(q)) == -2
    assert L.ojasx_kv_cache_append(kv._handle, 0, None, p(q)) == -1


def test_quantiser_codes_bit_exact(pkg):
    """One token per head through the reference C-ABI; with a one-hot query on
    coordinate 16g the attention output over a single token recovers
    (code_v - 128) * vs exactly, and both codes match the oracle quantiser."""
    r = gen.rng(40)
    kv = pkg.native.NativeKVCache(1, 128, 4)
    k = r.normal(0, 3, size=128).astype(np.float32)
    v = r.normal(0, 3, size=128).astype(np.float32)
    v[32] = 0.5 * np.abs(v).max() / np.float32(127.0) * 3   # an exact half step
    kv.append(0, k, v)
    out = kv.attention(0, np.ones(128, np.float32))
    vc, vs = cpu.kv_quantize_token(v)
    want = np.zeros(128, np.float32)
    want[::16] = (vc.astype(np.float32) - 128.0) * vs
    assert np.array_equal(out, want)


def decode(pkg, d, T, Hq, Hkv, sf=-1.0, hd=128, D=16):
    import torch
    dev = torch.device("cuda:0")
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k])).to(dev)
         for k in ("q", "k_codes", "k_scales", "v_codes", "v_scales", "k_cb", "v_cb",
                   "block_table")}
    out = torch.empty(Hq, hd, device=dev)
    rc = pkg.lib().ojasx_kv_decode_paged_device(
        vp(t["q"]), vp(t["k_codes"]), vp(t["k_scales"]), vp(t["v_codes"]), vp(t["v_scales"]),
        vp(t["k_cb"]), vp(t["v_cb"]), vp(t["block_table"]), T, d["page"], Hq, Hkv, hd, D, sf,
        vp(out), None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("T,shuffle", [(2048, False), (32768, True), (1000, True), (1, False),
                                       (17, True)])
def test_paged_decode_gqa(pkg, dev, T, shuffle):
    """rel <= 1e-5 against the exact (fp64) attention of the same codes.  The
    oracle -- the reference's sequential fp32 two-pass softmax -- itself
    drifts up to ~1e-5 from the exact value at T = 32768 (its 32768-term fp32
    sums), so against the oracle the bar is 1e-5 plus the oracle's own error."""
    d = gen.kv(H_kv=8, H_q=32, T=T, seed=T, shuffle_pages=shuffle)
    out = decode(pkg, d, T, 32, 8)
    worst = dict(exact=0.0, oracle=0.0, oracle_vs_exact=0.0)
    for j in range(32):
        h = j // 4
        kc, ks, vc, vs = gen.kv_logical(d, h)
        want = cpu.kv_attention_cb(d["q"][j], d["k_cb"][h], d["v_cb"][h], kc, ks, vc, vs)
        Kd = d["k_cb"][h][kc.astype(np.int64)].reshape(T, -1) * ks[:, None].astype(np.float64)
        Vd = d["v_cb"][h][vc.astype(np.int64)].reshape(T, -1) * vs[:, None].astype(np.float64)
        exact = no.full_softmax_attention(d["q"][j], Kd, Vd)
        e_exact, e_orc, e_oe = rel_err(out[j], exact), rel_err(out[j], want), rel_err(want, exact)
        for k, v in (("exact", e_exact), ("oracle", e_orc), ("oracle_vs_exact", e_oe)):
            worst[k] = max(worst[k], v)
        assert e_exact < 1e-5, j
        assert e_orc < 1e-5 + e_oe, j
    print(f"KV decode T={T}: worst rel err vs exact fp64 {worst['exact']:.3e}, vs the oracle "
          f"{worst['oracle']:.3e} (bar 1e-5 + the oracle's own {worst['oracle_vs_exact']:.3e})",
          flush=True)


def test_reference_codebook_special_case(pkg, dev):
    """C[c] = (c-128) e_0 reproduces the reference's scalar decode."""
    d = gen.kv(H_kv=2, H_q=2, T=300, seed=3)
    cb = np.zeros((2, 256, 16), np.float32)
    cb[:, :, 0] = np.arange(256) - 128
    d["k_cb"] = cb
    d["v_cb"] = cb
    out = decode(pkg, d, 300, 2, 2, sf=0.02)
    for j in range(2):
        kc, ks, vc, vs = gen.kv_logical(d, j)
        want = cpu.kv_attention_ref(d["q"][j], kc, ks, vc, vs, 0.02)
        assert rel_err(out[j], want) < 1e-5


def check_all_heads(d, out, T, Hq, Hkv):
    R = Hq // Hkv
    for j in range(Hq):
        h = j // R
        kc, ks, vc, vs = gen.kv_logical(d, h)
        Kd = d["k_cb"][h][kc.astype(np.int64)].reshape(T, -1) * ks[:, None].astype(np.float64)
        Vd = d["v_cb"][h][vc.astype(np.int64)].reshape(T, -1) * vs[:, None].astype(np.float64)
        exact = no.full_softmax_attention(d["q"][j], Kd, Vd)
        assert rel_err(out[j], exact) < 1e-5, j


@pytest.mark.parametrize("T,Hq,Hkv", [(3000, 16, 2),    # GQA 8: two workgroups of 4 heads (short path)
                                      (9000, 16, 2),    # GQA 8, long-context path
                                      (5000, 4, 4),     # no GQA, long-context path
                                      (64, 3, 1)])      # 3 query heads, one full chunk
def test_paged_decode_gqa_ratios(pkg, dev, T, Hq, Hkv):
    d = gen.kv(H_kv=Hkv, H_q=Hq, T=T, seed=T + Hq, shuffle_pages=True)
    out = decode(pkg, d, T, Hq, Hkv)
    check_all_heads(d, out, T, Hq, Hkv)


def test_paged_decode_runtime_shape(pkg, dev):
    """head_dim 64 with block 8 (8 groups): the runtime-shape kernel."""
    T, Hq, Hkv = 700, 4, 2
    d = gen.kv(H_kv=Hkv, H_q=Hq, T=T, head_dim=64, D=8, seed=21, shuffle_pages=True)
    out = decode(pkg, d, T, Hq, Hkv, hd=64, D=8)
    check_all_heads(d, out, T, Hq, Hkv)


def test_paged_decode_unaligned_query(pkg, dev):
    """q not 16-byte aligned takes the runtime-shape kernel."""
    import torch
    T, Hq, Hkv = 1500, 8, 2
    d = gen.kv(H_kv=Hkv, H_q=Hq, T=T, seed=22, shuffle_pages=True)
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k])).to(dev)
         for k in ("k_codes", "k_scales", "v_codes", "v_scales", "k_cb", "v_cb", "block_table")}
    qbuf = torch.empty(Hq * 128 + 1, device=dev)
    qt = qbuf[1:].view(Hq, 128)
    qt.copy_(torch.from_numpy(d["q"]).to(dev))
    out = torch.empty(Hq, 128, device=dev)
    rc = pkg.lib().ojasx_kv_decode_paged_device(
        vp(qt), vp(t["k_codes"]), vp(t["k_scales"]), vp(t["v_codes"]), vp(t["v_scales"]),
        vp(t["k_cb"]), vp(t["v_cb"]), vp(t["block_table"]), T, d["page"], Hq, Hkv, 128, 16, -1.0,
        vp(out), None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    check_all_heads(d, out.cpu().numpy(), T, Hq, Hkv)


def decode_device_len(pkg, t, d, seq_dev, Tmax, Hq, Hkv, tpl, out, stream=None):
    rc = pkg.lib().ojasx_kv_decode_paged_device_len(
        vp(t["q"]), vp(t["k_codes"]), vp(t["k_scales"]), vp(t["v_codes"]), vp(t["v_scales"]),
        vp(t["k_cb"]), vp(t["v_cb"]), vp(t["block_table"]), vp(seq_dev), Tmax, d["page"], Hq, Hkv,
        128, 16, -1.0, tpl, vp(out), stream)
    assert rc == 0, pkg.lib().ojasx_get_last_error()


def device_tensors(d, dev):
    import torch
    return {k: torch.from_numpy(np.ascontiguousarray(d[k])).to(dev)
            for k in ("q", "k_codes", "k_scales", "v_codes", "v_scales", "k_cb", "v_cb",
                      "block_table")}


def check_prefix(d, out, T, Hq=32, Hkv=8):
    """rel <= 1e-5 against the exact fp64 attention over the first T tokens,
    and against the oracle within 1e-5 plus the oracle's own fp32 error."""
    R = Hq // Hkv
    for j in range(Hq):
        h = j // R
        kc, ks, vc, vs = (a[:T] for a in gen.kv_logical(d, h))
        want = cpu.kv_attention_cb(d["q"][j], d["k_cb"][h], d["v_cb"][h], kc, ks, vc, vs)
        Kd = d["k_cb"][h][kc.astype(np.int64)].reshape(T, -1) * ks[:, None].astype(np.float64)
        Vd = d["v_cb"][h][vc.astype(np.int64)].reshape(T, -1) * vs[:, None].astype(np.float64)
        exact = no.full_softmax_attention(d["q"][j], Kd, Vd)
        assert rel_err(out[j], exact) < 1e-5, (T, j)
        assert rel_err(out[j], want) < 1e-5 + rel_err(want, exact), (T, j)


@pytest.mark.parametrize("T,Tmax,tpl", [(2048, 2048, 1), (3000, 4224, 2), (4100, 4224, 4),
                                        (1, 300, 2), (130, 4224, 0), (64, 64, 1), (4224, 4224, 0)])
def test_paged_decode_device_length(pkg, dev, T, Tmax, tpl):
    """Context length read on the device: chunks of 64, 128 or 256 tokens,
    the launch sized for Tmax and the chunks past T idle; equal to the oracle
    over the first T tokens."""
    import torch
    d = gen.kv(H_kv=8, H_q=32, T=Tmax, seed=T + Tmax, shuffle_pages=True)
    t = device_tensors(d, dev)
    seq = torch.tensor([T], dtype=torch.int32, device=dev)
    out = torch.empty(32, 128, device=dev)
    decode_device_len(pkg, t, d, seq, Tmax, 32, 8, tpl, out)
    torch.cuda.synchronize()
    check_prefix(d, out.cpu().numpy(), T)


def test_paged_decode_device_length_empty_and_errors(pkg, dev):
    import torch
    d = gen.kv(H_kv=8, H_q=32, T=300, seed=2)
    t = device_tensors(d, dev)
    out = torch.full((32, 128), 7.0, device=dev)
    seq = torch.zeros(1, dtype=torch.int32, device=dev)
    decode_device_len(pkg, t, d, seq, 300, 32, 8, 1, out)
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
    L = pkg.lib()
    rc = L.ojasx_kv_decode_paged_device_len(
        vp(t["q"]), vp(t["k_codes"]), vp(t["k_scales"]), vp(t["v_codes"]), vp(t["v_scales"]),
        vp(t["k_cb"]), vp(t["v_cb"]), vp(t["block_table"]), vp(seq), 300, 16, 32, 8, 128, 16,
        -1.0, 3, vp(out), None)
    assert rc == -3


def test_paged_decode_device_length_graph_replay(pkg, dev):
    """One captured HIP graph replayed as the device-side length grows: each
    replay equals the eager call at that length, bit for bit, and the oracle."""
    import torch
    Tmax = 4224
    d = gen.kv(H_kv=8, H_q=32, T=Tmax, seed=77, shuffle_pages=True)
    t = device_tensors(d, dev)
    seq = torch.tensor([100], dtype=torch.int32, device=dev)
    out = torch.empty(32, 128, device=dev)
    eager = torch.empty(32, 128, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        decode_device_len(pkg, t, d, seq, Tmax, 32, 8, 0, eager,
                          ctypes.c_void_p(s.cuda_stream))       # workspace before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        decode_device_len(pkg, t, d, seq, Tmax, 32, 8, 0, out,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for T in (100, 1000, 2500, 4224, 64):
        seq.fill_(T)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            decode_device_len(pkg, t, d, seq, Tmax, 32, 8, 0, eager, ctypes.c_void_p(s.cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(out, eager), T
        check_prefix(d, out.cpu().numpy(), T)

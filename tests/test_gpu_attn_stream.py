"""GPU parity of OnlineSoftmaxBlockAttention (ojasx_24x96/long_context.py:47-209)
through the streamed-attention C-ABI: the reference's M13 cases against the
fp64 full-matrix attention (its bar, max |diff| < 1e-5) and against the fp64
stream oracle (fp32 output within 1e-6 relative, fp64 output within 1e-12),
the int8 paged cache read in place against its dequantised pages, the report
fields, and the size-independent invariant of n identical tiles."""
import math

import numpy as np
import pytest

from conftest import rel_err
from oracle import numpy_oracle as no

pytestmark = pytest.mark.gpu


def randn(torch, *shape, seed, dtype=None):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g)
    return t if dtype is None else t.to(dtype)


def check(out, q, K, V, causal, qsp, bar_oracle=1e-6):
    """out against the stream oracle and the masked full attention (fp64)."""
    qn, Kn, Vn = (t.double().cpu().numpy() for t in (q, K, V))
    want = no.masked_full_attention(qn, Kn, Vn, causal, qsp)
    got = out.double().cpu().numpy()
    print(f"max |diff| vs full fp64 {np.abs(got - want).max():.3e}, rel {rel_err(got, want):.3e}")
    assert np.abs(got - want).max() < 1e-5
    assert rel_err(got, want) < bar_oracle


@pytest.mark.parametrize("causal", [True, False])
def test_mha_exact_parity(pkg, dev, causal):
    """T/test_m13_ultra_long_context_10m.py:110-133 (MHA, 256 tokens)."""
    import torch
    B, H, S, D = 2, 4, 256, 64
    q, k, v = (randn(torch, B, H, S, D, seed=s) for s in (1, 2, 3))
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(H, H, D, q_block_size=64,
                                                        kv_block_size=96, causal=causal)
    out = attn.forward(q.to(dev), k.to(dev), v.to(dev))
    assert out.dtype == torch.float32 and out.shape == (B, H, S, D)
    check(out, q, k, v, causal, 0)


def test_gqa_chunked_prefill_parity(pkg, dev):
    """GQA 8/2 with query_start_pos > 0 (the reference's :135-161)."""
    import torch
    B, Hq, Hkv, D, S_k, S_q, qsp = 1, 8, 2, 32, 500, 100, 400
    q = randn(torch, B, Hq, S_q, D, seed=4)
    k, v = randn(torch, B, Hkv, S_k, D, seed=5), randn(torch, B, Hkv, S_k, D, seed=6)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, q_block_size=32,
                                                        kv_block_size=64, causal=True)
    out = attn.forward(q.to(dev), k.to(dev), v.to(dev), query_start_pos=qsp)
    check(out, q, k, v, True, qsp)


def test_gqa_single_token_decode_parity(pkg, dev):
    """One query token at the end of a 1000-token context (:163-190)."""
    import torch
    B, Hq, Hkv, D, S = 2, 16, 4, 128, 1000
    q = randn(torch, B, Hq, 1, D, seed=7)
    k, v = randn(torch, B, Hkv, S, D, seed=8), randn(torch, B, Hkv, S, D, seed=9)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, causal=True)
    out = attn.forward(q.to(dev), k.to(dev), v.to(dev), query_start_pos=S - 1)
    check(out, q, k, v, True, S - 1)


@pytest.mark.parametrize("causal", [True, False])
def test_uneven_lengths_and_stream(pkg, dev, causal):
    """Lengths not divisible by the blocks (:192-222), and forward_stream over
    uneven tiles (one empty) with fp64 queries against the stream oracle."""
    import torch
    B, H, S_q, S_k, D = 1, 3, 77, 301, 16
    q = randn(torch, B, H, S_q, D, seed=10)
    k, v = randn(torch, B, H, S_k, D, seed=11), randn(torch, B, H, S_k, D, seed=12)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(H, H, D, q_block_size=20,
                                                        kv_block_size=45, causal=causal)
    out = attn.forward(q.to(dev), k.to(dev), v.to(dev), query_start_pos=S_k - S_q)
    check(out, q, k, v, causal, S_k - S_q)
    cuts = [0, 10, 10, 200, 301]
    qd = q.double().to(dev)
    tiles = [(k[:, :, a:b].double().to(dev), v[:, :, a:b].double().to(dev))
             for a, b in zip(cuts, cuts[1:])]
    out, rep = attn.forward_stream(qd, iter(tiles), query_start_pos=S_k - S_q)
    want, lse, n, nt = no.block_attention_stream(
        q.double().numpy(), [(a.cpu().numpy(), b.cpu().numpy()) for a, b in tiles], causal,
        S_k - S_q)
    assert out.dtype == torch.float64
    assert rel_err(out.cpu().numpy(), want) < 1e-12
    assert rep.query_tokens == S_q and rep.kv_tokens == n == S_k and rep.num_kv_blocks == nt == 3
    assert rep.peak_tile_elements == B * H * S_q * 190
    assert abs(rep.max_logsumexp - float(lse.max())) < 1e-10


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_half_tiles_and_queries(pkg, dev, dtype):
    """bf16 / fp16 query and tiles: values converted exactly to fp64, the fp64
    result rounded to the query's type through fp32 (torch's .to())."""
    import torch
    dt = getattr(torch, dtype)
    B, Hq, Hkv, S_q, S_k, D = 1, 4, 2, 3, 200, 64
    q = randn(torch, B, Hq, S_q, D, seed=13, dtype=dt)
    k, v = randn(torch, B, Hkv, S_k, D, seed=14, dtype=dt), randn(torch, B, Hkv, S_k, D, seed=15, dtype=dt)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, causal=True)
    out, _ = attn.forward_stream(q.to(dev), [(k[:, :, :120].to(dev), v[:, :, :120].to(dev)),
                                             (k[:, :, 120:].to(dev), v[:, :, 120:].to(dev))],
                                 query_start_pos=S_k - S_q)
    want, _, _, _ = no.block_attention_stream(q.double().numpy(), [(k.double().numpy(),
                                                                    v.double().numpy())],
                                              True, S_k - S_q)
    assert out.dtype == dt
    ref = torch.from_numpy(want).float().to(dt)           # fp64 -> fp32 -> half, as torch
    diff = (out.cpu().float() - ref.float()).abs().max().item()
    ulp = 2 ** -7 if dtype == "bfloat16" else 2 ** -10
    assert diff <= ulp * ref.float().abs().max().item()


def make_cache(pkg, dev, torch, B, H, D, page, pages, sink, chunks, seed):
    cache = pkg.long_context.PagedCompressedKVCache(page_size=page, max_resident_pages=pages,
                                                    sink_pages=sink)
    for i, n in enumerate(chunks):
        cache.append(randn(torch, B, H, n, D, seed=seed + 2 * i).to(dev) * (1 + i % 3),
                     randn(torch, B, H, n, D, seed=seed + 2 * i + 1).to(dev))
    return cache


@pytest.mark.parametrize("causal,qsp", [(False, 0), (True, 200)])
def test_paged_int8_in_place(pkg, dev, causal, qsp):
    """forward_stream over the cache itself (int8 pages read in place) equals
    the stream over its dequantised pages (the reference's own path,
    :312-331 of its M13 tests) and the fp64 oracle on those pages."""
    import torch
    B, Hq, Hkv, D = 2, 8, 2, 32
    cache = make_cache(pkg, dev, torch, B, Hkv, D, page=32, pages=8, sink=2,
                       chunks=[50, 64, 7, 100, 33, 90], seed=20)
    assert len(cache._pages) == 8
    q = randn(torch, B, Hq, 5, D, seed=19).double().to(dev)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, causal=causal)
    out, rep = attn.forward_stream(q, cache, query_start_pos=qsp)
    out2, rep2 = attn.forward_stream(q, cache.iter_dequantized_pages(torch.float32),
                                     query_start_pos=qsp)
    pages = [(no.paged_dequantize_int8(qk.cpu().numpy(), sk.cpu().numpy()),
              no.paged_dequantize_int8(qv.cpu().numpy(), sv.cpu().numpy()))
             for qk, sk, qv, sv in cache._pages]
    want, lse, n, nt = no.block_attention_stream(q.cpu().numpy(), pages, causal, qsp)
    print(f"int8 pages: rel {rel_err(out.cpu().numpy(), want):.3e}")
    assert rel_err(out.cpu().numpy(), want) < 1e-12
    assert rel_err(out2.cpu().numpy(), want) < 1e-12
    fields = lambda r: (r.query_tokens, r.kv_tokens, r.num_kv_blocks, r.peak_tile_elements)
    assert fields(rep) == fields(rep2)
    assert abs(rep.max_logsumexp - rep2.max_logsumexp) < 1e-10
    assert rep.kv_tokens == cache.resident_tokens == n and rep.num_kv_blocks == nt == 8
    assert abs(rep.max_logsumexp - float(lse.max())) < 1e-10


def test_identical_tiles_invariant(pkg, dev):
    """n copies of one tile (non-causal): the same attention output and
    max_logsumexp + log(n), at 2,000,000 streamed tokens."""
    import torch
    B, H, S_q, D, T = 1, 4, 2, 16, 20000
    q = randn(torch, B, H, S_q, D, seed=30).to(dev)
    k, v = randn(torch, B, H, T, D, seed=31).to(dev), randn(torch, B, H, T, D, seed=32).to(dev)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(H, H, D, causal=False)
    o1, r1 = attn.forward_stream(q, [(k, v)])
    n = 100
    on, rn = attn.forward_stream(q, ((k, v) for _ in range(n)))
    assert rn.kv_tokens == n * T and rn.num_kv_blocks == n
    assert torch.isfinite(on).all()
    assert rel_err(on.cpu().numpy(), o1.cpu().numpy()) < 1e-6
    assert abs(rn.max_logsumexp - (r1.max_logsumexp + math.log(n))) < 1e-9


def test_fully_masked_rows_and_errors(pkg, dev):
    """Causal rows that see no key give 0 (l = 0 -> 1); shape errors raise
    the reference's ValueError; a CPU query raises."""
    import torch
    lc = pkg.long_context
    attn = lc.OnlineSoftmaxBlockAttention(2, 1, 8, causal=True)
    q = randn(torch, 1, 2, 4, 8, seed=40).to(dev)
    k, v = randn(torch, 1, 1, 6, 8, seed=41).to(dev), randn(torch, 1, 1, 6, 8, seed=42).to(dev)
    out, rep = attn.forward_stream(q, [(k, v)], query_start_pos=-2)
    assert torch.all(out[:, :, :2] == 0)
    want, _, _, _ = no.block_attention_stream(q.double().cpu().numpy(),
                                              [(k.double().cpu().numpy(), v.double().cpu().numpy())],
                                              True, -2)
    assert rel_err(out.cpu().numpy(), want) < 1e-6
    out, rep = attn.forward_stream(q, [])
    assert torch.all(out == 0) and rep.kv_tokens == 0 and rep.max_logsumexp == 0.0
    with pytest.raises(ValueError, match="Expected query"):
        attn.forward_stream(q[0], [(k, v)])
    with pytest.raises(ValueError, match="Expected query heads"):
        lc.OnlineSoftmaxBlockAttention(4, 1, 8).forward_stream(q, [(k, v)])
    with pytest.raises(ValueError, match="must be divisible"):
        lc.OnlineSoftmaxBlockAttention(3, 2, 8)
    with pytest.raises(RuntimeError, match="GPU only"):
        attn.forward_stream(q.cpu(), [(k, v)])


@pytest.mark.parametrize("causal,qsp", [(False, 0), (True, 700)])
def test_paged_int8_in_place_head_dim_128(pkg, dev, causal, qsp):
    """The int8 head_dim-128 path (value words held in registers): GQA 32/8,
    partial pages (appends that end inside a page), a decode row and a short
    prefill, causal with a query offset and non-causal, against the fp64
    stream oracle over the dequantised pages."""
    import torch
    B, Hq, Hkv, D = 1, 32, 8, 128
    cache = make_cache(pkg, dev, torch, B, Hkv, D, page=256, pages=6, sink=1,
                       chunks=[300, 100, 250, 7, 400], seed=50)
    assert any(p[0].shape[2] < 256 for p in cache._pages)
    q = randn(torch, B, Hq, 3, D, seed=51).to(dev)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, causal=causal)
    for qq in (q.double(), q[:, :, :1].double()):
        out, rep = attn.forward_stream(qq, cache, query_start_pos=qsp)
        pages = [(no.paged_dequantize_int8(qk.cpu().numpy(), sk.cpu().numpy()),
                  no.paged_dequantize_int8(qv.cpu().numpy(), sv.cpu().numpy()))
                 for qk, sk, qv, sv in cache._pages]
        want, lse, n, nt = no.block_attention_stream(qq.cpu().numpy(), pages, causal, qsp)
        print(f"int8 hd128: rel {rel_err(out.cpu().numpy(), want):.3e}")
        assert rel_err(out.cpu().numpy(), want) < 1e-12
        assert rep.kv_tokens == n and rep.num_kv_blocks == nt
        assert abs(rep.max_logsumexp - float(lse.max())) < 1e-10


@pytest.mark.parametrize("D", [12, 20, 3])
def test_head_dim_not_multiple_of_8(pkg, dev, D):
    """Any positive head_dim, as the reference accepts: forward, forward_stream
    over tiles and over an int8 paged cache, against fp64 full attention."""
    import torch
    B, Hq, Hkv, S = 1, 4, 2, 150
    q = randn(torch, B, Hq, S, D, seed=60 + D)
    k, v = randn(torch, B, Hkv, S, D, seed=61 + D), randn(torch, B, Hkv, S, D, seed=62 + D)
    attn = pkg.long_context.OnlineSoftmaxBlockAttention(Hq, Hkv, D, q_block_size=64,
                                                        kv_block_size=48, causal=True)
    out = attn.forward(q.to(dev), k.to(dev), v.to(dev))
    assert out.shape == (B, Hq, S, D) and out.is_contiguous()
    check(out, q, k, v, True, 0)
    out, rep = attn.forward_stream(q.to(dev), [(k[:, :, :70].to(dev), v[:, :, :70].to(dev)),
                                               (k[:, :, 70:].to(dev), v[:, :, 70:].to(dev))])
    assert out.shape == (B, Hq, S, D) and rep.kv_tokens == S
    check(out, q, k, v, True, 0)
    cache = make_cache(pkg, dev, torch, B, Hkv, D, page=64, pages=8, sink=1,
                       chunks=[90, 60], seed=63 + D)
    qd = q[:, :, -2:].double().to(dev)
    out, rep = attn.forward_stream(qd, cache, query_start_pos=148)
    pages = [(no.paged_dequantize_int8(qk.cpu().numpy(), sk.cpu().numpy()),
              no.paged_dequantize_int8(qv.cpu().numpy(), sv.cpu().numpy()))
             for qk, sk, qv, sv in cache._pages]
    want, _, _, _ = no.block_attention_stream(qd.cpu().numpy(), pages, True, 148)
    assert out.shape == (B, Hq, 2, D)
    assert rel_err(out.cpu().numpy(), want) < 1e-12

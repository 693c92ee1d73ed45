"""GPU parity of the KV write path against the CPU oracle: the int8 page
quantiser and dequantiser bit-exact for float32, bfloat16, float16 and float64 input,
the PagedCompressedKVCache face (the reference's own M13 checks, including the
eviction known answer), the codebook encode-append codes and scales bit-exact
through a slot mapping, and PagedCodeKVCache append -> decode end to end."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from oracle import cpu, numpy_oracle as no

pytestmark = pytest.mark.gpu


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def edge_rows(torch, dtype, B, H, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(B, H, S, D, generator=g) * torch.logspace(-3, 3, S)[None, None, :, None]
    t[0, 0, 0] = 0.0 if dtype != torch.float16 else 1.0
    t[0, 0, 1] = torch.arange(D, dtype=torch.float32) - D // 2
    t[0, 0, 1, 0] = 127.0
    return t.to(dtype)


@pytest.mark.parametrize("kind", ["float32", "bfloat16", "float16", "float64"])
@pytest.mark.parametrize("shape", [(1, 4, 300, 64), (2, 3, 17, 130), (1, 1, 5, 8)])
def test_quantize_dequantize_int8(pkg, dev, kind, shape):
    import torch
    dtype = getattr(torch, kind)
    t = edge_rows(torch, dtype, *shape, seed=shape[2])
    lc = pkg.long_context
    q, s = lc.PagedCompressedKVCache._quantize_int8(t.to(dev))
    qn, sn = no.paged_quantize_int8(t.double().numpy() if kind == "float64" else
                                    t.float().numpy(), kind)
    assert q.dtype == torch.int8 and s.dtype == torch.float16 and s.shape == (*shape[:3], 1)
    assert np.array_equal(q.cpu().numpy(), qn)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), sn.view(np.uint16))
    for out_kind in ("float32", "bfloat16", "float16", "float64"):
        d = lc.PagedCompressedKVCache._dequantize_int8(q, s, getattr(torch, out_kind))
        dn = no.paged_dequantize_int8(qn, sn, out_kind)
        assert d.dtype == getattr(torch, out_kind)
        assert np.array_equal(d.double().cpu().numpy(), dn.astype(np.float64))


def test_quantize_int8_float64_scale_tie(pkg, dev):
    """A float64 row whose scale sits just above a float16 tie once rounded to
    float32: the stored scale follows torch's cast through float32."""
    import torch
    s_want = 1 + 2 ** -11 + 2 ** -40
    t = torch.tensor([[[[127.0 * s_want, 63.0, -1.0, 0.25]]]], dtype=torch.float64)
    q, s = pkg.long_context.PagedCompressedKVCache._quantize_int8(t.to(dev))
    qn, sn = no.paged_quantize_int8(t.numpy(), "float64")
    assert float(s.cpu()[0, 0, 0, 0]) == 1.0
    assert np.array_equal(s.cpu().numpy().view(np.uint16), sn.view(np.uint16))
    assert np.array_equal(q.cpu().numpy(), qn)


def test_paged_cache_compression_and_accuracy(pkg, dev):
    """The reference's M13 checks (T/test_m13_ultra_long_context_10m.py:347-398)
    plus every page bit-exact against the oracle."""
    import torch
    lc = pkg.long_context
    torch.manual_seed(42)
    B, H, S, D = 1, 4, 1024, 64
    k = torch.randn(B, H, S, D, dtype=torch.float32)
    v = torch.randn(B, H, S, D, dtype=torch.float32)
    cache = lc.PagedCompressedKVCache(page_size=256, max_resident_pages=16, sink_pages=2)
    cache.append(k.to(dev), v.to(dev))
    assert cache.resident_tokens == S and cache.total_tokens_seen == S
    qk, sk, qv, sv = cache._pages[0]
    assert qk.dtype == torch.int8 and qv.dtype == torch.int8
    assert sk.dtype == torch.float16 and sv.dtype == torch.float16
    assert 2 * (B * H * S * D * 4) / cache.storage_bytes >= 3.5
    assert cache.storage_bytes == 2 * (B * H * S * D + B * H * S * 2)
    pages = list(cache.iter_dequantized_pages(dtype=torch.float32))
    assert len(pages) == 4
    for i, (kd, vd) in enumerate(pages):
        sl = slice(256 * i, 256 * (i + 1))
        for src, got in ((k, kd), (v, vd)):
            qn, sn = no.paged_quantize_int8(src[:, :, sl].numpy())
            assert np.array_equal(got.cpu().numpy(), no.paged_dequantize_int8(qn, sn))

    torch.manual_seed(123)
    B, H, S, D = 1, 2, 128, 32
    k = torch.randn(B, H, S, D) * 5.0
    v = torch.randn(B, H, S, D) * 3.0
    cache = lc.PagedCompressedKVCache(page_size=128, max_resident_pages=4, sink_pages=1)
    cache.append(k.to(dev), v.to(dev))
    (k_rec, v_rec), = list(cache.iter_dequantized_pages(dtype=torch.float32))
    k_rec, v_rec = k_rec.cpu(), v_rec.cpu()
    assert torch.cosine_similarity(k.flatten(), k_rec.flatten(), dim=0).item() > 0.999
    assert torch.cosine_similarity(v.flatten(), v_rec.flatten(), dim=0).item() > 0.999
    assert torch.max(torch.abs(k - k_rec)).item() <= cache._pages[0][1].max().item() * 1.5


def test_paged_cache_eviction_known_answer(pkg, dev):
    """T/test_m13_ultra_long_context_10m.py:400-429: page means [1, 2, 10, 11, 12]."""
    import torch
    lc = pkg.long_context
    cache = lc.PagedCompressedKVCache(page_size=16, max_resident_pages=5, sink_pages=2)
    for i in range(12):
        k = torch.full((1, 1, 16, 8), float(i + 1), device=dev)
        cache.append(k, k.clone())
    assert cache.total_tokens_seen == 12 * 16
    assert len(cache._pages) == 5 and cache.resident_tokens == 5 * 16
    means = [round(p[0].mean().item(), 1) for p in cache.iter_dequantized_pages()]
    assert means == [1.0, 2.0, 10.0, 11.0, 12.0]


def test_paged_cache_evicted_page_kept_for_its_holder(pkg, dev):
    """The reference's pop (long_context.py:255-257) leaves a page that a
    caller still holds intact: later appends must not write into it.  Chunks
    in float64 (the reference accepts any float tensor)."""
    import torch
    lc = pkg.long_context
    cache = lc.PagedCompressedKVCache(page_size=16, max_resident_pages=3, sink_pages=1)
    held = None
    for i in range(8):
        k = torch.full((1, 2, 16, 8), float(i + 1), dtype=torch.float64, device=dev)
        cache.append(k, -k)
        if i == 1:
            held = cache._pages[1]                   # page 2, evicted at i == 3
            snap = [t.clone() for t in held]
    assert cache.total_tokens_seen == 8 * 16
    assert all(torch.equal(a, b) for a, b in zip(held, snap))
    assert all(p is not held for p in cache._pages)
    kd = lc.PagedCompressedKVCache._dequantize_int8(held[0], held[1], torch.float64)
    qn, sn = no.paged_quantize_int8(np.full((1, 2, 16, 8), 2.0), "float64")
    assert np.array_equal(kd.cpu().numpy(), no.paged_dequantize_int8(qn, sn, "float64"))
    means = [round(p[0].mean().item(), 1) for p in cache.iter_dequantized_pages(torch.float64)]
    assert means == [1.0, 7.0, 8.0]


def test_paged_cache_ragged_chunks_match_reference_pages(pkg, dev):
    """Ragged appends (partial pages, chunks spanning pages, evictions inside
    one append): the resident pages equal the reference's page list built by
    its append rule over the oracle's quantiser."""
    import torch
    lc = pkg.long_context
    r = np.random.default_rng(9)
    P, M, sink = 32, 4, 1
    cache = lc.PagedCompressedKVCache(page_size=P, max_resident_pages=M, sink_pages=sink)
    ref_pages = []
    for step in range(9):
        S = int(r.integers(1, 3 * P))
        k = (r.normal(size=(2, 3, S, 24)) * 10 ** r.uniform(-2, 2)).astype(np.float32)
        v = r.normal(size=(2, 3, S, 24)).astype(np.float32)
        cache.append(torch.from_numpy(k).to(dev).to(torch.bfloat16),
                     torch.from_numpy(v).to(dev).to(torch.bfloat16))
        kb = no.round_to(k, "bfloat16")
        vb = no.round_to(v, "bfloat16")
        for start in range(0, S, P):
            sl = slice(start, min(start + P, S))
            ref_pages.append((no.paged_quantize_int8(kb[:, :, sl], "bfloat16"),
                              no.paged_quantize_int8(vb[:, :, sl], "bfloat16")))
            if len(ref_pages) > M:
                ref_pages.pop(sink)
        assert len(cache._pages) == len(ref_pages)
        for (qk, sk, qv, sv), ((rqk, rsk), (rqv, rsv)) in zip(cache._pages, ref_pages):
            assert np.array_equal(qk.cpu().numpy(), rqk)
            assert np.array_equal(qv.cpu().numpy(), rqv)
            assert np.array_equal(sk.cpu().numpy().view(np.uint16), rsk.view(np.uint16))
            assert np.array_equal(sv.cpu().numpy().view(np.uint16), rsv.view(np.uint16))
        ref_bytes = sum(q.size + 2 * s.size for pair in ref_pages for q, s in pair)
        assert cache.storage_bytes == ref_bytes


def encode(pkg, dev, k, v, kcb, vcb, slots, P, pages, D, fill=0xAB):
    """Run ojasx_kv_encode_append_device into fresh paged buffers prefilled
    with a sentinel; returns the buffers on the host."""
    import torch
    n, Hkv, hd = k.shape
    G = hd // D
    kt, vt = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    kc = torch.full((pages, Hkv, P, G), fill, dtype=torch.uint8, device=dev)
    vc = kc.clone()
    ks = torch.full((pages, Hkv, P), -1.0, device=dev)
    vs = ks.clone()
    st = torch.from_numpy(np.asarray(slots, np.int32)).to(dev)
    cbk = cbv = None
    if kcb is not None:
        kcb_t, vcb_t = kcb.to(dev), vcb.to(dev)
        cbk, cbv = vp(kcb_t), vp(vcb_t)
    rc = pkg.lib().ojasx_kv_encode_append_device(vp(kt), vp(vt), n, Hkv, hd, D, cbk, cbv, vp(st),
                                                 P, pages, vp(kc), vp(ks), vp(vc), vp(vs), None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (kc, ks, vc, vs)]


def check_encoded(bufs, k, v, slots, P, want_k, want_v):
    """Every written slot holds want_*(token, head); every other slot keeps
    the sentinel."""
    kc, ks, vc, vs = bufs
    written = np.zeros(kc.shape[:3], bool)
    for i, sl in enumerate(slots):
        if sl < 0 or sl // P >= kc.shape[0]:
            continue
        pg, off = divmod(int(sl), P)
        for h in range(k.shape[1]):
            for src, want, codes, scales in ((k, want_k, kc, ks), (v, want_v, vc, vs)):
                c, s = want(src[i, h], h)
                assert np.array_equal(codes[pg, h, off], c), (i, h)
                assert scales[pg, h, off] == s, (i, h)
        written[pg, :, off] = True
    assert np.all(kc[~written] == 0xAB) and np.all(vc[~written] == 0xAB)
    assert np.all(ks[~written] == -1.0) and np.all(vs[~written] == -1.0)


@pytest.mark.parametrize("Hkv,hd,D,aligned", [(8, 128, 16, True), (2, 64, 8, True),
                                               (3, 128, 16, False), (1, 96, 32, True),
                                               # groups past one batch of 8: 16, 12 (a
                                               # partial second batch) and 64 (the most)
                                               (2, 128, 8, True), (1, 96, 8, False),
                                               (1, 1024, 16, True)])
def test_encode_append_codebook_bit_exact(pkg, dev, Hkv, hd, D, aligned):
    """Nearest-centroid codes and scales bit-exact against the oracle, tokens
    scattered through a slot mapping that also skips tokens (-1 and a slot past
    the pool).  aligned=False offsets the codebooks by one float, which takes
    the kernel's codebook-from-memory path."""
    import torch
    r = np.random.default_rng(hd + Hkv)
    n, P, pages = 45, 16, 6
    k = (r.normal(size=(n, Hkv, hd)) * r.uniform(0.01, 100, size=(n, 1, 1))).astype(np.float32)
    v = r.normal(size=(n, Hkv, hd)).astype(np.float32)
    k[3] = 0.0                                    # all-zero token: scale 1e-8 / 127
    cbs = r.normal(0, 40, size=(2, Hkv, 256, D)).astype(np.float32)
    cbs[:, :, 17] = cbs[:, :, 3]                  # duplicate centroid: ties go to 3
    flat = np.zeros(cbs.size + 1, np.float32)
    off = 0 if aligned else 1
    flat[off:off + cbs.size] = cbs.reshape(-1)
    dev_flat = torch.from_numpy(flat).to(dev)
    kcb, vcb = dev_flat[off:off + cbs[0].size], dev_flat[off + cbs[0].size:off + cbs.size]
    slots = r.permutation(pages * P)[:n].astype(np.int64)
    slots[5], slots[9] = -1, pages * P + 3
    bufs = encode(pkg, dev, k, v, kcb, vcb, slots, P, pages, D)
    check_encoded(bufs, k, v, slots, P,
                  lambda x, h: cpu.kv_encode_token(x, cbs[0, h], D),
                  lambda x, h: cpu.kv_encode_token(x, cbs[1, h], D))


def test_encode_append_reference_quantiser(pkg, dev):
    """Without codebooks the codes are the reference quantiser's
    (ojasx_lut_kv_cache.cpp:29-45), including exact half steps, which round
    away from zero there."""
    r = np.random.default_rng(77)
    n, Hkv, hd, P, pages = 20, 4, 128, 8, 3
    k = r.normal(0, 3, size=(n, Hkv, hd)).astype(np.float32)
    v = r.normal(0, 3, size=(n, Hkv, hd)).astype(np.float32)
    k[:, :, 0] = 127.0                            # scale 1: x = k exactly
    k[:, :, 16], k[:, :, 32], k[:, :, 48] = 2.5, -2.5, 0.5
    bufs = encode(pkg, dev, k, v, None, None, np.arange(n), P, pages, 16)
    check_encoded(bufs, k, v, np.arange(n), P,
                  lambda x, h: cpu.kv_quantize_token(x),
                  lambda x, h: cpu.kv_quantize_token(x))
    assert bufs[0][0, 0, 0, 1:4].tolist() == [131, 125, 129]


def test_encode_append_errors(pkg, dev):
    import torch
    L = pkg.lib()
    z = torch.zeros(64, device=dev)
    zi = torch.zeros(4, dtype=torch.int32, device=dev)
    zc = torch.zeros(64, dtype=torch.uint8, device=dev)
    args = lambda hd, D, kcb, vcb: (vp(z), vp(z), 1, 1, hd, D, kcb, vcb, vp(zi), 4, 1, vp(zc),
                                    vp(z), vp(zc), vp(z), None)
    assert L.ojasx_kv_encode_append_device(*args(16, 16, vp(z), None)) == -1
    assert L.ojasx_kv_encode_append_device(*args(20, 16, None, None)) == -3
    assert L.ojasx_kv_encode_append_device(*args(16 * 65, 16, None, None)) == -3
    assert L.ojasx_kv_encode_append_device(vp(z), vp(z), 0, 1, 16, 16, None, None, vp(zi), 4, 1,
                                           vp(zc), vp(z), vp(zc), vp(z), None) == 0


def test_code_cache_append_decode_with_eviction(pkg, dev):
    """PagedCodeKVCache: ragged appends through sink + sliding eviction, then
    decode.  The resident codes equal the oracle encoder's for the surviving
    tokens, in block-table order, and the decode output matches the oracle's
    attention over exactly those tokens (rel <= 1e-5)."""
    import torch
    lc = pkg.long_context
    r = np.random.default_rng(21)
    Hkv, Hq, hd, D, P, M, sink = 4, 16, 128, 16, 16, 12, 2
    cbs = r.normal(0, 30, size=(2, Hkv, 256, D)).astype(np.float32)
    cache = lc.PagedCodeKVCache(Hkv, hd, D, page_size=P, max_resident_pages=M, sink_pages=sink,
                                k_codebook=torch.from_numpy(cbs[0]),
                                v_codebook=torch.from_numpy(cbs[1]), device=dev)
    toks_k, toks_v, pages_model = [], [], []
    for step in range(14):
        S = int(r.integers(1, 40)) if step != 6 else 300      # one append evicts inside itself
        k = r.normal(size=(S, Hkv, hd)).astype(np.float32)
        v = r.normal(size=(S, Hkv, hd)).astype(np.float32)
        cache.append(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        for i in range(S):
            if not pages_model or len(pages_model[-1]) == P:
                if len(pages_model) == M:
                    pages_model.pop(sink)
                pages_model.append([])
            pages_model[-1].append(len(toks_k))
            toks_k.append(k[i])
            toks_v.append(v[i])
    resident = [t for page in pages_model for t in page]
    assert cache.seq_len == len(resident) and cache.total_tokens_seen == len(toks_k)
    kc, ks = cache.k_codes.cpu().numpy(), cache.k_scales.cpu().numpy()
    vc, vs = cache.v_codes.cpu().numpy(), cache.v_scales.cpu().numpy()
    q = r.normal(size=(Hq, hd)).astype(np.float32)
    out = cache.decode(torch.from_numpy(q).to(dev)).cpu().numpy()
    for h in range(Hkv):
        lk = np.empty((len(resident), hd // D), np.uint8)
        lks = np.empty(len(resident), np.float32)
        lv, lvs = np.empty_like(lk), np.empty_like(lks)
        for pos, t in enumerate(resident):
            pg, off = cache.table.pages[pos // P], pos % P
            ck, sk = cpu.kv_encode_token(toks_k[t][h], cbs[0, h], D)
            cv, sv = cpu.kv_encode_token(toks_v[t][h], cbs[1, h], D)
            assert np.array_equal(kc[pg, h, off], ck) and ks[pg, h, off] == sk
            assert np.array_equal(vc[pg, h, off], cv) and vs[pg, h, off] == sv
            lk[pos], lks[pos], lv[pos], lvs[pos] = ck, sk, cv, sv
        for j in range(h * (Hq // Hkv), (h + 1) * (Hq // Hkv)):
            want = cpu.kv_attention_cb(q[j], cbs[0, h], cbs[1, h], lk, lks, lv, lvs)
            assert rel_err(out[j], want) < 1e-5, j


def test_code_cache_reference_quantiser_decode(pkg, dev):
    """No codebooks: the scalar reference quantiser and its implicit codebook;
    the decode equals the reference's own decode of the same tokens."""
    import torch
    lc = pkg.long_context
    r = np.random.default_rng(8)
    cache = lc.PagedCodeKVCache(2, 128, 16, page_size=16, max_resident_pages=64, sink_pages=1,
                                device=dev)
    k = r.normal(0, 2, size=(150, 2, 128)).astype(np.float32)
    v = r.normal(0, 2, size=(150, 2, 128)).astype(np.float32)
    cache.append(torch.from_numpy(k[:7]).to(dev), torch.from_numpy(v[:7]).to(dev))
    cache.append(torch.from_numpy(k[7:]).to(dev), torch.from_numpy(v[7:]).to(dev))
    q = r.normal(size=(2, 128)).astype(np.float32)
    out = cache.decode(torch.from_numpy(q).to(dev)).cpu().numpy()
    for h in range(2):
        enc = [cpu.kv_quantize_token(k[t, h]) for t in range(150)]
        encv = [cpu.kv_quantize_token(v[t, h]) for t in range(150)]
        want = cpu.kv_attention_ref(q[h], np.array([c for c, _ in enc]),
                                    np.array([s for _, s in enc], np.float32),
                                    np.array([c for c, _ in encv]),
                                    np.array([s for _, s in encv], np.float32))
        assert rel_err(out[h], want) < 1e-5
    empty = lc.PagedCodeKVCache(2, 128, 16, device=dev)
    assert np.all(empty.decode(torch.from_numpy(q).to(dev)).cpu().numpy() == 0)

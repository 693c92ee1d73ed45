"""CPU side of the KV write path: the oracle's int8 page quantiser pinned
against the reference's own torch expression (long_context.py:234-244)
evaluated by torch on the CPU, the nearest-centroid encoder pinned against the
reference scalar quantiser and an fp64 brute force, and the host page logic
(validation, eviction order, slot planning)."""
import numpy as np
import pytest

from oracle import cpu, numpy_oracle as no


def torch_reference_quantise(t):
    """The reference's _quantize_int8 / _dequantize_int8 expressions
    (long_context.py:236-244), evaluated by torch in t's dtype."""
    import torch
    abs_max = t.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    scale = abs_max / 127.0
    q = torch.clamp(torch.round(t / scale), -127, 127).to(torch.int8)
    return q, scale.to(torch.float16)


def rows_with_edges(torch, dtype, n=512, d=40, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(n, d, generator=g) * torch.logspace(-4, 4, n)[:, None]
    t[0] = 0.0                                   # all-zero row: scale from the clamp
    t[1, :] = torch.arange(d, dtype=torch.float32) - 20.0   # many exact halves of s
    t[1, 0] = 127.0
    t[2, :] = 0.5                                # every element equals the max
    t[3, :4] = torch.tensor([127.0, 63.5, -63.5, 0.5])
    t[3, 4:] = 0.0
    return t.to(dtype)


@pytest.mark.parametrize("kind", ["float32", "bfloat16", "float16", "float64"])
def test_int8_oracle_matches_torch_expression(kind):
    """Bit-exact codes and scales, and the dequantised values, against the
    reference expressions evaluated by torch on rows that include zero rows,
    exact half steps and values spanning eight decades.  An all-zero float16
    row is the one case left out: there the reference divides 0 by 0."""
    import torch
    dtype = getattr(torch, kind)
    t = rows_with_edges(torch, dtype)
    if kind == "float16":
        t = t[1:]
    q, s = torch_reference_quantise(t)
    qn, sn = no.paged_quantize_int8(t.double().numpy() if kind == "float64" else
                                    t.float().numpy(), kind)
    assert np.array_equal(qn, q.numpy())
    assert np.array_equal(sn.view(np.uint16), s.numpy().view(np.uint16))
    d = (q.to(torch.float32) * s.to(torch.float32)).to(dtype)
    dn = no.paged_dequantize_int8(qn, sn, kind)
    assert np.array_equal(dn, d.double().numpy() if kind == "float64" else d.float().numpy())
    assert dn.dtype == (np.float64 if kind == "float64" else np.float32)


def test_int8_oracle_float64_scale_rounds_through_float32():
    """torch casts a float64 scale to float16 through float32; a direct cast
    rounds differently when the float32 value is a float16 tie.  A row whose
    scale is just above such a tie (1 + 2^-11 + 2^-40 in units of 2^k) pins
    the double rounding, and its codes pin the float64 division."""
    import torch
    s_want = 1 + 2 ** -11 + 2 ** -40
    t = torch.tensor([[127.0 * s_want, 63.0, -1.0]], dtype=torch.float64)
    q, s = torch_reference_quantise(t)
    qn, sn = no.paged_quantize_int8(t.numpy(), "float64")
    assert float(s[0, 0]) == 1.0 and float(np.float16(s_want)) != 1.0
    assert np.array_equal(sn.view(np.uint16), s.numpy().view(np.uint16))
    assert np.array_equal(qn, q.numpy())


def test_int8_oracle_rounding_steps():
    """Two steps a restatement could plausibly drop, each caught here.  In
    bfloat16 the quotient t / s is rounded to bfloat16 before torch.round:
    1.9765625 / bf16(100 / 127) = 2.50495 rounds to 2.5 and then to 2, where a
    single rounding gives 3.  And the scale itself is rounded to the input
    type: computing it in fp32 gives 127 instead of 126 for the row below."""
    import torch
    t = torch.tensor([[100.0, 1.9765625]], dtype=torch.bfloat16)
    q, s = torch_reference_quantise(t)
    qn, sn = no.paged_quantize_int8(t.float().numpy(), "bfloat16")
    assert np.array_equal(qn, q.numpy()) and q.tolist() == [[126, 2]]
    s_bf = no.round_to(np.float32(100.0) / np.float32(127.0), "bfloat16")
    assert np.rint(np.float32(1.9765625) / s_bf) == 3          # single rounding
    t2 = torch.tensor([[100.0, 1.0078125]], dtype=torch.bfloat16)
    q2, _ = torch_reference_quantise(t2)
    fp32_scale, _ = no.paged_quantize_int8(t2.float().numpy(), "float32")
    assert np.array_equal(no.paged_quantize_int8(t2.float().numpy(), "bfloat16")[0], q2.numpy())
    assert q2.tolist() == [[126, 1]] and fp32_scale.tolist() == [[127, 1]]


def test_encoder_reduces_to_reference_quantiser():
    """With C[c] = (c - 128) e_0 the nearest-centroid codes equal the
    reference quantiser's (ojasx_lut_kv_cache.cpp:36-45, pinned against the
    reference build in test_oracle.py) wherever x[gD] is not a half-way tie."""
    r = np.random.default_rng(5)
    cb = np.zeros((256, 16), np.float32)
    cb[:, 0] = np.arange(256) - 128
    for _ in range(200):
        k = r.normal(0, r.uniform(0.1, 10), size=128).astype(np.float32)
        c1, s1 = cpu.kv_encode_token(k, cb)
        c2, s2 = cpu.kv_quantize_token(k)
        assert s1 == s2
        x = k[::16] / s1
        ok = np.abs(np.abs(x - np.floor(x)) - 0.5) > 1e-3
        assert np.array_equal(c1[ok], c2[ok])


def test_encoder_matches_fp64_brute_force():
    """Random codebooks: the code is the fp64 argmin wherever the two nearest
    centroids are separated by more than fp32 rounding; a transposed codebook,
    a wrong group offset or a missing scale fails this."""
    r = np.random.default_rng(6)
    checked = 0
    for trial in range(40):
        D = (8, 16, 32)[trial % 3]
        cb = r.normal(0, 30, size=(256, D)).astype(np.float32)
        k = r.normal(0, 2, size=4 * D).astype(np.float32)
        codes, s = cpu.kv_encode_token(k, cb, block_dim=D)
        assert s == np.float32(max(np.float32(1e-8), np.abs(k).max()) / np.float32(127.0))
        x = (k.astype(np.float64) / np.float64(s)).reshape(4, D)
        dist = ((x[:, None, :] - cb[None].astype(np.float64)) ** 2).sum(-1)
        order = np.sort(dist, axis=1)
        clear = (order[:, 1] - order[:, 0]) > 1e-4 * order[:, 1]
        assert np.array_equal(codes[clear], dist.argmin(1)[clear])
        checked += clear.sum()
    assert checked > 100


def test_encoder_ties_to_lower_index():
    cb = np.zeros((256, 16), np.float32)
    cb[:, 0] = 500.0
    cb[7, 0] = cb[200, 0] = 0.0                  # two identical nearest centroids
    k = np.zeros(32, np.float32)
    k[0] = 1e-9
    codes, _ = cpu.kv_encode_token(k, cb)
    assert codes.tolist() == [7, 7]


def test_paged_cache_validation(pkg):
    lc = pkg.long_context
    for args in ((0, 4, 1), (16, 2, 2), (16, 1, 3)):
        with pytest.raises(ValueError, match="Invalid page configuration for PagedCompressedKVCache"):
            lc.PagedCompressedKVCache(*args)
    c = lc.PagedCompressedKVCache(16, 5, 2)
    assert c.resident_tokens == 0 and c.storage_bytes == 0 and c.total_tokens_seen == 0


def test_paged_cache_cpu_tensors_raise(pkg):
    import torch
    c = pkg.long_context.PagedCompressedKVCache(16, 5, 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        c.append(torch.zeros(1, 1, 4, 8), torch.zeros(1, 1, 4, 8))




def test_page_table_plan_matches_token_model(pkg):
    """PageTable places tokens into token-filled pages with the reference's
    eviction rule; the resident tokens, in block-table order, are the last
    ones of a token-level model, every written slot is unique, and tokens
    evicted within their own call are skipped (-1)."""
    lc = pkg.long_context
    r = np.random.default_rng(3)
    for P, M, sink in ((4, 5, 2), (16, 3, 0), (1, 4, 1), (8, 2, 1)):
        table = lc.PageTable(P, M, sink)
        slot_of = {}
        model = []                       # token-filled pages of token ids
        next_id = 0
        for _ in range(30):
            n = int(r.integers(0, 3 * P * M))
            slots = table.plan(n)
            ids = list(range(next_id, next_id + n))
            next_id += n
            for tid, sl in zip(ids, slots):
                if not model or len(model[-1]) == P:
                    if len(model) == M:
                        model.pop(sink)
                    model.append([])
                model[-1].append(tid)
                slot_of[tid] = int(sl)
            live = [s for s in slots if s >= 0]
            assert len(set(live)) == len(live)
            resident = [t for page in model for t in page]
            assert table.seq_len == len(resident)
            for lp, phys in enumerate(table.pages):
                for off, tid in enumerate(model[lp]):
                    assert slot_of[tid] == phys * P + off
            assert sorted(table.pages) == sorted(set(table.pages))
            assert all(0 <= p < M for p in table.pages)


def test_page_table_validation(pkg):
    lc = pkg.long_context
    with pytest.raises(ValueError, match="Invalid page configuration"):
        lc.PageTable(16, 2, 2)
    with pytest.raises(ValueError, match="Invalid page configuration"):
        lc.PageTable(0, 4, 1)

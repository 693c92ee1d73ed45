"""GPU parity of the LUT decoder (csrc/decoder.hip) through the C-ABI: the
fused linear variants against fp64 (rel <= 1e-5), then a small decoder stack
step by step against the fp64 oracle step (logits rel <= 1e-4 over two layers
of fp32 arithmetic; greedy tokens equal; the new token's KV codes equal the
oracle encoder's on the oracle's rotated k / v wherever the nearest centroid is
not a near tie), and the graph replay bit-identical to eager steps."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from oracle import cpu, numpy_oracle as no

pytestmark = pytest.mark.gpu


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def make_linear(pkg, r, M, K, density=0.0038, scales="u"):
    cb = r.normal(0, 0.05, size=(256, 16)).astype(np.float32)
    codes = r.integers(0, 256, size=(M, K // 16), dtype=np.uint8)
    sc = r.uniform(0.5, 1.5, size=M).astype(np.float32) if scales == "u" else np.ones(M, np.float32)
    csr = pkg.synthetic.csr_outliers(r, M, K, density)
    lin = pkg.native.NativeSplitManifoldLinear(K, M, 16, 256)
    lin.initialize_weights(cb, codes, sc)
    lin.set_outliers(*csr)
    W = no.dequantize(cb, codes, sc, csr=csr)
    return lin, W


@pytest.mark.parametrize("M,K,pro,res", [(700, 2560, 1, False), (300, 9728, 2, True),
                                         (2560, 4096, 0, True), (97, 512, 1, True),
                                         (64, 9728, 2, False),
                                         # tall RMSNorm linears (MFMA-built LUT slices):
                                         # ragged rows; x longer than the first staging pass
                                         (65600, 2560, 1, False), (65536, 5120, 1, False),
                                         (65600, 512, 1, True),    # with a residual: in place
                                         # batch-1 workgroups of 3 - 5 row tiles
                                         (19456, 2560, 1, False), (9000, 9728, 2, True),
                                         (12289, 512, 0, True),
                                         # RMSNorm + SwiGLU epilogue (gate rows, then up rows):
                                         # the decoder's 2 x 9728; 1 - 4 tiles; a ragged last
                                         # workgroup; the 64-VGPR build (641 workgroups)
                                         (19456, 2560, 3, False), (700, 2560, 3, False),
                                         (9002, 1024, 3, False), (16384, 256, 3, False),
                                         (20482, 64, 3, False), (12290, 9728, 3, False),
                                         # 2048 .. 4095 rows: 8 - 15 rows per workgroup
                                         (2560, 9728, 0, True), (2050, 2560, 1, False),
                                         (3001, 4096, 2, True), (4000, 512, 1, True)])
def test_fused_linear(pkg, dev, M, K, pro, res):
    import torch
    r = np.random.default_rng(M + K + pro)
    lin, W = make_linear(pkg, r, M, K)
    xin = r.normal(size=(2 * K if pro == 2 else K)).astype(np.float32) * 3.0
    w = r.uniform(0.5, 1.5, size=K).astype(np.float32)
    n_out = M // 2 if pro == 3 else M
    resid = r.normal(size=n_out).astype(np.float32)
    x_t = torch.from_numpy(xin).to(dev)
    w_t = torch.from_numpy(w).to(dev)
    y_t = torch.from_numpy(resid.copy()).to(dev)      # residual in place (y == residual)
    out = y_t if res else torch.empty(n_out, device=dev)
    rc = pkg.lib().ojasx_linear_forward_fused_device(
        lin.handle, vp(x_t), vp(out), pro, vp(w_t) if pro in (1, 3) else None, 1e-6,
        vp(y_t) if res else None, None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    x64 = xin.astype(np.float64)
    if pro in (1, 3):
        x64 = no.rmsnorm(x64, w, 1e-6)
    elif pro == 2:
        x64 = no.silu(x64[:K]) * x64[K:]
    want = W @ x64 + (resid if res else 0.0)
    if pro == 3:
        want = no.silu(want[:n_out]) * want[n_out:]
    assert rel_err(out.cpu().numpy(), want) < 1e-5


def test_swiglu_epilogue_equals_two_step(pkg, dev):
    """The SwiGLU epilogue (prologue 3) gives the bits of the two-step form it
    replaces in the decoder: the RMSNorm linear's 2I outputs (prologue 1),
    then silu(gate) * up as the SwiGLU prologue computes it, fed to a down
    linear (prologue 2) against that linear on the epilogue's output
    (prologue 0): equal outputs, bit for bit, at the decoder's 2560 -> 2 x 9728."""
    import torch
    r = np.random.default_rng(97)
    I, H = 9728, 2560
    gu, _ = make_linear(pkg, r, 2 * I, H)
    dn, _ = make_linear(pkg, r, H, I)
    x_t = torch.from_numpy(r.normal(size=H).astype(np.float32)).to(dev)
    w_t = torch.from_numpy(r.uniform(0.5, 1.5, size=H).astype(np.float32)).to(dev)
    L = pkg.lib()
    z = torch.empty(2 * I, device=dev)
    h = torch.empty(I, device=dev)
    y2, y1 = torch.zeros(H, device=dev), torch.zeros(H, device=dev)
    assert L.ojasx_linear_forward_fused_device(gu.handle, vp(x_t), vp(z), 1, vp(w_t), 1e-6,
                                               None, None) == 0
    assert L.ojasx_linear_forward_fused_device(dn.handle, vp(z), vp(y2), 2, None, 0.0, None,
                                               None) == 0
    assert L.ojasx_linear_forward_fused_device(gu.handle, vp(x_t), vp(h), 3, vp(w_t), 1e-6,
                                               None, None) == 0
    assert L.ojasx_linear_forward_fused_device(dn.handle, vp(h), vp(y1), 0, None, 0.0, None,
                                               None) == 0
    torch.cuda.synchronize()
    zz = z.cpu().numpy()
    g, u = zz[:I], zz[I:]
    h_two_step = (g / (np.float32(1) + np.exp(-g))) * u      # float32 throughout
    assert np.abs(h.cpu().numpy() - h_two_step).max() <= 2e-6 * np.abs(h_two_step).max()
    assert torch.equal(y1, y2)


def test_fused_linear_tall_beyond_tall_kernel_lds(pkg, dev):
    """A tall RMSNorm linear whose input is too long for the tall kernel's LDS
    (x * w staged beside two LUT buffers: about 31000 inputs) runs on the
    in-place kernel instead: 65536 rows x 32768 inputs against the fp64 LUT
    gather (no dense matrix); one past the in-place kernel's LDS is refused
    with the LDS sizes named."""
    import torch
    r = np.random.default_rng(65536)
    M, K = 65536, 32768
    cb = r.normal(0, 0.05, size=(256, 16)).astype(np.float32)
    codes = r.integers(0, 256, size=(M, K // 16), dtype=np.uint8)
    sc = r.uniform(0.5, 1.5, size=M).astype(np.float32)
    csr = pkg.synthetic.csr_outliers(r, M, K, 2e-5)
    lin = pkg.native.NativeSplitManifoldLinear(K, M, 16, 256)
    lin.initialize_weights(cb, codes, sc)
    lin.set_outliers(*csr)
    xin = r.normal(size=K).astype(np.float32) * 3.0
    w = r.uniform(0.5, 1.5, size=K).astype(np.float32)
    x_t = torch.from_numpy(xin).to(dev)
    w_t = torch.from_numpy(w).to(dev)
    out = torch.empty(M, device=dev)
    L = pkg.lib()
    rc = L.ojasx_linear_forward_fused_device(lin.handle, vp(x_t), vp(out), 1, vp(w_t), 1e-6,
                                             None, None)
    assert rc == 0, L.ojasx_get_last_error()
    torch.cuda.synchronize()
    want = no.engine_forward_rows(no.rmsnorm(xin.astype(np.float64), w, 1e-6), cb, codes, sc, csr)
    assert rel_err(out.cpu().numpy(), want) < 1e-5
    big, _ = make_linear(pkg, r, 64, 40960)
    xb = torch.zeros(40960, device=dev)
    wb = torch.ones(40960, device=dev)
    yb = torch.zeros(64, device=dev)
    assert L.ojasx_linear_forward_fused_device(big.handle, vp(xb), vp(yb), 1, vp(wb), 1e-6, None,
                                               None) == -3
    assert b"does not fit the LDS" in L.ojasx_get_last_error()


def test_fused_linear_errors(pkg, dev):
    import torch
    r = np.random.default_rng(3)
    lin, _ = make_linear(pkg, r, 32, 64)
    x = torch.zeros(64, device=dev)
    y = torch.zeros(32, device=dev)
    L = pkg.lib()
    w = torch.ones(64, device=dev)
    assert L.ojasx_linear_forward_fused_device(lin.handle, vp(x), vp(y), 1, None, 1e-6, None, None) == -1
    assert L.ojasx_linear_forward_fused_device(lin.handle, vp(x), vp(y), 3, None, 1e-6, None, None) == -1
    assert L.ojasx_linear_forward_fused_device(lin.handle, vp(x), vp(y), 4, vp(w), 1e-6, None, None) == -3
    # the SwiGLU epilogue takes no residual and an even out_features
    assert L.ojasx_linear_forward_fused_device(lin.handle, vp(x), vp(y), 3, vp(w), 1e-6, vp(y),
                                               None) == -3
    odd, _ = make_linear(pkg, r, 33, 64)
    assert L.ojasx_linear_forward_fused_device(odd.handle, vp(x), vp(y), 3, vp(w), 1e-6, None,
                                               None) == -3
    assert L.ojasx_linear_forward_fused_device(None, vp(x), vp(y), 0, None, 1e-6, None, None) == -1


SMALL = dict(hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=128, intermediate=384,
             vocab=500, max_context=96, page_size=16, max_steps=8, rms_eps=1e-6, rope_theta=1e6)


def oracle_check_step(pkg, decoder, weights, cfg, pos, x_emb, dense, linear="dense"):
    """Compare the decoder state after the step at `pos` with the oracle step."""
    caches = [decoder.read_kv(l, 0, pos + 1) for l in range(cfg.layers)]
    logits, new_kv = no.decoder_step(x_emb, weights, cfg, pos, caches, dense, linear)
    pg, off = divmod(pos, cfg.page_size)
    for l in range(cfg.layers):
        kc, ks, vc, vs = caches[l]
        w = weights["layers"][l]
        for h in range(cfg.kv_heads):
            for src, codes, scales, cb in ((new_kv[l][0][h], kc, ks, w["k_codebook"]),
                                           (new_kv[l][1][h], vc, vs, w["v_codebook"])):
                want, s = cpu.kv_encode_token(src.astype(np.float32), cb[h])
                got = codes[pg, h, off]
                assert abs(scales[pg, h, off] - s) <= 1e-5 * s
                if not np.array_equal(got, want):
                    # allowed only where the two nearest centroids are within
                    # the fp32-vs-fp64 difference of the inputs
                    x = src / s
                    for g in np.nonzero(got != want)[0]:
                        d = ((x[g * 16:(g + 1) * 16][None] - cb[h]) ** 2).sum(1)
                        a, b = d[int(got[g])], d[int(want[g])]
                        assert abs(a - b) <= 1e-4 * max(a, b), (l, h, g)
    return logits


@pytest.mark.parametrize("context", [70, 0, 63, 64])
def test_decoder_matches_oracle_and_graph_replay(pkg, dev, context):
    """Three steps from `context` cached tokens: two 64-token chunks (70), the
    new token alone (0), a step onto a chunk boundary (63 -> 64) and one
    starting at it (64: the chunk holding the new token has no cached token)."""
    dec = pkg.decoder
    cfg = dec.DecoderConfig(**SMALL)
    d, weights = dec.synthetic_decoder(cfg, context=context, seed=11, device=dev,
                                       keep_weights=True)
    emb = weights["embedding"]
    dense = {}
    token = 7
    eager_tokens, eager_logits = [], None
    for step in range(3):
        toks, logits = d.generate(token, 1, use_graph=False, return_logits=True)
        want = oracle_check_step(pkg, d, weights, cfg, context + step, emb[token], dense)
        assert rel_err(logits, want) < 1e-4, step
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 1e-3 * np.abs(want).max():
            assert int(toks[0]) == int(np.argmax(want)), step
        eager_tokens.append(int(toks[0]))
        eager_logits = logits
        token = int(toks[0])
    # the same three steps as one generate call, eager and graph: identical
    for use_graph in (False, True, True):
        for l, w in enumerate(weights["layers"]):
            if context:
                d.set_context(l, w["k_codes"], w["k_scales"], w["v_codes"], w["v_scales"], context)
        d.reset(context)
        toks, logits = d.generate(7, 3, use_graph=use_graph, return_logits=True)
        assert toks.tolist() == eager_tokens, use_graph
        assert np.array_equal(logits, eager_logits), use_graph
    d.close()


@pytest.mark.timeout(600)
def test_decoder_full_size_matches_oracle(pkg, dev):
    """BASELINE.json configs[4] at full size: hidden 2560, 36 layers, 32 q /
    8 kv heads, MLP 9728, vocab 151936, every linear LUT with 0.38 % CSR, a
    4096-token code context.  One eager step, then two more in one graph
    generate (an eager step, the capture, a replay); the first and the last
    step are checked against the fp64 oracle step, whose linears gather from
    the LUT in fp64 (engine_forward_rows) and whose attention reads the codes
    the GPU wrote: logits rel <= 1e-4 after 36 layers of fp32 arithmetic,
    tokens equal where the top-2 margin allows, new KV codes equal to the
    oracle encoder's away from near ties."""
    dec = pkg.decoder
    ctx = 4096
    cfg = dec.DecoderConfig(max_steps=4, max_context=ctx + 8)
    print(f"full-size decoder: build, context {ctx}", flush=True)
    d, weights = dec.synthetic_decoder(cfg, context=ctx, seed=3, device=dev, keep_weights=True)
    emb = weights["embedding"]
    ops = {}

    def check(pos, token_in, logits, token_out):
        want = oracle_check_step(pkg, d, weights, cfg, pos, emb[token_in], ops, linear="lut")
        err = rel_err(logits, want)
        print(f"full-size decoder: step at {pos}: logits rel err {err:.3e}", flush=True)
        assert err < 1e-4, pos
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 1e-3 * np.abs(want).max():
            assert token_out == int(np.argmax(want)), pos

    toks, logits = d.generate(1, 1, use_graph=False, return_logits=True)
    check(ctx, 1, logits, int(toks[0]))
    t1 = int(toks[0])
    toks2, logits2 = d.generate(t1, 2, use_graph=True, return_logits=True)
    check(ctx + 2, int(toks2[0]), logits2, int(toks2[1]))
    d.close()


def test_decoder_errors(pkg, dev):
    dec = pkg.decoder
    cfg = dec.DecoderConfig(**SMALL)
    d = dec.LUTDecoder(cfg, device=dev)
    with pytest.raises(pkg.OjasxError, match="set every layer"):
        d.generate(1, 1)
    r = np.random.default_rng(4)
    wrong, _ = make_linear(pkg, r, 64, 256)
    ok = [make_linear(pkg, r, M, K)[0] for M, K in ((1024, 256), (256, 512), (768, 256),
                                                     (256, 384))]
    norms = [np.ones(256, np.float32), np.ones(256, np.float32), np.ones(128, np.float32),
             np.ones(128, np.float32)]
    cbs = [np.zeros((2, 256, 16), np.float32)] * 2
    with pytest.raises(pkg.OjasxError, match="qkv linear"):
        d.set_layer(0, wrong, *ok[1:], *norms, *cbs)
    d.set_layer(0, *ok, *norms, *cbs)
    with pytest.raises(pkg.OjasxError):
        d.set_layer(5, *ok, *norms, *cbs)
    with pytest.raises(pkg.OjasxError, match="position"):
        d.reset(96)
    d.close()


def test_decoder_graph_recaptured_after_layer_swap(pkg, dev):
    """A captured step holds the linear handles' device pointers: after
    set_layer / set_head replace handles, graph generation must follow the
    new weights (the decoder drops its graph and captures again)."""
    dec = pkg.decoder
    cfg = dec.DecoderConfig(**SMALL)
    d, _ = dec.synthetic_decoder(cfg, context=20, seed=5, device=dev)
    _, before = d.generate(7, 2, use_graph=True, return_logits=True)     # captures
    r = np.random.default_rng(99)
    qd, kvd = cfg.q_heads * 128, cfg.kv_heads * 128
    shapes = ((qd + 2 * kvd, cfg.hidden), (cfg.hidden, qd), (2 * cfg.intermediate, cfg.hidden),
              (cfg.hidden, cfg.intermediate))
    lins = [dec._linear(r, M, K, 0.05, 0.0038, 0.05, False)[0] for M, K in shapes]
    norms = [r.uniform(0.8, 1.2, size=n).astype(np.float32)
             for n in (cfg.hidden, cfg.hidden, 128, 128)]
    cbs = [r.normal(0, 40, size=(cfg.kv_heads, 256, 16)).astype(np.float32) for _ in range(2)]
    d.set_layer(1, *lins, *norms, *cbs)
    lm = dec._linear(r, cfg.vocab, cfg.hidden, 0.05, 0.0038, 0.05, False)[0]
    d.set_head(lm, np.ones(cfg.hidden, np.float32),
               r.normal(size=(cfg.vocab, cfg.hidden)).astype(np.float32))
    res = {}
    for use_graph in (False, True, True):
        d.reset(20)
        res[use_graph] = d.generate(7, 2, use_graph=use_graph, return_logits=True)
    assert res[True][0].tolist() == res[False][0].tolist()
    assert np.array_equal(res[True][1], res[False][1])
    assert not np.array_equal(res[True][1], before)
    d.close()

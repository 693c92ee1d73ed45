"""Pins of the decoder oracle's pieces (oracle/numpy_oracle.py) from their
mathematics, and the decoder's host-side validation."""
import math

import numpy as np
import pytest

from oracle import numpy_oracle as no


def test_rmsnorm_closed_form():
    r = np.random.default_rng(0)
    x = r.normal(size=300) * 7.0
    y = no.rmsnorm(x, np.ones(300), 0.0)
    assert abs(np.mean(y * y) - 1.0) < 1e-12
    w = r.uniform(0.5, 2.0, size=300)
    assert np.allclose(no.rmsnorm(x, w, 1e-6), x / math.sqrt(np.mean(x * x) + 1e-6) * w, rtol=1e-14)
    assert np.allclose(no.rmsnorm(3 * x, w, 0.0), no.rmsnorm(x, w, 0.0), rtol=1e-12)


def test_rope_tables_and_rotation():
    cos, sin = no.rope_tables(64, 128, 1e6)
    assert cos.dtype == np.float32 and cos.shape == (64, 64)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # frequency 0 is 1 rad per position; the last is theta^(-126/128)
    assert abs(float(cos[1, 0]) - math.cos(1.0)) < 1e-7
    assert abs(float(sin[5, 63]) - math.sin(5 * 1e6 ** (-126 / 128))) < 1e-7
    r = np.random.default_rng(1)
    x = r.normal(size=128)
    assert np.allclose(no.rope(x, cos[0], sin[0]), x)
    y = no.rope(x, cos[7], sin[7])
    # a rotation of each (i, i + 64) pair: pair norms kept, and rotating by the
    # negative angle restores x
    assert np.allclose(x[:64] ** 2 + x[64:] ** 2, y[:64] ** 2 + y[64:] ** 2)
    assert np.allclose(no.rope(y, cos[7], -sin[7]), x)
    # pair 0 (frequency 1) at position 7 turns by 7 rad
    lo, hi = y[0], y[64]
    c, s = math.cos(7.0), math.sin(7.0)
    assert abs(lo - (x[0] * c - x[64] * s)) < 1e-6 and abs(hi - (x[64] * c + x[0] * s)) < 1e-6


def test_decoder_step_single_token_context():
    """With one cached token the attention output is that token's V, so one
    layer reduces to x + Wo V + Wdown(SwiGLU(...)), composed here from
    the dense matrices."""
    class C:
        head_dim, q_heads, kv_heads, rms_eps, rope_theta = 128, 2, 1, 1e-6, 1e4

    r = np.random.default_rng(2)
    hid, inter = 32, 48

    def lin(M, K):
        return dict(codebook=r.normal(0, 0.1, size=(256, 16)).astype(np.float32),
                    codes=r.integers(0, 256, size=(M, K // 16), dtype=np.uint8),
                    csr=(np.zeros(M + 1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32)))

    layer = dict(qkv=lin(4 * 128, hid), o=lin(hid, 256), gate_up=lin(2 * inter, hid),
                 down=lin(hid, inter), input_norm=np.ones(hid), post_norm=np.ones(hid),
                 q_norm=np.ones(128), k_norm=np.ones(128),
                 k_codebook=r.normal(size=(1, 256, 16)), v_codebook=r.normal(size=(1, 256, 16)))
    weights = dict(layers=[layer], lm_head=lin(10, hid), final_norm=np.ones(hid))
    kc = r.integers(0, 256, size=(1, 1, 16, 8), dtype=np.uint8)
    vc = r.integers(0, 256, size=(1, 1, 16, 8), dtype=np.uint8)
    ks = np.full((1, 1, 16), 0.5, np.float32)
    vs = np.full((1, 1, 16), 2.0, np.float32)
    x = r.normal(size=hid)
    logits, _ = no.decoder_step(x, weights, C, 0, [(kc, ks, vc, vs)])
    V0 = layer["v_codebook"][0][vc[0, 0, 0].astype(np.int64)].reshape(-1) * 2.0
    attn = np.concatenate([V0, V0])
    W = {k: no.lut_dense(layer[k]) for k in ("o", "gate_up", "down")}
    x1 = x + W["o"] @ attn
    gu = W["gate_up"] @ no.rmsnorm(x1, np.ones(hid), 1e-6)
    x2 = x1 + W["down"] @ (no.silu(gu[:inter]) * gu[inter:])
    want = no.lut_dense(weights["lm_head"]) @ no.rmsnorm(x2, np.ones(hid), 1e-6)
    assert np.allclose(logits, want, rtol=1e-12, atol=1e-12)


def test_decoder_config_validation(pkg):
    dec = pkg.decoder
    bad = dec.DecoderConfig(hidden=256, layers=1, q_heads=4, kv_heads=2, head_dim=64,
                            intermediate=128, vocab=10, max_context=32)
    with pytest.raises(RuntimeError, match="head_dim must be 128"):
        dec.LUTDecoder(bad, device="cpu")


def _lut_linear(r, M, K, density=0.01):
    from oracle import gen
    return dict(codebook=r.normal(0, 0.1, size=(256, 16)).astype(np.float32),
                codes=r.integers(0, 256, size=(M, K // 16), dtype=np.uint8),
                csr=gen.csr_outliers(r, M, K, density))


def test_engine_forward_rows_equals_dense():
    """The row-blocked fp64 LUT gather equals the dense x . W^T (the identity
    LUT-gather = x . W^T), across row blocks, with scales, CSR and bias; an
    off-by-one code (planted) is far outside the bar."""
    r = np.random.default_rng(5)
    for M, K, blk in ((300, 256, 64), (1000, 4096, 4096), (77, 48, 10)):
        w = _lut_linear(r, M, K)
        sc = r.uniform(0.5, 1.5, size=M)
        bias = r.normal(size=M)
        x = r.normal(size=K)
        got = no.engine_forward_rows(x, w["codebook"], w["codes"], sc, w["csr"], bias, blk)
        want = no.linear_fp64(x, w["codebook"], w["codes"], sc, bias, w["csr"])[0]
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
        assert np.allclose(no.LUTOp(w) @ x, no.lut_dense(w) @ x, rtol=1e-12,
                           atol=1e-12 * np.abs(want).max())
        bad = dict(w, codes=(w["codes"].astype(np.int64) + 1).astype(np.uint8) % 255)
        assert np.abs(no.LUTOp(bad) @ x - no.lut_dense(w) @ x).max() > 1e-3 * np.abs(want).max()


def test_decoder_step_lut_equals_dense():
    class C:
        head_dim, q_heads, kv_heads, rms_eps, rope_theta = 128, 4, 2, 1e-6, 1e6

    r = np.random.default_rng(6)
    hid, inter, T = 64, 96, 40
    layers = []
    caches = []
    for _ in range(2):
        layers.append(dict(qkv=_lut_linear(r, 8 * 128, hid), o=_lut_linear(r, hid, 512),
                           gate_up=_lut_linear(r, 2 * inter, hid), down=_lut_linear(r, hid, inter),
                           input_norm=r.uniform(0.8, 1.2, hid), post_norm=r.uniform(0.8, 1.2, hid),
                           q_norm=r.uniform(0.8, 1.2, 128), k_norm=r.uniform(0.8, 1.2, 128),
                           k_codebook=r.normal(size=(2, 256, 16)),
                           v_codebook=r.normal(size=(2, 256, 16))))
        kc = r.integers(0, 256, size=(3, 2, 16, 8), dtype=np.uint8)
        vc = r.integers(0, 256, size=(3, 2, 16, 8), dtype=np.uint8)
        caches.append((kc, r.uniform(0.01, 0.03, size=(3, 2, 16)), vc,
                       r.uniform(0.01, 0.03, size=(3, 2, 16))))
    weights = dict(layers=layers, lm_head=_lut_linear(r, 50, hid), final_norm=np.ones(hid))
    x = r.normal(size=hid)
    a, kv_a = no.decoder_step(x, weights, C, T - 1, caches)
    b, kv_b = no.decoder_step(x, weights, C, T - 1, caches, linear="lut")
    assert np.allclose(a, b, rtol=1e-10, atol=1e-10 * np.abs(a).max())
    for (ka, va), (kb, vb) in zip(kv_a, kv_b):
        assert np.allclose(ka, kb, rtol=1e-10) and np.allclose(va, vb, rtol=1e-10)

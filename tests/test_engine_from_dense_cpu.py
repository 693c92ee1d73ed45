"""SplitManifoldLUTLinear.from_dense (split_manifold_engine.py:90-183) on the
CPU: the offline fit runs in torch on the weight's device, so these tests
need no GPU.  They pin the algorithm by what it must produce, not by
retyping it:
  * a weight built from 256 distinct unit-scale blocks laid out in 256 equal
    runs is recovered exactly (the evenly spaced initial picks land one in
    each run, so the first assignment is exact and Lloyd's steps keep it);
    a wrong block partition, pick rule or code order fails it;
  * the outlier set is {|W - mean| >= tau * std} with torch's unbiased std
    (split_manifold_engine.py:113-117), the row scales are the max |w| of
    the manifold (outliers zeroed), and the residuals are exact at the
    outlier coordinates (dequantised W equals W there);
  * every code is a nearest centroid of its normalised block (fp64 brute
    force), the fixed point the final assignment must reach;
  * the reference's own float64 property (tests/test_split_manifold_lut.py:
    88-109): the LUT forward equals x @ dequantize_weights().T + b to 1e-12,
    here through the fp64 oracle forward.
"""
import numpy as np
import pytest
import torch

from oracle import numpy_oracle as no


@pytest.fixture(scope="module")
def engine(pkg):
    import importlib
    return importlib.import_module(pkg.__name__ + ".engine")


def _exact_case(out_f=64, in_f=512, seed=7):
    """W whose blocks take 256 distinct values in 256 equal runs of the
    row-major block order.  Entries are multiples of 1/128 and every block
    holds a +-1, so each row scale is exactly 1 and the Lloyd means of equal
    vectors are exact."""
    g = np.random.default_rng(seed)
    G = in_f // 16
    n = out_f * G
    assert n % 256 == 0
    V = (g.integers(-127, 128, size=(256, 16)) / 128.0).astype(np.float32)
    V[:, 0] = (np.arange(256) - 128) / 128.0                  # all distinct
    V[:, 1] = np.where(g.integers(0, 2, 256) > 0, 1.0, -1.0)  # max |v| = 1 in every block
    run = n // 256
    ids = np.repeat(np.arange(256), run)                       # block k -> vector k // run
    V2 = V[ids]
    return V2.reshape(out_f, in_f), V2, ids


def test_from_dense_recovers_exact_blocks(engine):
    W, V2, ids = _exact_case()
    layer = engine.SplitManifoldLUTLinear.from_dense(torch.from_numpy(W), block_dim=16,
                                                     codebook_size=256, outlier_tau=9999.0)
    assert layer.num_outliers == 0
    assert torch.equal(layer.scales, torch.ones(W.shape[0]))
    codes = layer.codes.numpy().reshape(-1)
    cb = layer.codebook.numpy()
    # each block's centroid is the block itself
    assert np.array_equal(cb[codes], V2)
    # one code per distinct vector: blocks equal iff their codes are equal
    assert len(np.unique(codes)) == len(np.unique(V2, axis=0))
    assert np.array_equal(layer.dequantize_weights().numpy(), W)


@pytest.mark.parametrize("tau", [2.5, 3.0, 3.5])
def test_from_dense_outliers_scales_residuals(engine, tau):
    torch.manual_seed(11)
    W = torch.randn(96, 256) * 0.05
    W[3, 17] = 2.0
    W[50, 200] = -1.5
    layer = engine.SplitManifoldLUTLinear.from_dense(W, block_dim=16, codebook_size=256,
                                                     outlier_tau=tau)
    Wd = W.double().numpy()
    thr = tau * W.std().item()
    mask = np.abs(W.numpy() - W.mean().item()) >= thr
    oi = layer.outlier_indices.numpy()
    got = np.zeros_like(mask)
    got[oi[0], oi[1]] = True
    assert np.array_equal(got, mask)
    assert mask[3, 17] and mask[50, 200]
    # row scales: max |w| of the manifold
    man = np.where(mask, 0.0, W.numpy())
    assert np.array_equal(layer.scales.numpy(), np.maximum(np.abs(man).max(axis=1), 1e-8).astype(np.float32))
    # exact residual at the outlier coordinates (one fp32 rounding at most)
    Wq = layer.dequantize_weights().double().numpy()
    err = np.abs(Wq[mask] - Wd[mask])
    assert np.all(err <= np.abs(Wd[mask]) * 2.0 ** -23 + 1e-12)


def test_from_dense_codes_are_nearest(engine):
    torch.manual_seed(3)
    W = torch.randn(128, 512)
    layer = engine.SplitManifoldLUTLinear.from_dense(W, block_dim=16, codebook_size=256,
                                                     outlier_tau=3.5)
    oi = layer.outlier_indices.numpy()
    man = W.numpy().copy()
    man[oi[0], oi[1]] = 0.0
    blocks = man.reshape(128, 32, 16) / layer.scales.numpy().reshape(128, 1, 1)
    v = blocks.reshape(-1, 16).astype(np.float64)
    cb = layer.codebook.numpy().astype(np.float64)
    d2 = (v * v).sum(1)[:, None] + (cb * cb).sum(1)[None, :] - 2.0 * v @ cb.T
    codes = layer.codes.numpy().reshape(-1).astype(np.int64)
    best = d2.min(axis=1)
    mine = d2[np.arange(len(codes)), codes]
    # torch.cdist works in fp32: a chosen code may trail the fp64 best by rounding only
    assert np.all(mine - best <= 1e-5 * (1.0 + best))
    assert (mine == best).mean() > 0.99


def test_from_dense_float64_forward_identity(engine):
    torch.manual_seed(1337)
    W = torch.randn(128, 256, dtype=torch.float64)
    b = torch.randn(128, dtype=torch.float64)
    x = torch.randn(4, 256, dtype=torch.float64)
    layer = engine.SplitManifoldLUTLinear.from_dense(W, b, block_dim=16, codebook_size=256,
                                                     outlier_tau=3.0)
    assert layer.codebook.dtype == torch.float64 and layer.codes.dtype == torch.uint8
    want = (x @ layer.dequantize_weights().t() + layer.bias.detach()).numpy()
    y = no.engine_forward(x.numpy(), layer.codebook.numpy(), layer.codes.numpy(),
                          layer.scales.numpy(), layer.outlier_indices.numpy(),
                          layer.outlier_values.numpy(), layer.bias.detach().numpy())
    assert np.abs(y - want).max() < 1e-12

"""GPU parity of the math-engine drop-in (subspace_lut_rvq_gemm, pack_codes,
unpack_codes) against the numpy restatement of ojasx_24x96/math_engine.py:136-208
and codec.py:176-214, itself pinned to the dense product x.W^T in test_oracle.

Bars: bit-exact for packing and for integer-valued inputs; rel <= 1e-5
(max-abs error / max |ref|) for fp32 inputs, <= 1e-2 for bf16 inputs.
"""
import numpy as np
import pytest

from conftest import rel_err
from oracle import gen
from oracle import numpy_oracle as no

pytestmark = pytest.mark.gpu


def make_encoded(me, torch, dev, rows, cols, block, bits, stages, seed, integer=False, cb_scale=1.0):
    r = gen.rng(seed)
    G = (cols + block - 1) // block
    if integer:
        cbs = r.integers(-3, 4, size=(stages, 1 << bits, block)).astype(np.float32)
        scales = r.integers(1, 3, size=rows).astype(np.float32)
    else:
        cbs = (r.normal(size=(stages, 1 << bits, block)) * cb_scale).astype(np.float32)
        scales = r.uniform(0.5, 1.5, size=rows).astype(np.float32)
    codes = r.integers(0, 1 << bits, size=(stages, rows, G))
    packed = np.stack([no.pack_codes(codes[s], bits) for s in range(stages)])
    enc = me.QuantizedWeight((rows, cols), block, bits, torch.from_numpy(packed).to(dev),
                             torch.from_numpy(cbs).to(dev), torch.from_numpy(scales).to(dev), {})
    return enc, cbs, packed, scales


@pytest.mark.parametrize("rows,cols,block,bits,stages", [
    (333, 2560, 16, 8, 1),     # the linear layer's code format, no outliers
    (257, 1003, 8, 4, 2),      # K padding; stage 1 starts at an odd byte
    (130, 100, 24, 2, 3),      # block 24: runtime-block path
    (64, 37, 4, 1, 2),         # 1-bit codes, tiny rows
    (6912, 2560, 16, 8, 2),    # 2-stage gate/up size
    (50, 96, 32, 4, 1),        # block 32
])
@pytest.mark.parametrize("B", [1, 5])
def test_lut_gemm_matches_oracle(pkg, dev, rows, cols, block, bits, stages, B):
    import torch
    me = pkg.math_engine
    enc, cbs, packed, scales = make_encoded(me, torch, dev, rows, cols, block, bits, stages,
                                            seed=rows + cols + bits + B)
    r = gen.rng(7 + B)
    x = r.normal(size=(B, cols)).astype(np.float32)
    bias = r.normal(size=rows).astype(np.float32)
    y = me.subspace_lut_rvq_gemm(torch.from_numpy(x).to(dev), enc, torch.from_numpy(bias).to(dev))
    want = no.subspace_lut_rvq_gemm(x, cbs, packed, bits, rows, cols, block, scales, bias)
    assert y.dtype == torch.float32 and tuple(y.shape) == (B, rows)
    assert rel_err(y.cpu().numpy(), want) < 1e-5


def test_lut_gemm_integer_bit_exact(pkg, dev):
    import torch
    me = pkg.math_engine
    rows, cols, block, bits, stages = 300, 1000, 8, 4, 3
    enc, cbs, packed, scales = make_encoded(me, torch, dev, rows, cols, block, bits, stages, seed=3,
                                            integer=True)
    x = gen.rng(4).integers(-4, 5, size=(3, cols)).astype(np.float32)
    y = me.subspace_lut_rvq_gemm(torch.from_numpy(x).to(dev), enc).cpu().numpy()
    G = (cols + block - 1) // block
    W = np.zeros((rows, G * block), np.int64)
    for s in range(stages):
        c = no.unpack_codes(packed[s], bits, rows * G).reshape(rows, G).astype(np.int64)
        W += cbs[s][c].reshape(rows, G * block).astype(np.int64)
    want = (x.astype(np.int64) @ W[:, :cols].T) * scales.astype(np.int64)
    assert np.array_equal(y, want.astype(np.float32))


def test_lut_gemm_shapes_dtypes_and_errors(pkg, dev):
    import torch
    me = pkg.math_engine
    rows, cols = 96, 200
    enc, cbs, packed, scales = make_encoded(me, torch, dev, rows, cols, 8, 8, 2, seed=11)
    x = gen.rng(12).normal(size=(2, 3, cols)).astype(np.float32)
    xt = torch.from_numpy(x).to(dev)
    y = me.subspace_lut_rvq_gemm(xt, enc)
    assert tuple(y.shape) == (2, 3, rows)
    want = no.subspace_lut_rvq_gemm(x.reshape(6, cols), cbs, packed, 8, rows, cols, 8, scales)
    assert rel_err(y.reshape(6, rows).cpu().numpy(), want) < 1e-5
    yb = me.subspace_lut_rvq_gemm(xt.to(torch.bfloat16), enc)
    assert yb.dtype == torch.bfloat16
    wantb = no.subspace_lut_rvq_gemm(xt.to(torch.bfloat16).float().reshape(6, cols).cpu().numpy(),
                                     cbs, packed, 8, rows, cols, 8, scales)
    assert rel_err(yb.float().reshape(6, rows).cpu().numpy(), wantb) < 1e-2
    with pytest.raises(ValueError, match="Input feature mismatch"):
        me.subspace_lut_rvq_gemm(xt[..., :-1], enc)
    with pytest.raises(RuntimeError, match="GPU only"):
        me.subspace_lut_rvq_gemm(torch.from_numpy(x), enc)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_pack_unpack_bit_exact(pkg, dev, bits):
    import torch
    me = pkg.math_engine
    codes = gen.rng(bits).integers(0, 1 << bits, size=1001)
    ct = torch.from_numpy(codes.astype(np.int32)).to(dev)
    packed = me.pack_codes(ct, bits)
    assert np.array_equal(packed.cpu().numpy(), no.pack_codes(codes, bits))
    back = me.unpack_codes(packed, bits, 1001)
    assert np.array_equal(back.cpu().numpy(), codes.astype(np.uint8))
    # 7 rows x 143 blocks = 1001 codes in one stage: codes_range over unaligned bits
    enc = me.QuantizedWeight((7, 143 * bits), bits, bits, packed[None, :].clone(),
                             torch.zeros(1, 1 << bits, bits, device=dev), torch.ones(7, device=dev), {})
    for start, count in ((333, 100), (0, 1), (1, 7), (7, 9), (995, 6), (1000, 1), (5, 0), (0, 1001)):
        got = enc.codes_range(0, start, count).cpu().numpy()
        assert np.array_equal(got, codes[start:start + count].astype(np.uint8)), (start, count)
    assert np.array_equal(enc.codes(0).cpu().numpy(), codes.astype(np.uint8))
    for bad in ((-1, 2), (1000, 2), (3, -1)):
        with pytest.raises(IndexError):
            enc.codes_range(0, *bad)
    with pytest.raises(IndexError):
        enc.codes(1)
    with pytest.raises(ValueError, match="exceeds"):
        me.pack_codes(ct + (1 << bits), bits)

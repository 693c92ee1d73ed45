"""Host-side logic of the math-engine drop-in: the QuantizedWeight container's
validation (ojasx_24x96/codec.py:77-134) and the GPU-only guard."""
import numpy as np
import pytest


def _enc(me, torch, rows=4, cols=20, block=8, bits=4, stages=2, **kw):
    G = (cols + block - 1) // block
    nbytes = (rows * G * bits + 7) // 8
    args = dict(original_shape=(rows, cols), block_size=block, bits_per_stage=bits,
                packed_codes=torch.zeros(stages, nbytes, dtype=torch.uint8),
                codebooks=torch.zeros(stages, 1 << bits, block),
                row_scales=torch.ones(rows), metrics={})
    args.update(kw)
    return me.QuantizedWeight(**args)


def test_container_properties(pkg):
    import torch
    me = pkg.math_engine
    e = _enc(me, torch)
    assert e.stages == 2 and e.blocks_per_row == 3 and e.vector_count == 12
    assert e.storage_bytes == 2 * 6 + 2 * 16 * 8 * 4 + 4 * 4
    assert e.nominal_bits_per_weight == 2 * 4 / 8
    assert np.isclose(e.measured_bits_per_weight, 8.0 * e.storage_bytes / 80)


@pytest.mark.parametrize("kw,exc", [
    (dict(bits_per_stage=3), ValueError),
    (dict(original_shape=(4, 20, 1)), ValueError),
    (dict(packed_codes=None), TypeError),
    (dict(row_scales=None), ValueError),
    (dict(codebooks=None), ValueError),
])
def test_container_validation(pkg, kw, exc):
    import torch
    me = pkg.math_engine
    if "packed_codes" in kw:
        kw = dict(packed_codes=torch.zeros(2, 6, dtype=torch.int32))
    if "row_scales" in kw:
        kw = dict(row_scales=torch.ones(5))
    if "codebooks" in kw:
        kw = dict(codebooks=torch.zeros(2, 16, 4))
    with pytest.raises(exc):
        _enc(me, torch, **kw)


def test_gemm_refuses_cpu_tensors(pkg):
    import torch
    me = pkg.math_engine
    e = _enc(me, torch)
    with pytest.raises(RuntimeError, match="GPU only"):
        me.subspace_lut_rvq_gemm(torch.zeros(1, 20), e)
    with pytest.raises(ValueError, match="Input feature mismatch"):
        me.subspace_lut_rvq_gemm(torch.zeros(1, 19), e)

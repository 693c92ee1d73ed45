"""oqpack.v1 layers loaded onto the GPU: each residual-VQ linear's forward
through the math-engine kernel, and a single-stage 8-bit block-16 layer
repacked into the tiled LUT-GEMV handle, against the fp64 oracle (rel 1e-5)."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import numpy_oracle as no
from test_oqpack_cpu import make_weight

pytestmark = pytest.mark.gpu


def test_package_layers_on_gpu(pkg, dev, tmp_path):
    import torch
    me, oq = pkg.math_engine, pkg.oqpack
    r = np.random.default_rng(5)
    layers = {"a": make_weight(me, torch, r, 300, 200, 8, 4, 2),
              "b": make_weight(me, torch, r, 257, 512, 16, 8, 1),
              "c": make_weight(me, torch, r, 64, 45, 16, 2, 3)}
    biases = {"b": torch.from_numpy(r.normal(size=257).astype(np.float32))}
    oq.save_oqpack(layers, tmp_path / "p", biases=biases, max_shard_bytes=4096)
    loaded, manifest = oq.load_lut_layers(tmp_path / "p", device=dev)
    assert len(manifest.shards) >= 2
    for name, w in layers.items():
        lay = loaded[name]
        assert lay.weight.packed_codes.is_cuda
        rows, cols = w.original_shape
        x = r.normal(size=(3, cols)).astype(np.float32)
        y = lay(torch.from_numpy(x).to(dev)).cpu().numpy()
        b = biases.get(name)
        want = no.subspace_lut_rvq_gemm(x, w.codebooks.numpy(), w.packed_codes.numpy(),
                                        w.bits_per_stage, rows, cols, w.block_size,
                                        w.row_scales.numpy(), None if b is None else b.numpy())
        assert rel_err(y, want) < 1e-5, name
    nat = loaded["b"].native_linear()
    x = r.normal(size=(2, 512)).astype(np.float32)
    w = layers["b"]
    want = no.subspace_lut_rvq_gemm(x, w.codebooks.numpy(), w.packed_codes.numpy(), 8, 257, 512,
                                    16, w.row_scales.numpy(), biases["b"].numpy())
    assert rel_err(nat.forward(x), want) < 1e-5
    with pytest.raises(ValueError, match="one 8-bit stage"):
        loaded["a"].native_linear()


def test_reference_written_package_on_gpu(pkg, dev):
    """The reference's own package (tests/golden/make_oqpack_golden.py): its
    layers on the GPU reproduce the reference modules' outputs, through the
    math-engine kernel and, for the 8-bit block-16 layer, the LUT-GEMV handle."""
    import os
    import torch
    from conftest import GOLDEN
    exp = np.load(os.path.join(GOLDEN, "oqpack_ref_expected.npz"))
    layers, _ = pkg.oqpack.load_lut_layers(os.path.join(GOLDEN, "oqpack_ref_small"), device=dev)
    for name, x, y in (("0", exp["x0"], exp["y0"]), ("2", exp["x2"], exp["y2"])):
        got = layers[name](torch.from_numpy(x).to(dev)).cpu().numpy()
        assert rel_err(got, y) < 1e-5, name
    assert rel_err(layers["0"].native_linear().forward(exp["x0"]), exp["y0"]) < 1e-5

"""Writes ``oqpack_ref_small/``, a package written by the reference's own
``save_oqpack`` (ojasx_24x96/oqpack.py:383-548), and
``oqpack_ref_expected.npz``: inputs and the reference modules' outputs.

It also writes the same two layers with this repository's ``save_oqpack``
(from the tensors of the reference's package, on the CPU), loads that package
with the reference's ``load_quantized_model_from_oqpack`` (:688-754) into a
fresh two-linear skeleton and stores its outputs on the same inputs
(``ours_by_ref_y0``, ``ours_by_ref_y2``): the reference reads this build's
packages as its own.

The model is two ``nn.Linear`` layers quantised by the reference's
``quantize_model`` (ojasx_24x96/module.py:947) into adaptive residual-VQ
linears: ``0`` (64 -> 96, bias, block 16, one 8-bit stage: the tiled LUT-GEMV
handle applies) and ``2`` (96 -> 40, no bias, block 8, up to three 4-bit
stages).  The expected outputs are the quantised modules' own forward passes
(``ResidualVQLinear.forward``, fp32, on the CPU) for 5 seeded input rows.

This imports the reference package from /root/reference and runs only in
the build container (the reference does not exist on the GPU box).  Run from
the repository root:  python tests/golden/make_oqpack_golden.py
"""
import os
import shutil
import sys

import numpy as np
import torch
import torch.nn as nn

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(HERE, "oqpack_ref_small")
OUT = os.path.join(HERE, "oqpack_ref_expected.npz")


def main():
    sys.path.insert(0, "/root/reference")
    from ojasx_24x96.codec import QuantizationConfig
    from ojasx_24x96.module import quantize_model
    from ojasx_24x96.oqpack import save_oqpack

    torch.manual_seed(2041)
    model = nn.Sequential(nn.Linear(64, 96, bias=True), nn.ReLU(), nn.Linear(96, 40, bias=False))
    common = dict(max_relative_error=None, require_compression=False, min_weight_elements=16,
                  kmeans_iterations=6, max_codebook_samples=2048)
    quantize_model(model, QuantizationConfig(block_size=16, bits_per_stage=8, max_stages=1,
                                             **common), include=("0",))
    quantize_model(model, QuantizationConfig(block_size=8, bits_per_stage=4, max_stages=3,
                                             **common), include=("2",))
    kinds = [type(m).__name__ for m in (model[0], model[2])]
    assert kinds == ["ResidualVQLinear", "ResidualVQLinear"], kinds
    if os.path.isdir(PKG_DIR):
        shutil.rmtree(PKG_DIR)
    manifest = save_oqpack(model, PKG_DIR, model_id="ojasx-lut-interchange-fixture")
    x0 = torch.from_numpy(np.random.default_rng(7).normal(size=(5, 64)).astype(np.float32))
    x2 = torch.from_numpy(np.random.default_rng(8).normal(size=(5, 96)).astype(np.float32))
    with torch.no_grad():
        y0 = model[0](x0)
        y2 = model[2](x2)
    # this build's writer -> the reference's loader
    import tempfile
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    import __graft_entry__
    from ojasx_24x96.oqpack import load_quantized_model_from_oqpack
    ours = __graft_entry__.load_package()
    layers, _ = ours.oqpack.load_lut_layers(PKG_DIR, device="cpu")
    with tempfile.TemporaryDirectory() as tmp:
        ours.oqpack.save_oqpack({k: v.weight for k, v in layers.items()}, tmp,
                                biases={"0": layers["0"].bias})
        skel = nn.Sequential(nn.Linear(64, 96, bias=True), nn.ReLU(),
                             nn.Linear(96, 40, bias=False))
        back, _ = load_quantized_model_from_oqpack(skel, tmp)
        with torch.no_grad():
            r0, r2 = back[0](x0), back[2](x2)
    assert torch.equal(r0, y0) and torch.equal(r2, y2), "the reference read our package differently"
    np.savez_compressed(OUT, x0=x0.numpy(), y0=y0.numpy(), x2=x2.numpy(), y2=y2.numpy(),
                        stages=np.array([model[0].stages, model[2].stages]),
                        ours_by_ref_y0=r0.numpy(), ours_by_ref_y2=r2.numpy())
    print(f"wrote {PKG_DIR} ({manifest.format_version}, {len(manifest.shards)} shard(s)) and "
          f"{OUT}; stages {model[0].stages}, {model[2].stages}; torch {torch.__version__}")


if __name__ == "__main__":
    main()

"""Writes ``engine_bf16_2560x6912.npz``: outputs of the reference's own PyTorch
LUT module with bfloat16 buffers (split_manifold_lut_experiment/engine/
split_manifold_engine.py:22-250), the path whose arithmetic no restatement
here pins: its LUT matmul, gather sum, scale product, outlier scatter-add and
bias add all run in bf16 through torch's CPU kernels (:199, :227, :236-247).

Inputs are the repo's seeded generator (``oracle.gen.linear``: 2560 -> 6912,
64 tokens, scales U[0.5, 1.5], bias, 0.38 % CSR outliers as the module's
row-major COO), each array rounded to bf16 by torch (round to nearest even).
They are regenerated at test time, so only a digest of them is stored, with
the outputs: every column at 1 and 8 tokens, every 7th column at 64 tokens,
as bf16 bit patterns (uint16).

This imports the reference module from /root/reference and runs only in the
build container (the reference does not exist on the GPU box).  Run from the
repository root:  python tests/golden/make_bf16_golden.py
"""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import gen  # noqa: E402

M, K, B, SEED = 6912, 2560, 64, 2031
COL_STRIDE_B64 = 7


def bf16_inputs():
    """The generator's arrays rounded to bf16, as CPU torch tensors; the GPU
    test imports this function to rebuild the same inputs."""
    d = gen.linear(M, K, B=B, seed=SEED, scales="u", bias=True)
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    rp, cl, vl = d["csr"]
    rows = np.repeat(np.arange(M), np.diff(rp)).astype(np.int64)
    return dict(codebook=bf(d["codebook"]), codes=torch.from_numpy(d["codes"]),
                scales=bf(d["scales"]), bias=bf(d["bias"]),
                outlier_indices=torch.from_numpy(np.stack([rows, cl.astype(np.int64)])),
                outlier_values=bf(vl), x=bf(d["x"]))


def digest(t):
    h = hashlib.sha256()
    for k in sorted(t):
        a = t[k]
        h.update(k.encode())
        h.update((a.view(torch.int16) if a.dtype == torch.bfloat16 else a).numpy().tobytes())
    return h.hexdigest()


def main():
    sys.path.insert(0, "/root/reference/split_manifold_lut_experiment/engine")
    import split_manifold_engine as sme

    t = bf16_inputs()
    layer = sme.SplitManifoldLUTLinear(K, M, bias=True, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.codebook.copy_(t["codebook"])
        layer.codes.copy_(t["codes"])
        layer.scales.copy_(t["scales"])
        layer.bias.data.copy_(t["bias"])
        layer.outlier_indices = t["outlier_indices"]
        layer.outlier_values = t["outlier_values"]
        layer.num_outliers = int(t["outlier_values"].numel())
        out = {}
        for b in (1, 8, 64):
            y = layer(t["x"][:b])
            assert y.dtype == torch.bfloat16 and y.shape == (b, M)
            if b == 64:
                y = y[:, ::COL_STRIDE_B64]
            out[f"y_b{b}"] = y.contiguous().view(torch.int16).numpy().view(np.uint16)
    path = os.path.join(HERE, "engine_bf16_2560x6912.npz")
    np.savez_compressed(path, inputs_sha256=np.array(digest(t)), seed=np.array(SEED),
                        col_stride_b64=np.array(COL_STRIDE_B64), **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes), torch {torch.__version__}")


if __name__ == "__main__":
    main()

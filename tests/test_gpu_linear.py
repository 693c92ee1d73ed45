"""GPU parity of the LUT linear layer against the CPU oracle, through the HIP
C-ABI: the single-kernel path (block_dim 16, aligned x) and the two-kernel
LUT-build + gather path (other block sizes, unaligned x).

Bars: bit-exact on integer-valued inputs (every partial sum exact in fp32,
so any summation order gives the same bits) and on the reference's CSR known
answer; rel <= 1e-5 (max-abs error / max |ref|) for fp32 activations and
<= 1e-2 for bf16 activations on random inputs.
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err
from oracle import cpu, gen
from test_oracle import integer_case

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 1e-2


def native_linear(pkg, d, M, K, D=16, Kcb=256):
    nat = pkg.native.NativeSplitManifoldLinear(K, M, D, Kcb)
    nat.initialize_weights(d["codebook"], d["codes"],
                           d["scales"] if d.get("scales") is not None else np.ones(M, np.float32),
                           d.get("bias"))
    if d.get("csr") is not None:
        nat.set_outliers(*d["csr"])
    return nat


def dev_forward(pkg, nat, x_t, dtype_tag, out_dtype):
    import torch
    y = torch.empty(x_t.shape[0], nat.out_features, device=x_t.device, dtype=out_dtype)
    rc = pkg.lib().ojasx_linear_forward_device(
        nat.handle, ctypes.c_void_p(x_t.data_ptr()), ctypes.c_void_p(y.data_ptr()),
        x_t.shape[0], dtype_tag, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("name", ["linear_k256_m200_b3", "linear_d8_k128_m96_b2_cb64",
                                  "linear_k2560_m64_b1", "linear_d64_k512_m72_b3",
                                  "linear_d48_k480_m40_b2_cb100"])
def test_host_api_golden(pkg, name):
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    M, G = g["codes"].shape
    D = g["codebook"].shape[1]
    d = dict(codebook=g["codebook"], codes=g["codes"], scales=g["scales"],
             bias=g["bias"] if "bias" in g else None, csr=(g["row_ptrs"], g["cols"], g["vals"]))
    nat = native_linear(pkg, d, M, G * D, D, g["codebook"].shape[0])
    y = nat.forward(g["x"])
    assert rel_err(y, g["y"]) < F32_TOL


def test_reference_t3_exact(pkg):
    t3 = gen.reference_t3()
    nat = native_linear(pkg, t3, 32, 64)
    y = nat.forward(t3["x"])
    assert np.all(y == 5.0)


def test_reference_t2(pkg):
    t2 = gen.reference_t2()
    nat = native_linear(pkg, t2, 128, 256)
    y = nat.forward(t2["x"])
    g = np.load(os.path.join(GOLDEN, "ref_t2_linear.npz"))["y"][0]
    assert np.abs(y - g).max() < 1e-4
    assert rel_err(y, g) < F32_TOL


@pytest.mark.parametrize("M,K,B", [(97, 640, 2), (6912, 2560, 1), (6912, 2560, 3),
                                   (2560, 2560, 8), (1000, 2560, 64),
                                   (333, 2000, 5),    # 125 groups: partial last slice
                                   (1000, 8192, 3),   # 32 slices: two per wave
                                   (257, 5120, 2),    # 20 slices: one or two per wave
                                   (64, 16, 7),       # one group, one wave
                                   (333, 2000, 35),   # MFMA path: ragged rows, tokens, slices
                                   (70, 464, 33),
                                   (333, 2000, 9),    # MFMA, one row tile per workgroup
                                   (517, 1040, 27),   # MFMA, two row tiles per workgroup
                                   # batch 1, tall: 3 / 4 / 5 row tiles per workgroup
                                   # (48- and 80-row workgroups end past the padded rows)
                                   (9000, 1024, 1), (12289, 256, 1), (19456, 2560, 1),
                                   (20481, 64, 1),    # past 5 tiles: 32-row workgroups
                                   # batch 1, 2048 .. 4095 rows: ceil(M / 256) rows per
                                   # workgroup (8 - 15), the last workgroup ragged
                                   (2048, 512, 1), (2049, 1024, 1), (3001, 2560, 1),
                                   (4095, 256, 1)])
def test_integer_inputs_bit_exact(pkg, dev, M, K, B):
    import torch
    c = integer_case(M * 7 + B, M=M, K=K, B=B)
    nat = native_linear(pkg, dict(codebook=c["codebook"], codes=c["codes"], csr=c["csr"]), M, K)
    y = dev_forward(pkg, nat, torch.from_numpy(c["x"]).to(dev), 0, torch.float32)
    assert np.array_equal(y.cpu().numpy(), c["y"])


@pytest.mark.parametrize("M,K,B", [(2560, 2560, 1), (6912, 2560, 1), (6912, 2560, 8),
                                   (6912, 2560, 64)])
def test_baseline_configs_fp32(pkg, dev, M, K, B):
    import torch
    d = gen.linear(M, K, B=B, seed=M + B, scales="u")
    nat = native_linear(pkg, d, M, K)
    y = dev_forward(pkg, nat, torch.from_numpy(d["x"]).to(dev), 0, torch.float32).cpu().numpy()
    y_ref = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], None, *d["csr"])
    assert rel_err(y, y_ref) < F32_TOL


@pytest.mark.parametrize("M,K,B,dt,density", [
    (700, 2000, 32, 0, 0.02),      # dense outliers: more than the LDS stage holds
    (129, 4096, 40, 0, 0.02),
    (6912, 2560, 36, 1, 0.0038),   # outliers staged in LDS, added slice by slice
    (300, 256, 48, 1, 0.02),
    (1000, 2560, 33, 0, 0.0038),
    (333, 1040, 9, 0, 0.0038),     # one row tile per workgroup, 5 slices (a tail of 1)
    (70, 4096, 16, 1, 0.02),       # one row tile, 16 slices (no tail)
    (95, 2560, 14, 0, 0.05),       # one row tile, outliers past the LDS stage
    (2049, 768, 20, 0, 0.0038),    # two row tiles, 3 slices (main loop skipped)
    (517, 3072, 31, 1, 0.0038),    # two row tiles, 12 slices
    (257, 9728, 65, 0, 0.0038),    # 38 slices (a tail of 2); five 16-token tiles, the last of 1
    (64, 176, 100, 0, 0.02),       # 11 groups in one slice; 100 tokens
    (40, 2560, 128, 1, 0.0038),    # eight full 16-token tiles
    (333, 2000, 9, 1, 0.0038),     # bf16 from 9 tokens on 32 x 32 tiles (9 of 32 tokens)
    (1000, 2560, 57, 0, 0.0038)])  # fp32 two row tiles: a ragged 64-row block and token tile
def test_mfma_batched_shapes(pkg, dev, M, K, B, dt, density):
    """Many tokens (x . W^T on MFMA): ragged rows, tokens and slices, bias,
    outliers given with each row's columns shuffled (the handle sorts them),
    fp32 (rel 1e-5) and bf16 activations (rel 1e-2)."""
    import torch
    d = gen.linear(M, K, B=B, seed=M + K + B, scales="u", bias=True, density=density)
    rp, cl, vl = d["csr"]
    r = np.random.default_rng(M)
    cl, vl = cl.copy(), vl.copy()
    for m in range(M):
        perm = r.permutation(rp[m + 1] - rp[m]) + rp[m]
        cl[rp[m]:rp[m + 1]], vl[rp[m]:rp[m + 1]] = cl[perm], vl[perm]
    d["csr"] = (rp, cl, vl)
    nat = native_linear(pkg, d, M, K)
    x = torch.from_numpy(d["x"]).to(dev)
    if dt:
        x = x.to(torch.bfloat16)
    y = dev_forward(pkg, nat, x, dt, x.dtype).float().cpu().numpy()
    y_ref = cpu.linear_forward(x.float().cpu().numpy(), d["codebook"], d["codes"], d["scales"],
                               d["bias"], *d["csr"])
    assert rel_err(y, y_ref) < (BF16_TOL if dt else F32_TOL)


@pytest.mark.parametrize("B,M", [(1, 6912), (8, 6912), (64, 6912), (1, 19456)])
def test_baseline_gate_up_bf16(pkg, dev, B, M):
    import torch
    d = gen.linear(M, 2560, B=B, seed=50 + B)
    nat = native_linear(pkg, d, M, 2560)
    xb = torch.from_numpy(d["x"]).to(dev).to(torch.bfloat16)
    y = dev_forward(pkg, nat, xb, 1, torch.bfloat16).float().cpu().numpy()
    x_rounded = xb.float().cpu().numpy()
    y_ref = cpu.linear_forward(x_rounded, d["codebook"], d["codes"], d["scales"], None, *d["csr"])
    assert rel_err(y, y_ref) < BF16_TOL


@pytest.mark.parametrize("M,K,D,Kcb,bias", [(300, 200, 8, 256, True), (513, 384, 24, 100, False),
                                            (64, 32, 32, 256, True), (1, 16, 16, 256, False),
                                            (200, 768, 64, 256, True), (96, 1536, 512, 64, False),
                                            (40, 300, 300, 256, True)])
def test_odd_shapes(pkg, dev, M, K, D, Kcb, bias):
    """Groups not a multiple of 16, block_dim != 16 (up to groups wider than
    the 256-thread LUT-build workgroup and a single group), small codebooks,
    one row."""
    d = gen.linear(M, K, B=5, D=D, Kcb=Kcb, seed=M + K, scales="u", bias=bias, density=0.02)
    nat = native_linear(pkg, d, M, K, D, Kcb)
    y = nat.forward(d["x"])
    y_ref = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *d["csr"])
    assert rel_err(y, y_ref) < F32_TOL


@pytest.mark.parametrize("M,K,B", [(130, 1024, 3), (70, 4096, 1)])
def test_dense_outlier_rows(pkg, dev, M, K, B):
    """Rows with more CSR entries than the lanes that share them (4 per wave)."""
    import torch
    d = gen.linear(M, K, B=B, seed=K + B, scales="u", bias=True, density=0.08)
    assert np.diff(d["csr"][0]).max() > 4 * min(K // 256, 16)
    nat = native_linear(pkg, d, M, K)
    y = dev_forward(pkg, nat, torch.from_numpy(d["x"]).to(dev), 0, torch.float32).cpu().numpy()
    y_ref = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *d["csr"])
    assert rel_err(y, y_ref) < F32_TOL


@pytest.mark.parametrize("dtype_tag", [0, 1])
def test_unaligned_activations(pkg, dev, dtype_tag):
    """x that is not 16-byte aligned (fp32) / 8-byte aligned (bf16) takes the
    two-kernel path; results stay within tolerance."""
    import torch
    M, K, B = 300, 512, 3
    d = gen.linear(M, K, B=B, seed=31, scales="u")
    nat = native_linear(pkg, d, M, K)
    tdt = torch.float32 if dtype_tag == 0 else torch.bfloat16
    buf = torch.empty(B * K + 1, device=dev, dtype=tdt)
    xt = buf[1:].view(B, K)
    xt.copy_(torch.from_numpy(d["x"]).to(dev).to(tdt))
    y = dev_forward(pkg, nat, xt, dtype_tag, tdt).float().cpu().numpy()
    x_used = xt.float().cpu().numpy()
    y_ref = cpu.linear_forward(x_used, d["codebook"], d["codes"], d["scales"], None, *d["csr"])
    assert rel_err(y, y_ref) < (F32_TOL if dtype_tag == 0 else BF16_TOL)


def test_repeat_calls_deterministic_and_outlier_reset(pkg):
    """Fixed reduction order: repeated calls give identical bits; nnz = 0
    clears the outliers."""
    d = gen.linear(6912, 2560, B=2, seed=77, scales="u", bias=True)
    nat = native_linear(pkg, d, 6912, 2560)
    ys = [nat.forward(d["x"]) for _ in range(5)]
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    y1 = nat.forward(d["x"][:1])
    assert rel_err(y1[None] if y1.ndim == 1 else y1, ys[0][:1]) < F32_TOL
    nat.set_outliers(np.zeros(6913, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    y0 = nat.forward(d["x"])
    want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"])
    assert rel_err(y0, want) < F32_TOL


def test_host_calls_from_threads(pkg):
    """Host-pointer calls stage through a per-thread pinned buffer and stream:
    four threads, each with its own layer and batch sizes that grow and shrink
    the buffer, give the same results as the oracle."""
    import threading
    cases = [gen.linear(256 + 64 * i, 512, B=1 + 7 * i, seed=90 + i, scales="u", bias=True)
             for i in range(4)]
    errs = [None] * 4

    def run(i):
        try:
            d = cases[i]
            M = d["codes"].shape[0]
            nat = native_linear(pkg, d, M, 512)
            want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"],
                                      *d["csr"])
            for rep in range(6):
                b = d["x"].shape[0] if rep % 2 == 0 else 1
                y = nat.forward(d["x"][:b])
                y = y.reshape(b, M)
                assert rel_err(y, want[:b]) < F32_TOL, (i, rep)
        except BaseException as e:   # reported by the main thread
            errs[i] = e

    ts = [threading.Thread(target=run, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    for e in errs:
        if e is not None:
            raise e


def test_invalid_outliers_rejected(pkg):
    d = gen.linear(64, 256, seed=3)
    nat = native_linear(pkg, dict(codebook=d["codebook"], codes=d["codes"]), 64, 256)
    rp = np.zeros(65, np.int32)
    rp[1:] = 1
    with pytest.raises(pkg.OjasxError):
        nat.set_outliers(rp, np.array([256], np.int32), np.array([1.0], np.float32))
    L = pkg.lib()
    assert L.ojasx_linear_forward(None, None, None, 1, 0) == -1
    assert L.ojasx_set_linear_outliers(None, 0, None, None, None) == -1


def test_zero_batch_noop(pkg, dev):
    import torch
    d = gen.linear(64, 256, seed=4)
    nat = native_linear(pkg, d, 64, 256)
    y = torch.full((1, 64), 3.0, device=dev)
    rc = pkg.lib().ojasx_linear_forward_device(nat.handle, ctypes.c_void_p(y.data_ptr()),
                                               ctypes.c_void_p(y.data_ptr()), 0, 0, None)
    torch.cuda.synchronize()
    assert rc == 0 and bool((y == 3.0).all())


def test_build_lut_device(pkg, dev):
    import torch
    eng = pkg.engine
    d = gen.linear(8, 2560, B=3, seed=5)
    layer = eng.SplitManifoldLUTLinear(2560, 8).to(dev)
    layer.codebook.copy_(torch.from_numpy(d["codebook"]))
    lut = layer.build_lut(torch.from_numpy(d["x"]).to(dev)).cpu().numpy()
    for b in range(3):
        assert rel_err(lut[b], cpu.build_lut(d["x"][b], d["codebook"])) < 1e-6


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_engine_module(pkg, dev, dtype):
    """SplitManifoldLUTLinear API: COO outliers, bias, leading batch dims."""
    import torch
    dt = getattr(torch, dtype)
    d = gen.linear(640, 1024, B=6, seed=9, scales="u", bias=True)
    layer = pkg.engine.SplitManifoldLUTLinear(1024, 640, bias=True, dtype=dt).to(dev)
    layer.codebook.copy_(torch.from_numpy(d["codebook"]))
    layer.codes.copy_(torch.from_numpy(d["codes"]))
    layer.scales.copy_(torch.from_numpy(d["scales"]))
    layer.bias.data.copy_(torch.from_numpy(d["bias"]))
    rp, cl, vl = d["csr"]
    rows = np.repeat(np.arange(640), np.diff(rp))
    layer.outlier_indices = torch.from_numpy(np.stack([rows, cl]).astype(np.int64)).to(dev)
    layer.outlier_values = torch.from_numpy(vl).to(dev).to(dt)
    layer.num_outliers = vl.size
    x = torch.from_numpy(d["x"]).to(dev).to(dt).view(2, 3, 1024)
    y = layer(x)
    assert y.shape == (2, 3, 640) and y.dtype == dt
    # reference semantics on the module's own (possibly bf16-rounded) buffers
    f = lambda t: t.detach().float().cpu().numpy()
    y_ref = cpu.linear_forward(f(x).reshape(6, 1024), f(layer.codebook), d["codes"],
                               f(layer.scales), f(layer.bias), rp, cl, f(layer.outlier_values))
    tol = F32_TOL if dt == torch.float32 else BF16_TOL
    assert rel_err(f(y).reshape(6, 640), y_ref) < tol
    # the diagnostic dense weight reproduces the same layer
    W = f(layer.dequantize_weights()).astype(np.float64)
    assert rel_err(f(y).reshape(6, 640), f(x).reshape(6, 1024) @ W.T + f(layer.bias)) < tol * 10


@pytest.mark.parametrize("B", [1, 8, 64])
def test_bf16_matches_reference_bf16_module(pkg, dev, B):
    """bf16 parity against the reference's own bf16 path: outputs of its
    PyTorch module with bf16 buffers (split_manifold_engine.py:22-250, LUT
    matmul and gather sum in bf16), written in the build container by
    tests/golden/make_bf16_golden.py from the same seeded inputs.  The HIP
    path keeps the LUT and its sums in fp32, so it agrees to the bf16 bar
    (rel 1e-2, max-abs error over max |ref|) rather than bit for bit."""
    import sys
    import torch
    sys.path.insert(0, GOLDEN)
    from make_bf16_golden import M, K, bf16_inputs
    g = np.load(os.path.join(GOLDEN, "engine_bf16_2560x6912.npz"))
    t = bf16_inputs()
    layer = pkg.engine.SplitManifoldLUTLinear(K, M, bias=True, dtype=torch.bfloat16).to(dev)
    with torch.no_grad():
        for k in ("codebook", "codes", "scales"):
            getattr(layer, k).copy_(t[k])
        layer.bias.data.copy_(t["bias"])
    layer.outlier_indices = t["outlier_indices"].to(dev)
    layer.outlier_values = t["outlier_values"].to(dev)
    layer.num_outliers = int(t["outlier_values"].numel())
    y = layer(t["x"][:B].to(dev))
    assert y.dtype == torch.bfloat16
    y = y.float().cpu().numpy()
    if B == 64:
        y = y[:, ::int(g["col_stride_b64"])]
    want = torch.from_numpy(g[f"y_b{B}"].view(np.int16)).view(torch.bfloat16).float().numpy()
    err = rel_err(y, want)
    print(f"bf16 2560->6912 B={B}: rel err vs the reference bf16 module {err:.2e}", flush=True)
    assert err < BF16_TOL


def test_cpu_tensor_fails_loudly(pkg):
    import torch
    layer = pkg.engine.SplitManifoldLUTLinear(32, 8)
    with pytest.raises(RuntimeError, match="GPU only"):
        layer(torch.zeros(1, 32))


@pytest.mark.parametrize("B", [1, 2, 5])
def test_large_m_tile_loop(pkg, dev, B):
    """60000 output rows: more row tiles than resident workgroups, so each
    workgroup walks several tiles with the codebook and x staged once."""
    import torch
    M, K = 60000, 2560
    d = gen.linear(M, K, B=B, seed=60 + B, scales="u", bias=True)
    nat = native_linear(pkg, d, M, K)
    x_t = torch.from_numpy(d["x"]).to(dev)
    y = dev_forward(pkg, nat, x_t, 0, torch.float32).cpu().numpy()
    want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *d["csr"])
    assert rel_err(y, want) < F32_TOL


def test_grouped_linears(pkg, dev):
    """Many linears of different shapes in one launch (MFMA-built LUT slices)
    against the oracle, each rel <= 1e-5: partial row blocks, one-slice and
    38-slice inputs, with and without outliers and bias."""
    import torch
    shapes = [(6912, 2560, True, False), (700, 256, False, True), (513, 9728, True, True),
              (40, 64, True, False), (1025, 4096, False, False)]
    nats, xs, ys, ds = [], [], [], []
    for i, (M, K, outl, bias) in enumerate(shapes):
        d = gen.linear(M, K, B=1, seed=90 + i, scales="u", bias=bias, outliers=outl)
        nats.append(native_linear(pkg, d, M, K))
        xs.append(torch.from_numpy(d["x"][0]).to(dev))
        ys.append(torch.full((M,), 7.0, device=dev))
        ds.append(d)
    n = len(shapes)
    H = (ctypes.c_void_p * n)(*[nat.handle for nat in nats])
    X = (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs])
    Y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    rc = pkg.lib().ojasx_linear_forward_grouped_device(H, n, X, Y, None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    for (M, K, outl, bias), d, y in zip(shapes, ds, ys):
        csr = d["csr"] if outl else (np.zeros(M + 1, np.int32), np.zeros(0, np.int32),
                                     np.zeros(0, np.float32))
        want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"], *csr)
        assert rel_err(y.cpu().numpy()[None], want) < F32_TOL, (M, K)


def test_grouped_linears_wide_inputs(pkg, dev):
    """Items whose input exceeds the bank kernel's LDS (K > 16384, e.g. an
    18944-wide down projection) run on the single-linear path inside the same
    grouped call; the others stay on the bank kernel.  Also a call of wide
    items only."""
    import torch
    shapes = [(300, 18944, True), (700, 2560, True), (96, 20480, False), (64, 16384, True)]
    nats, xs, ys, ds = [], [], [], []
    for i, (M, K, outl) in enumerate(shapes):
        d = gen.linear(M, K, B=1, seed=150 + i, scales="u", bias=True, outliers=outl)
        nats.append(native_linear(pkg, d, M, K))
        xs.append(torch.from_numpy(d["x"][0]).to(dev))
        ys.append(torch.full((M,), 7.0, device=dev))
        ds.append(d)
    for sel in ([0, 1, 2, 3], [2, 0]):
        n = len(sel)
        H = (ctypes.c_void_p * n)(*[nats[i].handle for i in sel])
        X = (ctypes.c_void_p * n)(*[xs[i].data_ptr() for i in sel])
        Y = (ctypes.c_void_p * n)(*[ys[i].data_ptr() for i in sel])
        rc = pkg.lib().ojasx_linear_forward_grouped_device(H, n, X, Y, None)
        assert rc == 0, pkg.lib().ojasx_get_last_error()
        torch.cuda.synchronize()
        for i in sel:
            M, K, outl = shapes[i]
            d = ds[i]
            csr = d["csr"] if outl else (np.zeros(M + 1, np.int32), np.zeros(0, np.int32),
                                         np.zeros(0, np.float32))
            want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"],
                                      *csr)
            assert rel_err(ys[i].cpu().numpy()[None], want) < F32_TOL, (M, K)


def test_grouped_linears_repeat_and_errors(pkg, dev):
    """Two grouped calls in a row (the second with fewer linears reuses the
    staged item buffer), an empty call, and the argument checks."""
    import torch
    L = pkg.lib()
    shapes = [(300, 512), (1100, 1024), (64, 160)]
    nats, xs, ds = [], [], []
    for i, (M, K) in enumerate(shapes):
        d = gen.linear(M, K, B=1, seed=130 + i, scales="u", bias=True, outliers=True)
        nats.append(native_linear(pkg, d, M, K))
        xs.append(torch.from_numpy(d["x"][0]).to(dev))
        ds.append(d)

    def run(sel):
        ys = [torch.full((shapes[i][0],), -1.0, device=dev) for i in sel]
        n = len(sel)
        H = (ctypes.c_void_p * n)(*[nats[i].handle for i in sel])
        X = (ctypes.c_void_p * n)(*[xs[i].data_ptr() for i in sel])
        Y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        assert L.ojasx_linear_forward_grouped_device(H, n, X, Y, None) == 0, L.ojasx_get_last_error()
        torch.cuda.synchronize()
        for i, y in zip(sel, ys):
            d = ds[i]
            want = cpu.linear_forward(d["x"], d["codebook"], d["codes"], d["scales"], d["bias"],
                                      *d["csr"])
            assert rel_err(y.cpu().numpy()[None], want) < F32_TOL, shapes[i]

    run([0, 1, 2])
    run([2, 0])
    one = (ctypes.c_void_p * 1)(nats[0].handle)
    xp = (ctypes.c_void_p * 1)(xs[0].data_ptr())
    y = torch.empty(shapes[0][0], device=dev)
    yp = (ctypes.c_void_p * 1)(y.data_ptr())
    assert L.ojasx_linear_forward_grouped_device(one, 0, xp, yp, None) == 0
    assert L.ojasx_linear_forward_grouped_device(None, 1, xp, yp, None) != 0
    bad = (ctypes.c_void_p * 1)(xs[0].data_ptr() + 4)
    assert L.ojasx_linear_forward_grouped_device(one, 1, bad, yp, None) != 0
    assert b"aligned" in L.ojasx_get_last_error()


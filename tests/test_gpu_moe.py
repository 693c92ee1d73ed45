"""GPU parity of the top-k MoE path (K4) and the router, through the C-ABI.

Bars: router indices bit-exact (ties to the lower index); router weights
rel <= 1e-6; MoE outputs rel <= 1e-5 (fp32) / 1e-2 (bf16 activations)
against the CPU oracle (itself bit-exact with the reference engine).
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err
from oracle import cpu, gen

pytestmark = pytest.mark.gpu


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def make_native(pkg, m, E, H, I, k=10):
    nat = pkg.native.NativeSplitManifoldMoE(E, H, I, k, m["cb_in"].shape[1])
    nat.initialize_weights(m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                           m["dn_codes"], m["dn_scales"])
    return nat


def test_host_api_golden_skip_rules(pkg):
    g = np.load(os.path.join(GOLDEN, "moe_e32_h128_i64.npz"))
    nat = make_native(pkg, g, 32, 128, 64, 6)
    y = nat.forward(g["x"], g["idx"], g["w"])
    assert rel_err(y, g["y"]) < 1e-5


@pytest.mark.parametrize("name", ["moe_d24_e16_h96_i72", "moe_d64_e8_h256_i128"])
def test_host_api_golden_block_sizes(pkg, name):
    """block_dim 24 (not dividing 32) and 64 against the compiled reference."""
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    E, two_i, _ = g["gu_codes"].shape
    H = g["dn_codes"].shape[1]
    nat = make_native(pkg, g, E, H, two_i // 2, g["idx"].size)
    y = nat.forward(g["x"], g["idx"], g["w"])
    assert rel_err(y, g["y"]) < 1e-5


def test_host_api_reference_t6(pkg):
    t6 = gen.reference_t6()
    nat = make_native(pkg, t6, 512, 256, 64)
    y = nat.forward(t6["x"], t6["idx"], t6["w"])
    want = np.load(os.path.join(GOLDEN, "ref_t6_moe.npz"))["y"]
    assert rel_err(y, want) < 1e-5


def test_k_active_zero_leaves_output(pkg):
    g = np.load(os.path.join(GOLDEN, "moe_e32_h128_i64.npz"))
    nat = make_native(pkg, g, 32, 128, 64, 6)
    y = np.full(128, 7.0, np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    x, idx, w = (np.ascontiguousarray(g[n]) for n in ("x", "idx", "w"))
    assert pkg.lib().ojasx_moe_forward(nat.handle, p(x), p(idx), p(w), p(y), 0) == 0
    assert np.all(y == 7.0)


def route(pkg, logits_t, k, renorm):
    import torch
    T, E = logits_t.shape
    idx = torch.empty(T, k, dtype=torch.int32, device=logits_t.device)
    w = torch.empty(T, k, dtype=torch.float32, device=logits_t.device)
    rc = pkg.lib().ojasx_moe_route_device(vp(logits_t), T, E, k, int(renorm), vp(idx), vp(w),
                                          None)
    assert rc == 0
    torch.cuda.synchronize()
    return idx, w


@pytest.mark.parametrize("renorm", [False, True])
def test_router_bit_exact_indices(pkg, dev, renorm):
    import torch
    m = gen.moe(E=512, H=16, I=16, T=16, seed=30)
    lg = m["logits"].copy()
    lg[3, [7, 300, 301]] = 5.0                       # ties at the top
    lg[4, :] = 0.25                                  # all equal
    idx, w = route(pkg, torch.from_numpy(lg).to(dev), 10, renorm)
    i_ref, w_ref = cpu.router_topk(lg, 10, renorm)
    assert np.array_equal(idx.cpu().numpy(), i_ref)
    assert rel_err(w.cpu().numpy(), w_ref) < 1e-6


@pytest.fixture(scope="module")
def baseline_moe(pkg):
    m = gen.moe(E=512, H=2048, I=768, T=32, seed=2024, scales="u")
    nat = make_native(pkg, m, 512, 2048, 768)
    return m, nat


@pytest.mark.parametrize("T", [1, 16, 32])
def test_baseline_moe_fp32(pkg, dev, baseline_moe, T):
    import torch
    m, nat = baseline_moe
    logits = torch.from_numpy(m["logits"][:T]).to(dev)
    idx, w = route(pkg, logits, 10, False)
    x = torch.from_numpy(m["x"][:T]).to(dev)
    y = torch.empty(T, 2048, device=dev)
    rc = pkg.lib().ojasx_moe_forward_device(nat.handle, vp(x), vp(idx), vp(w), vp(y), T, 10, 0,
                                            None)
    assert rc == 0
    torch.cuda.synchronize()
    idx_h, w_h = idx.cpu().numpy(), w.cpu().numpy()
    i_ref, _ = cpu.router_topk(m["logits"][:T], 10)
    assert np.array_equal(idx_h, i_ref)
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx_h[t], w_h[t])
        assert rel_err(y[t].cpu().numpy(), want) < 1e-5, t


@pytest.mark.parametrize("T", [4, 32])   # grouped-per-slot path; token-major + pair-major kernels
def test_baseline_moe_bf16(pkg, dev, baseline_moe, T):
    import torch
    m, nat = baseline_moe
    idx, w = route(pkg, torch.from_numpy(m["logits"][:T]).to(dev), 10, True)
    x = torch.from_numpy(m["x"][:T]).to(dev).to(torch.bfloat16)
    y = torch.empty(T, 2048, device=dev, dtype=torch.bfloat16)
    rc = pkg.lib().ojasx_moe_forward_device(nat.handle, vp(x), vp(idx), vp(w), vp(y), T, 10, 1,
                                            None)
    assert rc == 0
    torch.cuda.synchronize()
    xr = x.float().cpu().numpy()
    for t in range(T):
        want = cpu.moe_forward(xr[t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t].cpu().numpy(),
                               w[t].cpu().numpy())
        assert rel_err(y[t].float().cpu().numpy(), want) < 1e-2


@pytest.mark.parametrize("T", [1, 4, 20, 28])   # in-place, grouped-per-slot, by-expert, token-major
def test_repeat_deterministic_and_skips(pkg, dev, baseline_moe, T):
    """Skipped slots (id out of range, |w| < 1e-8) and repeated experts within a
    token; repeated calls return identical bits."""
    import torch
    m, nat = baseline_moe
    row_i = np.array([5, 600, 5, 9, -3, 11, 12, 13, 14, 15], np.int32)
    row_w = np.array([0.2, 0.3, 0.1, 1e-9, 0.1, 0.05, 0.05, 0.05, 0.1, 0.05], np.float32)
    idx = np.stack([np.roll(row_i, t) for t in range(T)])
    w = np.stack([np.roll(row_w, t) for t in range(T)])
    it, wt = torch.from_numpy(idx).to(dev), torch.from_numpy(w).to(dev)
    x = torch.from_numpy(m["x"][:T]).to(dev)
    ys = []
    for _ in range(3):
        y = torch.empty(T, 2048, device=dev)
        assert pkg.lib().ojasx_moe_forward_device(nat.handle, vp(x), vp(it), vp(wt), vp(y), T, 10,
                                                  0, None) == 0
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(ys[0][t], want) < 1e-5, t
    assert all(np.array_equal(ys[0], yy) for yy in ys[1:])


def device_moe(pkg, dev, nat, x_t, idx, w, k, dtype_tag=0):
    import torch
    T, H = x_t.shape
    y = torch.empty(T, H, device=dev, dtype=x_t.dtype)
    it = torch.from_numpy(np.ascontiguousarray(idx, np.int32)).to(dev)
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(dev)
    rc = pkg.lib().ojasx_moe_forward_device(nat.handle, vp(x_t), vp(it), vp(wt), vp(y), T, k,
                                            dtype_tag, None)
    assert rc == 0, pkg.lib().ojasx_get_last_error()
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


# below / from the token count that selects the grouped path; from the one
# that groups the routed pairs by expert (bank kernel: partial slices, rows)
@pytest.mark.parametrize("T", [2, 6, 20, 28])
@pytest.mark.parametrize("E,H,I,k,D", [
    (40, 480, 208, 20, 16),    # partial input/intermediate slices; 20 slots > 16 waves
    (64, 512, 256, 32, 16),    # the largest k of the single-kernel stages
    (48, 256, 96, 6, 8),       # block_dim 8: LUT-build + gather path
    (16, 96, 72, 6, 24),       # block_dim 24 (does not divide 32)
    (12, 640, 384, 4, 128),    # block_dim 128
    (24, 4352, 1152, 4, 16),   # 17 input slices, 5 intermediate slices
])
def test_moe_shapes(pkg, dev, E, H, I, k, D, T):
    import torch
    m = gen.moe(E=E, H=H, I=I, T=T, D=D, seed=E + k, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    idx[0, 1] = idx[0, 0]                           # a repeated expert within a token
    y = device_moe(pkg, dev, nat, torch.from_numpy(m["x"]).to(dev), idx, w, k)
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < 1e-5, t


@pytest.mark.parametrize("dtype_tag", [0, 1])
def test_moe_unaligned_activations(pkg, dev, baseline_moe, dtype_tag):
    """x not aligned for vector loads takes the LUT-build path."""
    import torch
    m, nat = baseline_moe
    T = 2
    tdt = torch.float32 if dtype_tag == 0 else torch.bfloat16
    buf = torch.empty(T * 2048 + 1, device=dev, dtype=tdt)
    xt = buf[1:].view(T, 2048)
    xt.copy_(torch.from_numpy(m["x"][:T]).to(dev).to(tdt))
    idx, w = cpu.router_topk(m["logits"][:T], 10)
    y = device_moe(pkg, dev, nat, xt, idx, w, 10, dtype_tag)
    xr = xt.float().cpu().numpy()
    for t in range(T):
        want = cpu.moe_forward(xr[t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < (1e-5 if dtype_tag == 0 else 1e-2)


@pytest.mark.parametrize("T", [64, 160])
@pytest.mark.parametrize("dtype_tag", [0, 1])
def test_moe_by_expert_many_pairs_per_expert(pkg, dev, dtype_tag, T):
    """256 and 640 routed pairs over 8 experts (32 and 80 per expert on
    average) on the token-major gate/up and pair-major down kernels; skipped
    slots, fp32 and bf16."""
    import torch
    E, H, I, k = 8, 256, 96, 4
    m = gen.moe(E=E, H=H, I=I, T=T, seed=77, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    idx[3, 2] = E + 5                                # out of range: skipped
    w[7, 1] = 0.0                                    # below 1e-8: skipped
    tdt = torch.float32 if dtype_tag == 0 else torch.bfloat16
    xt = torch.from_numpy(m["x"]).to(dev).to(tdt)
    y = device_moe(pkg, dev, nat, xt, idx, w, k, dtype_tag)
    xr = xt.float().cpu().numpy()
    for t in range(T):
        want = cpu.moe_forward(xr[t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < (1e-5 if dtype_tag == 0 else 1e-2), t


def test_token_major_rows_equal_bank_rows(pkg, dev, baseline_moe):
    """Gate/up runs per (pair, row block) below 24 tokens and token-major from
    24: a token's output row is the same bits either way."""
    import torch
    m, nat = baseline_moe
    idx, w = cpu.router_topk(m["logits"], 10)
    x = torch.from_numpy(m["x"]).to(dev)
    y16 = device_moe(pkg, dev, nat, x[:16].contiguous(), idx[:16], w[:16], 10)
    y32 = device_moe(pkg, dev, nat, x, idx, w, 10)
    assert np.array_equal(y16, y32[:16])


@pytest.mark.parametrize("dtype_tag", [0, 1])
def test_moe_token_major_full_workgroups(pkg, dev, dtype_tag):
    """72 tokens x 8 slots x 4 gate/up row blocks (the last one partial):
    eight units per token-major workgroup, the last workgroup of each token
    short; down over 3 row blocks (the last partial) and a partial second
    slice; skipped and repeated slots."""
    import torch
    E, H, I, k, T = 32, 1200, 1008, 8, 72
    m = gen.moe(E=E, H=H, I=I, T=T, seed=4321, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    idx[4, 3] = -1                                   # out of range: skipped
    idx[10, 0] = E                                   # out of range: skipped
    w[20, 7] = 5e-9                                  # below 1e-8: skipped
    idx[30, 2] = idx[30, 5]                          # repeated expert within a token
    tdt = torch.float32 if dtype_tag == 0 else torch.bfloat16
    xt = torch.from_numpy(m["x"]).to(dev).to(tdt)
    y = device_moe(pkg, dev, nat, xt, idx, w, k, dtype_tag)
    xr = xt.float().cpu().numpy()
    for t in range(T):
        want = cpu.moe_forward(xr[t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < (1e-5 if dtype_tag == 0 else 1e-2), t


def test_moe_plan_sorted_down(pkg, dev):
    """160 tokens with 1152 intermediate values (beyond the pair-major down
    kernel's two slices): the plan sorts the pairs by expert and down runs on
    the bank kernel's work list, gate/up token-major."""
    import torch
    E, H, I, k, T = 8, 256, 1152, 4, 160
    m = gen.moe(E=E, H=H, I=I, T=T, seed=99, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    idx[11, 0] = -2                                  # out of range: skipped
    y = device_moe(pkg, dev, nat, torch.from_numpy(m["x"]).to(dev), idx, w, k)
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < 1e-5, t


@pytest.mark.parametrize("case", range(8))
def test_moe_seeded_shapes_around_thresholds(pkg, dev, case):
    """Seeded shapes around the path thresholds (16, 24, 128 tokens) with
    hidden and intermediate sizes any multiple of 16 (partial slices, partial
    64- and 512-row blocks), on the bank, token-major and pair-major kernels."""
    import torch
    r = np.random.default_rng(900 + case)
    T = (16, 23, 24, 25, 47, 130, 24, 130)[case]
    E = int(r.integers(3, 40))
    k = int(r.integers(1, min(E, 8) + 1))
    H = 16 * int(r.integers(1, 129))                 # up to 2048
    I = 16 * int(r.integers(1, 65))                  # up to 1024
    m = gen.moe(E=E, H=H, I=I, T=T, seed=1000 + case, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    tdt = torch.bfloat16 if case % 3 == 2 else torch.float32
    xt = torch.from_numpy(m["x"]).to(dev).to(tdt)
    y = device_moe(pkg, dev, nat, xt, idx, w, k, 1 if tdt == torch.bfloat16 else 0)
    xr = xt.float().cpu().numpy()
    for t in range(T):
        want = cpu.moe_forward(xr[t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        tol = 1e-2 if tdt == torch.bfloat16 else 1e-5
        assert rel_err(y[t], want) < tol, (case, T, E, k, H, I, t)


@pytest.mark.parametrize("T", [16, 64])
def test_moe_graph_replay_matches_eager(pkg, dev, T):
    """The T >= 16 launch sequence (bank or token-major gate/up, pair-major
    down, combine) captured in a HIP graph: every replay, with eager calls
    and synchronisations between replays, returns the eager bits."""
    import torch
    E, H, I, k = 64, 512, 256, 8
    m = gen.moe(E=E, H=H, I=I, T=T, seed=321 + T, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    x = torch.from_numpy(m["x"]).to(dev)
    it = torch.from_numpy(np.ascontiguousarray(idx, np.int32)).to(dev)
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(dev)
    y = torch.empty(T, H, device=dev)
    L = pkg.lib()

    def call(stream):
        return L.ojasx_moe_forward_device(nat.handle, vp(x), vp(it), vp(wt), vp(y), T, k, 0, stream)

    assert call(None) == 0                          # eager: sizes the workspaces
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        assert call(ctypes.c_void_p(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    other = torch.empty_like(y)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), rep
        # eager work between replays (a call into another buffer)
        assert L.ojasx_moe_forward_device(nat.handle, vp(x), vp(it), vp(wt), vp(other), T, k, 0,
                                          None) == 0
        torch.cuda.synchronize()
        assert torch.equal(other, eager), rep
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(eager[t].cpu().numpy(), want) < 1e-5, t
    del g


@pytest.mark.parametrize("H,I", [(18432, 64), (256, 17408), (36864, 48)])
def test_moe_wide_hidden_or_intermediate(pkg, dev, H, I):
    """16 tokens with a hidden (or intermediate) size beyond the by-expert
    kernel's LDS: the call takes a path that fits (the per-slot kernels, or
    the L2-LUT kernels where even their staged input does not fit)."""
    import torch
    E, k, T = 6, 2, 16
    m = gen.moe(E=E, H=H, I=I, T=T, seed=H % 89, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    y = device_moe(pkg, dev, nat, torch.from_numpy(m["x"]).to(dev), idx, w, k)
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < 1e-5, t


@pytest.mark.parametrize("E,T", [(4096, 16), (16384, 16), (4096, 128), (16384, 128)])
def test_moe_many_experts(pkg, dev, E, T):
    """Large expert counts: at 16 tokens the gate/up bank kernel maps
    workgroups to (pair, row block) directly; at 128 tokens both stages run
    the resident-LUT kernels, which need no plan (no per-expert LDS)."""
    import torch
    H, I, k = 64, 32, 4
    m = gen.moe(E=E, H=H, I=I, T=T, seed=E % 97, scales="u")
    nat = make_native(pkg, m, E, H, I, k)
    idx, w = cpu.router_topk(m["logits"], k, renorm=True)
    idx[2, 3] = idx[2, 0]                            # a repeated expert within a token
    idx[5, 1] = idx[9, 2]                            # and across tokens
    y = device_moe(pkg, dev, nat, torch.from_numpy(m["x"]).to(dev), idx, w, k)
    for t in range(T):
        want = cpu.moe_forward(m["x"][t], m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"], idx[t], w[t])
        assert rel_err(y[t], want) < 1e-5, t

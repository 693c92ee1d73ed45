"""Seeded synthetic inputs for the benchmark configurations (NumPy PCG64).

TEST INFRASTRUCTURE ONLY.  Inputs are generated once here and fed to both the
GPU path and the CPU oracle, so both see identical bytes.  Shapes and
distributions follow the benchmark configurations:

* linear:  x ~ N(0,1); codebook [256,16] ~ N(0, 0.02); codes uniform {0..255}
           [M, K/16]; CSR outliers at 0.38 % of entries, drawn without
           replacement, |v| ~ U[15 sigma, 36 sigma] (sigma = 0.02), random sign
* moe:     codebooks [256,16] ~ N(0, 0.02) shared by all experts; gate/up codes
           [E, 2I, H/16], down codes [E, H, I/16] uniform; router logits ~ N(0,1)
* kv:      per kv head K and V codebooks [256,16] ~ N(0,1); codes uniform;
           per-token scales ~ U[0.5, 1.5]; q ~ N(0,1)
"""
import numpy as np

OUTLIER_DENSITY = 0.0038
SIGMA = 0.02


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def csr_outliers(r, M, K, density=OUTLIER_DENSITY, sigma=SIGMA):
    """Distinct (row, col) positions sorted row-major, CSR int32/int32/fp32."""
    nnz = int(round(density * M * K))
    if nnz == 0:
        return (np.zeros(M + 1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    pos = np.sort(r.choice(M * K, size=nnz, replace=False))
    rows = (pos // K).astype(np.int64)
    cols = (pos % K).astype(np.int32)
    mag = r.uniform(15.0 * sigma, 36.0 * sigma, size=nnz)
    sign = np.where(r.integers(0, 2, size=nnz) == 0, -1.0, 1.0)
    vals = (mag * sign).astype(np.float32)
    row_ptrs = np.zeros(M + 1, np.int64)
    np.add.at(row_ptrs, rows + 1, 1)
    row_ptrs = np.cumsum(row_ptrs).astype(np.int32)
    return row_ptrs, cols, vals


def linear(M, K, B=1, D=16, Kcb=256, seed=0, outliers=True, scales="one", bias=False,
           cb_sigma=SIGMA, density=OUTLIER_DENSITY):
    r = rng(seed)
    G = K // D
    codebook = r.normal(0.0, cb_sigma, size=(Kcb, D)).astype(np.float32)
    codes = r.integers(0, Kcb, size=(M, G), dtype=np.int64).astype(np.uint8)
    if scales == "one":
        sc = np.ones(M, np.float32)
    else:
        sc = r.uniform(0.5, 1.5, size=M).astype(np.float32)
    bs = r.normal(0.0, 0.1, size=M).astype(np.float32) if bias else None
    csr = csr_outliers(r, M, K, density) if outliers else None
    x = r.normal(0.0, 1.0, size=(B, K)).astype(np.float32)
    return dict(codebook=codebook, codes=codes, scales=sc, bias=bs, csr=csr, x=x)


def moe(E=512, H=2048, I=768, T=1, D=16, Kcb=256, seed=0, scales="one"):
    r = rng(seed)
    cb_in = r.normal(0.0, SIGMA, size=(Kcb, D)).astype(np.float32)
    cb_down = r.normal(0.0, SIGMA, size=(Kcb, D)).astype(np.float32)
    gu_codes = r.integers(0, Kcb, size=(E, 2 * I, H // D), dtype=np.int64).astype(np.uint8)
    dn_codes = r.integers(0, Kcb, size=(E, H, I // D), dtype=np.int64).astype(np.uint8)
    if scales == "one":
        gu_scales = np.ones((E, 2 * I), np.float32)
        dn_scales = np.ones((E, H), np.float32)
    else:
        gu_scales = r.uniform(0.5, 1.5, size=(E, 2 * I)).astype(np.float32)
        dn_scales = r.uniform(0.5, 1.5, size=(E, H)).astype(np.float32)
    x = r.normal(0.0, 1.0, size=(T, H)).astype(np.float32)
    logits = r.normal(0.0, 1.0, size=(T, E)).astype(np.float32)
    return dict(cb_in=cb_in, cb_down=cb_down, gu_codes=gu_codes, gu_scales=gu_scales,
                dn_codes=dn_codes, dn_scales=dn_scales, x=x, logits=logits)


def kv(H_kv=8, H_q=32, T=2048, head_dim=128, D=16, page=16, seed=0, shuffle_pages=False,
       unit_scales=False):
    """Paged code-domain KV cache: codes [n_pages_total, H_kv, page, G], scales
    [n_pages_total, H_kv, page], with a block table mapping logical page ->
    physical page."""
    r = rng(seed)
    G = head_dim // D
    n_pages = (T + page - 1) // page
    k_cb = r.normal(0.0, 1.0, size=(H_kv, 256, D)).astype(np.float32)
    v_cb = r.normal(0.0, 1.0, size=(H_kv, 256, D)).astype(np.float32)
    k_codes = r.integers(0, 256, size=(n_pages, H_kv, page, G), dtype=np.int64).astype(np.uint8)
    v_codes = r.integers(0, 256, size=(n_pages, H_kv, page, G), dtype=np.int64).astype(np.uint8)
    if unit_scales:
        k_scales = np.ones((n_pages, H_kv, page), np.float32)
        v_scales = np.ones((n_pages, H_kv, page), np.float32)
    else:
        k_scales = r.uniform(0.5, 1.5, size=(n_pages, H_kv, page)).astype(np.float32)
        v_scales = r.uniform(0.5, 1.5, size=(n_pages, H_kv, page)).astype(np.float32)
    block_table = np.arange(n_pages, dtype=np.int32)
    if shuffle_pages:
        block_table = r.permutation(n_pages).astype(np.int32)
    q = r.normal(0.0, 1.0, size=(H_q, head_dim)).astype(np.float32)
    return dict(k_cb=k_cb, v_cb=v_cb, k_codes=k_codes, v_codes=v_codes, k_scales=k_scales,
                v_scales=v_scales, block_table=block_table, q=q, T=T, page=page)


def kv_logical(d, kv_head):
    """Gather one kv head's logical token stream [T, G] from the paged layout."""
    T, page = d["T"], d["page"]
    bt = d["block_table"]
    kc = d["k_codes"][bt][:, kv_head].reshape(-1, d["k_codes"].shape[-1])[:T]
    vc = d["v_codes"][bt][:, kv_head].reshape(-1, d["v_codes"].shape[-1])[:T]
    ks = d["k_scales"][bt][:, kv_head].reshape(-1)[:T]
    vs = d["v_scales"][bt][:, kv_head].reshape(-1)[:T]
    return kc, ks, vc, vs


def reference_t2():
    """Fully formula-determined setup of the reference's linear test
    (NAT/tests/test_native_lut.cpp:30-93): 256 -> 128, D = 16."""
    in_f, out_f, D, Kcb = 256, 128, 16, 256
    G = in_f // D
    k = np.arange(Kcb, dtype=np.float32)[:, None]
    d = np.arange(D, dtype=np.float32)[None, :]
    codebook = (((k % 17) - 8) * np.float32(0.1) + d * np.float32(0.01)).astype(np.float32)
    m = np.arange(out_f)[:, None]
    g = np.arange(G)[None, :]
    codes = ((m * 3 + g * 7) % 256).astype(np.uint8)
    scales = (1.0 + 0.01 * np.arange(out_f, dtype=np.float32)).astype(np.float32)
    x = np.sin(np.arange(in_f, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    return dict(codebook=codebook, codes=codes, scales=scales, x=x)


def reference_t3():
    """CSR known answer (NAT/tests/test_native_lut.cpp:95-126): 64 -> 32, zero
    codebook, two outliers per row (+10 at col 2m mod 64, -5 at 2m+1 mod 64),
    x = 1, so y == 5 exactly."""
    in_f, out_f = 64, 32
    row_ptrs = (np.arange(out_f + 1) * 2).astype(np.int32)
    cols = np.empty(2 * out_f, np.int32)
    cols[0::2] = (np.arange(out_f) * 2) % in_f
    cols[1::2] = (np.arange(out_f) * 2 + 1) % in_f
    vals = np.tile(np.array([10.0, -5.0], np.float32), out_f)
    return dict(codebook=np.zeros((256, 16), np.float32),
                codes=np.zeros((out_f, in_f // 16), np.uint8),
                scales=np.ones(out_f, np.float32), csr=(row_ptrs, cols, vals),
                x=np.ones(in_f, np.float32))


def reference_t6():
    """MoE setup of NAT/tests/test_native_lut.cpp:186-248 (512 experts, H=256,
    I=64, top-10 with fixed indices and weights, x = 0.5)."""
    E, H, I, D = 512, 256, 64, 16
    k = np.arange(256, dtype=np.float32)[:, None]
    cb_in = np.repeat(np.float32(0.05) * ((k % 11) - 5), D, axis=1).astype(np.float32)
    cb_down = np.repeat(np.float32(0.03) * ((k % 7) - 3), D, axis=1).astype(np.float32)
    n_gu = E * 2 * I * (H // D)
    n_dn = E * H * (I // D)
    gu = (np.arange(n_gu) % 256).astype(np.uint8).reshape(E, 2 * I, H // D)
    dn = ((np.arange(n_dn, dtype=np.int64) * 3) % 256).astype(np.uint8).reshape(E, H, I // D)
    idx = np.array([4, 12, 57, 103, 199, 255, 340, 412, 480, 511], np.int32)
    w = np.array([0.25, 0.20, 0.15, 0.10, 0.08, 0.07, 0.05, 0.04, 0.03, 0.03], np.float32)
    return dict(cb_in=cb_in, cb_down=cb_down, gu_codes=gu, gu_scales=np.ones((E, 2 * I), np.float32),
                dn_codes=dn, dn_scales=np.ones((E, H), np.float32), x=np.full(H, 0.5, np.float32),
                idx=idx, w=w)

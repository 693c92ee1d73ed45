"""Seeded synthetic inputs of the benchmark configurations (NumPy PCG64).

Used by bench.py and, through oracle/gen.py, by the tests, so the GPU path and
the CPU oracle see identical bytes.  Shapes and distributions:

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

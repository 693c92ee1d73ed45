"""NumPy restatements of the Python side of the reference LUT path.

TEST INFRASTRUCTURE ONLY (tests, smoke() checker, bench.py cpu_baseline).

Each function cites the reference routine it restates (paths relative to the
reference tree).  All of them accept a ``dtype`` so they can be evaluated in
float64 as a brute-force reference.
"""
import math

import numpy as np


# --- split_manifold_lut_experiment/engine/split_manifold_engine.py ---------------

def engine_build_lut(x, codebook, dtype=np.float64):
    """LUT[..., g, k] = <x_g, C[k]>.  split_manifold_engine.py:185-200."""
    x = np.asarray(x, dtype)
    cb = np.asarray(codebook, dtype)
    d = cb.shape[1]
    xb = x.reshape(*x.shape[:-1], x.shape[-1] // d, d)
    return xb @ cb.T


def engine_forward(x, codebook, codes, scales, outlier_indices=None, outlier_values=None,
                   bias=None, dtype=np.float64):
    """SplitManifoldLUTLinear.forward: gather-sum, * scales, + COO outliers
    (index_add over rows), + bias.  split_manifold_engine.py:202-250."""
    x = np.asarray(x, dtype)
    shp = x.shape
    xf = x.reshape(-1, shp[-1])
    lut = engine_build_lut(xf, codebook, dtype)            # [B, G, K]
    codes = np.asarray(codes).astype(np.int64)              # [M, G]
    g = np.arange(codes.shape[1])[None, :]
    gathered = lut[:, g, codes]                             # [B, M, G]
    y = gathered.sum(axis=2) * np.asarray(scales, dtype)[None, :]
    if outlier_values is not None and np.asarray(outlier_values).size:
        m_idx = np.asarray(outlier_indices[0], np.int64)
        k_idx = np.asarray(outlier_indices[1], np.int64)
        prod = xf[:, k_idx] * np.asarray(outlier_values, dtype)[None, :]
        yo = np.zeros_like(y)
        for b in range(y.shape[0]):
            np.add.at(yo[b], m_idx, prod[b])
        y = y + yo
    if bias is not None:
        y = y + np.asarray(bias, dtype)[None, :]
    return y.reshape(*shp[:-1], codes.shape[0])


def dequantize(codebook, codes, scales, csr=None, dtype=np.float64):
    """Dense W = s_m * C[codes] (+ outliers).  split_manifold_engine.py:252-267."""
    cb = np.asarray(codebook, dtype)
    codes = np.asarray(codes).astype(np.int64)
    M, G = codes.shape
    W = (cb[codes] * np.asarray(scales, dtype)[:, None, None]).reshape(M, G * cb.shape[1])
    if csr is not None:
        rp, cl, vl = csr
        rows = np.repeat(np.arange(M), np.diff(np.asarray(rp)))
        W[rows, np.asarray(cl)] += np.asarray(vl, dtype)
    return W


def csr_to_coo(csr):
    rp, cl, vl = csr
    rows = np.repeat(np.arange(len(rp) - 1), np.diff(np.asarray(rp)))
    return np.stack([rows, np.asarray(cl, np.int64)]), np.asarray(vl)


def linear_fp64(x, codebook, codes, scales, bias=None, csr=None):
    """Brute force y = x W^T + bias in float64 (the identity LUT-gather = x.W^T)."""
    W = dequantize(codebook, codes, scales, csr, np.float64)
    y = np.asarray(x, np.float64).reshape(-1, W.shape[1]) @ W.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


# --- MoE brute force ------------------------------------------------------------

def silu(v):
    return v / (1.0 + np.exp(-v))


def moe_fp64(x, cb_in, cb_down, gu_codes, gu_scales, dn_codes, dn_scales, idx, w, E=None):
    """Top-k SwiGLU FFN in float64 from dequantised experts, with the skip rule
    of NAT/src/ojasx_lut_cpu.cpp:284-286."""
    x = np.asarray(x, np.float64).reshape(-1)
    E = gu_codes.shape[0] if E is None else E
    I = gu_codes.shape[1] // 2
    y = np.zeros(dn_codes.shape[1], np.float64)
    for e, we in zip(np.asarray(idx).reshape(-1), np.asarray(w, np.float32).reshape(-1)):
        if e < 0 or e >= E or abs(float(we)) < 1e-8:
            continue
        Wgu = dequantize(cb_in, gu_codes[e], gu_scales[e])
        gu = Wgu @ x
        inter = silu(gu[:I]) * gu[I:]
        Wd = dequantize(cb_down, dn_codes[e], dn_scales[e])
        y += float(we) * (Wd @ inter)
    return y


# --- router ---------------------------------------------------------------------

def router_topk(logits, k, renorm=False):
    """Stable descending top-k (ties -> lower index), softmax weights in fp64."""
    lg = np.asarray(logits, np.float32)
    if lg.ndim == 1:
        lg = lg[None]
    idx = np.argsort(-lg, axis=1, kind="stable")[:, :k].astype(np.int32)
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    w = np.take_along_axis(p, idx.astype(np.int64), axis=1)
    if renorm:
        w = w / w.sum(axis=1, keepdims=True)
    return idx, w


# --- ojasx_24x96/long_context.py --------------------------------------------------

def online_softmax_attention(q, k_tiles, v_tiles, scale=None):
    """fp64 online-softmax attention of one query row over streamed (K, V)
    tiles, non-causal (decode).  Restates OnlineSoftmaxBlockAttention.
    forward_stream (long_context.py:92-176): running (m, l, acc), alpha =
    exp(m_old - m_new) with the -inf guard, final acc / l."""
    q = np.asarray(q, np.float64).reshape(-1)
    D = q.size
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    m, l, acc = -math.inf, 0.0, np.zeros(D)
    for kt, vt in zip(k_tiles, v_tiles):
        kt = np.asarray(kt, np.float64)
        vt = np.asarray(vt, np.float64)
        if kt.shape[0] == 0:
            continue
        s = (kt @ q) * scale
        m_new = max(m, float(s.max()))
        safe = 0.0 if math.isinf(m_new) else m_new
        alpha = 0.0 if math.isinf(m) else math.exp(m - safe)
        p = np.where(np.isinf(s), 0.0, np.exp(s - safe))
        l = alpha * l + p.sum()
        acc = alpha * acc + p @ vt
        m = m_new
    return acc / (l if l > 0 else 1.0)


def block_attention_stream(q, tiles, causal=True, query_start_pos=0, scale=None):
    """fp64 OnlineSoftmaxBlockAttention.forward_stream (long_context.py:92-176)
    for q [B, Hq, Sq, D] over (K, V) tiles [B, Hkv, S_k, D] in order, query
    head h reading kv head h // (Hq // Hkv) (:80-89).  Per tile: scores
    (q @ K^T) * scale, -inf where key position > query position when causal
    (:133-139), then the running (m, l, acc) update with the -inf guards
    (:141-163).  Returns (out [B, Hq, Sq, D] fp64, lse [B, Hq, Sq] fp64 =
    m + log(l) with l = 0 -> 1, kv tokens, tiles)."""
    q = np.asarray(q, np.float64)
    B, Hq, Sq, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    m = np.full((B, Hq, Sq, 1), -np.inf)
    l = np.zeros((B, Hq, Sq, 1))
    acc = np.zeros((B, Hq, Sq, D))
    qpos = (query_start_pos + np.arange(Sq)).reshape(1, 1, Sq, 1)
    off = n_tiles = 0
    for K, V in tiles:
        K = np.asarray(K, np.float64)
        V = np.asarray(V, np.float64)
        S = K.shape[2]
        if S == 0:
            continue
        n_tiles += 1
        rep = Hq // K.shape[1]
        K = np.repeat(K, rep, axis=1)
        V = np.repeat(V, rep, axis=1)
        s = (q @ np.swapaxes(K, -1, -2)) * scale
        if causal:
            kpos = (off + np.arange(S)).reshape(1, 1, 1, S)
            s = np.where(kpos > qpos, -np.inf, s)
        m_new = np.maximum(m, s.max(axis=-1, keepdims=True))
        safe = np.where(np.isinf(m_new), 0.0, m_new)
        with np.errstate(invalid="ignore"):
            alpha = np.where(np.isinf(m), 0.0, np.exp(m - safe))
            p = np.where(np.isinf(s), 0.0, np.exp(s - safe))
        l = alpha * l + p.sum(axis=-1, keepdims=True)
        acc = alpha * acc + p @ V
        m = m_new
        off += S
    sl = np.where(l > 0.0, l, 1.0)
    with np.errstate(invalid="ignore"):
        lse = (m + np.log(sl))[..., 0]
    return acc / sl, lse, off, n_tiles


def masked_full_attention(q, K, V, causal=True, query_start_pos=0, scale=None):
    """fp64 full-matrix attention with the causal mask and GQA head mapping
    (tests/test_m13_ultra_long_context_10m.py:49-103): rows whose keys are
    all hidden give 0."""
    q = np.asarray(q, np.float64)
    B, Hq, Sq, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    rep = Hq // np.asarray(K).shape[1]
    K = np.repeat(np.asarray(K, np.float64), rep, axis=1)
    V = np.repeat(np.asarray(V, np.float64), rep, axis=1)
    s = (q @ np.swapaxes(K, -1, -2)) * scale
    if causal:
        kpos = np.arange(K.shape[2]).reshape(1, 1, 1, -1)
        qpos = (query_start_pos + np.arange(Sq)).reshape(1, 1, Sq, 1)
        s = np.where(kpos > qpos, -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    safe = np.where(np.isinf(mx), 0.0, mx)
    e = np.where(np.isinf(s), 0.0, np.exp(s - safe))
    tot = e.sum(axis=-1, keepdims=True)
    return (e / np.where(tot > 0.0, tot, 1.0)) @ V


def full_softmax_attention(q, K, V, scale=None):
    """fp64 full-softmax reference (tests/test_m13_ultra_long_context_10m.py:49-103)."""
    q = np.asarray(q, np.float64).reshape(-1)
    scale = 1.0 / math.sqrt(q.size) if scale is None else scale
    s = (np.asarray(K, np.float64) @ q) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ np.asarray(V, np.float64)


def round_to(a, kind):
    """fp32 values rounded to nearest even in ``kind`` ("float32", "bfloat16",
    "float16") and returned as fp32: the result of a torch elementwise op on
    tensors of that type (finite inputs)."""
    a = np.asarray(a, np.float32)
    if kind == "float32":
        return a
    if kind == "float16":
        return a.astype(np.float16).astype(np.float32)
    if kind == "bfloat16":
        u = a.view(np.uint32).astype(np.uint64)
        u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        return u.astype(np.uint32).view(np.float32)
    raise ValueError(kind)


def paged_quantize_int8(t, kind="float32"):
    """PagedCompressedKVCache._quantize_int8 (long_context.py:234-240) on a
    tensor of element type ``kind`` (t holds values of that type):
    a = max(|t|_D, T(1e-8)), s = T(a / 127), q = clamp(round_half_even(T(t / s)),
    -127, 127) int8 with every elementwise result T() rounded to the type as
    torch does; s returned as float16.  An all-zero float16 row gives s = 0
    and 0/0 in the reference; q is 0 there.  For "float64" every step is
    float64 and s reaches float16 as torch casts it: through float32."""
    if kind == "float64":
        t = np.asarray(t, np.float64)
        s = np.maximum(np.abs(t).max(axis=-1, keepdims=True), 1e-8) / 127.0
        q = np.clip(np.rint(t / s), -127, 127).astype(np.int8)
        return q, s.astype(np.float32).astype(np.float16)
    t = round_to(t, kind)
    amax = np.maximum(np.abs(t).max(axis=-1, keepdims=True), round_to(np.float32(1e-8), kind))
    s = round_to(amax / np.float32(127.0), kind)
    with np.errstate(invalid="ignore", divide="ignore"):
        v = np.rint(round_to(t / s, kind))
    v = np.where(np.isnan(v), 0, v)
    q = np.clip(v, -127, 127).astype(np.int8)
    return q, s.astype(np.float16)


def paged_dequantize_int8(q, s, kind="float32"):
    """PagedCompressedKVCache._dequantize_int8 (long_context.py:242-244):
    float(q) * float(s) in fp32, then rounded to ``kind``."""
    v = np.asarray(q, np.float32) * np.asarray(s, np.float16).astype(np.float32)
    return v.astype(np.float64) if kind == "float64" else round_to(v, kind)


def code_domain_kv_decode(q_heads, kv_group, k_cb, v_cb, k_codes, k_scales, v_codes, v_scales,
                          scale=None, tile=256):
    """fp64 general-codebook decode for the query heads of one kv head, as an
    online softmax over tiles of the dequantised stream: K_t = s_t * Ck[code],
    V_t = vs_t * Cv[code]."""
    k_cb = np.asarray(k_cb, np.float64)
    v_cb = np.asarray(v_cb, np.float64)
    T, G = k_codes.shape
    Kd = (k_cb[k_codes.astype(np.int64)].reshape(T, -1)) * np.asarray(k_scales, np.float64)[:, None]
    Vd = (v_cb[v_codes.astype(np.int64)].reshape(T, -1)) * np.asarray(v_scales, np.float64)[:, None]
    outs = []
    for q in q_heads:
        kt = [Kd[i:i + tile] for i in range(0, T, tile)]
        vt = [Vd[i:i + tile] for i in range(0, T, tile)]
        outs.append(online_softmax_attention(q, kt, vt, scale))
    return np.stack(outs)


# --- ojasx_24x96/codec.py + math_engine.py ---------------------------------------

def pack_codes(codes, bits):
    """Little-endian bit packing (codec.py:176-195); identity for 8 bits."""
    flat = np.asarray(codes).reshape(-1).astype(np.int64)
    if bits not in (1, 2, 4, 8):
        raise ValueError("Only 1-, 2-, 4-, and 8-bit codes are supported")
    if flat.size and (flat.min() < 0 or flat.max() >= (1 << bits)):
        raise ValueError("A code exceeds the requested bit width")
    if bits == 8:
        return flat.astype(np.uint8)
    per = 8 // bits
    n = (flat.size + per - 1) // per * per
    pad = np.zeros(n, np.int64)
    pad[:flat.size] = flat
    grp = pad.reshape(-1, per)
    return (grp << (np.arange(per) * bits)).sum(axis=1).astype(np.uint8)


def unpack_codes(packed, bits, count):
    """Inverse of pack_codes with explicit count (codec.py:198-214)."""
    packed = np.asarray(packed, np.uint8)
    if (count * bits + 7) // 8 != packed.size:
        raise ValueError("packed size mismatch")
    per = 8 // bits
    vals = (packed.astype(np.int64)[:, None] >> (np.arange(per) * bits)) & ((1 << bits) - 1)
    return vals.reshape(-1)[:count].astype(np.uint8)


def subspace_lut_rvq_gemm(x, codebooks, packed_codes, bits, rows, cols, block, row_scales,
                          bias=None, dtype=np.float64):
    """Y[b,m] = s_m * sum_{s,g} LUT[b,s,g,code_s[m,g]] + bias with K zero-padded
    to G*block (math_engine.py:136-208)."""
    x = np.asarray(x, dtype)
    shp = x.shape
    xf = x.reshape(-1, cols)
    G = (cols + block - 1) // block
    if G * block > cols:
        xf = np.pad(xf, ((0, 0), (0, G * block - cols)))
    xb = xf.reshape(xf.shape[0], G, block)
    cbs = np.asarray(codebooks, dtype)                      # [S, Q, block]
    lut = np.einsum("bgd,sqd->bsgq", xb, cbs)
    y = np.zeros((xf.shape[0], rows), dtype)
    gi = np.arange(G)[None, :]
    for s in range(cbs.shape[0]):
        c = unpack_codes(packed_codes[s], bits, rows * G).reshape(rows, G).astype(np.int64)
        y += lut[:, s][:, gi, c].sum(axis=2)
    y = y * np.asarray(row_scales, dtype)[None, :]
    if bias is not None:
        y = y + np.asarray(bias, dtype)[None, :]
    return y.reshape(*shp[:-1], rows)


# --- the LUT decoder (ojasx-vector-24x96_amd/csrc/decoder.hip) ------------------
# Not a reference function: the reference runs its 4B-shaped configuration only
# as a benchmark description.  Each piece below is textbook arithmetic
# (RMSNorm, RoPE by rotate-half, softmax attention, SwiGLU) composed with the
# pinned pieces of this oracle: the dequantised LUT linear (engine_forward /
# linear_fp64) and the code-domain KV dequantisation K_t = s_t * C[code_t].

def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def rope_tables(max_pos, head_dim, theta):
    """cos / sin [max_pos][head_dim/2]: angle = fp32(pos) * fp32(1 / theta^(2i/hd)),
    cos and sin of that fp32 angle rounded to fp32."""
    half = head_dim // 2
    inv = (1.0 / np.power(np.float64(theta), np.arange(half, dtype=np.float64) * 2 / head_dim))
    inv = inv.astype(np.float32)
    ang = np.arange(max_pos, dtype=np.float32)[:, None] * inv[None, :]
    return np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)


def rope(x, cos, sin):
    """Rotate-half RoPE of one head vector x [hd] with the position's cos/sin [hd/2]."""
    x = np.asarray(x, np.float64)
    half = x.shape[-1] // 2
    c, s = np.asarray(cos, np.float64), np.asarray(sin, np.float64)
    lo, hi = x[:half], x[half:]
    return np.concatenate([lo * c - hi * s, hi * c + lo * s])


def lut_dense(w):
    """Dense fp64 matrix of a LUT linear {codebook, codes, csr} with unit scales."""
    return dequantize(w["codebook"], w["codes"], np.ones(w["codes"].shape[0]), csr=w["csr"])


def engine_forward_rows(x, codebook, codes, scales=None, csr=None, bias=None, row_block=4096):
    """SplitManifoldLUTLinear.forward for one token in fp64 without a dense
    matrix (split_manifold_engine.py:202-250): LUT[g, k] = <x_g, C[k]>, then
    y_m = s_m * sum_g LUT[g, codes[m, g]] + sum_j val_j * x[col_j] (+ bias),
    gathered ``row_block`` rows at a time so [M, G] fp64 never materialises."""
    x = np.asarray(x, np.float64).reshape(-1)
    cb = np.asarray(codebook, np.float64)
    d = cb.shape[1]
    lut = x.reshape(-1, d) @ cb.T                           # [G, 256]
    M, G = codes.shape
    gi = np.arange(G)[None, :]
    y = np.empty(M, np.float64)
    for r0 in range(0, M, row_block):
        blk = np.asarray(codes[r0:r0 + row_block]).astype(np.intp)
        y[r0:r0 + blk.shape[0]] = lut[gi, blk].sum(axis=1)
    if scales is not None:
        y *= np.asarray(scales, np.float64)
    if csr is not None and np.asarray(csr[2]).size:
        rp, cl, vl = csr
        rows = np.repeat(np.arange(M), np.diff(np.asarray(rp, np.int64)))
        y += np.bincount(rows, weights=x[np.asarray(cl, np.int64)] * np.asarray(vl, np.float64),
                         minlength=M)
    if bias is not None:
        y += np.asarray(bias, np.float64)
    return y


class LUTOp:
    """A LUT linear {codebook, codes, csr} with unit scales that applies as
    ``op @ x`` through engine_forward_rows: the decoder oracle's linear at
    sizes where a dense fp64 matrix would not fit in memory."""

    def __init__(self, w):
        self.w = w

    def __matmul__(self, x):
        w = self.w
        return engine_forward_rows(x, w["codebook"], w["codes"], None, w["csr"])


def decoder_step(x, weights, cfg, pos, caches, dense=None, linear="dense"):
    """One greedy step of the LUT decoder in fp64 from the residual x (the
    token's embedding row) at position `pos`.  caches[l] = (kc, ks, vc, vs)
    holds every layer's code cache for tokens 0..pos in the paged layout with
    the identity block table, including the new token's codes (written by the
    step under test).  ``linear`` = "dense" applies each LUT linear as its
    dense fp64 matrix, "lut" through engine_forward_rows (same values to fp64
    rounding, for shapes whose dense matrices would not fit in memory), or a
    callable w -> op with ``op @ x`` (another implementation of the linear).
    Returns (logits, new_kv) with new_kv[l] = (k_rot, v) of
    the new token per kv head, for checking its codes."""
    hd, Hq, Hkv = cfg.head_dim, cfg.q_heads, cfg.kv_heads
    R = Hq // Hkv
    make = {"dense": lut_dense, "lut": LUTOp}.get(linear, linear)
    cos, sin = rope_tables(pos + 1, hd, cfg.rope_theta)
    dense = dense if dense is not None else {}
    x = np.asarray(x, np.float64)
    new_kv = []
    T = pos + 1
    for l, w in enumerate(weights["layers"]):
        W = {k: dense.get((l, k)) for k in ("qkv", "o", "gate_up", "down")}
        for k in W:
            if W[k] is None:
                W[k] = dense[(l, k)] = make(w[k])
        h = rmsnorm(x, w["input_norm"], cfg.rms_eps)
        qkv = W["qkv"] @ h
        q = qkv[:Hq * hd].reshape(Hq, hd)
        k = qkv[Hq * hd:(Hq + Hkv) * hd].reshape(Hkv, hd)
        v = qkv[(Hq + Hkv) * hd:].reshape(Hkv, hd)
        q = np.stack([rope(rmsnorm(q[j], w["q_norm"], cfg.rms_eps), cos[pos], sin[pos])
                      for j in range(Hq)])
        k = np.stack([rope(rmsnorm(k[j], w["k_norm"], cfg.rms_eps), cos[pos], sin[pos])
                      for j in range(Hkv)])
        new_kv.append((k, v))
        kc, ks, vc, vs = caches[l]
        attn = np.zeros((Hq, hd))
        for h_ in range(Hkv):
            kcl = kc[:, h_].reshape(-1, kc.shape[-1])[:T].astype(np.int64)
            vcl = vc[:, h_].reshape(-1, vc.shape[-1])[:T].astype(np.int64)
            Kd = w["k_codebook"][h_][kcl].reshape(T, hd) * ks[:, h_].reshape(-1)[:T, None].astype(np.float64)
            Vd = w["v_codebook"][h_][vcl].reshape(T, hd) * vs[:, h_].reshape(-1)[:T, None].astype(np.float64)
            for j in range(h_ * R, (h_ + 1) * R):
                attn[j] = full_softmax_attention(q[j], Kd, Vd, 1.0 / math.sqrt(hd))
        x = x + W["o"] @ attn.reshape(-1)
        h2 = rmsnorm(x, w["post_norm"], cfg.rms_eps)
        gu = W["gate_up"] @ h2
        I = gu.shape[0] // 2
        a = silu(gu[:I]) * gu[I:]
        x = x + W["down"] @ a
    Wl = dense.get("lm")
    if Wl is None:
        Wl = dense["lm"] = make(weights["lm_head"])
    logits = Wl @ rmsnorm(x, weights["final_norm"], cfg.rms_eps)
    return logits, new_kv


/*
 * lut_oracle.c -- CPU restatement of the OjasX split-manifold LUT path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle: it is built into
 * oracle/liblut_oracle.so and may be loaded only by tests/, by
 * __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg.
 * The product (the HIP C-ABI library) never links, loads or calls it.
 *
 * Every function restates, in plain C and in the reference's own loop and
 * accumulation order, one routine of the reference engine.  Citations are to
 * files under split_manifold_lut_experiment/native/ ("NAT/") of the
 * reference tree.  The code is written from the formulas; nothing is copied.
 * Build flags: -O2 -ffp-contract=off, no -march (scalar path, no FMA
 * contraction), which is what the reference's own Makefile flags give on x86
 * (NAT/Makefile:5; NAT/include/ojasx_lut.h:26-32 selects no SIMD path).
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   orc_build_lut        closed form / one-hot special case (bit-exact),
 *                        fp64 brute force, compiled reference (bit-exact)
 *   orc_linear_forward   reference T2/T3 known answers, integer-exact cases,
 *                        fp64 dequantised GEMV, compiled reference (bit-exact)
 *   orc_moe_forward      fp64 brute force, skip rules, compiled reference
 *   orc_kv_*             closed form per token, compiled reference (bit-exact)
 *   orc_kv_attention_cb  reduces to orc_kv_attention_ref for C[c]=(c-128)e0,
 *                        fp64 full-softmax brute force
 *   orc_router_topk      numpy stable argsort brute force (bit-exact indices)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* LUT[g][k] = sum_d x[g*D+d] * C[k*D+d], d ascending, fp32.
 * NAT/src/ojasx_lut_cpu.cpp:92-100 (portable path taken by x86 builds). */
ORC_API void orc_build_lut(const float *x, const float *codebook, int G, int D,
                           int Kcb, float *lut) {
    for (int g = 0; g < G; ++g) {
        const float *xg = x + (size_t)g * D;
        float *lg = lut + (size_t)g * Kcb;
        for (int k = 0; k < Kcb; ++k) {
            const float *c = codebook + (size_t)k * D;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += xg[d] * c[d];
            lg[k] = dot;
        }
    }
}

/* y[b][m] = (sum_g LUT_b[g][codes[m][g]]) * s[m] (+ bias[m]), groups in
 * ascending order, then y[b][m] += sum_j val_j * x[b][col_j] over the CSR row.
 * NAT/src/ojasx_lut_cpu.cpp:132-206 (row loop :160-184, epilogue :178-182),
 * outliers :104-130 (applied after the epilogue, not scaled). */
ORC_API void orc_linear_forward(const float *x, int B, int K, int M, int D,
                                int Kcb, const float *codebook,
                                const uint8_t *codes, const float *scales,
                                const float *bias, int nnz,
                                const int *row_ptrs, const int *cols,
                                const float *vals, float *y) {
    const int G = K / D;
    float *lut = (float *)malloc(sizeof(float) * (size_t)G * Kcb);
    for (int b = 0; b < B; ++b) {
        const float *xb = x + (size_t)b * K;
        float *yb = y + (size_t)b * M;
        orc_build_lut(xb, codebook, G, D, Kcb, lut);
        for (int m = 0; m < M; ++m) {
            const uint8_t *row = codes + (size_t)m * G;
            float sum = 0.0f;
            for (int g = 0; g < G; ++g) sum += lut[(size_t)g * Kcb + row[g]];
            float r = sum * (scales ? scales[m] : 1.0f);
            if (bias) r += bias[m];
            yb[m] = r;
        }
    }
    free(lut);
    if (nnz > 0 && row_ptrs && cols && vals) {
        for (int b = 0; b < B; ++b) {
            const float *xb = x + (size_t)b * K;
            float *yb = y + (size_t)b * M;
            for (int m = 0; m < M; ++m) {
                float acc = 0.0f;
                for (int j = row_ptrs[m]; j < row_ptrs[m + 1]; ++j)
                    acc += vals[j] * xb[cols[j]];
                yb[m] += acc;
            }
        }
    }
}

/* x / (1 + exp(-x)) in fp32 with libm expf.  NAT/src/ojasx_lut_cpu.cpp:209-211 */
static float orc_silu(float v) { return v / (1.0f + expf(-v)); }

static float orc_row_gather(const float *lut, int Kcb, const uint8_t *row, int G) {
    float s = 0.0f;
    for (int g = 0; g < G; ++g) s += lut[(size_t)g * Kcb + row[g]];
    return s;
}

/* Top-k SwiGLU expert FFN in the code domain, batch 1.
 * NAT/src/ojasx_lut_cpu.cpp:213-365.  k_active <= 0 leaves y untouched
 * (:220); otherwise y is zeroed (:223); an expert id outside [0,E) or a
 * weight with |w| < 1e-8 is skipped (:284-286).  gate rows are 0..I-1 and
 * up rows I..2I-1 of the expert's [2I][G_in] block (:295,:310). */
ORC_API void orc_moe_forward(const float *x, int E, int H, int I, int D,
                             int Kcb, const float *cb_in, const float *cb_down,
                             const uint8_t *gu_codes, const float *gu_scales,
                             const uint8_t *dn_codes, const float *dn_scales,
                             const int *idx, const float *w, int k_active,
                             float *y) {
    if (k_active <= 0) return;
    for (int h = 0; h < H; ++h) y[h] = 0.0f;
    const int Gin = H / D, Gi = I / D;
    float *lut_in = (float *)malloc(sizeof(float) * (size_t)Gin * Kcb);
    float *lut_dn = (float *)malloc(sizeof(float) * (size_t)Gi * Kcb);
    float *inter = (float *)malloc(sizeof(float) * (size_t)I);
    orc_build_lut(x, cb_in, Gin, D, Kcb, lut_in);
    for (int k = 0; k < k_active; ++k) {
        const int e = idx[k];
        const float we = w[k];
        if (e < 0 || e >= E || fabsf(we) < 1e-8f) continue;
        const uint8_t *gu = gu_codes + (size_t)e * 2 * I * Gin;
        const float *gus = gu_scales + (size_t)e * 2 * I;
        for (int i = 0; i < I; ++i) {
            float gate = orc_row_gather(lut_in, Kcb, gu + (size_t)i * Gin, Gin) * gus[i];
            float up = orc_row_gather(lut_in, Kcb, gu + (size_t)(I + i) * Gin, Gin) * gus[I + i];
            inter[i] = orc_silu(gate) * up;
        }
        /* LUT_down, built with the same scalar dot (:330-342) */
        orc_build_lut(inter, cb_down, Gi, D, Kcb, lut_dn);
        const uint8_t *dn = dn_codes + (size_t)e * H * Gi;
        const float *dns = dn_scales + (size_t)e * H;
        for (int h = 0; h < H; ++h) {
            float v = orc_row_gather(lut_dn, Kcb, dn + (size_t)h * Gi, Gi) * dns[h];
            y[h] += v * we; /* :361-362 */
        }
    }
    free(lut_in);
    free(lut_dn);
    free(inter);
}

/* Reference KV quantiser for one token of one head.
 * NAT/src/ojasx_lut_kv_cache.cpp:29-46: s = max(1e-8, max_d |k_d|) / 127;
 * code[g] = clamp(round(k[g*D] / s), -128, 127) + 128, where round() rounds
 * halves away from zero (std::round); only coordinate g*D of each group is
 * used. */
ORC_API void orc_kv_quantize_token(const float *k, int head_dim, int D,
                                   uint8_t *codes, float *scale) {
    float mx = 1e-8f;
    for (int d = 0; d < head_dim; ++d) {
        float a = fabsf(k[d]);
        mx = mx > a ? mx : a;
    }
    const float s = mx / 127.0f;
    *scale = s;
    const int G = head_dim / D;
    for (int g = 0; g < G; ++g) {
        int q = (int)roundf(k[g * D] / s);
        if (q < -128) q = -128;
        if (q > 127) q = 127;
        codes[g] = (uint8_t)(q + 128);
    }
}

/* Codebook KV encoder for one token of one head (defined by this build; the
 * step before the general-codebook decode).  Scale as orc_kv_quantize_token
 * (NAT/src/ojasx_lut_kv_cache.cpp:29-34); x_d = k_d / s;
 * code[g] = argmin_c sum_{d<D} (x[gD+d] - cb[c][d])^2 over the 256 rows of
 * cb [256][D], the sum accumulated with fmaf in d order from 0, ties to the
 * lower c.  With cb[c] = (c - 128) e_0 and other coordinates zero this is the
 * reference quantiser away from half-way ties. */
ORC_API void orc_kv_encode_token(const float *k, int head_dim, int D, const float *cb,
                                 uint8_t *codes, float *scale) {
    float mx = 1e-8f;
    for (int d = 0; d < head_dim; ++d) {
        float a = fabsf(k[d]);
        mx = mx > a ? mx : a;
    }
    const float s = mx / 127.0f;
    *scale = s;
    const int G = head_dim / D;
    for (int g = 0; g < G; ++g) {
        float best = 0.0f;
        int bi = 0;
        for (int c = 0; c < 256; ++c) {
            float dist = 0.0f;
            for (int d = 0; d < D; ++d) {
                const float df = k[g * D + d] / s - cb[c * D + d];
                dist = fmaf(df, df, dist);
            }
            if (c == 0 || dist < best) {
                best = dist;
                bi = c;
            }
        }
        codes[g] = (uint8_t)bi;
    }
}

/* Reference decode attention for one head over T tokens.
 * logits: NAT/src/ojasx_lut_kv_cache.cpp:67-108 (LUT_q[g][c] = q[g*D]*(c-128),
 * sum over g ascending, times s_t times sf; sf <= 0 means 1/sqrt(head_dim)).
 * softmax: NAT/src/ojasx_lut_c_api.cpp:178-191 (max, exp and sum in t order,
 * multiply by 1/sum).  context: NAT/src/ojasx_lut_kv_cache.cpp:110-132
 * (out[g*D] += (code-128) * (p_t*vs_t), zero weights skipped, all other
 * coordinates 0).  T == 0 leaves out untouched (c_api.cpp:172-173). */
ORC_API void orc_kv_attention_ref(const float *q, int T, int head_dim, int D,
                                  const uint8_t *k_codes, const float *k_scales,
                                  const uint8_t *v_codes, const float *v_scales,
                                  float sf, float *out) {
    if (T <= 0) return;
    if (sf <= 0.0f) sf = 1.0f / sqrtf((float)head_dim);
    const int G = head_dim / D;
    float *lut = (float *)malloc(sizeof(float) * (size_t)G * 256);
    float *p = (float *)malloc(sizeof(float) * (size_t)T);
    for (int g = 0; g < G; ++g) {
        const float qv = q[g * D];
        for (int c = 0; c < 256; ++c) lut[g * 256 + c] = qv * (float)(c - 128);
    }
    for (int t = 0; t < T; ++t) {
        const uint8_t *row = k_codes + (size_t)t * G;
        float s = 0.0f;
        for (int g = 0; g < G; ++g) s += lut[g * 256 + row[g]];
        p[t] = s * k_scales[t] * sf;
    }
    float mx = p[0];
    for (int t = 1; t < T; ++t) mx = mx > p[t] ? mx : p[t];
    float sum = 0.0f;
    for (int t = 0; t < T; ++t) {
        p[t] = expf(p[t] - mx);
        sum += p[t];
    }
    const float inv = 1.0f / sum;
    for (int t = 0; t < T; ++t) p[t] *= inv;
    for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
    for (int t = 0; t < T; ++t) {
        const float wt = p[t] * v_scales[t];
        if (wt == 0.0f) continue;
        const uint8_t *row = v_codes + (size_t)t * G;
        for (int g = 0; g < G; ++g) out[g * D] += (float)((int)row[g] - 128) * wt;
    }
    free(lut);
    free(p);
}

/* General-codebook form of the same decode for one query head:
 * LUT_q[g][c] = q_g . Ck[c] (scalar dot, d ascending), logit_t =
 * (sum_g LUT_q[g][code_k[t][g]]) * s_t * sf, two-pass softmax as above, and
 * out[g*D+d] = sum_t (p_t * vs_t) * Cv[code_v[t][g]][d].  With
 * Ck = Cv = (c-128) e_0 it is exactly orc_kv_attention_ref. */
ORC_API void orc_kv_attention_cb(const float *q, int T, int head_dim, int D,
                                 const float *k_cb, const float *v_cb,
                                 const uint8_t *k_codes, const float *k_scales,
                                 const uint8_t *v_codes, const float *v_scales,
                                 float sf, float *out) {
    if (T <= 0) return;
    if (sf <= 0.0f) sf = 1.0f / sqrtf((float)head_dim);
    const int G = head_dim / D;
    float *lut = (float *)malloc(sizeof(float) * (size_t)G * 256);
    float *p = (float *)malloc(sizeof(float) * (size_t)T);
    orc_build_lut(q, k_cb, G, D, 256, lut);
    for (int t = 0; t < T; ++t) {
        const uint8_t *row = k_codes + (size_t)t * G;
        float s = 0.0f;
        for (int g = 0; g < G; ++g) s += lut[g * 256 + row[g]];
        p[t] = s * k_scales[t] * sf;
    }
    float mx = p[0];
    for (int t = 1; t < T; ++t) mx = mx > p[t] ? mx : p[t];
    float sum = 0.0f;
    for (int t = 0; t < T; ++t) {
        p[t] = expf(p[t] - mx);
        sum += p[t];
    }
    const float inv = 1.0f / sum;
    for (int t = 0; t < T; ++t) p[t] *= inv;
    for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
    for (int t = 0; t < T; ++t) {
        const float wt = p[t] * v_scales[t];
        if (wt == 0.0f) continue;
        const uint8_t *row = v_codes + (size_t)t * G;
        for (int g = 0; g < G; ++g) {
            const float *c = v_cb + (size_t)row[g] * D;
            for (int d = 0; d < D; ++d) out[g * D + d] += c[d] * wt;
        }
    }
    free(lut);
    free(p);
}

/* Router (absent from the reference, whose callers pass indices and weights:
 * ojasx_24x96/module.py:653-657, NAT/src/ojasx_run.cpp:171-174).  Defined
 * here as: select the k largest logits, descending, ties to the lower expert
 * index; weight = softmax over all E logits (fp32: max, expf(l-max), sum in
 * index order) at the selected experts; renorm != 0 divides the k weights by
 * their sum (in selection order). */
ORC_API void orc_router_topk(const float *logits, int T, int E, int k,
                             int renorm, int *idx, float *w) {
    for (int t = 0; t < T; ++t) {
        const float *l = logits + (size_t)t * E;
        int *it = idx + (size_t)t * k;
        float *wt = w + (size_t)t * k;
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                int used = 0;
                for (int u = 0; u < j; ++u) used |= (it[u] == e);
                if (used) continue;
                if (best < 0 || l[e] > l[best]) best = e;
            }
            it[j] = best;
        }
        float mx = l[0];
        for (int e = 1; e < E; ++e) mx = mx > l[e] ? mx : l[e];
        float sum = 0.0f;
        for (int e = 0; e < E; ++e) sum += expf(l[e] - mx);
        for (int j = 0; j < k; ++j) wt[j] = expf(l[it[j]] - mx) / sum;
        if (renorm) {
            float s = 0.0f;
            for (int j = 0; j < k; ++j) s += wt[j];
            for (int j = 0; j < k; ++j) wt[j] = wt[j] / s;
        }
    }
}

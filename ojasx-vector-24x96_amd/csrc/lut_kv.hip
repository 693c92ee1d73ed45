// lut_kv.hip -- code-domain paged KV decode attention on gfx950.
//
// For query head j (kv head h = j / (Hq/Hkv)) over tokens t < T:
//   LUT_q[g][c] = <q_j[gD:(g+1)D], Ck_h[c]>
//   l_t = sf * s_t * sum_g LUT_q[g, kcode_t[g]]
//   p = softmax(l)
//   o[gD+d] = sum_t p_t * vs_t * Cv_h[vcode_t[g]][d]
// This is the computation of split_manifold_lut_experiment/native/src/
// ojasx_lut_kv_cache.cpp:67-132 with ojasx_lut_c_api.cpp:160-196 (two-pass
// softmax), generalised from the reference's implicit codebook
// C[c] = (c - 128) e_0 to a per-kv-head 256 x D codebook; the reference
// C-ABI (ojasx_kv_cache_*) runs on the same kernels with that special
// codebook, which reproduces its arithmetic exactly (the other coordinates
// contribute exact zeros).
//
// Kernels:
//  * kv_append: the reference quantiser (ojasx_lut_kv_cache.cpp:16-65) for one
//    token of one head: s = max(1e-8, max|k|) / 127, code[g] =
//    clamp(round(k[gD] / s), -128, 127) + 128 (round half away from zero).
//  * kv_decode_chunk: workgroup = (chunk of 256 tokens, kv head, the query
//    heads of its GQA group); thread = token and centroid.  Builds LUT_q for
//    its query heads in LDS (centroid in registers), computes the chunk's
//    scores from the K codes (page-table indirection), the chunk max and exp
//    (wave shuffles), then accumulates V in the code domain: a histogram
//    W[j][g][c] += p_t * vs_t over the chunk (LDS atomics) followed by one
//    [heads*groups x 256] x [256 x D] contraction with the V codebook.  A
//    context of at most 256 tokens writes the normalised output directly;
//    otherwise (max, sum, o) per chunk.
//  * kv_merge: log-sum-exp merge of the chunks in chunk order (the online
//    softmax combine of ojasx_24x96/long_context.py:133-166).
// Cache layout (device): codes [pages][Hkv][page][G] uint8, scales
// [pages][Hkv][page] fp32, so a page of one kv head is contiguous.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;
constexpr int kMaxRG = 32;   // query heads per workgroup x groups per head
constexpr int kMaxD = 32;
// Histogram row pitch: 257 floats, so the rows of different groups that one
// wave reads in the contraction sit in different LDS banks.
constexpr int kHP = 257;
}  // namespace

__global__ __launch_bounds__(128) void kv_append_kernel(const float *__restrict__ k,
                                                       const float *__restrict__ v, int hd, int D,
                                                       uint8_t *kc, uint8_t *vc, float *ks,
                                                       float *vs) {
    __shared__ float red[2][128];
    const int tid = threadIdx.x;
    float mk = 0.f, mv = 0.f;
    for (int d = tid; d < hd; d += 128) {
        mk = fmaxf(mk, fabsf(k[d]));
        mv = fmaxf(mv, fabsf(v[d]));
    }
    red[0][tid] = mk;
    red[1][tid] = mv;
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
        if (tid < st) {
            red[0][tid] = fmaxf(red[0][tid], red[0][tid + st]);
            red[1][tid] = fmaxf(red[1][tid], red[1][tid + st]);
        }
        __syncthreads();
    }
    const float sk = fmaxf(1e-8f, red[0][0]) / 127.0f;
    const float sv = fmaxf(1e-8f, red[1][0]) / 127.0f;
    const int G = hd / D;
    for (int g = tid; g < G; g += 128) {
        int qk = (int)roundf(k[g * D] / sk);
        int qv = (int)roundf(v[g * D] / sv);
        kc[g] = (uint8_t)(min(127, max(-128, qk)) + 128);
        vc[g] = (uint8_t)(min(127, max(-128, qv)) + 128);
    }
    if (tid == 0) {
        *ks = sk;
        *vs = sv;
    }
}

struct KVParams {
    const float *q;
    const uint8_t *kc, *vc;
    const float *ks, *vs, *kcb, *vcb;
    const int *bt;
    float *part_o;   // [Hq][n_chunks][hd]
    float *part_ml;  // [Hq][n_chunks][2]
    float *out;      // [Hq][hd] (written directly when n_chunks == 1)
    int T, P, Hq, Hkv, hd, D, G, Tc, RS, n_chunks;
    float sf;
};

// One workgroup = (chunk of 256 tokens, kv head, group of RS query heads);
// thread tid owns token t_begin + tid and centroid tid.  LDS: q rows, V
// codebook [256][D], LUT_q [RS][G][256], histogram [RS][G][256], scores
// [RS][256].  GT = G (groups per head) and DT = D when specialised (8 and 16:
// head_dim 128), 0 for the runtime fallback; HM = most query heads per
// workgroup (4 on the GQA-4 fast path).
template <int GT, int DT, int HM, int NTT>
__global__ __launch_bounds__(kNT) void kv_decode_chunk_kernel(KVParams p) {
    extern __shared__ float sm[];
    constexpr int DM = DT > 0 ? DT : kMaxD;
    constexpr int GM = GT > 0 ? GT : kMaxRG;
    constexpr int GW = (GM + 3) / 4;
    const int G = GT > 0 ? GT : p.G;
    const int D = DT > 0 ? DT : p.D;
    const int R = p.Hq / p.Hkv;
    const int h = blockIdx.y;
    const int j0 = h * R + blockIdx.z * p.RS;
    const int nj = min(p.RS, R - (int)blockIdx.z * p.RS);
    const int hd = p.hd;
    float *qs = sm;                                 // [RS][hd]
    float *cv = qs + p.RS * hd;                     // [256][D]
    float *lutq = cv + 256 * D;                     // [RS][G][256]
    float *hist = lutq + p.RS * G * 256;            // [RS][G][kHP] (padded rows)
    __shared__ float wred[2][HM][kNT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c = blockIdx.x;
    const int t_begin = c * (kNT * NTT);

    // ---- round trip 1: block table, codebook row of centroid tid, q, Cv
    int pg[NTT];
#pragma unroll
    for (int i = 0; i < NTT; ++i) pg[i] = p.bt[min(t_begin + tid + kNT * i, p.T - 1) / p.P];
    float ck[DM];
    {
        const float *kr = p.kcb + ((size_t)h * 256 + tid) * D;
#pragma unroll
        for (int d = 0; d < DM; ++d) ck[d] = kr[min(d, D - 1)];
    }
    stage_to_lds<kNT, 4>(qs, p.q + (size_t)j0 * hd, nj * hd);
    stage_to_lds<kNT, 4>(cv, p.vcb + (size_t)h * 256 * D, 256 * D);
    // ---- round trip 2: the tokens' codes and scales
    float ksv[NTT], vsv[NTT];
    uint32_t kw[NTT][GW], vw[NTT][GW];
#pragma unroll
    for (int i = 0; i < NTT; ++i) {
        const int t = min(t_begin + tid + kNT * i, p.T - 1);
        const size_t slot = ((size_t)pg[i] * p.Hkv + h) * p.P + (t % p.P);
        ksv[i] = p.ks[slot];
        vsv[i] = p.vs[slot];
        if (GT == 8) {
            const uint2 a2 = *reinterpret_cast<const uint2 *>(p.kc + slot * 8);
            const uint2 b2 = *reinterpret_cast<const uint2 *>(p.vc + slot * 8);
            kw[i][0] = a2.x;
            kw[i][1] = a2.y;
            vw[i][0] = b2.x;
            vw[i][1] = b2.y;
        } else {
#pragma unroll
            for (int u = 0; u < GW; ++u) kw[i][u] = vw[i][u] = 0;
            for (int g = 0; g < G; ++g) {
                kw[i][g >> 2] |= (uint32_t)p.kc[slot * G + g] << ((g & 3) * 8);
                vw[i][g >> 2] |= (uint32_t)p.vc[slot * G + g] << ((g & 3) * 8);
            }
        }
    }
    if (!(DT == 16 && GT == 8 && HM == 4))
        for (int i = tid; i < nj * G * kHP; i += kNT) hist[i] = 0.f;
    __syncthreads();
    // ---- LUT_q[j][g][tid] = <q_j[gD:(g+1)D], Ck[tid]>
    if (DT == 16) {
#pragma unroll 2
        for (int jg = 0; jg < nj * G; ++jg) {
            const int j = jg / G, g = jg - j * G;
            const float4 *q4 = reinterpret_cast<const float4 *>(qs + j * hd + g * 16);
            const float4 a0 = q4[0], a1 = q4[1], a2 = q4[2], a3 = q4[3];
            const float qv[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                  a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
            float dot = 0.f;
#pragma unroll
            for (int d = 0; d < 16; ++d) dot = fmaf(qv[d], ck[d], dot);
            lutq[jg * 256 + tid] = dot;
        }
    } else {
        for (int jg = 0; jg < nj * G; ++jg) {
            const int j = jg / G, g = jg - j * G;
            const float *qv = qs + j * hd + g * D;
            float dot = 0.f;
#pragma unroll
            for (int d = 0; d < DM; ++d)
                if (d < D) dot = fmaf(qv[d], ck[d], dot);
            lutq[jg * 256 + tid] = dot;
        }
    }
    __syncthreads();
    // ---- scores of this thread's tokens for the RS heads
    float sc[NTT][HM];
#pragma unroll
    for (int i = 0; i < NTT; ++i) {
        const bool live = t_begin + tid + kNT * i < p.T;
#pragma unroll
        for (int j = 0; j < HM; ++j) {
            sc[i][j] = -INFINITY;
            if (j < nj && live) {
                const float *L = lutq + j * G * 256;
                float v[GM];
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    v[g] = g < G ? L[g * 256 + ((kw[i][g >> 2] >> ((g & 3) * 8)) & 0xffu)] : 0.f;
                float a = 0.f;
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (g < G) a += v[g];
                sc[i][j] = a * (ksv[i] * p.sf);
            }
        }
    }
    // ---- per-head max and sum of exp over the chunk (shuffles + LDS)
    float mx[HM];
#pragma unroll
    for (int j = 0; j < HM; ++j) {
        float m = sc[0][j];
#pragma unroll
        for (int i = 1; i < NTT; ++i) m = fmaxf(m, sc[i][j]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        mx[j] = m;
    }
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < HM; ++j) wred[0][j][wv] = mx[j];
    __syncthreads();
    float e[NTT][HM];
#pragma unroll
    for (int j = 0; j < HM; ++j) {
        float m = wred[0][j][0];
#pragma unroll
        for (int q = 1; q < kNT / 64; ++q) m = fmaxf(m, wred[0][j][q]);
        mx[j] = m;
        float l = 0.f;
#pragma unroll
        for (int i = 0; i < NTT; ++i) {
            e[i][j] = sc[i][j] == -INFINITY ? 0.f : expf(sc[i][j] - m);
            l += e[i][j];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) wred[1][j][wv] = l;
    }
    if (DT == 16 && GT == 8 && HM == 4) {
        // ---- V, code domain, no atomics: token weights p_jt * vs_t and the
        // token's V code words go to LDS; thread (token group tg, group g,
        // d-quad dq) accumulates o[j][g][4dq..4dq+3] over its tokens from the
        // V codebook rows, then the 8 token groups are summed in LDS.
        float4 *pw = reinterpret_cast<float4 *>(hist);              // [Tc] head weights
        uint2 *vcw = reinterpret_cast<uint2 *>(pw + kNT * NTT);     // [Tc] V code words
#pragma unroll
        for (int i = 0; i < NTT; ++i) {
            const bool live = t_begin + tid + kNT * i < p.T;
            const float f = live ? vsv[i] : 0.f;
            pw[tid + kNT * i] = make_float4(e[i][0] * f, nj > 1 ? e[i][1] * f : 0.f,
                                            nj > 2 ? e[i][2] * f : 0.f, nj > 3 ? e[i][3] * f : 0.f);
            vcw[tid + kNT * i] = make_uint2(vw[i][0], vw[i][1]);
        }
        __syncthreads();
        const int tg = tid >> 5, r = tid & 31, g = r >> 2, dq = r & 3;
        float acc[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[j][k] = 0.f;
        const int per = kNT * NTT / 8;
        const float4 *cv4 = reinterpret_cast<const float4 *>(cv);
#pragma unroll 4
        for (int u = 0; u < per; ++u) {
            const int tl = tg * per + u;
            const uint2 cwv = vcw[tl];
            const uint32_t code = ((g < 4 ? cwv.x : cwv.y) >> ((g & 3) * 8)) & 0xffu;
            const float4 cq = cv4[code * 4 + dq];
            const float4 wj = pw[tl];
            const float wa[4] = {wj.x, wj.y, wj.z, wj.w};
            const float ca[4] = {cq.x, cq.y, cq.z, cq.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[j][k] = fmaf(wa[j], ca[k], acc[j][k]);
        }
        __syncthreads();
        float *part = hist;                                           // [8][32][16]
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) part[(tg * 32 + r) * 16 + j * 4 + k] = acc[j][k];
        __syncthreads();
    } else {
        // ---- V in the code domain: W[j][g][c] += p_t * vs_t (LDS atomics)
#pragma unroll
        for (int i = 0; i < NTT; ++i) {
            if (t_begin + tid + kNT * i >= p.T) break;
#pragma unroll
            for (int j = 0; j < HM; ++j) {
                if (j >= nj) break;
                const float w = e[i][j] * vsv[i];
                float *Hj = hist + j * G * kHP;
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (g < G) atomicAdd(&Hj[g * kHP + ((vw[i][g >> 2] >> ((g & 3) * 8)) & 0xffu)], w);
            }
        }
        __syncthreads();
    }
    // ---- o[j][g*D + d] = sum_c W[j][g][c] * Cv[c][d]
    float lsum[HM];
#pragma unroll
    for (int j = 0; j < HM; ++j) {
        float l = 0.f;
        if (j < nj) {
            l = wred[1][j][0];
#pragma unroll
            for (int q = 1; q < kNT / 64; ++q) l += wred[1][j][q];
        }
        lsum[j] = l;
    }
    if (DT == 16 && GT == 8 && HM == 4) {
        // output (j, g, d): sum of the 8 token-group partials, in order
        const float *part = hist;
        for (int i = tid; i < nj * hd; i += kNT) {
            const int j = i / hd;
            const int od = i - j * hd;
            const int g = od >> 4, d = od & 15;
            const int r = g * 4 + (d >> 2);
            float a = 0.f;
#pragma unroll
            for (int tg = 0; tg < 8; ++tg) a += part[(tg * 32 + r) * 16 + j * 4 + (d & 3)];
            float l = lsum[0];
#pragma unroll
            for (int q = 1; q < HM; ++q)
                if (j == q) l = lsum[q];
            if (p.n_chunks == 1)
                p.out[(size_t)(j0 + j) * hd + od] = a / l;
            else
                p.part_o[((size_t)(j0 + j) * p.n_chunks + c) * hd + od] = a;
        }
    } else {
#pragma unroll 1
        for (int i = tid; i < nj * hd; i += kNT) {
            const int j = i / hd;
            const int od = i - j * hd;
            const int g = od / D, d = od - g * D;
            const float *Hjg = hist + (j * G + g) * kHP;
            float a = 0.f;
            for (int cc = 0; cc < 256; ++cc) a = fmaf(Hjg[cc], cv[cc * D + d], a);
            float l = lsum[0];
            for (int q = 1; q < HM; ++q)
                if (j == q) l = lsum[q];
            if (p.n_chunks == 1)
                p.out[(size_t)(j0 + j) * hd + od] = a / l;
            else
                p.part_o[((size_t)(j0 + j) * p.n_chunks + c) * hd + od] = a;
        }
    }
    if (p.n_chunks > 1 && tid < nj) {
        float l = lsum[0];
#pragma unroll
        for (int q = 1; q < HM; ++q)
            if (tid == q) l = lsum[q];
        float m = mx[0];
#pragma unroll
        for (int q = 1; q < HM; ++q)
            if (tid == q) m = mx[q];
        float *ml = p.part_ml + ((size_t)(j0 + tid) * p.n_chunks + c) * 2;
        ml[0] = m;
        ml[1] = l;
    }
}

// Log-sum-exp merge of the chunks of one query head, chunks in order:
// (max, sum) pairs staged in LDS, max and normaliser by wave shuffles, then
// each thread sums one output coordinate over the chunks.
__global__ __launch_bounds__(kNT) void kv_merge_kernel(const float *part_o, const float *part_ml,
                                                      int n_chunks, int hd, float *out) {
    extern __shared__ float wsm[];   // [n_chunks] chunk weights
    __shared__ float red[kNT / 64];
    const int j = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float *ml = part_ml + (size_t)j * n_chunks * 2;
    float m = -INFINITY;
    for (int c = tid; c < n_chunks; c += kNT) m = fmaxf(m, ml[2 * c]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int q = 1; q < kNT / 64; ++q) m = fmaxf(m, red[q]);
    __syncthreads();
    float l = 0.f;
    for (int c = tid; c < n_chunks; c += kNT) {
        const float mc = ml[2 * c];
        const float wc = mc == -INFINITY ? 0.f : expf(mc - m);
        wsm[c] = wc;
        l += ml[2 * c + 1] * wc;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    if (lane == 0) red[wv] = l;
    __syncthreads();
    l = red[0];
#pragma unroll
    for (int q = 1; q < kNT / 64; ++q) l += red[q];
    const float inv = 1.f / l;
    for (int d = tid; d < hd; d += kNT) {
        const float *po = part_o + (size_t)j * n_chunks * hd + d;
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int c = 0;
        for (; c + 8 <= n_chunks; c += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = po[(size_t)(c + u) * hd];
#pragma unroll
            for (int u = 0; u < 8; ++u) o[u] = fmaf(v[u], wsm[c + u], o[u]);
        }
        for (; c < n_chunks; ++c) o[0] = fmaf(po[(size_t)c * hd], wsm[c], o[0]);
        out[(size_t)j * hd + d] = (((o[0] + o[1]) + (o[2] + o[3])) + ((o[4] + o[5]) + (o[6] + o[7]))) * inv;
    }
}

// Workspace for the decode partials, one per thread of the host (device
// entry points called from several host threads each get their own).
struct KVWork {
    DevBuf o, ml;
    ~KVWork() {
        o.release();
        ml.release();
    }
};
static thread_local KVWork t_work;

int kv_decode(const float *q, const uint8_t *kc, const float *ks, const uint8_t *vc,
              const float *vs, const float *kcb, const float *vcb, const int *bt, int T, int P,
              int Hq, int Hkv, int hd, int D, float sf, float *out, hipStream_t st,
              KVWork &wk) {
    if (T <= 0) return OJASX_OK;
    if (Hkv <= 0 || Hq <= 0 || Hq % Hkv || D <= 0 || D > kMaxD || hd <= 0 || hd % D || P <= 0 ||
        hd > 1024) {
        set_error("invalid KV decode shape Hq=%d Hkv=%d hd=%d D=%d page=%d", Hq, Hkv, hd, D, P);
        return OJASX_ERR_INVALID;
    }
    if (sf <= 0.f) sf = 1.0f / sqrtf((float)hd);
    const int G = hd / D;
    const int R = Hq / Hkv;
    if (G > kMaxRG) {
        set_error("head_dim / block_dim must be <= %d", kMaxRG);
        return OJASX_ERR_INVALID;
    }
    // Query heads per workgroup (all of a GQA group when they fit): the codes
    // of a chunk are read once per workgroup.
    const int RS = std::max(1, std::min({R, kMaxRG / G, 8}));
    const int nz = (R + RS - 1) / RS;
    // Tokens per thread: 1 for short contexts (more workgroups), 4 for long
    // ones (the chunk's LUT_q build is amortised over 1024 tokens).
    const int ntt = T > 8192 ? 4 : 1;
    const int Tc = kNT * ntt;
    const int n_chunks = (T + Tc - 1) / Tc;
    int rc = OJASX_OK;
    if (n_chunks > 1) {
        rc = wk.o.ensure((size_t)Hq * n_chunks * hd * 4);
        if (!rc) rc = wk.ml.ensure((size_t)Hq * n_chunks * 2 * 4);
        if (rc) return rc;
    }
    KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, wk.o.as<float>(), wk.ml.as<float>(), out, T, P,
               Hq, Hkv, hd, D, G, Tc, RS, n_chunks, sf};
    const size_t tail = std::max<size_t>((size_t)RS * G * kHP * 4,
                                         std::max<size_t>((size_t)Tc * 24, 8 * 32 * 16 * 4));
    const size_t lds = ((size_t)RS * hd + 256 * D + (size_t)RS * G * 256) * 4 + tail;
    dim3 grid(n_chunks, Hkv, nz);
    static size_t g1 = 0, g4 = 0, g0 = 0;
    const bool fast = G == 8 && D == 16 && RS <= 4;
    if (fast && ntt == 1) {
        rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_chunk_kernel<8, 16, 4, 1>), lds, &g1);
        if (rc) return rc;
        OJX_LAUNCH((kv_decode_chunk_kernel<8, 16, 4, 1>), grid, dim3(kNT), lds, st, p);
    } else if (fast) {
        rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_chunk_kernel<8, 16, 4, 4>), lds, &g4);
        if (rc) return rc;
        OJX_LAUNCH((kv_decode_chunk_kernel<8, 16, 4, 4>), grid, dim3(kNT), lds, st, p);
    } else {
        // runtime-shape fallback: one token per thread
        p.Tc = kNT;
        p.n_chunks = (T + kNT - 1) / kNT;
        if (p.n_chunks > 1) {
            rc = wk.o.ensure((size_t)Hq * p.n_chunks * hd * 4);
            if (!rc) rc = wk.ml.ensure((size_t)Hq * p.n_chunks * 2 * 4);
            if (rc) return rc;
            p.part_o = wk.o.as<float>();
            p.part_ml = wk.ml.as<float>();
        }
        grid.x = p.n_chunks;
        rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_chunk_kernel<0, 0, 8, 1>), lds, &g0);
        if (rc) return rc;
        OJX_LAUNCH((kv_decode_chunk_kernel<0, 0, 8, 1>), grid, dim3(kNT), lds, st, p);
    }
    const int nch = p.n_chunks;
    if (nch > 1)
        OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)nch * 4, st,
                           wk.o.as<float>(), wk.ml.as<float>(), nch, hd, out);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}


// ---- reference-API KV cache: one code stream per head ---------------------
struct KVHead {
    DevBuf kc, vc, ks, vs;
    int len = 0, cap = 0;
};

struct KVCache {
    int heads = 0, hd = 0, D = 0, G = 0, max_seq = 0;
    std::vector<KVHead> h;
    DevBuf cb, bt, kstage, vstage, qstage, ostage;
    int bt_pages = 0;
    KVWork work;
    ~KVCache() {
        for (auto &x : h)
            for (DevBuf *b : {&x.kc, &x.vc, &x.ks, &x.vs}) b->release();
        for (DevBuf *b : {&cb, &bt, &kstage, &vstage, &qstage, &ostage}) b->release();
    }
};

static int grow(DevBuf &b, size_t old_bytes, size_t new_bytes) {
    DevBuf nb;
    int rc = nb.ensure(new_bytes);
    if (rc) return rc;
    OJX_HIP(hipMemset(nb.ptr, 0, new_bytes));
    if (old_bytes) OJX_HIP(hipMemcpy(nb.ptr, b.ptr, old_bytes, hipMemcpyDeviceToDevice));
    b.release();
    b = nb;
    nb.ptr = nullptr;
    return OJASX_OK;
}

static int ensure_pages(KVCache *c, int pages) {
    if (pages <= c->bt_pages) return OJASX_OK;
    std::vector<int> id(pages);
    for (int i = 0; i < pages; ++i) id[i] = i;
    int rc = upload(c->bt, id.data(), id.size() * 4);
    if (rc) return rc;
    c->bt_pages = pages;
    return OJASX_OK;
}

}  // namespace ojx

using ojx::KVCache;

extern "C" {

OJASX_API OjasxKVHandle ojasx_create_kv_cache(int num_heads, int head_dim, int max_seq_len,
                                              int block_dim) {
    using namespace ojx;
    if (num_heads <= 0 || head_dim <= 0 || block_dim <= 0 || block_dim > kMaxD ||
        head_dim % block_dim || head_dim / block_dim > kMaxRG || max_seq_len < 0 ||
        head_dim > 1024) {
        set_error("invalid KV cache shape");
        return nullptr;
    }
    KVCache *c = new (std::nothrow) KVCache;
    if (!c) return nullptr;
    c->heads = num_heads;
    c->hd = head_dim;
    c->D = block_dim;
    c->G = head_dim / block_dim;
    c->max_seq = max_seq_len;
    c->h.resize(num_heads);
    // The reference's implicit codebook: C[c] = (c - 128) e_0.
    std::vector<float> cb((size_t)256 * block_dim, 0.f);
    for (int i = 0; i < 256; ++i) cb[(size_t)i * block_dim] = (float)(i - 128);
    int rc = upload(c->cb, cb.data(), cb.size() * 4);
    for (auto &hh : c->h) {
        if (rc) break;
        const int cap = (int)round_up(std::max(max_seq_len, 1), 16);
        rc = grow(hh.kc, 0, (size_t)cap * c->G);
        if (!rc) rc = grow(hh.vc, 0, (size_t)cap * c->G);
        if (!rc) rc = grow(hh.ks, 0, (size_t)cap * 4);
        if (!rc) rc = grow(hh.vs, 0, (size_t)cap * 4);
        hh.cap = cap;
    }
    if (!rc) rc = c->kstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->vstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->qstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->ostage.ensure((size_t)head_dim * 4);
    if (rc) {
        delete c;
        return nullptr;
    }
    return c;
}

OJASX_API int ojasx_kv_cache_append(OjasxKVHandle handle, int head_idx, const float *k,
                                    const float *v) {
    using namespace ojx;
    if (!handle || !k || !v) return OJASX_ERR_NULL;
    KVCache *c = static_cast<KVCache *>(handle);
    if (head_idx < 0 || head_idx >= c->heads) return OJASX_ERR_HEAD;
    KVHead &hh = c->h[head_idx];
    if (hh.len >= hh.cap) {  // ojasx_lut_kv_cache.cpp:17-25: grow to max(1024, 2 * cap)
        const int nc = (int)round_up(std::max(1024, hh.cap * 2), 16);
        int rc = grow(hh.kc, (size_t)hh.cap * c->G, (size_t)nc * c->G);
        if (!rc) rc = grow(hh.vc, (size_t)hh.cap * c->G, (size_t)nc * c->G);
        if (!rc) rc = grow(hh.ks, (size_t)hh.cap * 4, (size_t)nc * 4);
        if (!rc) rc = grow(hh.vs, (size_t)hh.cap * 4, (size_t)nc * 4);
        if (rc) return rc;
        hh.cap = nc;
    }
    OJX_HIP(hipMemcpy(c->kstage.ptr, k, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    OJX_HIP(hipMemcpy(c->vstage.ptr, v, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    OJX_LAUNCH(kv_append_kernel, dim3(1), dim3(128), 0, nullptr, c->kstage.as<float>(),
                       c->vstage.as<float>(), c->hd, c->D, hh.kc.as<uint8_t>() + (size_t)hh.len * c->G,
                       hh.vc.as<uint8_t>() + (size_t)hh.len * c->G, hh.ks.as<float>() + hh.len,
                       hh.vs.as<float>() + hh.len);
    OJX_HIP(hipGetLastError());
    OJX_HIP(hipDeviceSynchronize());
    hh.len++;
    return OJASX_OK;
}

OJASX_API int ojasx_kv_cache_attention(OjasxKVHandle handle, int head_idx, const float *q,
                                       float *out_context, float scale_factor) {
    using namespace ojx;
    if (!handle || !q || !out_context) return OJASX_ERR_NULL;
    KVCache *c = static_cast<KVCache *>(handle);
    if (head_idx < 0 || head_idx >= c->heads) return OJASX_ERR_HEAD;
    KVHead &hh = c->h[head_idx];
    if (hh.len == 0) return OJASX_OK;
    int rc = ensure_pages(c, hh.cap / 16);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(c->qstage.ptr, q, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    rc = kv_decode(c->qstage.as<float>(), hh.kc.as<uint8_t>(), hh.ks.as<float>(),
                   hh.vc.as<uint8_t>(), hh.vs.as<float>(), c->cb.as<float>(), c->cb.as<float>(),
                   c->bt.as<int>(), hh.len, 16, 1, 1, c->hd, c->D, scale_factor,
                   c->ostage.as<float>(), nullptr, c->work);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(out_context, c->ostage.ptr, (size_t)c->hd * 4, hipMemcpyDeviceToHost));
    return OJASX_OK;
}

OJASX_API size_t ojasx_kv_cache_get_memory_size(OjasxKVHandle handle) {
    if (!handle) return 0;
    const KVCache *c = static_cast<const KVCache *>(handle);
    size_t b = 0;
    for (const auto &hh : c->h)  // ojasx_lut_kv_cache.h:40-44 accounting
        b += (size_t)hh.cap * c->G * 2 + (size_t)hh.cap * 4 * 2 + (size_t)256 * c->D * 4 * 2;
    return b;
}

OJASX_API float ojasx_kv_cache_get_compression_ratio(OjasxKVHandle handle) {
    if (!handle) return 0.f;
    const KVCache *c = static_cast<const KVCache *>(handle);
    if (c->heads == 0) return 0.f;
    const size_t len = c->h[0].len;
    const size_t dense = 2 * (size_t)c->hd * len * 4;
    const size_t comp = len * (c->G * 2 + 2 * 4);
    return (float)dense / (float)(comp ? comp : 1);
}

OJASX_API void ojasx_destroy_kv_cache(OjasxKVHandle handle) {
    delete static_cast<KVCache *>(handle);
}

OJASX_API int ojasx_kv_decode_paged_device(const float *q, const uint8_t *k_codes,
                                           const float *k_scales, const uint8_t *v_codes,
                                           const float *v_scales, const float *k_cb,
                                           const float *v_cb, const int *block_table, int seq_len,
                                           int page_size, int num_q_heads, int num_kv_heads,
                                           int head_dim, int block_dim, float scale_factor,
                                           float *out, void *stream) {
    using namespace ojx;
    if (!q || !k_codes || !k_scales || !v_codes || !v_scales || !k_cb || !v_cb || !block_table ||
        !out)
        return OJASX_ERR_NULL;
    return kv_decode(q, k_codes, k_scales, v_codes, v_scales, k_cb, v_cb, block_table, seq_len,
                     page_size, num_q_heads, num_kv_heads, head_dim, block_dim, scale_factor, out,
                     static_cast<hipStream_t>(stream), t_work);
}

}  // extern "C"

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
//  * head_dim 128 as 8 groups of 16 (all configured shapes), inputs aligned
//    for vector loads, two kernels by context length:
//    - kv_decode_small (T <= 4096): chunks of 64 tokens, one wave per query
//      head; scores computed directly from the K codebook in LDS (4x fewer
//      FMAs than building LUT_q for 64 tokens), in-wave softmax statistics,
//      V accumulated per output dim pair;
//    - kv_decode_wide (longer): chunks of up to 1024 tokens in 1024-thread
//      workgroups (about one per CU); LUT_q per chunk, scores by LUT
//      gathers, V accumulated in the code domain without atomics.
//  * kv_decode_chunk: any other shape (runtime groups and block size) or
//    unaligned inputs: chunks of 256 tokens, LUT_q, codes read bytewise, V as
//    a code histogram (LDS atomics) contracted with the V codebook.
//  Every kernel writes the normalised output when the context is one chunk,
//  otherwise (max, sum, o) per chunk.
//  * kv_merge: log-sum-exp merge of the chunks in chunk order (the online
//    softmax combine of ojasx_24x96/long_context.py:133-166).
// Cache layout (device): codes [pages][Hkv][page][G] uint8, scales
// [pages][Hkv][page] fp32, so a page of one kv head is contiguous.
#include <algorithm>
#include <cmath>
#include <mutex>
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
    // Context length read on the device, *len_dev + len_add, when len_dev is
    // set (kv_decode_small_kernel only): n_chunks then covers the longest
    // context and chunks past the current one exit at once.
    const int *len_dev;
    int len_add;
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
#pragma unroll
        for (int u = 0; u < GW; ++u) kw[i][u] = vw[i][u] = 0;
        for (int g = 0; g < G; ++g) {
            kw[i][g >> 2] |= (uint32_t)p.kc[slot * G + g] << ((g & 3) * 8);
            vw[i][g >> 2] |= (uint32_t)p.vc[slot * G + g] << ((g & 3) * 8);
        }
    }
    for (int i = tid; i < nj * G * kHP; i += kNT) hist[i] = 0.f;
    __syncthreads();
    // ---- LUT_q[j][g][tid] = <q_j[gD:(g+1)D], Ck[tid]>
    for (int jg = 0; jg < nj * G; ++jg) {
        const int j = jg / G, g = jg - j * G;
        const float *qv = qs + j * hd + g * D;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < DM; ++d)
            if (d < D) dot = fmaf(qv[d], ck[d], dot);
        lutq[jg * 256 + tid] = dot;
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

// Fast path (G = 8 groups of D = 16, head_dim 128, up to 4 query heads per kv
// head): 1024 threads, one token per thread, chunk of C <= 1024 tokens.
//  * round trip 1: the token's block-table entry, q, one float4 of the V
//    codebook and, for waves 0-7, their operand of the K codebook; round
//    trip 2: the token's K/V code words and scales;
//  * LUT_q^T[256 x 32] = Ck[256 x 16] . Q^T[16 x 32] (column n = (j, g):
//    dims 16g .. 16g + 15 of query head j) on v_mfma_f32_32x32x16_bf16 over
//    exact bf16 splits (fp32 accuracy), wave w < 8 taking centroids
//    32w .. 32w + 31;
//  * scores (8 LUT gathers per head), chunk max and sum of exp per head by
//    DPP wave reductions and 16 per-wave values in LDS (fixed order);
//  * V in the code domain: thread (token group tg of 32, group g, d-quad dq)
//    adds p_jt * vs_t * Cv[code][4dq..4dq+3] for the 4 heads over tokens
//    tg, tg+32, ... (code rows addressed by byte offsets staged per token);
//    the two token groups of a wave are added with one shuffle, the 16 waves'
//    partials in LDS in a fixed order.  Measured and not kept: code
//    histograms contracted on MFMA (3x slower: LDS float atomics on
//    colliding bins serialise) and 8 dims per lane (the cross-lane sums cost
//    more than the shared weight reads save).
constexpr int kWideNT = 1024;
constexpr int kLutP = 257;    // LUT_q row pitch (one row per (j, g)): conflict-free stores

__global__ __launch_bounds__(kWideNT) void kv_decode_wide_kernel(KVParams p) {
    extern __shared__ float sm[];
    float *qs = sm;                                          // [4][128]
    float *cv = qs + 4 * 128;                                // [256][16]
    float *lutq = cv + 256 * 16;                             // [32][kLutP]
    float4 *pw = reinterpret_cast<float4 *>(lutq + 32 * kLutP + 32);   // [C] weights of 4 heads
    uint4 *vof = reinterpret_cast<uint4 *>(pw + kWideNT);   // [C][8] V codebook row offsets, u16
    float *part = reinterpret_cast<float *>(vof + kWideNT); // [16 waves][32][16]
    __shared__ __align__(16) float wred[2][4][kWideNT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int R = p.Hq / p.Hkv;
    const int h = blockIdx.y;
    const int j0 = h * R + blockIdx.z * 4;
    const int nj = min(4, R - (int)blockIdx.z * 4);
    const int C = p.Tc;
    const int c = blockIdx.x;
    const int t = c * C + tid;
    const bool live = tid < C && t < p.T;
    const int tc = min(t, p.T - 1);

    // ---- round trip 1
    const int pg = p.bt[tc / p.P];
    float af[8];   // K codebook row 32 (wv % 8) + lane % 32, dims 8 (lane / 32) ..
    {
        const int cr = (wv & 7) * 32 + (lane & 31);
        const float4 *kr =
            reinterpret_cast<const float4 *>(p.kcb + ((size_t)h * 256 + cr) * 16 + 8 * (lane >> 5));
        const float4 u = kr[0], v = kr[1];
        af[0] = u.x; af[1] = u.y; af[2] = u.z; af[3] = u.w;
        af[4] = v.x; af[5] = v.y; af[6] = v.z; af[7] = v.w;
    }
    const float4 cvv = reinterpret_cast<const float4 *>(p.vcb + (size_t)h * 256 * 16)[tid];
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < nj * 32) qv = reinterpret_cast<const float4 *>(p.q + (size_t)j0 * 128)[tid];
    // ---- round trip 2: the token's codes and scales
    const size_t slot = ((size_t)pg * p.Hkv + h) * p.P + (tc % p.P);
    const uint2 kw = *reinterpret_cast<const uint2 *>(p.kc + slot * 8);
    const uint2 vw = *reinterpret_cast<const uint2 *>(p.vc + slot * 8);
    const float ksv = p.ks[slot], vsv = p.vs[slot];
    if (tid < 128) reinterpret_cast<float4 *>(qs)[tid] = qv;   // zero rows past nj
    reinterpret_cast<float4 *>(cv)[tid] = cvv;
    __syncthreads();

    // ---- LUT_q on MFMA: wave w < 8, centroids 32w .. 32w + 31
    if (wv < 8) {
        const int n = lane & 31, hh = lane >> 5;
        const float4 *qp =
            reinterpret_cast<const float4 *>(qs + (n >> 3) * 128 + 16 * (n & 7) + 8 * hh);
        const float4 b0 = qp[0], b1 = qp[1];
        const float bf[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        bf16x8_t a[3], b[3];
        split3_bf16(af, a);
        split3_bf16(bf, b);
        const f32x16_t d = mfma32_bf16x3(a, b);
        float *L = lutq + n * kLutP + 32 * wv + 4 * hh;
#pragma unroll
        for (int r = 0; r < 16; ++r) L[8 * (r / 4) + (r % 4)] = d[r];
    }
    __syncthreads();

    // ---- scores, chunk max and sum of exp per head (the 4 heads' wave
    //      reductions interleaved)
    const uint32_t kwd[2] = {kw.x, kw.y};
    float s[4], wm[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = -INFINITY;
        if (live && j < nj) {
            const float *L = lutq + j * 8 * kLutP;
            float v[8];
#pragma unroll
            for (int g = 0; g < 8; ++g)
                v[g] = L[g * kLutP + ((kwd[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
            float a = 0.f;
#pragma unroll
            for (int g = 0; g < 8; ++g) a += v[g];
            s[j] = a * (ksv * p.sf);
        }
        wm[j] = s[j];
    }
    wave_max_n(wm);
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < 4; ++j) wred[0][j][wv] = wm[j];
    __syncthreads();
    float mx[4], e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 *w4 = reinterpret_cast<const float4 *>(wred[0][j]);
        float m = -INFINITY;
#pragma unroll
        for (int q = 0; q < kWideNT / 256; ++q) {
            const float4 u = w4[q];
            m = fmaxf(m, fmaxf(fmaxf(u.x, u.y), fmaxf(u.z, u.w)));
        }
        mx[j] = m;
        e[j] = s[j] == -INFINITY ? 0.f : expf(s[j] - m);
        wm[j] = e[j];
    }
    wave_sum_n(wm);
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < 4; ++j) wred[1][j][wv] = wm[j];
    const float f = live ? vsv : 0.f;
    pw[tid] = make_float4(e[0] * f, e[1] * f, e[2] * f, e[3] * f);
    // the token's V codes as byte offsets of their codebook rows (code * 64),
    // 16 bits each, group g at element g
    {
        const uint32_t x = vw.x, y = vw.y;
        auto pair = [](uint32_t wd, int sh) {
            return (((wd >> sh) & 0xffu) << 6) | (((wd >> (sh + 8)) & 0xffu) << 22);
        };
        vof[tid] = make_uint4(pair(x, 0), pair(x, 16), pair(y, 0), pair(y, 16));
    }
    __syncthreads();

    // ---- V in the code domain
    {
        const int tg = tid >> 5, r = tid & 31, g = r >> 2, dq = r & 3;
        float acc[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[j][k] = 0.f;
        const char *cvq = reinterpret_cast<const char *>(cv) + 16 * dq;
        const unsigned short *vo = reinterpret_cast<const unsigned short *>(vof) + g;
#pragma unroll 4
        for (int tl = tg; tl < C; tl += 32) {
            const float4 cq = *reinterpret_cast<const float4 *>(cvq + vo[8 * tl]);
            const float4 wj = pw[tl];
            const float wa[4] = {wj.x, wj.y, wj.z, wj.w};
            const float ca[4] = {cq.x, cq.y, cq.z, cq.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[j][k] = fmaf(wa[j], ca[k], acc[j][k]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[j][k] += __shfl_xor(acc[j][k], 32);
        if (lane < 32)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < 4; ++k) part[(wv * 32 + r) * 16 + j * 4 + k] = acc[j][k];
    }
    __syncthreads();

    // ---- outputs (j, g*16 + d): the 16 waves' partials in order
    float lsum[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float l = wred[1][j][0];
#pragma unroll
        for (int q = 1; q < kWideNT / 64; ++q) l += wred[1][j][q];
        lsum[j] = l;
    }
    if (tid < nj * 128) {
        const int j = tid >> 7, od = tid & 127;
        const int g = od >> 4, d = od & 15, r = g * 4 + (d >> 2), k = d & 3;
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < kWideNT / 64; ++w) a += part[(w * 32 + r) * 16 + j * 4 + k];
        const float l = j == 0 ? lsum[0] : j == 1 ? lsum[1] : j == 2 ? lsum[2] : lsum[3];
        if (p.n_chunks == 1)
            p.out[(size_t)(j0 + j) * 128 + od] = a / l;
        else
            p.part_o[((size_t)(j0 + j) * p.n_chunks + c) * 128 + od] = a;
    }
    if (p.n_chunks > 1 && tid < nj) {
        const float l = tid == 0 ? lsum[0] : tid == 1 ? lsum[1] : tid == 2 ? lsum[2] : lsum[3];
        const float m = tid == 0 ? mx[0] : tid == 1 ? mx[1] : tid == 2 ? mx[2] : mx[3];
        float *ml = p.part_ml + ((size_t)(j0 + tid) * p.n_chunks + c) * 2;
        ml[0] = m;
        ml[1] = l;
    }
}

// Short-context fast path (G = 8, D = 16, up to 4 query heads per kv head):
// chunks of 64 * TPL tokens, 256 threads.  A short chunk costs 4x fewer FMAs
// computing scores directly, <q_j,g, Ck[code]> from the K codebook in LDS,
// than building LUT_q.  Every codebook row a token selects is read from LDS
// once for all the workgroup's query heads:
//  * scores: four lanes per token, each a quarter of the 16 dims, a quad
//    shuffle sum per head; the scores pass through LDS to wave j = head j;
//  * softmax statistics of head j: in-wave DPP reductions over the chunk;
//  * V: wave w takes a quarter of the chunk's tokens for all heads, lane l
//    owning output dims 2l, 2l+1; the four waves' sums are added in LDS in
//    wave order.
// Wave u < TPL loads the codes and scales of tokens 64u .. 64u + 63.  The
// per-head form (each wave reading the rows for its own head) measured 8.3
// vs 7.4 us at 2048 tokens (8 kv / 32 q heads).
constexpr int kSmallC = 64;
// Longest context for the 64-token chunks: measured 13.9 vs 14.7 us (wide)
// at 4096 tokens and 22.1 vs 15.0 us at 8192 (8 kv / 32 q heads).
constexpr int kSmallMaxT = 4096;

template <int TPL>
__global__ __launch_bounds__(kNT) void kv_decode_small_kernel(KVParams p) {
    constexpr int C = kSmallC * TPL;     // tokens per chunk
    __shared__ float4 ck4[256 * 4];      // K codebook [256][16], rows swizzled (cb_slot)
    __shared__ float4 cv4[256 * 4];      // V codebook [256][16]
    __shared__ float4 q4s[4 * 32];       // q [4][128]
    __shared__ uint2 kcw[C], vcw[C];
    __shared__ float wsc[4][C];          // K scale * sf and V scale, then p_jt * vs_t
    __shared__ float ssc[4][C];          // scores of the chunk's tokens per head
    __shared__ float2 ored[4][4][64];    // V sums per wave, head and dim pair
    const int tid = threadIdx.x, lane = tid & 63, j = tid >> 6;
    const int R = p.Hq / p.Hkv;
    const int h = blockIdx.y;
    const int j0 = h * R + blockIdx.z * 4;
    const int nj = min(4, R - (int)blockIdx.z * 4);
    const int c = blockIdx.x;
    // ---- round trip 1, none of it waiting for the device length: the length,
    // codebooks, q, and the block-table entry of wave j's token (the table
    // covers the launch's longest context p.T)
    const int len = p.len_dev ? *p.len_dev : 0;
    const float4 *gk = reinterpret_cast<const float4 *>(p.kcb + (size_t)h * 256 * 16);
    const float4 *gv = reinterpret_cast<const float4 *>(p.vcb + (size_t)h * 256 * 16);
    float4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        a[u] = gk[tid + u * kNT];
        b[u] = gv[tid + u * kNT];
    }
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < nj * 32) qv = reinterpret_cast<const float4 *>(p.q + (size_t)j0 * 128)[tid];
    const int tw = c * C + j * kSmallC + lane;   // the token wave j loads (j < TPL)
    const int pg = j < TPL ? p.bt[min(tw, p.T - 1) / p.P] : 0;
    // device length clamped to the launch's longest context p.T
    const int T = p.len_dev ? min(len + p.len_add, p.T) : p.T;
    if (c * C >= T) return;              // whole workgroup: a chunk past the context
    const bool wlive = j < TPL && tw < T;
    // ---- round trip 2: codes and scales of the live tokens
    uint2 kw = make_uint2(0, 0), vw = make_uint2(0, 0);
    float ksv = 0.f, vsv = 0.f;
    if (wlive) {
        const size_t slot = ((size_t)pg * p.Hkv + h) * p.P + (tw % p.P);
        kw = *reinterpret_cast<const uint2 *>(p.kc + slot * 8);
        vw = *reinterpret_cast<const uint2 *>(p.vc + slot * 8);
        ksv = p.ks[slot];
        vsv = p.vs[slot];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid + u * kNT;
        ck4[cb_slot(i >> 2, i & 3)] = a[u];
        cv4[tid + u * kNT] = b[u];
    }
    if (tid < 128) q4s[tid] = qv;
    if (j < TPL) {
        const int tl = j * kSmallC + lane;
        kcw[tl] = kw;
        vcw[tl] = vw;
        wsc[0][tl] = wlive ? ksv * p.sf : 0.f;
        wsc[1][tl] = wlive ? vsv : 0.f;
    }
    __syncthreads();

    // ---- scores: pass u, lane (token tq = 64 u + 16 j + lane / 4, quarter
    //      k4 = lane % 4) reads its token's K codebook quarter once per group
    //      for every head of the workgroup; a quad sum completes each score,
    //      then the scores go through LDS to a head per wave
    const int k4 = lane & 3;
#pragma unroll
    for (int u = 0; u < TPL; ++u) {
        const int tq = u * kSmallC + 16 * j + (lane >> 2);
        float pq[4] = {0.f, 0.f, 0.f, 0.f};
        const uint2 kq = kcw[tq];
        const uint32_t kd[2] = {kq.x, kq.y};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t code = (kd[g >> 2] >> ((g & 3) * 8)) & 0xffu;
            const float4 cq = ck4[cb_slot(code, k4)];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                if (jj >= nj) break;
                const float4 qq = q4s[jj * 32 + g * 4 + k4];
                float dot = pq[jj];
                dot = fmaf(qq.x, cq.x, dot);
                dot = fmaf(qq.y, cq.y, dot);
                dot = fmaf(qq.z, cq.z, dot);
                dot = fmaf(qq.w, cq.w, dot);
                pq[jj] = dot;
            }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            pq[jj] += __shfl_xor(pq[jj], 1);
            pq[jj] += __shfl_xor(pq[jj], 2);
        }
        const float kfq = wsc[0][tq];
        if (k4 == 0) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) ssc[jj][tq] = c * C + tq < T ? pq[jj] * kfq : -INFINITY;
        }
    }
    float vf[TPL];
#pragma unroll
    for (int u = 0; u < TPL; ++u) vf[u] = wsc[1][u * kSmallC + lane];
    __syncthreads();   // the scores are in; wsc is rewritten with the weights below

    // ---- softmax of head j over the chunk (lane = token lane + 64 u)
    float sc[TPL];
#pragma unroll
    for (int u = 0; u < TPL; ++u) sc[u] = j < nj ? ssc[j][u * kSmallC + lane] : -INFINITY;
    float smax = sc[0];
#pragma unroll
    for (int u = 1; u < TPL; ++u) smax = fmaxf(smax, sc[u]);
    const float m = wave_max_f(smax);
    float esum = 0.f;
#pragma unroll
    for (int u = 0; u < TPL; ++u) {
        const float e = (sc[u] == -INFINITY) ? 0.f : expf(sc[u] - m);
        esum += e;
        wsc[j][u * kSmallC + lane] = e * vf[u];
    }
    const float l = wave_sum_f(esum);
    __syncthreads();

    // ---- V: lane owns dims 2 lane, 2 lane + 1 (group g = lane / 8) of every
    //      head; wave j takes tokens j C / 4 .. (j + 1) C / 4 - 1 (each V
    //      codebook row read once for all heads); the waves' sums meet in LDS,
    //      added in wave order
    {
        const int g = lane >> 3, d0 = (lane & 7) * 2;
        const float *cvf = reinterpret_cast<const float *>(cv4);
        float o[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
        constexpr int TW = C / 4;
#pragma unroll 4
        for (int tl = TW * j; tl < TW * j + TW; ++tl) {
            const uint2 cw = vcw[tl];
            const uint32_t code = ((g < 4 ? cw.x : cw.y) >> ((g & 3) * 8)) & 0xffu;
            const float2 cvv = *reinterpret_cast<const float2 *>(cvf + code * 16 + d0);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const float wgt = wsc[jj][tl];
                o[jj][0] = fmaf(wgt, cvv.x, o[jj][0]);
                o[jj][1] = fmaf(wgt, cvv.y, o[jj][1]);
            }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) ored[j][jj][lane] = make_float2(o[jj][0], o[jj][1]);
    }
    __syncthreads();
    if (j < nj) {
        float2 o = ored[0][j][lane];
#pragma unroll
        for (int u = 1; u < 4; ++u) {
            const float2 t = ored[u][j][lane];
            o.x += t.x;
            o.y += t.y;
        }
        const int od = lane * 2;
        if (p.n_chunks == 1) {
            p.out[(size_t)(j0 + j) * 128 + od] = o.x / l;
            p.out[(size_t)(j0 + j) * 128 + od + 1] = o.y / l;
        } else {
            float *po = p.part_o + ((size_t)(j0 + j) * p.n_chunks + c) * 128 + od;
            po[0] = o.x;
            po[1] = o.y;
            if (lane == 0) {
                float *ml = p.part_ml + ((size_t)(j0 + j) * p.n_chunks + c) * 2;
                ml[0] = m;
                ml[1] = l;
            }
        }
    }
}

// Log-sum-exp merge of the chunks of one query head, chunks in order:
// (max, sum) pairs staged in LDS, max and normaliser by wave shuffles, then
// each thread sums one output coordinate over the chunks.
// With len_dev set, only the first ceil((*len_dev + len_add) / chunk) of the
// chunks (the partials' stride) are merged.  With extra set, the stride's last
// slot holds one more partial, merged after the live chunks (it is not one of
// them).
__global__ __launch_bounds__(kNT) void kv_merge_kernel(const float *part_o, const float *part_ml,
                                                      int stride_chunks, int hd, float *out,
                                                      const int *len_dev, int len_add, int chunk,
                                                      int extra) {
    extern __shared__ float wsm[];   // [n_chunks] chunk weights
    __shared__ float red[kNT / 64];
    const int j = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n_slots = stride_chunks - extra;
    const int n_live =
        len_dev ? min(n_slots, (*len_dev + len_add + chunk - 1) / chunk) : n_slots;
    const int n_chunks = max(n_live, 0) + extra;   // chunk c < n_live at slot c, then the extra
    if (n_chunks <= 0) return;                      // empty context: out untouched
    auto slot = [&](int c) { return c < n_live ? c : stride_chunks - 1; };
    // The statistics of chunk tid first, then the partials of the first
    // 2 * kMergePre chunks for the two-threads-per-coordinate sum (even and odd
    // chunks) used when 2 * hd <= kNT.  Every load is unconditional, at clamped
    // indices, so the code stays straight-line and the max reduction waits
    // for the statistics only (vmcnt counts loads in issue order).
    const float *ml = part_ml + (size_t)j * stride_chunks * 2;
    float2 st0 = *reinterpret_cast<const float2 *>(ml + 2 * slot(min(tid, n_chunks - 1)));
    constexpr int kMergePre = 36;
    const bool pair = 2 * hd <= kNT;
    const int hf = tid / hd, d = tid - hf * hd;
    const float *po = part_o + (size_t)j * stride_chunks * hd + d;
    float pre[kMergePre];
#pragma unroll
    for (int u = 0; u < kMergePre; ++u)
        pre[u] = po[(size_t)slot(min(min(hf, 1) + 2 * u, n_chunks - 1)) * hd];
    if (tid >= n_chunks) st0 = make_float2(-INFINITY, 0.f);
    float m = st0.x;
    for (int c = tid + kNT; c < n_chunks; c += kNT) m = fmaxf(m, ml[2 * slot(c)]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int q = 1; q < kNT / 64; ++q) m = fmaxf(m, red[q]);
    __syncthreads();
    float l = 0.f;
    if (tid < n_chunks) {
        const float wc = st0.x == -INFINITY ? 0.f : expf(st0.x - m);
        wsm[tid] = wc;
        l = st0.y * wc;
    }
    for (int c = tid + kNT; c < n_chunks; c += kNT) {
        const float mc = ml[2 * slot(c)];
        const float wc = mc == -INFINITY ? 0.f : expf(mc - m);
        wsm[c] = wc;
        l += ml[2 * slot(c) + 1] * wc;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    if (lane == 0) red[wv] = l;
    __syncthreads();
    l = red[0];
#pragma unroll
    for (int q = 1; q < kNT / 64; ++q) l += red[q];
    const float inv = 1.f / l;
    if (pair) {
        // the prefetched chunks, then the rest 16 loads in flight at a time
        __shared__ float half_sum[kNT / 2];
        float acc = 0.f;
        if (hf < 2) {
            float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < kMergePre; ++u) {
                const int c = hf + 2 * u;
                if (c < n_chunks) o[u & 3] = fmaf(pre[u], wsm[c], o[u & 3]);
            }
            int c = hf + 2 * kMergePre;
            for (; c + 30 < n_chunks; c += 32) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = po[(size_t)slot(c + 2 * u) * hd];
#pragma unroll
                for (int u = 0; u < 16; ++u) o[u & 3] = fmaf(v[u], wsm[c + 2 * u], o[u & 3]);
            }
            for (; c < n_chunks; c += 2) o[0] = fmaf(po[(size_t)slot(c) * hd], wsm[c], o[0]);
            acc = (o[0] + o[1]) + (o[2] + o[3]);
            if (hf == 1) half_sum[d] = acc;
        }
        __syncthreads();
        if (hf == 0) out[(size_t)j * hd + d] = (acc + half_sum[d]) * inv;
        return;
    }
    for (int d = tid; d < hd; d += kNT) {
        const float *po = part_o + (size_t)j * stride_chunks * hd + d;
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int c = 0;
        for (; c + 8 <= n_chunks; c += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = po[(size_t)slot(c + u) * hd];
#pragma unroll
            for (int u = 0; u < 8; ++u) o[u] = fmaf(v[u], wsm[c + u], o[u]);
        }
        for (; c < n_chunks; ++c) o[0] = fmaf(po[(size_t)slot(c) * hd], wsm[c], o[0]);
        out[(size_t)j * hd + d] = (((o[0] + o[1]) + (o[2] + o[3])) + ((o[4] + o[5]) + (o[6] + o[7]))) * inv;
    }
}

// Workspace for the decode partials (part_o, part_ml), one per thread of the
// host (device entry points called from several host threads each get their
// own).  reserve() grows the buffers and sets po / pml; a workspace built on
// fixed memory (fixed_o, non-null) never allocates and refuses a request
// beyond its capacity instead.
struct KVWork {
    DevBuf o, ml;
    float *po = nullptr, *pml = nullptr;
    float *fixed_o = nullptr, *fixed_ml = nullptr;
    size_t fixed_o_bytes = 0, fixed_ml_bytes = 0;
    int reserve(size_t o_bytes, size_t ml_bytes) {
        if (fixed_o) {
            if (o_bytes > fixed_o_bytes || ml_bytes > fixed_ml_bytes) {
                set_error("decode partials need %zu + %zu bytes; the no-allocation scratch holds "
                          "%zu + %zu (num_q_heads x chunks too large)",
                          o_bytes, ml_bytes, fixed_o_bytes, fixed_ml_bytes);
                return OJASX_ERR_INVALID;
            }
            po = fixed_o;
            pml = fixed_ml;
            return OJASX_OK;
        }
        int rc = grow(o, o_bytes);
        if (!rc) rc = grow(ml, ml_bytes);
        if (rc) return rc;
        po = o.as<float>();
        pml = ml.as<float>();
        return OJASX_OK;
    }
    // A buffer that grows is retired, not freed, until the thread exits: a
    // graph captured over an earlier (smaller) call still owns valid memory.
    // Growth at least doubles, so the retired buffers total less than the
    // live one.
    std::vector<DevBuf> retired;
    int grow(DevBuf &b, size_t n) {
        if (n <= b.bytes && b.ptr) return OJASX_OK;
        if (b.ptr) {
            retired.push_back(b);
            n = std::max(n, 2 * b.bytes);
            b.ptr = nullptr;
            b.bytes = 0;
        }
        return b.ensure(n);
    }
    ~KVWork() {
        o.release();
        ml.release();
        for (DevBuf &b : retired) b.release();
    }
};
static thread_local KVWork t_work;

// Scratch of the no-allocation decode (ojasx_kv_decode_paged_device_noalloc):
// partial outputs [Hq][chunks][hd] fp32 in the first kScratchO bytes, then
// partial (max, sum) pairs [Hq][chunks][2].  Every GPU holds its own copy
// until the process ends; its device address is looked up once per device.
constexpr size_t kScratchO = (size_t)4 << 20;
constexpr size_t kScratchML = (size_t)64 << 10;
static __device__ __align__(256) unsigned char scratch[kScratchO + kScratchML];

// Decode with the context length read on the device (*len_dev + len_add, at
// most T_max): the short-context kernel over ceil(T_max / 64) chunks, the
// chunks past the current length exiting at once, then the merge of the live
// chunks.  Head dim 128, block dim 16; partials part_o [Hq][n][128] and
// part_ml [Hq][n][2] with n = ceil(T_max / 64).  Launches a fixed grid, so a
// captured graph can replay it as the context grows.
// Tokens per lane of the short-context kernel for a device-length decode of
// up to T_max tokens (chunks of 64 * TPL).  64-token chunks measured fastest
// in the decoder at 4224 tokens: 12.5 us per call against 15.6 us with 128
// (the merge shrinks less than the per-workgroup work grows).
int kv_device_len_tpl(int T_max) {
    (void)T_max;
    return 1;
}

int kv_decode_device_len(const float *q, const uint8_t *kc, const float *ks, const uint8_t *vc,
                         const float *vs, const float *kcb, const float *vcb, const int *bt,
                         const int *len_dev, int len_add, int T_max, int P, int Hq, int Hkv,
                         float sf, float *part_o, float *part_ml, float *out, hipStream_t st,
                         int tpl) {
    if (Hkv <= 0 || Hq <= 0 || Hq % Hkv || P <= 0 || T_max <= 0) {
        set_error("invalid KV decode shape Hq=%d Hkv=%d page=%d T_max=%d", Hq, Hkv, P, T_max);
        return OJASX_ERR_INVALID;
    }
    if (tpl == 0) tpl = kv_device_len_tpl(T_max);
    if (tpl != 1 && tpl != 2 && tpl != 4) {
        set_error("tokens per lane must be 0, 1, 2 or 4 (got %d)", tpl);
        return OJASX_ERR_INVALID;
    }
    const int C = kSmallC * tpl;
    const int n_chunks = (T_max + C - 1) / C;
    const int nz = (Hq / Hkv + 3) / 4;
    KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, part_o, part_ml, out, T_max, P,
               Hq, Hkv, 128, 16, 8, C, 4, n_chunks, sf, len_dev, len_add};
    const dim3 grid(n_chunks, Hkv, nz);
    if (tpl == 1) OJX_LAUNCH(kv_decode_small_kernel<1>, grid, dim3(kNT), 0, st, p);
    else if (tpl == 2) OJX_LAUNCH(kv_decode_small_kernel<2>, grid, dim3(kNT), 0, st, p);
    else OJX_LAUNCH(kv_decode_small_kernel<4>, grid, dim3(kNT), 0, st, p);
    if (n_chunks > 1)
        OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)n_chunks * 4, st, part_o, part_ml,
                   n_chunks, 128, out, len_dev, len_add, C, 0);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

int kv_merge_device_len(const float *part_o, const float *part_ml, int stride_chunks, int chunk,
                        int Hq, const int *len_dev, int len_add, int extra, float *out,
                        hipStream_t st) {
    if (stride_chunks < 1 + (extra ? 1 : 0) || Hq <= 0 || chunk <= 0) {
        set_error("invalid KV merge shape Hq=%d chunks=%d", Hq, stride_chunks);
        return OJASX_ERR_INVALID;
    }
    OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)stride_chunks * 4, st, part_o, part_ml,
               stride_chunks, 128, out, len_dev, len_add, chunk, extra ? 1 : 0);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

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
    auto aligned = [](const void *ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; };
    if (G == 8 && D == 16 && aligned(q, 16) && aligned(kcb, 16) && aligned(vcb, 16) && aligned(kc, 8) &&
        aligned(vc, 8)) {
        const int nz = (R + 3) / 4;
        if (T <= kSmallMaxT) {
            const int n_chunks = (T + kSmallC - 1) / kSmallC;
            if (n_chunks > 1) {
                const int rc = wk.reserve((size_t)Hq * n_chunks * hd * 4, (size_t)Hq * n_chunks * 2 * 4);
                if (rc) return rc;
            }
            KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, wk.po, wk.pml, out, T, P,
                       Hq, Hkv, hd, D, G, kSmallC, 4, n_chunks, sf, nullptr, 0};
            OJX_LAUNCH(kv_decode_small_kernel<1>, dim3(n_chunks, Hkv, nz), dim3(kNT), 0, st, p);
            if (n_chunks > 1)
                OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)n_chunks * 4, st,
                           wk.po, wk.pml, n_chunks, hd, out, nullptr, 0, 1, 0);
            OJX_HIP(hipGetLastError());
            return OJASX_OK;
        }
        // wide fast path: 1024-thread workgroups, chunk size chosen for about
        // one workgroup per CU; small problems take one chunk (no merge)
        const long units = (long)Hkv * nz;
        auto pow2 = [](long v) { long c = 1; while (c < v) c <<= 1; return c; };
        long C = pow2((T * units + 255) / 256);
        C = std::min<long>(1024, std::max<long>(64, C));
        if (T <= 1024 && units <= 16) C = std::max<long>(64, pow2(T));
        const int n_chunks = (int)((T + C - 1) / C);
        if (n_chunks > 1) {
            const int rc = wk.reserve((size_t)Hq * n_chunks * hd * 4, (size_t)Hq * n_chunks * 2 * 4);
            if (rc) return rc;
        }
        KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, wk.po, wk.pml, out, T, P,
                   Hq, Hkv, hd, D, G, (int)C, 4, n_chunks, sf, nullptr, 0};
        const size_t lds = (size_t)(4 * 128 + 256 * 16 + 32 * kLutP + 32) * 4 + (size_t)kWideNT * 16 +
                           (size_t)kWideNT * 16 + (size_t)16 * 32 * 16 * 4;
        static size_t gw = 0;
        int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_wide_kernel), lds, &gw);
        if (rc) return rc;
        OJX_LAUNCH(kv_decode_wide_kernel, dim3(n_chunks, Hkv, nz), dim3(kWideNT), lds, st, p);
        if (n_chunks > 1)
            OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)n_chunks * 4, st,
                       wk.po, wk.pml, n_chunks, hd, out, nullptr, 0, 1, 0);
        OJX_HIP(hipGetLastError());
        return OJASX_OK;
    }
    // Runtime-shape path (other group counts / block sizes, or inputs not
    // aligned for vector loads): 256 tokens per workgroup, query heads per
    // workgroup as many of the GQA group as fit, codes read bytewise.
    const int RS = std::max(1, std::min({R, kMaxRG / G, 8}));
    const int nz = (R + RS - 1) / RS;
    const int n_chunks = (T + kNT - 1) / kNT;
    int rc = OJASX_OK;
    if (n_chunks > 1) {
        rc = wk.reserve((size_t)Hq * n_chunks * hd * 4, (size_t)Hq * n_chunks * 2 * 4);
        if (rc) return rc;
    }
    KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, wk.po, wk.pml, out, T, P,
               Hq, Hkv, hd, D, G, kNT, RS, n_chunks, sf, nullptr, 0};
    const size_t lds = ((size_t)RS * hd + 256 * D + (size_t)RS * G * 256) * 4 + (size_t)RS * G * kHP * 4;
    static size_t g0 = 0;
    rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_chunk_kernel<0, 0, 8, 1>), lds, &g0);
    if (rc) return rc;
    OJX_LAUNCH((kv_decode_chunk_kernel<0, 0, 8, 1>), dim3(n_chunks, Hkv, nz), dim3(kNT), lds, st, p);
    const int nch = p.n_chunks;
    if (nch > 1)
        OJX_LAUNCH(kv_merge_kernel, dim3(Hq), dim3(kNT), (size_t)nch * 4, st,
                           wk.po, wk.pml, nch, hd, out, nullptr, 0, 1, 0);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}


// Device address of `scratch` on the current device, looked up once per
// device with that device current (host code must never pass the array's
// name itself: on the host it is only a stand-in for the symbol).
static int scratch_address(unsigned char **out) {
    static std::mutex mu;
    static unsigned char *addr[64] = {};
    int dev = 0;
    OJX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) {
        set_error("no-allocation scratch: device %d out of range", dev);
        return OJASX_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        OJX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        addr[dev] = static_cast<unsigned char *>(p);
    }
    *out = addr[dev];
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
    DevBuf cb, bt, kstage, qstage, ostage;   // kstage holds k | v of one append
    int bt_pages = 0;
    KVWork work;
    ~KVCache() {
        for (auto &x : h)
            for (DevBuf *b : {&x.kc, &x.vc, &x.ks, &x.vs}) b->release();
        for (DevBuf *b : {&cb, &bt, &kstage, &qstage, &ostage}) b->release();
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
    if (!rc) rc = c->kstage.ensure((size_t)head_dim * 8);
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
    // one upload: k [hd] | v [hd]
    const size_t hb = (size_t)c->hd * 4;
    HostIO &io = host_io();
    int rc = io.reserve(2 * hb);
    if (rc) return rc;
    memcpy(io.pin, k, hb);
    memcpy(io.pin + hb, v, hb);
    OJX_HIP(hipMemcpyAsync(c->kstage.ptr, io.pin, 2 * hb, hipMemcpyHostToDevice, io.st));
    OJX_LAUNCH(kv_append_kernel, dim3(1), dim3(128), 0, io.st, c->kstage.as<float>(),
                       c->kstage.as<float>() + c->hd, c->hd, c->D,
                       hh.kc.as<uint8_t>() + (size_t)hh.len * c->G,
                       hh.vc.as<uint8_t>() + (size_t)hh.len * c->G, hh.ks.as<float>() + hh.len,
                       hh.vs.as<float>() + hh.len);
    OJX_HIP(hipGetLastError());
    OJX_HIP(hipStreamSynchronize(io.st));
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
    const size_t hb = (size_t)c->hd * 4, oo = round_up(hb, 256);
    HostIO &io = host_io();
    rc = io.reserve(oo + hb);
    if (rc) return rc;
    memcpy(io.pin, q, hb);
    OJX_HIP(hipMemcpyAsync(c->qstage.ptr, io.pin, hb, hipMemcpyHostToDevice, io.st));
    rc = kv_decode(c->qstage.as<float>(), hh.kc.as<uint8_t>(), hh.ks.as<float>(),
                   hh.vc.as<uint8_t>(), hh.vs.as<float>(), c->cb.as<float>(), c->cb.as<float>(),
                   c->bt.as<int>(), hh.len, 16, 1, 1, c->hd, c->D, scale_factor,
                   c->ostage.as<float>(), io.st, c->work);
    if (!rc) OJX_HIP(hipMemcpyAsync(io.pin + oo, c->ostage.ptr, hb, hipMemcpyDeviceToHost, io.st));
    OJX_HIP(hipStreamSynchronize(io.st));
    if (rc) return rc;
    memcpy(out_context, io.pin + oo, hb);
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

OJASX_API int ojasx_kv_decode_paged_device_noalloc(const float *q, const uint8_t *k_codes,
                                                   const float *k_scales, const uint8_t *v_codes,
                                                   const float *v_scales, const float *k_cb,
                                                   const float *v_cb, const int *block_table,
                                                   int seq_len, int page_size, int num_q_heads,
                                                   int num_kv_heads, int head_dim, int block_dim,
                                                   float scale_factor, float *out, void *stream) {
    using namespace ojx;
    if (!q || !k_codes || !k_scales || !v_codes || !v_scales || !k_cb || !v_cb || !block_table ||
        !out)
        return OJASX_ERR_NULL;
    unsigned char *base = nullptr;
    const int rc = scratch_address(&base);
    if (rc) return rc;
    KVWork wk;   // no DevBuf is touched: reserve() hands out the scratch only
    wk.fixed_o = reinterpret_cast<float *>(base);
    wk.fixed_ml = reinterpret_cast<float *>(base + kScratchO);
    wk.fixed_o_bytes = kScratchO;
    wk.fixed_ml_bytes = kScratchML;
    return kv_decode(q, k_codes, k_scales, v_codes, v_scales, k_cb, v_cb, block_table, seq_len,
                     page_size, num_q_heads, num_kv_heads, head_dim, block_dim, scale_factor, out,
                     static_cast<hipStream_t>(stream), wk);
}

OJASX_API int ojasx_kv_decode_paged_device_len(const float *q, const uint8_t *k_codes,
                                               const float *k_scales, const uint8_t *v_codes,
                                               const float *v_scales, const float *k_cb,
                                               const float *v_cb, const int *block_table,
                                               const int *seq_len_dev, int max_seq_len,
                                               int page_size, int num_q_heads, int num_kv_heads,
                                               int head_dim, int block_dim, float scale_factor,
                                               int tokens_per_lane, float *out, void *stream) {
    using namespace ojx;
    if (!q || !k_codes || !k_scales || !v_codes || !v_scales || !k_cb || !v_cb || !block_table ||
        !seq_len_dev || !out)
        return OJASX_ERR_NULL;
    auto aligned = [](const void *ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; };
    if (head_dim != 128 || block_dim != 16 || num_kv_heads <= 0 || num_q_heads <= 0 ||
        num_q_heads % num_kv_heads || max_seq_len <= 0 || page_size <= 0 || !aligned(q, 16) ||
        !aligned(k_cb, 16) || !aligned(v_cb, 16) || !aligned(k_codes, 8) || !aligned(v_codes, 8)) {
        set_error("device-length decode: head_dim 128, block_dim 16, 16-byte aligned q and "
                  "codebooks, 8-byte aligned codes");
        return OJASX_ERR_INVALID;
    }
    if (tokens_per_lane != 0 && tokens_per_lane != 1 && tokens_per_lane != 2 &&
        tokens_per_lane != 4) {
        set_error("tokens_per_lane must be 0, 1, 2 or 4 (got %d)", tokens_per_lane);
        return OJASX_ERR_INVALID;
    }
    const int n = kv_device_len_chunks(max_seq_len, tokens_per_lane);
    const int rc = t_work.reserve((size_t)num_q_heads * n * 128 * 4, (size_t)num_q_heads * n * 2 * 4);
    if (rc) return rc;
    if (scale_factor <= 0.f) scale_factor = 1.0f / sqrtf(128.f);
    return kv_decode_device_len(q, k_codes, k_scales, v_codes, v_scales, k_cb, v_cb, block_table,
                                seq_len_dev, 0, max_seq_len, page_size, num_q_heads, num_kv_heads,
                                scale_factor, t_work.po, t_work.pml, out,
                                static_cast<hipStream_t>(stream), tokens_per_lane);
}

}  // extern "C"

// kv_encode.h -- the KV cache's per-token encoder as a device function, used
// by the append kernel (kv_pages.hip; the decoder's attention prologue has
// its own copy of the same arithmetic).
//
// For one token of one kv head, K or V (a workgroup each):
//   s = max(1e-8, max_d |k_d|) / 127            (ojasx_lut_kv_cache.cpp:29-34),
//   x_d = k_d / s,
// then per group g of D coordinates either the nearest of the head's 256
// centroids (squared distance accumulated with fmaf in d order from 0, ties to
// the lower index) or, without a codebook, the reference quantiser
// clamp(round_half_away(x[gD]), -128, 127) + 128 (ojasx_lut_kv_cache.cpp:36-45).
// Run by a whole 256-thread workgroup; thread c holds centroid c.
#pragma once

#include "common.h"

namespace ojx {

constexpr int kEncNT = 256;
constexpr int kEncNW = kEncNT / 64;
constexpr int kMaxEncGroups = 64;

// Centroid row tid of one head's codebook into registers (DT > 0, 16-byte
// aligned rows).  Issued early so the loads overlap the caller's work.
template <int DT>
__device__ __forceinline__ void enc_load_centroid(const float *cb, float *creg) {
    if constexpr (DT > 0) {
        const float *cr = cb + (size_t)threadIdx.x * DT;
#pragma unroll
        for (int d = 0; d < DT; d += 4) {
            const float4 a = *reinterpret_cast<const float4 *>(cr + d);
            creg[d] = a.x, creg[d + 1] = a.y, creg[d + 2] = a.z, creg[d + 3] = a.w;
        }
    }
}

// Squared distance of x (D floats in LDS) to the thread's centroid: from
// registers (DT > 0) or from memory (DT == 0).
template <int DT>
__device__ __forceinline__ float centroid_dist(const float *x, const float *creg, const float *cmem,
                                               int D) {
    float dist = 0.f;
    if constexpr (DT > 0) {
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            const float df = x[d] - creg[d];
            dist = fmaf(df, df, dist);
        }
    } else {
        for (int d = 0; d < D; ++d) {
            const float df = x[d] - cmem[d];
            dist = fmaf(df, df, dist);
        }
    }
    return dist;
}

// Encode one row (K or V) of one token of one kv head.  r: hd floats (global
// memory or LDS); cb: the head's [256][D] codebook, or null for the scalar
// quantiser; creg: this thread's centroid row from enc_load_centroid (DT >
// 0); xs: LDS scratch of hd floats.  Writes G codes to code and the scale to
// *scale.  Every thread of the workgroup must call it.
template <int DT>
__device__ void encode_row(const float *r, const float *cb, const float *creg, int hd, int D,
                           int G, uint8_t *code, float *scale, float *xs) {
    __shared__ float red[kEncNW];
    __shared__ float wd[kMaxEncGroups][kEncNW];   // per-wave minimum distance
    __shared__ int wi[kMaxEncGroups][kEncNW];     // and its lowest centroid
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float m = 0.f;
    for (int d = tid; d < hd; d += kEncNT) m = fmaxf(m, fabsf(r[d]));
    m = wave_max_f(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = fmaxf(1e-8f, m) / 127.0f;
    for (int d = tid; d < hd; d += kEncNT) xs[d] = r[d] / s;
    if (tid == 0) *scale = s;
    __syncthreads();                             // xs complete
    if (cb == nullptr) {
        for (int g = tid; g < G; g += kEncNT) {
            int q = (int)roundf(xs[g * D]);
            q = max(-128, min(127, q));
            code[g] = (uint8_t)(q + 128);
        }
        return;
    }
    const int c = tid;
    const float *cr = cb + (size_t)c * D;
    // 8 groups at a time: 8 distances per centroid, then their 8 wave minima
    // and lowest centroids as interleaved reductions
    for (int g0 = 0; g0 < G; g0 += 8) {
        float dd[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) dd[u] = centroid_dist<DT>(xs + min(g0 + u, G - 1) * D, creg, cr, D);
        float mn[8];
        int id[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) mn[i] = dd[i];
        wave_min_n(mn);
#pragma unroll
        for (int i = 0; i < 8; ++i) id[i] = dd[i] == mn[i] ? c : 0x7fffffff;
        wave_min_n(id);
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (g0 + u < G) {
                    wd[g0 + u][w] = mn[u];
                    wi[g0 + u][w] = id[u];
                }
        }
    }
    __syncthreads();
    for (int g = tid; g < G; g += kEncNT) {
        float bm = wd[g][0];
        int bi = wi[g][0];
#pragma unroll
        for (int q = 1; q < kEncNW; ++q)
            if (wd[g][q] < bm) {   // strictly smaller: earlier waves hold lower indices
                bm = wd[g][q];
                bi = wi[g][q];
            }
        code[g] = (uint8_t)bi;
    }
}

}  // namespace ojx

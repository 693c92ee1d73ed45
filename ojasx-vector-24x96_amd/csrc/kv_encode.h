// kv_encode.h -- the KV cache's per-token encoder as a device function, shared
// by the append kernel (kv_pages.hip) and the decoder's attention prologue
// (decoder.hip).
//
// For one token of one kv head, K and V alike:
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

// Centroid row tid of the K and V codebooks of one head into registers (DT > 0,
// 16-byte aligned rows).  Issued early so the loads overlap the caller's work.
template <int DT>
__device__ __forceinline__ void enc_load_centroids(const float *kcb, const float *vcb, float *kreg,
                                                   float *vreg) {
    if constexpr (DT > 0) {
        const float *kcr = kcb + (size_t)threadIdx.x * DT;
        const float *vcr = vcb + (size_t)threadIdx.x * DT;
#pragma unroll
        for (int d = 0; d < DT; d += 4) {
            const float4 a = *reinterpret_cast<const float4 *>(kcr + d);
            const float4 b = *reinterpret_cast<const float4 *>(vcr + d);
            kreg[d] = a.x, kreg[d + 1] = a.y, kreg[d + 2] = a.z, kreg[d + 3] = a.w;
            vreg[d] = b.x, vreg[d + 1] = b.y, vreg[d + 2] = b.z, vreg[d + 3] = b.w;
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

// Encode one token of one kv head.  kr / vr: hd floats (global memory or
// LDS); kcb / vcb: the head's [256][D] codebooks, or both null for the scalar
// quantiser; kreg / vreg: this thread's centroid rows from enc_load_centroids
// (DT > 0); xs: LDS scratch of 2 * hd floats.  Writes G codes to kc and vc
// and one scale to *ks and *vs.  Every thread of the workgroup must call it.
template <int DT>
__device__ void encode_kv_token(const float *kr, const float *vr, const float *kcb,
                                const float *vcb, const float *kreg, const float *vreg, int hd,
                                int D, int G, uint8_t *kc, uint8_t *vc, float *ks, float *vs,
                                float *xs) {
    __shared__ float red[2][kEncNW];
    __shared__ float wd[2][kMaxEncGroups][kEncNW];  // per-wave minimum distance
    __shared__ int wi[2][kMaxEncGroups][kEncNW];    // and its lowest centroid
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float mk = 0.f, mv = 0.f;
    for (int d = tid; d < hd; d += kEncNT) {
        mk = fmaxf(mk, fabsf(kr[d]));
        mv = fmaxf(mv, fabsf(vr[d]));
    }
    mk = wave_max_f(mk);
    mv = wave_max_f(mv);
    if (lane == 0) {
        red[0][w] = mk;
        red[1][w] = mv;
    }
    __syncthreads();
    mk = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    mv = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const float sk = fmaxf(1e-8f, mk) / 127.0f;
    const float sv = fmaxf(1e-8f, mv) / 127.0f;
    for (int d = tid; d < hd; d += kEncNT) {
        xs[d] = kr[d] / sk;
        xs[hd + d] = vr[d] / sv;
    }
    if (tid == 0) {
        *ks = sk;
        *vs = sv;
    }
    __syncthreads();                             // xs complete
    if (kcb == nullptr) {
        for (int e = tid; e < 2 * G; e += kEncNT) {
            const int kv = e >= G, g = e - kv * G;
            int q = (int)roundf(xs[kv * hd + g * D]);
            q = max(-128, min(127, q));
            (kv ? vc : kc)[g] = (uint8_t)(q + 128);
        }
        return;
    }
    const int c = tid;
    const float *kcr = kcb + (size_t)c * D;
    const float *vcr = vcb + (size_t)c * D;
    // 8 groups at a time: 16 distances per centroid, then their 16 wave
    // minima and lowest centroids as interleaved reductions
    for (int g0 = 0; g0 < G; g0 += 8) {
        float dd[16];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int g = min(g0 + u, G - 1);
            dd[u] = centroid_dist<DT>(xs + g * D, kreg, kcr, D);
            dd[8 + u] = centroid_dist<DT>(xs + hd + g * D, vreg, vcr, D);
        }
        float mn[16];
        int id[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) mn[i] = dd[i];
        wave_min_n(mn);
#pragma unroll
        for (int i = 0; i < 16; ++i) id[i] = dd[i] == mn[i] ? c : 0x7fffffff;
        wave_min_n(id);
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (g0 + u < G) {
                    wd[0][g0 + u][w] = mn[u];
                    wi[0][g0 + u][w] = id[u];
                    wd[1][g0 + u][w] = mn[8 + u];
                    wi[1][g0 + u][w] = id[8 + u];
                }
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < 2 * G; e += kEncNT) {
        const int kv = e >= G, g = e - kv * G;
        float bm = wd[kv][g][0];
        int bi = wi[kv][g][0];
#pragma unroll
        for (int q = 1; q < kEncNW; ++q)
            if (wd[kv][g][q] < bm) {   // strictly smaller: earlier waves hold lower indices
                bm = wd[kv][g][q];
                bi = wi[kv][g][q];
            }
        (kv ? vc : kc)[g] = (uint8_t)bi;
    }
}

}  // namespace ojx

// lut_linear.hip -- split-manifold LUT linear layer on gfx950.
//
// Computes, for every token b and output row m,
//   y[b,m] = (s_m * sum_g LUT_b[g, codes[m,g]] + bias[m]) + sum_j val_j * x[b,col_j]
// with LUT_b[g,k] = <x_b[gD:(g+1)D], C[k]>, the formula and epilogue order of
// split_manifold_lut_experiment/native/src/ojasx_lut_cpu.cpp:18-206 (LUT build
// :18-102, row gather :160-184, epilogue :178-182, CSR outliers :104-130,
// added after the epilogue and not scaled) and of
// split_manifold_lut_experiment/engine/split_manifold_engine.py:185-250.
//
// block_dim 16 (the reference default and every configured shape): one
// kernel, lut_dec_kernel.  At small batch a call is latency-bound (1.1 MB of
// codes is ~0.14 us of HBM time against a ~1.3 us kernel floor and a ~1.6 us
// gap between dependent launches), so the LUT entries a workgroup needs are
// computed where they are used instead of in a second kernel:
// LUT[g][code] = <x_g, C[code]>, with the codebook (16 KB) and x staged in
// LDS.  Workgroup = 16*RPL output rows x all G groups; wave w owns the 16-group
// slices w, w+NW, ... (NW = min(S, 16) waves); lane (r, j) owns row r (and
// r+16 when RPL = 2) and the quarter j (4 floats) of every 16-float dot, so an
// 8-lane LDS group reads two codebook rows.  The row's quarters and slices
// are summed with DPP quad adds and an LDS reduction in a fixed order; the
// row's CSR entries are split over its 4*NW lanes; the epilogue applies
// (s_m * sum + bias) + outliers in the reference's order.  Round trip 1
// issues the L2-resident staging loads before the HBM code loads so the LDS
// writes do not wait for HBM.
//
// Other block sizes use two kernels and no cross-workgroup synchronisation:
//  K1 lut_build: the LUT of every token, LUT[b][g][k] for all 256 centroids,
//     into a workspace (workgroup = (1 group, 1 token), thread k owns
//     centroid k): x and the codebook, then one store.
//  K2 lut_gather: workgroup = 32 output rows x 8 slice groups x up to 4
//     tokens (216 workgroups at 6912 rows: every CU busy; 16- and 64-row
//     variants measured slower).  Thread (q, r) owns row r and the 16-group
//     slices q, q+8, ...  Round trip 1: its rows' 16 codes per slice with one
//     16-byte load each (a wave reads contiguous 512-byte runs of the
//     slice-major tiles [S][Mp][16]), the CSR row bounds and x (staged in
//     LDS).  Round trip 2: the 16 LUT entries per slice and token from the
//     L2-resident LUT and the thread's share of the row's CSR entries.  The
//     slice-group partials (manifold and outlier sums) are reduced in LDS in
//     a fixed order and the epilogue applies (s_m * sum + bias) + outliers in
//     the reference's order: deterministic results.
#include <algorithm>
#include <type_traits>
#include <cstring>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;        // threads per workgroup (4 waves)
constexpr int kGS = 16;         // groups per slice: 16 code bytes per row
constexpr int kRowAlign = 1024; // rows padded for the tile layout
constexpr int kCB = 256;        // centroids in the (zero-padded) codebook
constexpr int kRows = 32;       // rows per gather workgroup
constexpr int kOB = 32;         // outlier entries loaded per batch
constexpr size_t kXLdsBytes = 48 * 1024;  // x staged in LDS up to this size
constexpr int kMaxDecWaves = 16;          // waves (slice owners) per decode workgroup
constexpr int kTallRowsPerTile = 16 * 256;  // batch-1 rows per row tile per workgroup: one per CU
constexpr int kMaxTallTiles = 5;          // row tiles of 16 per batch-1 workgroup, at most
                                          // (6 spills at the 128-VGPR limit)
constexpr size_t kMaxLds = 160 * 1024;    // LDS per workgroup on gfx950
}  // namespace

struct GatherParams {
    const uint8_t *codes;   // [S][Mp][16]
    const float *lut;       // [B][Gp][256]
    const float *scales;    // [M]
    const float *bias;      // [M] or null
    const int *rowp;        // [M+1] CSR row pointers (null: no outliers)
    const int *col;         // [nnz]
    const float *val;       // [nnz]
    const void *x;          // [B][K]
    void *y;                // [B][M]
    int K, M, Mp, S, Gp, B, nnz, x_lds;
};

// K1: LUT of token b for group blockIdx.x (zero for padded groups >= G).
// DT = 16 holds the codebook row in registers; DT = 0 takes any group width
// D, staging the group 256 values at a time.
template <int DT, typename T>
__global__ __launch_bounds__(kCB) void lut_build_kernel(const T *__restrict__ x,
                                                      const float *__restrict__ cb, int K, int D,
                                                      int G, int Gp, float *__restrict__ lut) {
    __shared__ float xs[kCB];
    const int b = blockIdx.y, g = blockIdx.x, k = threadIdx.x;
    float dot = 0.f;
    if constexpr (DT > 0) {
        float c[DT];
#pragma unroll
        for (int d = 0; d < DT; ++d) c[d] = cb[k * DT + d];
        if (k < DT) xs[k] = g < G ? load_act(x, (size_t)b * K + (size_t)g * DT + k) : 0.f;
        __syncthreads();
#pragma unroll
        for (int d = 0; d < DT; ++d) dot = fmaf(xs[d], c[d], dot);
    } else {
        dot = staged_group_dot(x + (size_t)b * K + (size_t)min(g, G - 1) * D, g < G,
                               cb + (size_t)k * D, D, xs);
    }
    lut[((size_t)b * Gp + g) * kCB + k] = dot;
}

// K2 + K3: gather-accumulate, outliers and epilogue.  Workgroup = R rows x
// QG = 256/R slice groups: thread (q, r) owns row r and slices q, q+QG, ...;
// a wave holds two (or more) slice groups of consecutive rows, so its code
// loads are contiguous 16-byte rows.  A row's CSR entries are split over its
// QG threads (entry j0 + q + QG*u).  Loads are branch-free (clamped indices,
// results masked at use) so each thread's loads of a round trip are all in
// flight together; partial sums are reduced over the slice groups in LDS in
// a fixed order.
template <int R, int BT, typename T>
__global__ __launch_bounds__(kNT) void lut_gather_kernel(GatherParams p) {
    constexpr int QG = kNT / R;
    constexpr int NSB = 2;                // slices per thread per batch
    constexpr int NU = (kOB + QG - 1) / QG;  // outlier entries per thread in batch 1
    extern __shared__ float xs[];         // [BT][K] when p.x_lds
    __shared__ float red[2][QG][BT][R];
    const int tid = threadIdx.x;
    const int r = tid % R, q = tid / R;
    const int m = blockIdx.x * R + r;     // < Mp: codes need no clamp
    const int mr = min(m, p.M - 1);
    const int t0 = blockIdx.y * BT;
    const int nt = min(BT, p.B - t0);
    const bool outl = p.rowp != nullptr;
    const T *__restrict__ x = static_cast<const T *>(p.x);
    const int nsq = q < p.S ? (p.S - 1 - q) / QG + 1 : 0;   // slices of this thread

    // ---- round trip 1: codes of the first batch, row bounds, x
    uint4 cv[NSB];
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
        const int s = min(q + QG * i, p.S - 1);
        cv[i] = *reinterpret_cast<const uint4 *>(p.codes + ((size_t)s * p.Mp + m) * kGS);
    }
    int j0 = 0, j1 = 0;
    if (outl) {
        j0 = p.rowp[mr];
        j1 = p.rowp[mr + 1];
    }
    if (outl && p.x_lds) stage_to_lds<kNT>(xs, x + (size_t)t0 * p.K, nt * p.K);

    // ---- round trip 2: outlier entries of this thread, LUT entries
    int oc[NU];
    float ov[NU];
    if (outl) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int j = min(j0 + q + QG * u, p.nnz - 1);
            oc[u] = p.col[j];
            ov[u] = p.val[j];
        }
    }
    float acc[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) acc[t] = 0.f;
    for (int i0 = 0; i0 < nsq; i0 += NSB) {
        float lv[NSB][BT][kGS];
#pragma unroll
        for (int i = 0; i < NSB; ++i) {
            const int s = min(q + QG * (i0 + i), p.S - 1);
            const uint32_t w4[4] = {cv[i].x, cv[i].y, cv[i].z, cv[i].w};
#pragma unroll
            for (int t = 0; t < BT; ++t) {
                const int tt = min(t, nt - 1);
                const float *L = p.lut + ((size_t)(t0 + tt) * p.Gp + s * kGS) * kCB;
#pragma unroll
                for (int g = 0; g < kGS; ++g)
                    lv[i][t][g] = L[g * kCB + ((w4[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
            }
        }
        if (i0 + NSB < nsq) {  // next batch of codes
#pragma unroll
            for (int i = 0; i < NSB; ++i) {
                const int s = min(q + QG * (i0 + NSB + i), p.S - 1);
                cv[i] = *reinterpret_cast<const uint4 *>(p.codes + ((size_t)s * p.Mp + m) * kGS);
            }
        }
#pragma unroll
        for (int i = 0; i < NSB; ++i) {
            if (i0 + i < nsq) {
#pragma unroll
                for (int t = 0; t < BT; ++t) {
                    float a = acc[t];
#pragma unroll
                    for (int g = 0; g < kGS; ++g) a += lv[i][t][g];
                    acc[t] = a;
                }
            }
        }
    }
    float oac[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) oac[t] = 0.f;
    if (outl) {
        if (p.x_lds) __syncthreads();
        const int n0 = j1 - j0;
#pragma unroll
        for (int t = 0; t < BT; ++t) {
            const int tt = min(t, nt - 1);
            float o = 0.f;
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const float xv = p.x_lds ? xs[tt * p.K + oc[u]]
                                         : load_act(x, (size_t)(t0 + tt) * p.K + oc[u]);
                o += q + QG * u < n0 ? ov[u] * xv : 0.f;
            }
            oac[t] = o;
        }
        // entries beyond the first QG*NU of a row (rare)
        for (int j = j0 + q + QG * NU; j < j1; j += QG) {
            const int c = p.col[j];
            const float v = p.val[j];
#pragma unroll
            for (int t = 0; t < BT; ++t)
                if (t < nt)
                    oac[t] += v * (p.x_lds ? xs[t * p.K + c] : load_act(x, (size_t)(t0 + t) * p.K + c));
        }
    }
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        red[0][q][t][r] = acc[t];
        red[1][q][t][r] = oac[t];
    }
    __syncthreads();
    if (q != 0 || m >= p.M) return;
    const float sc = p.scales[m];
    const float bs = p.bias ? p.bias[m] : 0.f;
    T *y = static_cast<T *>(p.y);
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        if (t >= nt) break;
        float a = red[0][0][t][r], o = red[1][0][t][r];
#pragma unroll
        for (int k = 1; k < QG; ++k) {
            a += red[0][k][t][r];
            o += red[1][k][t][r];
        }
        float v = a * sc;
        if (p.bias) v += bs;
        v += o;
        store_act(y, (size_t)(t0 + t) * p.M + m, v);
    }
}

struct DecParams {
    const uint8_t *codes;   // [S][Mp][16]
    const float *cb;        // [256][16]
    const float *scales;    // [M]
    const float *bias;      // [M] or null
    const int *rowp;        // [M+1] (null: no outliers)
    const uint16_t *col;    // [nnz] 16-bit columns (the staged x bounds K far below 65536)
    const float *val;       // [nnz]
    const void *x;          // [B][xrow], 16-byte aligned (fp32) / 8-byte (bf16)
    void *y;                // [B][M]
    const float *pro_w;     // RMSNorm weight [K] (prologue 1)
    const float *res;       // residual [B][M] added to y (may alias y)
    float eps;              // RMSNorm epsilon
    int K, M, Mp, S, B, nnz, NW;
    int xrow;               // elements per token row of x: K, or 2K for SwiGLU
};

// Prologues of the fused decoder variants, applied as x is staged in LDS:
//   kProNone    x as given;
//   kProRms     RMSNorm: the row is staged as x * w and r = 1/sqrt(mean(x^2) + eps)
//               multiplies the manifold and outlier sums in the epilogue (r is a
//               per-token scalar, so it factors out of the linear map);
//   kProSwiglu  x[i] = silu(a[i]) * a[K + i] from a row a of 2K elements
//               (gate half, then up half), silu(v) = v / (1 + exp(-v));
//   kProRmsGlu  the RMSNorm prologue and a SwiGLU epilogue: of the M = 2I
//               outputs (gate rows, then up rows) y holds silu(y[i]) * y[I + i],
//               i < I, the kProSwiglu input of the next linear computed once.
//               A workgroup owns 8 RPL gate rows and their up rows.
enum { kProNone = 0, kProRms = 1, kProSwiglu = 2, kProRmsGlu = 3 };

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float4 swiglu4(float4 g, float4 u) {
    return make_float4(silu_f(g.x) * u.x, silu_f(g.y) * u.y, silu_f(g.z) * u.z, silu_f(g.w) * u.w);
}
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float sumsq4(float4 a) {
    return fmaf(a.w, a.w, fmaf(a.z, a.z, fmaf(a.y, a.y, a.x * a.x)));
}

// Single-kernel forward for block_dim 16 (see the file comment).  x is staged
// as [BT][S*256] with zeros past K, so groups past G contribute 0.  PRO selects
// a prologue (kPro*), RES adds p.res to the output.  HO (high occupancy) caps
// the kernel at 64 VGPRs, so three workgroups of up to 10 waves share a CU:
// for grids with more workgroups than fit twice per CU, where the 76-VGPR
// build would run a second round (gate/up 2560 -> 19456: 13.1 -> ~10 us);
// smaller grids keep the faster per-workgroup build.
template <typename T, int BT, int RPL, int PRO = kProNone, bool RES = false, bool HO = false>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(HO ? 8 : 1))) void lut_dec_kernel(DecParams p) {
    constexpr int R = 16 * RPL;            // rows per workgroup
    constexpr bool RMS = PRO == kProRms || PRO == kProRmsGlu;
    constexpr bool GLU = PRO == kProRmsGlu;
    static_assert(!GLU || (BT == 1 && !RES), "SwiGLU epilogue: batch 1, no residual");
    constexpr int RH = R / 2;              // GLU: gate rows per workgroup
    // code rows past Mp only where R does not divide the row padding, or GLU
    constexpr bool CLAMP = GLU || (kRowAlign % R) != 0;
    extern __shared__ float sm[];
    float *cbs = sm;                       // [256][16]
    float *xs = sm + kCB * 16;             // [BT][S*256]
    __shared__ float part[2][16][R][BT];   // [manifold|outlier][wave][row][token]
    __shared__ float ssq_part[16][BT];     // per-wave sums of x^2 (RMSNorm prologue)
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, w = tid >> 6;
    const int r = lane >> 2, j = lane & 3;
    const int NW = p.NW, S = p.S, KS = S * 256;
    const int base = (int)blockIdx.x * (GLU ? RH : R);
    const int I = p.M / 2;                 // GLU: gate rows [0, I), up rows [I, M)
    // output row of the workgroup's row rr: GLU takes gate rows base + rr and,
    // from rr = RH on, their up rows I + base + rr - RH
    auto grow = [&](int rr) { return GLU ? (rr < RH ? base + rr : I + base + rr - RH) : base + rr; };
    // code row of the lane's row i, < Mp
    auto crow = [&](int i) { return CLAMP ? min(grow(r + 16 * i), p.Mp - 1) : base + r + 16 * i; };
    const int t0 = (int)blockIdx.y * BT;
    const int nt = min(BT, p.B - t0);
    const bool outl = p.rowp != nullptr;
    const T *__restrict__ x = static_cast<const T *>(p.x);

    // ---- round trip 1: codebook and x (L2) first, then codes (HBM), row data
    float4 cv4[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        cv4[u] = reinterpret_cast<const float4 *>(p.cb)[min(tid + u * nthr, 1023)];
    const int nx4 = KS / 4;
    float4 xv4[BT][2];
    float4 av4[PRO == kProNone ? 1 : BT][2];   // RMSNorm weight or SwiGLU up half
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        const int tt = min(t, nt - 1);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = min(tid + u * nthr, nx4 - 1) * 4;
            const int ec = min(e, p.K - 4);
            xv4[t][u] = load4_act(x, (size_t)(t0 + tt) * p.xrow + ec);
            if constexpr (RMS)
                av4[t][u] = *reinterpret_cast<const float4 *>(p.pro_w + ec);
            if constexpr (PRO == kProSwiglu)
                av4[t][u] = load4_act(x, (size_t)(t0 + tt) * p.xrow + p.K + ec);
            if (e >= p.K) xv4[t][u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    uint4 cw[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i)
        cw[i] = *reinterpret_cast<const uint4 *>(p.codes + ((size_t)w * p.Mp + crow(i)) * kGS);
    // the epilogue thread of (row tid % R, token tid / R) when tid < R * BT
    // (GLU: thread tid < RH also takes the scale and bias of its up row)
    float sc = 0.f, bs = 0.f, sc2 = 0.f, bs2 = 0.f;
    if (tid < R * BT) {
        const int mm = min(grow(tid % R), p.M - 1);
        sc = p.scales[mm];
        bs = p.bias ? p.bias[mm] : 0.f;
    }
    if (GLU && tid < RH) {
        const int mm = min(grow(tid + RH), p.M - 1);
        sc2 = p.scales[mm];
        bs2 = p.bias ? p.bias[mm] : 0.f;
    }
    int j0[RPL], j1[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) j0[i] = j1[i] = 0;
    if (outl) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int mm = min(grow(r + 16 * i), p.M - 1);
            j0[i] = p.rowp[mm];
            j1[i] = p.rowp[mm + 1];
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) reinterpret_cast<float4 *>(cbs)[min(tid + u * nthr, 1023)] = cv4[u];
    if (2 * nthr < 1024) {  // fewer than 512 threads: the rest of the codebook, 8 loads in flight
        const float4 *c4 = reinterpret_cast<const float4 *>(p.cb);
        for (int b = tid + 2 * nthr; b < 1024; b += 8 * nthr) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = c4[min(b + u * nthr, 1023)];
#pragma unroll
            for (int u = 0; u < 8; ++u) reinterpret_cast<float4 *>(cbs)[min(b + u * nthr, 1023)] = v[u];
        }
    }
    float ssq[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        ssq[t] = 0.f;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float4 v = xv4[t][u];
            if constexpr (RMS) {
                // x^2 once per element: the clamped duplicate indices past nx4 count 0
                if (tid + u * nthr < nx4) ssq[t] += sumsq4(v);
                v = mul4(v, av4[t][u]);
            }
            if constexpr (PRO == kProSwiglu) v = swiglu4(v, av4[t][u]);
            if constexpr (PRO == kProSwiglu)
                if (min(tid + u * nthr, nx4 - 1) * 4 >= p.K) v = make_float4(0.f, 0.f, 0.f, 0.f);
            reinterpret_cast<float4 *>(xs + t * KS)[min(tid + u * nthr, nx4 - 1)] = v;
        }
    }
    if (2 * nthr < nx4) {  // more than two float4 of x per thread (K > 8192)
        for (int t = 0; t < nt; ++t)
            for (int i = tid + 2 * nthr; i < nx4; i += nthr) {
                const int e = i * 4;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (e < p.K) {
                    v = load4_act(x, (size_t)(t0 + t) * p.xrow + e);
                    if constexpr (RMS) {
                        ssq[t] += sumsq4(v);
                        v = mul4(v, *reinterpret_cast<const float4 *>(p.pro_w + e));
                    }
                    if constexpr (PRO == kProSwiglu)
                        v = swiglu4(v, load4_act(x, (size_t)(t0 + t) * p.xrow + p.K + e));
                }
                reinterpret_cast<float4 *>(xs + t * KS)[i] = v;
            }
    }
    if constexpr (RMS) {
#pragma unroll
        for (int t = 0; t < BT; ++t) {
            const float v = wave_sum_f(ssq[t]);
            if (lane == 0) ssq_part[w][t] = v;
        }
    }
    // ---- the lane's first CSR entry of each of its rows: j0 + lq (of 4*NW)
    const int lq = w * 4 + j, LQ = NW * 4;
    int oc[RPL];
    float ov[RPL];
    if (outl) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int jj = min(j0[i] + lq, p.nnz - 1);
            oc[i] = p.col[jj];
            ov[i] = p.val[jj];
        }
    }
    __syncthreads();

    // ---- dots: lane (r, j) adds x_t[g][4j..4j+3] . C[code][4j..4j+3]
    float acc[RPL][BT][2];
#pragma unroll
    for (int i = 0; i < RPL; ++i)
#pragma unroll
        for (int t = 0; t < BT; ++t) acc[i][t][0] = acc[i][t][1] = 0.f;
    const float *cbj = cbs + 4 * j;
    for (int s = w; s < S; s += NW) {
        uint32_t wd[RPL][4];
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            wd[i][0] = cw[i].x;
            wd[i][1] = cw[i].y;
            wd[i][2] = cw[i].z;
            wd[i][3] = cw[i].w;
        }
        if (s + NW < S) {
#pragma unroll
            for (int i = 0; i < RPL; ++i)
                cw[i] = *reinterpret_cast<const uint4 *>(
                    p.codes + ((size_t)(s + NW) * p.Mp + crow(i)) * kGS);
        }
        const float *xsj = xs + s * 256 + 4 * j;
#pragma unroll
        for (int g = 0; g < kGS; ++g) {
            float4 c[RPL];
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                const int code = (wd[i][g >> 2] >> ((g & 3) * 8)) & 0xffu;
                c[i] = *reinterpret_cast<const float4 *>(cbj + code * 16);
            }
#pragma unroll
            for (int t = 0; t < BT; ++t) {
                const float4 xv = *reinterpret_cast<const float4 *>(xsj + t * KS + g * 16);
#pragma unroll
                for (int i = 0; i < RPL; ++i) {
                    float a = acc[i][t][g & 1];
                    a = fmaf(xv.x, c[i].x, a);
                    a = fmaf(xv.y, c[i].y, a);
                    a = fmaf(xv.z, c[i].z, a);
                    a = fmaf(xv.w, c[i].w, a);
                    acc[i][t][g & 1] = a;
                }
            }
        }
    }
    // ---- outliers of this lane; rows with more than 4*NW entries loop
    float oa[RPL][BT];
#pragma unroll
    for (int i = 0; i < RPL; ++i)
#pragma unroll
        for (int t = 0; t < BT; ++t) oa[i][t] = 0.f;
    if (outl) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const bool on = lq < j1[i] - j0[i];
#pragma unroll
            for (int t = 0; t < BT; ++t) oa[i][t] = on ? ov[i] * xs[min(t, nt - 1) * KS + oc[i]] : 0.f;
            for (int jj = j0[i] + lq + LQ; jj < j1[i]; jj += LQ) {
                const int c = p.col[jj];
                const float v = p.val[jj];
#pragma unroll
                for (int t = 0; t < BT; ++t) oa[i][t] += v * xs[min(t, nt - 1) * KS + c];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RPL; ++i)
#pragma unroll
        for (int t = 0; t < BT; ++t) {
            const float v = quad_sum(acc[i][t][0] + acc[i][t][1]);
            const float o = quad_sum(oa[i][t]);
            if (j == 0) {
                part[0][w][r + 16 * i][t] = v;
                part[1][w][r + 16 * i][t] = o;
            }
        }
    __syncthreads();
    // ---- epilogue: one thread per (row, token), the waves' partials summed in
    // wave order (a launch has at least 64 threads; R * BT may be more)
    T *y = static_cast<T *>(p.y);
    if constexpr (GLU) {
        // thread tid < RH: gate row base + tid and its up row, each finished as
        // below, then silu(gate) * up (the kProSwiglu prologue's expression)
        if (tid >= RH || base + tid >= I) return;
        float a = 0.f, o = 0.f, a2 = 0.f, o2 = 0.f, q = 0.f;
        for (int k = 0; k < NW; ++k) {
            a += part[0][k][tid][0];
            o += part[1][k][tid][0];
            a2 += part[0][k][tid + RH][0];
            o2 += part[1][k][tid + RH][0];
            q += ssq_part[k][0];
        }
        const float rn = 1.0f / sqrtf(q / (float)p.K + p.eps);
        float g = (a * rn) * sc, u = (a2 * rn) * sc2;
        if (p.bias) {
            g += bs;
            u += bs2;
        }
        g += o * rn;
        u += o2 * rn;
        store_act(y, (size_t)(base + tid), silu_f(g) * u);
        return;
    }
    for (int e = tid; e < R * BT; e += nthr) {
        const int rr = e % R, t = e / R;
        const int m = base + rr;
        if (t >= nt || m >= p.M) continue;
        float a = 0.f, o = 0.f;
        for (int k = 0; k < NW; ++k) {
            a += part[0][k][rr][t];
            o += part[1][k][rr][t];
        }
        if constexpr (RMS) {
            float q = 0.f;
            for (int k = 0; k < NW; ++k) q += ssq_part[k][t];
            const float rn = 1.0f / sqrtf(q / (float)p.K + p.eps);
            a *= rn;
            o *= rn;
        }
        const float scm = e < nthr ? sc : p.scales[m];
        float v = a * scm;
        if (p.bias) v += e < nthr ? bs : p.bias[m];
        v += o;
        const size_t yi = (size_t)(t0 + t) * p.M + m;
        if constexpr (RES) v = p.res[yi] + v;
        store_act(y, yi, v);
    }
}

// Standalone LUT build with a codebook of Kcb rows: one workgroup per
// (group, token), thread k computes LUT[b][g][k].
template <typename T>
__global__ __launch_bounds__(kCB) void build_lut_kernel(const T *__restrict__ x,
                                                      const float *__restrict__ cb, int G, int D,
                                                      int Kcb, float *__restrict__ lut) {
    const int g = blockIdx.x, b = blockIdx.y, k = threadIdx.x;
    __shared__ float xs[kCB];
    const float dot = staged_group_dot(x + (size_t)b * G * D + (size_t)g * D, true,
                                       cb + (size_t)min(k, Kcb - 1) * D, D, xs);
    if (k < Kcb) lut[((size_t)b * G + g) * Kcb + k] = dot;
}

// ---------------------------------------------------------------------------
struct Linear {
    int K = 0, M = 0, D = 0, Kcb = 0, G = 0, S = 0, Mp = 0;
    bool has_bias = false;
    size_t nnz = 0;
    DevBuf codes, codes_b, codebook, cb3, scales, bias, rowp, col, col16, val;
    DevBuf lut, xstage, ystage;
    ~Linear() {
        for (DevBuf *b : {&codes, &codes_b, &codebook, &cb3, &scales, &bias, &rowp, &col, &col16,
                          &val, &lut, &xstage, &ystage})
            b->release();
    }
};

namespace {

template <int BT, typename T>
int launch_gather(const GatherParams &gp, int M, dim3 grid_y, size_t lds, hipStream_t st) {
    constexpr int R = kRows;
    static size_t granted = 0;
    const void *fn = reinterpret_cast<const void *>(&lut_gather_kernel<R, BT, T>);
    int rc = ensure_dyn_lds(fn, lds, &granted);
    if (rc) return rc;
    dim3 grid((M + R - 1) / R, grid_y.y);
    OJX_LAUNCH((lut_gather_kernel<R, BT, T>), grid, dim3(kNT), lds, st, gp);
    return OJASX_OK;
}

// Fused prologue / epilogue of a decoder call (kPro*, residual); none for
// the reference-facing entry points.
struct Fuse {
    int pro = kProNone;
    const float *w = nullptr;
    float eps = 0.f;
    const float *res = nullptr;
};

template <typename T, int BT, int RPL, int PRO, bool RES, bool HO>
int launch_dec_g(const DecParams &dp, dim3 grid, size_t lds, hipStream_t st) {
    static size_t granted = 0;
    const void *fn = reinterpret_cast<const void *>(&lut_dec_kernel<T, BT, RPL, PRO, RES, HO>);
    int rc = ensure_dyn_lds(fn, lds, &granted);
    if (rc) return rc;
    OJX_LAUNCH((lut_dec_kernel<T, BT, RPL, PRO, RES, HO>), grid, dim3(64 * dp.NW), lds, st, dp);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// Workgroups above which a batch-1 launch takes the 64-VGPR build: twice the
// CUs of an MI355X (256).
constexpr long kHighOccWorkgroups = 512;

template <typename T, int BT, int RPL, int PRO, bool RES>
int launch_dec_v(const DecParams &dp, int M, int B, size_t lds, hipStream_t st) {
    // rows per workgroup 16 RPL (SwiGLU epilogue: 8 RPL gate rows and their up rows)
    const int rows = PRO == kProRmsGlu ? 8 * RPL : 16 * RPL;
    dim3 grid(((PRO == kProRmsGlu ? M / 2 : M) + rows - 1) / rows, (B + BT - 1) / BT);
    if constexpr (BT == 1 && RPL <= 2) {
        if ((long)grid.x * grid.y > kHighOccWorkgroups)
            return launch_dec_g<T, BT, RPL, PRO, RES, true>(dp, grid, lds, st);
    }
    return launch_dec_g<T, BT, RPL, PRO, RES, false>(dp, grid, lds, st);
}

template <typename T, int BT, int RPL>
int launch_dec(Linear *L, const void *x, void *y, int B, size_t lds, hipStream_t st,
               const Fuse &f) {
    DecParams dp{};
    dp.codes = L->codes.as<uint8_t>();
    dp.cb = L->codebook.as<float>();
    dp.scales = L->scales.as<float>();
    dp.bias = L->has_bias ? L->bias.as<float>() : nullptr;
    dp.rowp = L->nnz ? L->rowp.as<int>() : nullptr;
    dp.col = L->col16.as<uint16_t>();
    dp.val = L->val.as<float>();
    dp.x = x;
    dp.y = y;
    dp.K = L->K;
    dp.M = L->M;
    dp.Mp = L->Mp;
    dp.S = L->S;
    dp.B = B;
    dp.nnz = (int)L->nnz;
    dp.NW = std::min(L->S, kMaxDecWaves);
    dp.xrow = f.pro == kProSwiglu ? 2 * L->K : L->K;
    dp.pro_w = f.w;
    dp.eps = f.eps;
    dp.res = f.res;
    const bool fused = f.pro != kProNone || f.res;
    if constexpr (std::is_same<T, float>::value && BT == 1) {
        if (fused) {
            const bool r = f.res != nullptr;
            if (f.pro == kProRms)
                return r ? launch_dec_v<T, 1, RPL, kProRms, true>(dp, L->M, B, lds, st)
                         : launch_dec_v<T, 1, RPL, kProRms, false>(dp, L->M, B, lds, st);
            if (f.pro == kProSwiglu)
                return r ? launch_dec_v<T, 1, RPL, kProSwiglu, true>(dp, L->M, B, lds, st)
                         : launch_dec_v<T, 1, RPL, kProSwiglu, false>(dp, L->M, B, lds, st);
            if (f.pro == kProRmsGlu)
                return launch_dec_v<T, 1, RPL, kProRmsGlu, false>(dp, L->M, B, lds, st);
            return launch_dec_v<T, 1, RPL, kProNone, true>(dp, L->M, B, lds, st);
        }
    }
    if (fused) {
        set_error("fused prologue / residual: fp32 and batch 1 only");
        return OJASX_ERR_INVALID;
    }
    return launch_dec_v<T, BT, RPL, kProNone, false>(dp, L->M, B, lds, st);
}

// Single-kernel path when block_dim is 16, x is aligned for vector loads and
// the staged x fits LDS; returns 1 when the two-kernel path must run instead.
template <typename T>
int try_dec(Linear *L, const void *x, void *y, int B, hipStream_t st, const Fuse &f = Fuse{}) {
    const size_t align = sizeof(T) == 4 ? 16 : 8;
    if (L->D != 16 || (reinterpret_cast<uintptr_t>(x) % align)) return 1;
    if (L->nnz && !L->col16.ptr) return 1;   // the kernel reads the 16-bit columns
    // tokens per workgroup: all of them up to 8 (the codebook staged and the
    // codes read once per row block), fewer where the staged x does not fit
    // the LDS beside the per-wave partials (2 x 16 waves x 32 rows x bt floats)
    int bt = B >= 5 ? 8 : B >= 3 ? 4 : B;
    const size_t xrow = (size_t)L->S * 256 * sizeof(float);
    auto lds_of = [&](int b) {
        return kCB * 16 * sizeof(float) + b * xrow + (size_t)(2 * 16 * 32 + 16) * b * sizeof(float);
    };
    while (bt > 1 && lds_of(bt) > kMaxLds) bt /= 2;
    if (lds_of(bt) > kMaxLds) return 1;
    const size_t lds = kCB * 16 * sizeof(float) + bt * xrow;
    // 32-row workgroups when that still gives about one workgroup per CU
    const long wg32 = (long)((L->M + 31) / 32) * ((B + bt - 1) / bt);
    const bool r2 = wg32 >= 192;
    if (bt == 1) {
        // Batch 1 with 8193 .. 20480 rows: ceil(M / 4096) row tiles of 16 per
        // workgroup, one workgroup per CU of the 256 with the rows spread
        // evenly (the LDS gathers of a CU's rows set the time): 19456 rows run
        // as 244 workgroups of 80 rows in 8.7 us, against 9.9 us for 608 of 32
        // (up to three on a CU) and 12.8 us for 304 of 64 (two on 48 CUs).
        int rpl = r2 ? 2 : 1;
        const int tall = (L->M + kTallRowsPerTile - 1) / kTallRowsPerTile;
        if (L->M > 2 * kTallRowsPerTile && tall <= kMaxTallTiles &&
            kCB * 16 * sizeof(float) + xrow + (size_t)(2 * 16 * 16 * tall + 16) * sizeof(float) <= kMaxLds)
            rpl = tall;
        switch (rpl) {
            case 1: return launch_dec<T, 1, 1>(L, x, y, B, lds, st, f);
            case 2: return launch_dec<T, 1, 2>(L, x, y, B, lds, st, f);
            case 3: return launch_dec<T, 1, 3>(L, x, y, B, lds, st, f);
            case 4: return launch_dec<T, 1, 4>(L, x, y, B, lds, st, f);
            default: return launch_dec<T, 1, 5>(L, x, y, B, lds, st, f);
        }
    }
    switch (bt * 2 + (r2 ? 1 : 0)) {
        case 4: return launch_dec<T, 2, 1>(L, x, y, B, lds, st, f);
        case 5: return launch_dec<T, 2, 2>(L, x, y, B, lds, st, f);
        case 8: return launch_dec<T, 4, 1>(L, x, y, B, lds, st, f);
        case 9: return launch_dec<T, 4, 2>(L, x, y, B, lds, st, f);
        case 16: return launch_dec<T, 8, 1>(L, x, y, B, lds, st, f);
        default: return launch_dec<T, 8, 2>(L, x, y, B, lds, st, f);
    }
}

template <typename T>
int launch(Linear *L, const void *x, void *y, int B, hipStream_t st) {
    const int Gp = L->S * kGS;
    dim3 g1(Gp, B);
    if (L->D == 16)
        OJX_LAUNCH((lut_build_kernel<16, T>), g1, dim3(kCB), 0, st,
                           static_cast<const T *>(x), L->codebook.as<float>(), L->K, L->D, L->G,
                           Gp, L->lut.as<float>());
    else
        OJX_LAUNCH((lut_build_kernel<0, T>), g1, dim3(kCB), 0, st,
                           static_cast<const T *>(x), L->codebook.as<float>(), L->K, L->D, L->G,
                           Gp, L->lut.as<float>());

    const int bt = B >= 3 ? 4 : B;
    GatherParams gp{};
    gp.codes = L->codes.as<uint8_t>();
    gp.lut = L->lut.as<float>();
    gp.scales = L->scales.as<float>();
    gp.bias = L->has_bias ? L->bias.as<float>() : nullptr;
    gp.rowp = L->nnz ? L->rowp.as<int>() : nullptr;
    gp.col = L->col.as<int>();
    gp.val = L->val.as<float>();
    gp.x = x;
    gp.y = y;
    gp.K = L->K;
    gp.M = L->M;
    gp.Mp = L->Mp;
    gp.S = L->S;
    gp.Gp = Gp;
    gp.B = B;
    gp.nnz = (int)L->nnz;
    const size_t xbytes = (size_t)bt * L->K * sizeof(float);
    gp.x_lds = L->nnz && xbytes <= kXLdsBytes;
    const size_t lds = gp.x_lds ? xbytes : 0;
    dim3 g2(1, (B + bt - 1) / bt);
    int rc;
    switch (bt) {
        case 1: rc = launch_gather<1, T>(gp, L->M, g2, lds, st); break;
        case 2: rc = launch_gather<2, T>(gp, L->M, g2, lds, st); break;
        default: rc = launch_gather<4, T>(gp, L->M, g2, lds, st); break;
    }
    if (rc) return rc;
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// From this many tokens the block_dim-16 linear runs as x . W^T on MFMA:
// measured (2560->6912, fp32) 17.0 vs 18.7 us at 10 tokens, 17.1 vs 23.7 at
// 16, 22.8 vs 39.6 at 32; at 8 the in-place LUT kernel is faster (14.1 vs
// 17.0 us).
constexpr int kMmMinBatch = 9;

int forward(Linear *L, const void *x, void *y, int B, int dtype, hipStream_t st) {
    if (B <= 0) return OJASX_OK;
    if (dtype != OJASX_DTYPE_F32 && dtype != OJASX_DTYPE_BF16) {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    if (B > 65535) {
        set_error("batch %d exceeds 65535", B);
        return OJASX_ERR_INVALID;
    }
    if (L->D == 16 && B >= kMmMinBatch && L->K <= 65535 &&
        (dtype != OJASX_DTYPE_F32 || reinterpret_cast<uintptr_t>(x) % 16 == 0)) {
        MmParams mp{L->codes.as<uint8_t>(), L->codebook.as<float>(), L->scales.as<float>(),
                    L->has_bias ? L->bias.as<float>() : nullptr,
                    L->nnz ? L->rowp.as<int>() : nullptr, L->col.as<int>(), L->val.as<float>(),
                    x, y, L->K, L->M, L->Mp, L->S, B, L->cb3.ptr};
        return launch_mm(mp, dtype, st);
    }
    int rc = dtype == OJASX_DTYPE_F32 ? try_dec<float>(L, x, y, B, st)
                                      : try_dec<__hip_bfloat16>(L, x, y, B, st);
    if (rc != 1) return rc;
    const int Gp = L->S * kGS;
    rc = L->lut.ensure((size_t)B * Gp * kCB * sizeof(float));
    if (rc) return rc;
    return dtype == OJASX_DTYPE_F32 ? launch<float>(L, x, y, B, st)
                                    : launch<__hip_bfloat16>(L, x, y, B, st);
}

}  // namespace

int linear_forward(void *h, const void *x, void *y, int B, int dtype, hipStream_t st) {
    return forward(static_cast<Linear *>(h), x, y, B, dtype, st);
}

// The device arrays of a block_dim-16 handle for the grouped kernel
// (lut_group.hip); x and y are filled by the caller.
int linear_items(const void *h, GroupItem *it) {
    const Linear *L = static_cast<const Linear *>(h);
    if (L->D != 16 || L->K % 4) {
        set_error("grouped linear: block_dim 16 and in_features %% 4 == 0 needed (got %d, %d)",
                  L->D, L->K);
        return OJASX_ERR_INVALID;
    }
    it->codes = L->codes.as<uint8_t>();
    it->codes_b = L->codes_b.as<uint8_t>();
    it->S32 = (L->G + 31) / 32;
    it->cb = L->codebook.as<float>();
    it->cb3 = L->cb3.ptr;
    it->scales = L->scales.as<float>();
    it->bias = L->has_bias ? L->bias.as<float>() : nullptr;
    it->rowp = L->nnz ? L->rowp.as<int>() : nullptr;
    it->col = L->col.as<int>();
    it->col16 = L->nnz ? L->col16.as<uint16_t>() : nullptr;
    it->val = L->val.as<float>();
    it->K = L->K;
    it->M = L->M;
    it->Mp = L->Mp;
    it->S = L->S;
    return OJASX_OK;
}

int linear_shape(const void *h, int *K, int *M, int *D) {
    const Linear *L = static_cast<const Linear *>(h);
    *K = L->K;
    *M = L->M;
    *D = L->D;
    return OJASX_OK;
}

// From this many output rows a batch-1 RMSNorm linear (no residual) runs on
// lut_tall_rms_kernel: MFMA-built LUT slices, one build per 256 rows (an LM
// head of 151936 rows: measured about 15 vs 37 us).  Below it the in-place
// kernel is faster: each tall workgroup runs a chain of slices, and 19456
// rows (76 workgroups) took 11.8 vs 11.3 us.
constexpr int kTallMinRows = 65536;

// The fused forward; with n_part set, a tall launch also writes the argmax
// partials arg_part and their count (0 on the in-place path).
static int fused_forward(void *h, const float *x, float *y, int pro, const float *w, float eps,
                         const float *res, hipStream_t st, float2 *arg_part, int *n_part) {
    Linear *L = static_cast<Linear *>(h);
    if (n_part) *n_part = 0;
    if (pro < kProNone || pro > kProRmsGlu) {
        set_error("unknown prologue %d", pro);
        return OJASX_ERR_INVALID;
    }
    const bool rms = pro == kProRms || pro == kProRmsGlu;
    if (rms && !w) return OJASX_ERR_NULL;
    if (L->K % 4 || (rms && (reinterpret_cast<uintptr_t>(w) & 15))) {
        set_error("fused linear: in_features %% 4 == 0 and a 16-byte aligned norm weight needed");
        return OJASX_ERR_INVALID;
    }
    if (pro == kProRmsGlu && (L->M % 2 || res)) {
        set_error("fused linear: the SwiGLU epilogue needs an even out_features and no residual");
        return OJASX_ERR_INVALID;
    }
    // (the tall kernel stages x * w beside two LUT buffers: it fits the LDS up
    // to about 31000 inputs)
    const bool tall_fits = (size_t)L->S * 256 * sizeof(float) + 2 * 16 * 260 * sizeof(float) +
                               64 <= kMaxLds;
    if (pro == kProRms && !res && L->D == 16 && L->M >= kTallMinRows && tall_fits &&
        (!L->nnz || L->col16.ptr) && !(reinterpret_cast<uintptr_t>(x) & 15)) {
        GroupItem it{};
        int rc = linear_items(h, &it);
        if (rc) return rc;
        it.x = x;
        it.y = y;
        if (n_part) *n_part = (L->M + tall_rows_per_part() - 1) / tall_rows_per_part();
        return launch_tall_rms(it, w, eps, st, n_part ? arg_part : nullptr);
    }
    Fuse f;
    f.pro = pro;
    f.w = w;
    f.eps = eps;
    f.res = res;
    const int rc = try_dec<float>(L, x, y, 1, st, f);
    if (rc == 1) {
        if (L->D == 16 && !(reinterpret_cast<uintptr_t>(x) & 15))
            set_error("fused linear: in_features %d does not fit the LDS: the staged input and "
                      "codebook need %zu bytes, %zu available",
                      L->K, kCB * 16 * sizeof(float) + (size_t)L->S * 256 * sizeof(float) +
                                (size_t)(2 * 16 * 32 + 16) * sizeof(float),
                      kMaxLds);
        else
            set_error("fused linear: block_dim 16 and a 16-byte aligned x needed");
        return OJASX_ERR_INVALID;
    }
    return rc;
}

int linear_forward_fused(void *h, const float *x, float *y, int pro, const float *w, float eps,
                         const float *res, hipStream_t st) {
    return fused_forward(h, x, y, pro, w, eps, res, st, nullptr, nullptr);
}

int linear_forward_lm_head(void *h, const float *x, float *y, const float *w, float eps,
                           float2 *arg_part, int *n_part, hipStream_t st) {
    return fused_forward(h, x, y, kProRms, w, eps, nullptr, st, arg_part, n_part);
}

int launch_lut_build(const void *x, const float *cb, int B, int K, int D, int G, int Gp,
                     float *lut, int dtype, hipStream_t st) {
    dim3 g(Gp, B);
    const bool d16 = D == 16;
    if (dtype == OJASX_DTYPE_F32) {
        const float *xf = static_cast<const float *>(x);
        if (d16) OJX_LAUNCH((lut_build_kernel<16, float>), g, dim3(kCB), 0, st, xf, cb, K, D, G, Gp, lut);
        else OJX_LAUNCH((lut_build_kernel<0, float>), g, dim3(kCB), 0, st, xf, cb, K, D, G, Gp, lut);
    } else {
        const __hip_bfloat16 *xb = static_cast<const __hip_bfloat16 *>(x);
        if (d16) OJX_LAUNCH((lut_build_kernel<16, __hip_bfloat16>), g, dim3(kCB), 0, st, xb, cb, K, D, G, Gp, lut);
        else OJX_LAUNCH((lut_build_kernel<0, __hip_bfloat16>), g, dim3(kCB), 0, st, xb, cb, K, D, G, Gp, lut);
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // namespace ojx
using ojx::Linear;

extern "C" {

OJASX_API OjasxLinearHandle ojasx_create_linear(int in_features, int out_features, int block_dim,
                                                int codebook_size, const float *codebook_data,
                                                const uint8_t *codes_data,
                                                const float *scales_data, const float *bias_data) {
    using namespace ojx;
    if (in_features <= 0 || out_features <= 0 || block_dim <= 0 || codebook_size <= 0 ||
        codebook_size > 256 || in_features % block_dim) {
        set_error("invalid linear shape in=%d out=%d block=%d codebook=%d", in_features,
                  out_features, block_dim, codebook_size);
        return nullptr;
    }
    Linear *L = new (std::nothrow) Linear;
    if (!L) return nullptr;
    L->K = in_features;
    L->M = out_features;
    L->D = block_dim;
    L->Kcb = codebook_size;
    L->G = in_features / block_dim;
    L->S = (L->G + kGS - 1) / kGS;
    L->Mp = (int)round_up(out_features, kRowAlign);

    // Slice-major code tiles; padded groups and rows hold code 0, whose
    // LUT entry is 0 for padded groups (x is zero there) and unused for rows.
    std::vector<uint8_t> packed((size_t)L->S * L->Mp * kGS, 0);
    if (codes_data) {
        for (int m = 0; m < L->M; ++m) {
            const uint8_t *row = codes_data + (size_t)m * L->G;
            for (int g = 0; g < L->G; ++g)
                packed[((size_t)(g / kGS) * L->Mp + m) * kGS + (g % kGS)] = row[g];
        }
    }
    std::vector<float> cb((size_t)kCB * L->D, 0.f);
    if (codebook_data) memcpy(cb.data(), codebook_data, sizeof(float) * codebook_size * block_dim);
    std::vector<float> sc(L->M, 1.f);
    if (scales_data) memcpy(sc.data(), scales_data, sizeof(float) * L->M);
    int rc = upload(L->codes, packed.data(), packed.size());
    if (!rc && L->D == 16) {   // the grouped kernel's layout (block_dim 16 only)
        std::vector<uint8_t> bank(bank_codes_bytes(L->M, L->G) + kBankSlack, 0);
        if (codes_data) pack_bank_codes(codes_data, L->M, L->G, bank.data());
        rc = upload(L->codes_b, bank.data(), bank.size());
    }
    if (!rc) rc = upload(L->codebook, cb.data(), cb.size() * sizeof(float));
    if (!rc && L->D == 16) {   // the grouped kernel's MFMA operand
        std::vector<uint16_t> cb3(kCb3Bytes / 2);
        split_codebook_bf16x3(cb.data(), cb3.data());
        rc = upload(L->cb3, cb3.data(), kCb3Bytes);
    }
    if (!rc) rc = upload(L->scales, sc.data(), sc.size() * sizeof(float));
    if (!rc && bias_data) {
        L->has_bias = true;
        rc = upload(L->bias, bias_data, sizeof(float) * L->M);
    }
    if (rc) {
        delete L;
        return nullptr;
    }
    return L;
}

OJASX_API int ojasx_set_linear_outliers(OjasxLinearHandle handle, int nnz, const int *row_ptrs,
                                        const int *col_indices, const float *values) {
    using namespace ojx;
    if (!handle) return OJASX_ERR_NULL;
    Linear *L = static_cast<Linear *>(handle);
    if (nnz < 0) {
        set_error("negative nnz");
        return OJASX_ERR_INVALID;
    }
    if (nnz == 0) {
        L->nnz = 0;
        return OJASX_OK;
    }
    if (!row_ptrs || !col_indices || !values) return OJASX_ERR_NULL;
    if (row_ptrs[0] != 0 || row_ptrs[L->M] != nnz) {
        set_error("row_ptrs must run from 0 to nnz");
        return OJASX_ERR_INVALID;
    }
    for (int m = 0; m < L->M; ++m)
        if (row_ptrs[m + 1] < row_ptrs[m]) {
            set_error("row_ptrs not monotone at row %d", m);
            return OJASX_ERR_INVALID;
        }
    for (int j = 0; j < nnz; ++j)
        if (col_indices[j] < 0 || col_indices[j] >= L->K) {
            set_error("outlier column %d out of range", col_indices[j]);
            return OJASX_ERR_INVALID;
        }
    // Each row's entries are kept sorted by column (a stable sort: equal
    // columns keep their order), so a kernel can take a row's entries slice
    // by slice of the input; the row's outlier sum is then formed in column
    // order, a reordering of the same terms.
    std::vector<int> cs(col_indices, col_indices + nnz), order;
    std::vector<float> vs(values, values + nnz);
    for (int m = 0; m < L->M; ++m) {
        const int j0 = row_ptrs[m], j1 = row_ptrs[m + 1];
        if (std::is_sorted(col_indices + j0, col_indices + j1)) continue;
        order.resize(j1 - j0);
        for (int j = j0; j < j1; ++j) order[j - j0] = j;
        std::stable_sort(order.begin(), order.end(),
                         [&](int a, int b) { return col_indices[a] < col_indices[b]; });
        for (int j = j0; j < j1; ++j) {
            cs[j] = col_indices[order[j - j0]];
            vs[j] = values[order[j - j0]];
        }
    }
    int rc = upload(L->rowp, row_ptrs, (size_t)(L->M + 1) * sizeof(int));
    if (!rc) rc = upload(L->col, cs.data(), (size_t)nnz * sizeof(int));
    if (!rc) rc = upload(L->val, vs.data(), (size_t)nnz * sizeof(float));
    // 16-bit columns for the grouped kernel: 6 instead of 8 bytes per entry
    // where the outliers are a bandwidth term of their own
    if (!rc && L->K <= 65536) {
        std::vector<uint16_t> c16(cs.begin(), cs.end());
        rc = upload(L->col16, c16.data(), (size_t)nnz * sizeof(uint16_t));
    } else if (!rc) {
        L->col16.release();
    }
    if (rc) return rc;
    L->nnz = (size_t)nnz;
    return OJASX_OK;
}

OJASX_API int ojasx_linear_forward_device(OjasxLinearHandle handle, const void *x, void *y,
                                          int batch_size, int dtype, void *stream) {
    if (!handle || !x || !y) return OJASX_ERR_NULL;
    return ojx::linear_forward(handle, x, y, batch_size, dtype, static_cast<hipStream_t>(stream));
}

OJASX_API int ojasx_linear_forward_fused_device(OjasxLinearHandle handle, const float *x,
                                                float *y, int prologue, const float *norm_weight,
                                                float eps, const float *residual, void *stream) {
    if (!handle || !x || !y) return OJASX_ERR_NULL;
    return ojx::linear_forward_fused(handle, x, y, prologue, norm_weight, eps, residual,
                                     static_cast<hipStream_t>(stream));
}

OJASX_API int ojasx_build_lut_device(const void *x, const float *codebook, int batch_size,
                                     int groups, int block_dim, int codebook_size, float *lut,
                                     int dtype, void *stream) {
    using namespace ojx;
    if (!x || !codebook || !lut) return OJASX_ERR_NULL;
    if (batch_size <= 0 || groups <= 0) return OJASX_OK;
    if (block_dim <= 0 || codebook_size <= 0 || codebook_size > 256 || groups > 65535 ||
        batch_size > 65535) {
        set_error("invalid LUT build shape");
        return OJASX_ERR_INVALID;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    dim3 grid(groups, batch_size);
    if (dtype == OJASX_DTYPE_F32)
        OJX_LAUNCH(build_lut_kernel<float>, grid, dim3(kCB), 0, st,
                           static_cast<const float *>(x), codebook, groups, block_dim,
                           codebook_size, lut);
    else if (dtype == OJASX_DTYPE_BF16)
        OJX_LAUNCH(build_lut_kernel<__hip_bfloat16>, grid, dim3(kCB), 0, st,
                           static_cast<const __hip_bfloat16 *>(x), codebook, groups, block_dim,
                           codebook_size, lut);
    else {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API int ojasx_linear_forward(OjasxLinearHandle handle, const float *x, float *y,
                                   int batch_size, int num_threads) {
    using namespace ojx;
    (void)num_threads;
    if (!handle || !x || !y) return OJASX_ERR_NULL;
    if (batch_size <= 0) return OJASX_OK;
    Linear *L = static_cast<Linear *>(handle);
    const size_t xb = (size_t)batch_size * L->K * sizeof(float);
    const size_t yb = (size_t)batch_size * L->M * sizeof(float);
    int rc = L->xstage.ensure(xb);
    if (!rc) rc = L->ystage.ensure(yb);
    HostIO &io = host_io();
    const size_t yo = round_up(xb, 256);
    if (!rc) rc = io.reserve(yo + yb);
    if (rc) return rc;
    memcpy(io.pin, x, xb);
    OJX_HIP(hipMemcpyAsync(L->xstage.ptr, io.pin, xb, hipMemcpyHostToDevice, io.st));
    rc = forward(L, L->xstage.ptr, L->ystage.ptr, batch_size, OJASX_DTYPE_F32, io.st);
    if (!rc) OJX_HIP(hipMemcpyAsync(io.pin + yo, L->ystage.ptr, yb, hipMemcpyDeviceToHost, io.st));
    OJX_HIP(hipStreamSynchronize(io.st));
    if (rc) return rc;
    memcpy(y, io.pin + yo, yb);
    return OJASX_OK;
}

OJASX_API size_t ojasx_get_compressed_size(OjasxLinearHandle handle) {
    if (!handle) return 0;
    const Linear *L = static_cast<const Linear *>(handle);
    size_t b = (size_t)L->M * L->G + (size_t)L->Kcb * L->D * 4 + (size_t)L->M * 4;
    if (L->has_bias) b += (size_t)L->M * 4;
    if (L->nnz) b += L->nnz * 8 + (size_t)(L->M + 1) * 4;
    return b;
}

OJASX_API size_t ojasx_get_dense_size(OjasxLinearHandle handle) {
    if (!handle) return 0;
    const Linear *L = static_cast<const Linear *>(handle);
    return (size_t)L->M * L->K * sizeof(float);
}

OJASX_API size_t ojasx_get_lut_sram_size(OjasxLinearHandle handle) {
    if (!handle) return 0;
    const Linear *L = static_cast<const Linear *>(handle);
    return (size_t)L->G * L->Kcb * sizeof(float);
}

OJASX_API float ojasx_get_compression_ratio(OjasxLinearHandle handle) {
    if (!handle) return 0.f;
    const size_t c = ojasx_get_compressed_size(handle);
    return (float)ojasx_get_dense_size(handle) / (float)(c ? c : 1);
}

OJASX_API size_t ojasx_linear_device_weight_bytes(OjasxLinearHandle handle) {
    if (!handle) return 0;
    const Linear *L = static_cast<const Linear *>(handle);
    size_t b = (size_t)L->M * L->G + (size_t)L->Kcb * L->D * 4 + (size_t)L->M * 4;
    if (L->has_bias) b += (size_t)L->M * 4;
    // outliers as the batch-1 and grouped kernels read them: 16-bit columns
    // and fp32 values (the batched MFMA kernels read 32-bit columns)
    if (L->nnz) b += L->nnz * (L->col16.ptr ? 6 : 8) + (size_t)(L->M + 1) * 4;
    return b;
}

OJASX_API void ojasx_destroy_linear(OjasxLinearHandle handle) {
    delete static_cast<Linear *>(handle);
}

}  // extern "C"

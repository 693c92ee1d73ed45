// lut_mm.hip -- the LUT linear (block_dim 16, 256 centroids) for many tokens
// as x . W^T on fp32 MFMA.
//
// y[b][m] = (s_m * sum_g LUT_b[g, codes[m, g]] + bias_m) + sum_j val_j x_b[col_j]
// with LUT_b[g, k] = <x_b[16g..16g+16), C[k]> (ojasx_lut_cpu.cpp:132-206).  By
// the identity LUT-gather = x . W^T, with W[m][16g + d] = C[codes[m, g]][d],
// the sum over groups is a GEMM against W decoded from the codes: the
// per-token LUTs grow with the batch (1 KB per group and token), W does not
// (64 bytes per group and row, decoded in registers from the codebook in
// LDS).  A workgroup owns 64 rows (16 per wave) and 16 tokens; per 256-wide
// input slice it stages the 16 tokens' x in LDS (two buffers, the next
// slice's loads in flight during the current one; codes kMmPF slices ahead,
// since they come from HBM), and per group each wave
// runs 4 MFMAs (v_mfma_f32_16x16x4f32) with
//   A[m][k] = C[code(m, g)][4k + ks]   (one 16-byte LDS read of the codebook row),
//   B[k][n] = x_n[16g + 4k + ks]       (one 16-byte LDS read of the staged x),
// for ks = 0..3: MFMA ks covers dims 4k + ks of the group, so a lane's four
// values are contiguous in both the codebook row and x.  Two accumulators
// (even and odd groups) keep the MFMA chains independent.  The CSR outliers
// of the workgroup's rows are staged in LDS; each lane adds those of its rows
// whose columns fall in the current slice from the staged x (a row's entries
// are sorted by column), so no x is read at random from memory.  The
// epilogue applies the scale and the bias: (s_m * sum + bias) + outliers.
//
// MFMA 16x16x4 fp32 operand layout: lane l supplies A[m = l % 16][k = l / 16]
// and B[k = l / 16][n = l % 16]; the result's value v of lane l is
// D[m = 4 (l / 16) + v][n = l % 16].
#include "common.h"

namespace ojx {

namespace {
constexpr int kMmNT = 256;       // 4 waves
constexpr int kMmRows = 64;      // rows per workgroup (16 per wave)
constexpr int kMmTok = 16;       // tokens per workgroup
constexpr int kXStride = 260;    // floats per staged x row (256 + pad)
constexpr int kMmPF = 4;         // slices of codes in flight
// CSR entries of a workgroup's 64 rows staged in LDS (columns as 16-bit:
// in_features <= 65535 on this path); three workgroups still fit a CU
constexpr int kCsrStage = 768;
constexpr int kOutPass = 3;      // outlier candidates per row per pass
typedef float v4f __attribute__((ext_vector_type(4)));
}  // namespace

// x of tokens n0..n0+15, inputs 256 s .. 256 s + 255 (zero past K and past B):
// thread t loads token t / 16, inputs 16 (t % 16) .. + 15.
template <typename T>
__device__ __forceinline__ void mm_load_x(const MmParams &p, int n0, int s, float (&r)[16]) {
    const int tt = threadIdx.x >> 4, k = s * 256 + (threadIdx.x & 15) * 16;
    const int n = n0 + tt;
    const bool ok = n < p.B && k < p.K;        // K is a multiple of 16
    const T *src = static_cast<const T *>(p.x) + (size_t)min(n, p.B - 1) * p.K + min(k, p.K - 16);
    if constexpr (sizeof(T) == 4) {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 f = gld(s4 + u);
            r[4 * u] = f.x;
            r[4 * u + 1] = f.y;
            r[4 * u + 2] = f.z;
            r[4 * u + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < 16; ++u) r[u] = load_act(src, u);
    }
    if (!ok) {
#pragma unroll
        for (int u = 0; u < 16; ++u) r[u] = 0.f;
    }
}

__device__ __forceinline__ void mm_store_x(float *xs, const float (&r)[16]) {
    float4 *d = reinterpret_cast<float4 *>(xs + (threadIdx.x >> 4) * kXStride + (threadIdx.x & 15) * 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) d[u] = make_float4(r[4 * u], r[4 * u + 1], r[4 * u + 2], r[4 * u + 3]);
}

template <typename T>
__global__ __launch_bounds__(kMmNT) void lut_mm_kernel(MmParams p) {
    __shared__ float4 cb4[256 * 4];                 // codebook [256][16]
    __shared__ float xs[2][kMmTok * kXStride];      // staged x slices
    __shared__ unsigned short lcol[kCsrStage];      // the workgroup's CSR outliers
    __shared__ float lval[kCsrStage];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ml = lane & 15, kk = lane >> 4;
    const int mb = blockIdx.x * kMmRows;
    const int m0 = mb + w * 16;
    const int n0 = blockIdx.y * kMmTok;
    const int row = min(m0 + ml, p.M - 1);          // rows past M: computed, never stored

    // ---- round trip 1: codebook, x slice 0, the CSR range of the rows, codes
    float4 c4[4];
    const float4 *gcb = reinterpret_cast<const float4 *>(p.cb);
#pragma unroll
    for (int u = 0; u < 4; ++u) c4[u] = gld(gcb + tid + u * kMmNT);
    float xr[16];
    mm_load_x<T>(p, n0, 0, xr);
    int e_lo = 0, e_hi = 0, j[4] = {0, 0, 0, 0}, je[4] = {0, 0, 0, 0};
    if (p.rowp) {
        e_lo = gld(p.rowp + mb);
        e_hi = gld(p.rowp + min(mb + kMmRows, p.M));
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = min(m0 + 4 * kk + v, p.M - 1);
            j[v] = gld(p.rowp + m);
            je[v] = m0 + 4 * kk + v < p.M ? gld(p.rowp + m + 1) : j[v];
        }
    }
    uint4 cr[kMmPF];   // codes of slices s .. s + kMmPF - 1, slot (s % kMmPF)
#pragma unroll
    for (int q = 0; q < kMmPF; ++q)
        cr[q] = gld(reinterpret_cast<const uint4 *>(p.codes + ((size_t)min(q, p.S - 1) * p.Mp + row) * 16));
    // ---- round trip 2: the CSR entries of the workgroup's rows into LDS when
    // they fit (the usual case: each row's entries sorted by column are then
    // added slice by slice from the staged x), else from memory at the end
    const bool staged = e_hi - e_lo <= kCsrStage;
    if (p.rowp && staged && e_hi > e_lo) {
#pragma unroll
        for (int u = 0; u < kCsrStage / kMmNT; ++u) {
            const int e = min(e_lo + tid + u * kMmNT, e_hi - 1);   // an entry of these rows
            const int c = gld(p.col + e);
            const float v = gld(p.val + e);
            if (e_lo + tid + u * kMmNT < e_hi) {
                lcol[tid + u * kMmNT] = (unsigned short)c;
                lval[tid + u * kMmNT] = v;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) cb4[tid + u * kMmNT] = c4[u];
    mm_store_x(xs[0], xr);
    __syncthreads();

    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        j[v] -= e_lo;
        je[v] -= e_lo;
    }
    // Slice s uses code slot s % kMmPF, a constant in the unrolled body (no
    // register moves of loads in flight); the slot is refilled with slice
    // s + kMmPF after its gathers, unconditionally (clamped to the last slice).
    for (int sb = 0; sb < p.S; sb += kMmPF) {
#pragma unroll
        for (int q = 0; q < kMmPF; ++q) {
            const int s = sb + q;
            if (s >= p.S) break;
            // the next slice's x in flight during this one (past the last
            // slice: a reload of the last, unused)
            mm_load_x<T>(p, n0, min(s + 1, p.S - 1), xr);
            const float *xt = xs[s & 1] + ml * kXStride;
            const float *xb = xt + 4 * kk;
            const uint32_t wd[4] = {cr[q].x, cr[q].y, cr[q].z, cr[q].w};
#pragma unroll
            for (int g = 0; g < 16; ++g) {
                const uint32_t code = (wd[g >> 2] >> ((g & 3) * 8)) & 0xffu;
                const float4 a = cb4[code * 4 + kk];
                const float4 b = *reinterpret_cast<const float4 *>(xb + 16 * g);
                v4f &acc = (g & 1) ? acc1 : acc0;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
            }
            // outliers of the lane's 4 rows whose columns fall in this slice:
            // kOutPass candidates per row per pass, all reads of a pass in
            // flight together (one pass covers a slice unless a row has more
            // than kOutPass entries in it); added in column order
            if (p.rowp && staged) {
                const int lim = (s + 1) * 256;
                bool more = true;
                while (more) {
                    int c[4][kOutPass];
                    float vv[4][kOutPass], xv[4][kOutPass];
                    bool in[4][kOutPass];
#pragma unroll
                    for (int v = 0; v < 4; ++v)
#pragma unroll
                        for (int u = 0; u < kOutPass; ++u) {
                            const int e = min(j[v] + u, kCsrStage - 1);
                            c[v][u] = lcol[e];
                            vv[v][u] = lval[e];
                        }
#pragma unroll
                    for (int v = 0; v < 4; ++v)
#pragma unroll
                        for (int u = 0; u < kOutPass; ++u) {
                            in[v][u] = j[v] + u < je[v] && c[v][u] < lim && (u == 0 || in[v][u - 1]);
                            xv[v][u] = xt[in[v][u] ? c[v][u] - s * 256 : 0];
                        }
                    more = false;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
#pragma unroll
                        for (int u = 0; u < kOutPass; ++u)
                            if (in[v][u]) o[v] += vv[v][u] * xv[v][u];
                        int took = 0;
#pragma unroll
                        for (int u = 0; u < kOutPass; ++u) took += in[v][u] ? 1 : 0;
                        j[v] += took;
                        more |= took == kOutPass;
                    }
                }
            }
            if (s + 1 < p.S) mm_store_x(xs[(s + 1) & 1], xr);
            cr[q] = gld(reinterpret_cast<const uint4 *>(
                p.codes + ((size_t)min(s + kMmPF, p.S - 1) * p.Mp + row) * 16));
            __syncthreads();   // slice s + 1 staged; slice s's reads done before it is overwritten
        }
    }

    // ---- epilogue: lane holds rows m0 + 4 kk + v of token n0 + ml
    const int n = n0 + ml;
    if (n >= p.B) return;
    const T *xn = static_cast<const T *>(p.x) + (size_t)n * p.K;
    T *yn = static_cast<T *>(p.y) + (size_t)n * p.M;
    if (p.rowp && !staged) {   // a dense-outlier block: entries and x from memory
#pragma unroll
        for (int v = 0; v < 4; ++v)
            for (int e = j[v]; e < je[v]; ++e) o[v] += gld(p.val + e_lo + e) * load_act(xn, gld(p.col + e_lo + e));
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int m = m0 + 4 * kk + v;
        if (m >= p.M) continue;
        float yv = (acc0[v] + acc1[v]) * gld(p.scales + m);
        if (p.bias) yv += gld(p.bias + m);
        store_act(yn, (size_t)m, yv + o[v]);
    }
}

int launch_mm(const MmParams &p, int dtype, hipStream_t st) {
    const dim3 grid((p.M + kMmRows - 1) / kMmRows, (p.B + kMmTok - 1) / kMmTok);
    if (grid.y > 65535) {
        set_error("batch %d too large for the MFMA path", p.B);
        return OJASX_ERR_INVALID;
    }
    if (dtype == OJASX_DTYPE_F32)
        OJX_LAUNCH(lut_mm_kernel<float>, grid, dim3(kMmNT), 0, st, p);
    else
        OJX_LAUNCH(lut_mm_kernel<__hip_bfloat16>, grid, dim3(kMmNT), 0, st, p);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // namespace ojx

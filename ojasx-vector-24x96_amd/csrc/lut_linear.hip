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
// Two kernels per call and no cross-workgroup synchronisation.  At batch 1
// both are latency-bound (1.1 MB of codes is ~0.14 us of HBM time against a
// ~1.3 us kernel floor), so each issues every independent load first and
// keeps the chain of dependent memory round trips to two:
//  K1 lut_build: the LUT of every token, LUT[b][g][k] for all 256 centroids,
//     into a workspace (workgroup = (1 group, 1 token), thread k owns
//     centroid k): x and the codebook, then one store.
//  K2 lut_gather: workgroup = 64 output rows x up to 4 tokens; lane = row, the
//     4 waves take interleaved 16-group slices.  Round trip 1: a lane reads
//     its row's 16 codes of each of its slices with one 16-byte load each (a
//     wave reads 1 KB contiguous from the slice-major tiles [S][Mp][16]),
//     together with scale, bias, CSR row bounds and x (staged in LDS).  Round
//     trip 2: the 16 LUT entries per slice and token from the L2-resident
//     LUT, and -- wave 0 -- the row's CSR outlier entries (32 per batch).
//     The four wave partials are summed in LDS in wave order and the epilogue
//     applies scale, bias and the outlier sum in the reference's order:
//     deterministic results.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;        // threads per workgroup (4 waves)
constexpr int kGS = 16;         // groups per slice: 16 code bytes per row
constexpr int kRowAlign = 1024; // rows padded for the tile layout
constexpr int kCB = 256;        // centroids in the (zero-padded) codebook
constexpr int kRows = 64;       // rows per gather workgroup (one per lane)
constexpr int kWaves = kNT / 64;
constexpr int kOB = 32;         // outlier entries loaded per batch
constexpr size_t kXLdsBytes = 48 * 1024;  // x staged in LDS up to this size
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
template <int DT, typename T>
__global__ __launch_bounds__(kCB) void lut_build_kernel(const T *__restrict__ x,
                                                      const float *__restrict__ cb, int K, int D,
                                                      int G, int Gp, float *__restrict__ lut) {
    constexpr int DMAX = DT > 0 ? DT : 32;
    const int Dr = DT > 0 ? DT : D;
    __shared__ float xs[32];
    const int b = blockIdx.y, g = blockIdx.x, k = threadIdx.x;
    float c[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) c[d] = d < Dr ? cb[k * Dr + d] : 0.f;
    if (k < Dr) xs[k] = g < G ? load_act(x, (size_t)b * K + (size_t)g * Dr + k) : 0.f;
    __syncthreads();
    float dot = 0.f;
#pragma unroll
    for (int d = 0; d < DMAX; ++d)
        if (d < Dr) dot = fmaf(xs[d], c[d], dot);
    lut[((size_t)b * Gp + g) * kCB + k] = dot;
}

// K2 + K3: gather-accumulate, outliers and epilogue, one row per lane.
// Loads are issued branch-free (clamped indices, results masked at use) so
// the compiler can keep them all in flight: round trip 1 = codes, scale,
// bias, CSR row bounds, x; round trip 2 = LUT entries and outlier entries.
template <int BT, typename T>
__global__ __launch_bounds__(kNT) void lut_gather_kernel(GatherParams p) {
    extern __shared__ float xs[];                 // [BT][K] when p.x_lds
    __shared__ float red[kWaves][BT][kRows];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int m = blockIdx.x * kRows + lane;      // < Mp: codes need no clamp
    const int mr = min(m, p.M - 1);               // clamped row for [M] arrays
    const int t0 = blockIdx.y * BT;
    const int nt = min(BT, p.B - t0);
    const bool outl = p.rowp != nullptr;
    const T *__restrict__ x = static_cast<const T *>(p.x);

    // ---- round trip 1
    uint4 cv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = min(w + i * kWaves, p.S - 1);
        cv[i] = *reinterpret_cast<const uint4 *>(p.codes + ((size_t)s * p.Mp + m) * kGS);
    }
    const float sc = p.scales[mr];
    const float bs = p.bias ? p.bias[mr] : 0.f;
    int j0 = 0, j1 = 0;
    if (outl) {
        j0 = p.rowp[mr];
        j1 = p.rowp[mr + 1];
    }
    if (outl && p.x_lds) stage_to_lds<kNT>(xs, x + (size_t)t0 * p.K, nt * p.K);

    // ---- round trip 2: first batch of outlier entries, LUT entries
    int oc[kOB];
    float ov[kOB];
    if (outl) {
#pragma unroll
        for (int u = 0; u < kOB; ++u) {
            const int j = min(j0 + u, p.nnz - 1);
            oc[u] = p.col[j];
            ov[u] = p.val[j];
        }
    }
    float acc[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) acc[t] = 0.f;
    for (int s0 = w;; s0 += kWaves * 4) {
        // (token, slice) pairs, 4 at a time: 64 LUT loads in flight, then the
        // adds (per token, slices ascending).
#pragma unroll
        for (int q0 = 0; q0 < BT * 4; q0 += 4) {
            float lv[4][kGS];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = (q0 + q) >> 2, i = (q0 + q) & 3;
                const int s = min(s0 + i * kWaves, p.S - 1);
                const int tt = min(t, nt - 1);
                const float *L = p.lut + ((size_t)(t0 + tt) * p.Gp + s * kGS) * kCB;
                const uint32_t w4[4] = {cv[i].x, cv[i].y, cv[i].z, cv[i].w};
#pragma unroll
                for (int g = 0; g < kGS; ++g)
                    lv[q][g] = L[g * kCB + ((w4[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = (q0 + q) >> 2, i = (q0 + q) & 3;
                if (s0 + i * kWaves < p.S) {
                    float a = acc[t];
#pragma unroll
                    for (int g = 0; g < kGS; ++g) a += lv[q][g];
                    acc[t] = a;
                }
            }
        }
        const int nx = s0 + kWaves * 4;
        if (nx >= p.S) break;
        // further slices (K > 64 groups * 4 waves): next batch of codes
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int s = min(nx + i * kWaves, p.S - 1);
            cv[i] = *reinterpret_cast<const uint4 *>(p.codes + ((size_t)s * p.Mp + m) * kGS);
        }
    }
#pragma unroll
    for (int t = 0; t < BT; ++t) red[w][t][lane] = acc[t];
    __syncthreads();
    if (w != 0 || m >= p.M) return;

    // Outliers in CSR order (x from LDS when staged).
    // First batch branch-free: entries past the row's end add an exact 0.
    float oac[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) oac[t] = 0.f;
    if (outl) {
        const int n0 = j1 - j0;
#pragma unroll
        for (int t = 0; t < BT; ++t) {
            const int tt = min(t, nt - 1);
            float xv[kOB];
#pragma unroll
            for (int u = 0; u < kOB; ++u)
                xv[u] = p.x_lds ? xs[tt * p.K + oc[u]] : load_act(x, (size_t)(t0 + tt) * p.K + oc[u]);
            float o = 0.f;
#pragma unroll
            for (int u = 0; u < kOB; ++u) o += u < n0 ? ov[u] * xv[u] : 0.f;
            oac[t] = o;
        }
        // rows with more than kOB outliers (rare): the rest in CSR order
        for (int j = j0 + kOB; j < j1; ++j) {
            const int c = p.col[j];
            const float v = p.val[j];
#pragma unroll
            for (int t = 0; t < BT; ++t)
                if (t < nt)
                    oac[t] += v * (p.x_lds ? xs[t * p.K + c] : load_act(x, (size_t)(t0 + t) * p.K + c));
        }
    }
    T *y = static_cast<T *>(p.y);
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        if (t >= nt) break;
        float a = red[0][t][lane];
#pragma unroll
        for (int q = 1; q < kWaves; ++q) a += red[q][t][lane];
        float r = a * sc;
        if (p.bias) r += bs;
        r += oac[t];
        store_act(y, (size_t)(t0 + t) * p.M + m, r);
    }
}

// Standalone LUT build with a codebook of Kcb rows: one workgroup per
// (group, token), thread k computes LUT[b][g][k].
template <typename T>
__global__ __launch_bounds__(kCB) void build_lut_kernel(const T *__restrict__ x,
                                                      const float *__restrict__ cb, int G, int D,
                                                      int Kcb, float *__restrict__ lut) {
    const int g = blockIdx.x, b = blockIdx.y, k = threadIdx.x;
    __shared__ float xs[32];
    if (k < D) xs[k] = load_act(x, (size_t)b * G * D + (size_t)g * D + k);
    __syncthreads();
    if (k >= Kcb) return;
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot = fmaf(xs[d], cb[(size_t)k * D + d], dot);
    lut[((size_t)b * G + g) * Kcb + k] = dot;
}

// ---------------------------------------------------------------------------
struct Linear {
    int K = 0, M = 0, D = 0, Kcb = 0, G = 0, S = 0, Mp = 0;
    bool has_bias = false;
    size_t nnz = 0;
    DevBuf codes, codebook, scales, bias, rowp, col, val;
    DevBuf lut, xstage, ystage;
    ~Linear() {
        for (DevBuf *b : {&codes, &codebook, &scales, &bias, &rowp, &col, &val, &lut, &xstage,
                          &ystage})
            b->release();
    }
};

namespace {

template <int BT, typename T>
int launch_gather(const GatherParams &gp, dim3 grid, size_t lds, hipStream_t st) {
    static size_t granted = 0;
    int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&lut_gather_kernel<BT, T>), lds, &granted);
    if (rc) return rc;
    hipLaunchKernelGGL((lut_gather_kernel<BT, T>), grid, dim3(kNT), lds, st, gp);
    return OJASX_OK;
}

template <typename T>
int launch(Linear *L, const void *x, void *y, int B, hipStream_t st) {
    const int Gp = L->S * kGS;
    dim3 g1(Gp, B);
    if (L->D == 16)
        hipLaunchKernelGGL((lut_build_kernel<16, T>), g1, dim3(kCB), 0, st,
                           static_cast<const T *>(x), L->codebook.as<float>(), L->K, L->D, L->G,
                           Gp, L->lut.as<float>());
    else
        hipLaunchKernelGGL((lut_build_kernel<0, T>), g1, dim3(kCB), 0, st,
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
    dim3 g2((L->M + kRows - 1) / kRows, (B + bt - 1) / bt);
    int rc;
    switch (bt) {
        case 1: rc = launch_gather<1, T>(gp, g2, lds, st); break;
        case 2: rc = launch_gather<2, T>(gp, g2, lds, st); break;
        default: rc = launch_gather<4, T>(gp, g2, lds, st); break;
    }
    if (rc) return rc;
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

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
    const int Gp = L->S * kGS;
    int rc = L->lut.ensure((size_t)B * Gp * kCB * sizeof(float));
    if (rc) return rc;
    return dtype == OJASX_DTYPE_F32 ? launch<float>(L, x, y, B, st)
                                    : launch<__hip_bfloat16>(L, x, y, B, st);
}

}  // namespace

int linear_forward(void *h, const void *x, void *y, int B, int dtype, hipStream_t st) {
    return forward(static_cast<Linear *>(h), x, y, B, dtype, st);
}

}  // namespace ojx
using ojx::Linear;

extern "C" {

OJASX_API OjasxLinearHandle ojasx_create_linear(int in_features, int out_features, int block_dim,
                                                int codebook_size, const float *codebook_data,
                                                const uint8_t *codes_data,
                                                const float *scales_data, const float *bias_data) {
    using namespace ojx;
    if (in_features <= 0 || out_features <= 0 || block_dim <= 0 || block_dim > 32 ||
        codebook_size <= 0 || codebook_size > 256 || in_features % block_dim) {
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
    if (!rc) rc = upload(L->codebook, cb.data(), cb.size() * sizeof(float));
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
    int rc = upload(L->rowp, row_ptrs, (size_t)(L->M + 1) * sizeof(int));
    if (!rc) rc = upload(L->col, col_indices, (size_t)nnz * sizeof(int));
    if (!rc) rc = upload(L->val, values, (size_t)nnz * sizeof(float));
    if (rc) return rc;
    L->nnz = (size_t)nnz;
    return OJASX_OK;
}

OJASX_API int ojasx_linear_forward_device(OjasxLinearHandle handle, const void *x, void *y,
                                          int batch_size, int dtype, void *stream) {
    if (!handle || !x || !y) return OJASX_ERR_NULL;
    return ojx::linear_forward(handle, x, y, batch_size, dtype, static_cast<hipStream_t>(stream));
}

OJASX_API int ojasx_build_lut_device(const void *x, const float *codebook, int batch_size,
                                     int groups, int block_dim, int codebook_size, float *lut,
                                     int dtype, void *stream) {
    using namespace ojx;
    if (!x || !codebook || !lut) return OJASX_ERR_NULL;
    if (batch_size <= 0 || groups <= 0) return OJASX_OK;
    if (block_dim <= 0 || block_dim > 32 || codebook_size <= 0 || codebook_size > 256 ||
        groups > 65535 || batch_size > 65535) {
        set_error("invalid LUT build shape");
        return OJASX_ERR_INVALID;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    dim3 grid(groups, batch_size);
    if (dtype == OJASX_DTYPE_F32)
        hipLaunchKernelGGL(build_lut_kernel<float>, grid, dim3(kCB), 0, st,
                           static_cast<const float *>(x), codebook, groups, block_dim,
                           codebook_size, lut);
    else if (dtype == OJASX_DTYPE_BF16)
        hipLaunchKernelGGL(build_lut_kernel<__hip_bfloat16>, grid, dim3(kCB), 0, st,
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
    if (rc) return rc;
    OJX_HIP(hipMemcpy(L->xstage.ptr, x, xb, hipMemcpyHostToDevice));
    rc = forward(L, L->xstage.ptr, L->ystage.ptr, batch_size, OJASX_DTYPE_F32, nullptr);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(y, L->ystage.ptr, yb, hipMemcpyDeviceToHost));
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
    if (L->nnz) b += L->nnz * 8 + (size_t)(L->M + 1) * 4;
    return b;
}

OJASX_API void ojasx_destroy_linear(OjasxLinearHandle handle) {
    delete static_cast<Linear *>(handle);
}

}  // extern "C"

// lut_linear.hip -- split-manifold LUT linear layer on gfx950.
//
// Computes, for every token b and output row m,
//   y[b,m] = s_m * sum_g LUT_b[g, codes[m,g]] + bias[m] + sum_j val_j * x[b,col_j]
// with LUT_b[g,k] = <x_b[gD:(g+1)D], C[k]>, the formula of
// split_manifold_lut_experiment/native/src/ojasx_lut_cpu.cpp:18-206 (LUT build
// :18-102, row gather :160-184, epilogue :178-182, CSR outliers :104-130) and
// of split_manifold_lut_experiment/engine/split_manifold_engine.py:185-250.
//
// Design (one kernel per call, K1+K2+K3 fused):
//  * Work tile = (row block of 256*RPT rows) x (slice of 16 groups) x (BT
//    tokens).  A workgroup owns a row block, a contiguous run of slices and a
//    token chunk.  For each slice it stages x for the slice's 16*D columns in
//    LDS, builds the slice's LUT (BT x 16 x 256 fp32, 16 KB per token) in LDS
//    from the 256 x D codebook (thread k owns centroid k), then every thread
//    gathers and sums the 16 LUT entries of each of its rows.
//  * Codes are repacked at handle creation into slice-major tiles
//    [S][Mp][16]: a thread reads its row's 16 codes of a slice with one 16-byte
//    load and a wave reads 1 KB contiguous.
//  * CSR outliers are re-bucketed at set_outliers() by (slice, row): a uint8
//    count per (slice,row), a uint32 base per (slice, 64-row group) and
//    (slice-local uint16 column, fp32 value) entries.  A lane finds its
//    entries by a wave prefix sum of the counts and reads x from the LDS
//    slice, so the outlier add is fused into the gather pass.
//  * When the row's slices are split over several workgroups, each writes a
//    partial (s_m * sum + outlier part) and the last workgroup to finish a row
//    block (atomic ticket) sums the partials in slice order and adds bias:
//    one launch, deterministic result.  The ticket counter is reset by that
//    workgroup, so the workspace needs no clearing between calls.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;        // threads per workgroup (4 waves)
constexpr int kGS = 16;         // groups per slice: 16 code bytes per row
constexpr int kRowAlign = 1024; // rows padded to the largest row block
constexpr int kCB = 256;        // centroids in the (zero-padded) codebook
}  // namespace

struct LinParams {
    const uint8_t *codes;    // [S][Mp][16]
    const uint8_t *ocnt;     // [S][Mp]
    const uint32_t *obase;   // [S][Mp/64]
    const uint16_t *ocol;    // [nnz] slice-local column
    const float *oval;       // [nnz]
    const float *codebook;   // [256][D]
    const float *scales;     // [M]
    const float *bias;       // [M] or null
    const void *x;           // [B][K]
    void *y;                 // [B][M]
    float *partial;          // [n_splits][B][Mp]
    unsigned *counters;      // [n_rb][token chunks]
    int K, M, Mp, D, S, B, spw, n_splits, has_out;
};

template <int BT, int RPT, int DT, typename T>
__global__ __launch_bounds__(kNT) void lut_gemv_kernel(LinParams p) {
    constexpr int DMAX = DT > 0 ? DT : 32;
    const int D = DT > 0 ? DT : p.D;
    const int slice_cols = kGS * D;
    extern __shared__ float smem[];
    float *lut = smem;                     // [BT][16][256]
    float *xs = smem + BT * kGS * kCB;     // [BT][16*D]
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int rb = blockIdx.x / p.n_splits;
    const int sp = blockIdx.x - rb * p.n_splits;
    const int t0 = blockIdx.y * BT;
    const int s0 = sp * p.spw;
    const int s1 = min(p.S, s0 + p.spw);
    const T *__restrict__ x = static_cast<const T *>(p.x);
    const int row0 = rb * kNT * RPT + tid;

    float cb[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) cb[d] = (d < D) ? p.codebook[tid * D + d] : 0.f;

    float acc[BT][RPT], oac[BT][RPT];
#pragma unroll
    for (int t = 0; t < BT; ++t)
#pragma unroll
        for (int j = 0; j < RPT; ++j) acc[t][j] = oac[t][j] = 0.f;

    for (int s = s0; s < s1; ++s) {
        uint4 cv[RPT];
        int oc[RPT];
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const size_t r = (size_t)s * p.Mp + row0 + j * kNT;
            cv[j] = *reinterpret_cast<const uint4 *>(p.codes + r * kGS);
            oc[j] = p.has_out ? p.ocnt[r] : 0;
        }
        for (int i = tid; i < BT * slice_cols; i += kNT) {
            const int t = i / slice_cols;
            const int c = i - t * slice_cols;
            const int tok = t0 + t;
            const int col = s * slice_cols + c;
            xs[i] = (tok < p.B && col < p.K) ? load_act(x, (size_t)tok * p.K + col) : 0.f;
        }
        __syncthreads();

        // K1: LUT[t][g][k = tid] = <x_t,g , C[k]>
#pragma unroll
        for (int t = 0; t < BT; ++t) {
#pragma unroll 4
            for (int g = 0; g < kGS; ++g) {
                const float *xg = xs + t * slice_cols + g * D;
                float dot = 0.f;
#pragma unroll
                for (int d = 0; d < DMAX; ++d)
                    if (d < D) dot = fmaf(xg[d], cb[d], dot);
                lut[(t * kGS + g) * kCB + tid] = dot;
            }
        }
        __syncthreads();

        // K2: gather-accumulate, groups in ascending order
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const uint32_t w4[4] = {cv[j].x, cv[j].y, cv[j].z, cv[j].w};
#pragma unroll
            for (int t = 0; t < BT; ++t) {
                const float *L = lut + t * kGS * kCB;
                float a = acc[t][j];
#pragma unroll
                for (int g = 0; g < kGS; ++g) {
                    const uint32_t code = (w4[g >> 2] >> ((g & 3) * 8)) & 0xffu;
                    a += L[g * kCB + code];
                }
                acc[t][j] = a;
            }
        }

        // K3: outliers of this slice (x from the LDS slice)
        if (p.has_out) {
#pragma unroll
            for (int j = 0; j < RPT; ++j) {
                const int c = oc[j];
                const int off = wave_excl_scan_u8(c);
                if (c) {
                    const int m = row0 + j * kNT;
                    const size_t base =
                        (size_t)p.obase[(size_t)s * (p.Mp >> 6) + (m >> 6)] + off;
                    for (int e = 0; e < c; ++e) {
                        const int col = p.ocol[base + e];
                        const float v = p.oval[base + e];
#pragma unroll
                        for (int t = 0; t < BT; ++t) oac[t][j] += v * xs[t * slice_cols + col];
                    }
                }
            }
        }
        __syncthreads();
    }

    T *y = static_cast<T *>(p.y);
    const bool split = p.n_splits > 1;
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        const int tok = t0 + t;
        if (tok >= p.B) break;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int m = row0 + j * kNT;
            if (m >= p.M) continue;
            const float sc = p.scales[m];
            if (!split) {
                float r = acc[t][j] * sc;
                if (p.bias) r += p.bias[m];
                r += oac[t][j];
                store_act(y, (size_t)tok * p.M + m, r);
            } else {
                p.partial[((size_t)sp * p.B + tok) * p.Mp + m] = acc[t][j] * sc + oac[t][j];
            }
        }
    }
    if (!split) return;

    // Ticket: the last workgroup of this (row block, token chunk) reduces.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned *ctr = p.counters + (size_t)rb * gridDim.y + blockIdx.y;
        const unsigned old = atomicAdd(ctr, 1u);
        s_last = (old == (unsigned)(p.n_splits - 1));
        if (s_last) atomicExch(ctr, 0u);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
#pragma unroll
    for (int t = 0; t < BT; ++t) {
        const int tok = t0 + t;
        if (tok >= p.B) break;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int m = row0 + j * kNT;
            if (m >= p.M) continue;
            float r = 0.f;
            for (int q = 0; q < p.n_splits; ++q)
                r += p.partial[((size_t)q * p.B + tok) * p.Mp + m];
            if (p.bias) r += p.bias[m];
            store_act(y, (size_t)tok * p.M + m, r);
        }
    }
}

// Standalone LUT build: one workgroup per (group, token), thread k computes
// LUT[b][g][k] = sum_d x[b][g*D+d] * C[k][d].
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
    DevBuf codes, codebook, scales, bias, ocnt, obase, ocol, oval;
    DevBuf partial, counters, xstage, ystage;
    size_t counters_n = 0;
    ~Linear() {
        for (DevBuf *b : {&codes, &codebook, &scales, &bias, &ocnt, &obase, &ocol, &oval,
                          &partial, &counters, &xstage, &ystage})
            b->release();
    }
};

namespace {

template <int BT, int RPT, int DT, typename T>
int launch_t(const LinParams &p, int grid_x, int grid_y, hipStream_t st) {
    const size_t lds = (size_t)BT * kGS * kCB * 4 + (size_t)BT * kGS * (DT > 0 ? DT : p.D) * 4;
    static bool attr_set = false;
    if (!attr_set) {
        OJX_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&lut_gemv_kernel<BT, RPT, DT, T>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    hipLaunchKernelGGL((lut_gemv_kernel<BT, RPT, DT, T>), dim3(grid_x, grid_y), dim3(kNT), lds, st, p);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

template <int BT, typename T>
int launch_bt(const LinParams &p, int gx, int gy, hipStream_t st) {
    return p.D == 16 ? launch_t<BT, 1, 16, T>(p, gx, gy, st) : launch_t<BT, 1, 0, T>(p, gx, gy, st);
}

template <typename T>
int launch_dtype(const LinParams &p, int bt, int gx, int gy, hipStream_t st) {
    switch (bt) {
        case 1: return launch_bt<1, T>(p, gx, gy, st);
        case 2: return launch_bt<2, T>(p, gx, gy, st);
        case 4: return launch_bt<4, T>(p, gx, gy, st);
        default: return launch_bt<8, T>(p, gx, gy, st);
    }
}

int forward(Linear *L, const void *x, void *y, int B, int dtype, hipStream_t st) {
    if (B <= 0) return OJASX_OK;
    if (dtype != OJASX_DTYPE_F32 && dtype != OJASX_DTYPE_BF16) {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    const int bt = B >= 8 ? 8 : B >= 3 ? 4 : B;
    const int chunks = (B + bt - 1) / bt;
    const int n_rb = (L->M + kNT - 1) / kNT;
    // Split the slices of a row over enough workgroups to fill the chip.
    const int base = n_rb * chunks;
    const int want = std::max(1, std::min(L->S, (512 + base - 1) / base));
    const int spw = (L->S + want - 1) / want;
    const int n_splits = (L->S + spw - 1) / spw;

    LinParams p{};
    p.codes = L->codes.as<uint8_t>();
    p.ocnt = L->ocnt.as<uint8_t>();
    p.obase = L->obase.as<uint32_t>();
    p.ocol = L->ocol.as<uint16_t>();
    p.oval = L->oval.as<float>();
    p.codebook = L->codebook.as<float>();
    p.scales = L->scales.as<float>();
    p.bias = L->has_bias ? L->bias.as<float>() : nullptr;
    p.x = x;
    p.y = y;
    p.K = L->K;
    p.M = L->M;
    p.Mp = L->Mp;
    p.D = L->D;
    p.S = L->S;
    p.B = B;
    p.spw = spw;
    p.n_splits = n_splits;
    p.has_out = L->nnz > 0;
    if (n_splits > 1) {
        int rc = L->partial.ensure((size_t)n_splits * B * L->Mp * sizeof(float));
        if (rc) return rc;
        const size_t nctr = (size_t)n_rb * chunks;
        if (nctr > L->counters_n) {
            rc = L->counters.ensure(nctr * sizeof(unsigned));
            if (rc) return rc;
            OJX_HIP(hipMemset(L->counters.ptr, 0, nctr * sizeof(unsigned)));
            L->counters_n = nctr;
        }
        p.partial = L->partial.as<float>();
        p.counters = L->counters.as<unsigned>();
    }
    const int gx = n_rb * n_splits;
    return dtype == OJASX_DTYPE_F32 ? launch_dtype<float>(p, bt, gx, chunks, st)
                                    : launch_dtype<__hip_bfloat16>(p, bt, gx, chunks, st);
}

}  // namespace

// Exposed for the stacked / MoE code paths and tests of the launch heuristics.
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
    const int slice_cols = kGS * L->D;
    std::vector<uint32_t> cnt((size_t)L->S * L->Mp, 0);
    for (int m = 0; m < L->M; ++m) {
        if (row_ptrs[m + 1] < row_ptrs[m]) {
            set_error("row_ptrs not monotone at row %d", m);
            return OJASX_ERR_INVALID;
        }
        for (int j = row_ptrs[m]; j < row_ptrs[m + 1]; ++j) {
            const int c = col_indices[j];
            if (c < 0 || c >= L->K) {
                set_error("outlier column %d out of range", c);
                return OJASX_ERR_INVALID;
            }
            if (++cnt[(size_t)(c / slice_cols) * L->Mp + m] > 255) {
                set_error("more than 255 outliers in one row slice");
                return OJASX_ERR_INVALID;
            }
        }
    }
    // Entry order: slice, row, CSR order.  base[s][grp] = first entry of the
    // 64-row group grp in slice s.
    const int ngrp = L->Mp / 64;
    std::vector<uint32_t> start((size_t)L->S * L->Mp);
    std::vector<uint32_t> base((size_t)L->S * ngrp);
    uint32_t off = 0;
    for (int s = 0; s < L->S; ++s)
        for (int m = 0; m < L->Mp; ++m) {
            const size_t i = (size_t)s * L->Mp + m;
            if ((m & 63) == 0) base[(size_t)s * ngrp + (m >> 6)] = off;
            start[i] = off;
            off += cnt[i];
        }
    std::vector<uint16_t> col((size_t)nnz);
    std::vector<float> val((size_t)nnz);
    std::vector<uint8_t> cnt8(cnt.size());
    for (size_t i = 0; i < cnt.size(); ++i) cnt8[i] = (uint8_t)cnt[i];
    for (int m = 0; m < L->M; ++m)
        for (int j = row_ptrs[m]; j < row_ptrs[m + 1]; ++j) {
            const int c = col_indices[j];
            const int s = c / slice_cols;
            const uint32_t at = start[(size_t)s * L->Mp + m]++;
            col[at] = (uint16_t)(c - s * slice_cols);
            val[at] = values[j];
        }
    int rc = upload(L->ocnt, cnt8.data(), cnt8.size());
    if (!rc) rc = upload(L->obase, base.data(), base.size() * sizeof(uint32_t));
    if (!rc) rc = upload(L->ocol, col.data(), col.size() * sizeof(uint16_t));
    if (!rc) rc = upload(L->oval, val.data(), val.size() * sizeof(float));
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
    if (L->nnz)
        b += L->nnz * 6 + (size_t)L->S * L->M + (size_t)L->S * (L->Mp / 64) * 4;
    return b;
}

OJASX_API void ojasx_destroy_linear(OjasxLinearHandle handle) {
    delete static_cast<Linear *>(handle);
}

}  // extern "C"

// lut_group.hip -- many independent LUT linears (block_dim 16, batch 1, fp32)
// in one launch: the sustained-throughput path.
//
// y_i[m] = (s_m * sum_g LUT_i[g, codes_i[m, g]] + bias_i[m]) + sum_j val_j x_i[col_j]
// for every instance i, with LUT_i[g, k] = <x_i[16g..16g+16), C_i[k]> (the
// formula and epilogue order of ojasx_lut_cpu.cpp:18-206).
//
// A single batch-1 call is latency-bound and runs lut_dec_kernel, which dots
// x with codebook rows read from LDS: 64 bytes of LDS per code byte, which
// caps it near 1.2 TB/s of code bytes on a full chip.  Here a workgroup owns
// 768 rows (3 per thread) of one instance and runs the MFMA-built LUT slice
// loop of lut_slices.h over the handles' slice-major code tiles: 4 bytes of
// LDS per code byte.  The MFMA build is a fixed 65,536 MACs per slice per
// workgroup, amortised over the workgroup's rows.  The grid is sized to run in
// one round: 72 VGPRs (one slice of codes in flight) and 27 KB of LDS give 6
// workgroups of 4 waves per CU, 1536 on the chip, and 160 x 2560->6912 is
// 1440 workgroups (measured 68.2 us; 4 rows per thread and two slices in
// flight: 1120 workgroups over 1024 places, 80.7 us; 5 or 6 rows: 74 or 84 us).
#include <algorithm>
#include <vector>

#include "common.h"
#include "lut_slices.h"

namespace ojx {

namespace {
constexpr int kPF = 1;                  // slices of codes in flight
constexpr int kGNT = 256;               // threads per workgroup (4 waves)
constexpr int kRPT = 3;                 // rows per thread
constexpr int kGRows = kGNT * kRPT;     // rows per workgroup
}  // namespace

__global__ __launch_bounds__(kGNT) __attribute__((amdgpu_waves_per_eu(6))) void lut_group_kernel(const GroupItem *__restrict__ items) {
    __shared__ float L[slices::kLutFloats];
    extern __shared__ float xs[];                     // [S * 256], zero past K
    const GroupItem it = items[blockIdx.y];
    const int base = (int)blockIdx.x * kGRows;
    if (base >= it.M) return;                         // whole workgroup
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int S = it.S, KS = S * 256;
    const bool outl = it.rowp != nullptr;

    // ---- round trip 1, L2-resident data first (vmcnt counts in order, so the
    //      x stores into LDS then do not wait for the HBM code loads): x, the
    //      codebook operands (wave w: centroid tiles 4w..4w+3), row bounds
    const int nx4 = KS / 4;
    float4 xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = min(tid + u * kGNT, nx4 - 1) * 4;
        xv[u] = gld(reinterpret_cast<const float4 *>(it.x + min(e, it.K - 4)));
        if (e >= it.K) xv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float bop[4][4];
    slices::load_cb_operands<4>(it.cb, w, lane, bop);
    int j0[kRPT] = {}, j1[kRPT] = {};               // the rows' CSR ranges
    if (outl) {
#pragma unroll
        for (int r2 = 0; r2 < kRPT; ++r2) {
            const int m = min(base + tid + kGNT * r2, it.M - 1);
            j0[r2] = gld(it.rowp + m);
            j1[r2] = gld(it.rowp + m + 1);
        }
    }
    // ---- then HBM: codes of slices 0..kPF-1 (rows past Mp clamp: loaded, never stored)
    int row[kRPT];
#pragma unroll
    for (int r2 = 0; r2 < kRPT; ++r2) row[r2] = min(base + tid + kGNT * r2, it.Mp - 1);
    uint4 ring[kPF][kRPT];
    slices::ring_start(it.codes, row, it.Mp, 0, S, ring);
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (tid + u * kGNT < nx4) reinterpret_cast<float4 *>(xs)[tid + u * kGNT] = xv[u];
    for (int i = tid + 4 * kGNT; i < nx4; i += kGNT) {   // K > 4096: the rest of x
        const int e = i * 4;
        reinterpret_cast<float4 *>(xs)[i] =
            e < it.K ? gld(reinterpret_cast<const float4 *>(it.x + e)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();

    float acc[kRPT] = {};
    slices::slice_loop<4, kRPT, false, kPF>(xs, L, bop, it.codes, row, it.Mp, 0, S, w, lane, ring, acc);

    // ---- epilogue: (s_m * sum + bias) + the row's CSR outliers (4 loads in
    //      flight; batching both rows' entries measured slower)
#pragma unroll
    for (int r2 = 0; r2 < kRPT; ++r2) {
        const int m = base + tid + kGNT * r2;
        if (m >= it.M) continue;
        float o = 0.f;
        if (outl) {
            int j = j0[r2];
            for (; j + 4 <= j1[r2]; j += 4) {
                int c[4];
                float v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    c[u] = gld(it.col + j + u);
                    v[u] = gld(it.val + j + u);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) o += v[u] * xs[c[u]];
            }
            for (; j < j1[r2]; ++j) o += gld(it.val + j) * xs[gld(it.col + j)];
        }
        float y = acc[r2] * gld(it.scales + m);
        if (it.bias) y += gld(it.bias + m);
        it.y[m] = y + o;
    }
}

// One tall batch-1 fp32 linear with the RMSNorm prologue (a decoder's gate/up
// and LM head): y[m] = ((s_m * r * sum_g LUT[g, code]) + bias_m) + r * outliers,
// r = 1 / sqrt(mean(x^2) + eps), with the LUT built from x * w (r factors out of
// the linear map, as in lut_dec_kernel's prologue).  Workgroup = 256 rows, one
// per thread, on the shared slice loop with two LUT buffers (few workgroups
// per CU: the build of slice s + 1 runs beside the gathers of s) and two
// slices of codes in flight.  For tall matrices this builds each LUT slice once
// per 256 rows instead of computing 64 bytes of codebook per code byte in
// place.
namespace {
constexpr int kTNT = 256;               // threads, one row each
constexpr int kTPF = 2;                 // slices of codes in flight
}  // namespace

__global__ __launch_bounds__(kTNT) void lut_tall_rms_kernel(GroupItem it, const float *w, float eps) {
    __shared__ float L[slices::lut_bytes(true) / sizeof(float)];
    extern __shared__ float xs[];                     // [S * 256]: x * w, zero past K
    __shared__ float red[kTNT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int base = (int)blockIdx.x * kTNT;
    const int S = it.S, KS = S * 256, nx4 = KS / 4;
    const bool outl = it.rowp != nullptr;
    // ---- round trip 1: x and w (L2), the codebook operands, the row's CSR
    //      range, scale and bias, then the codes of the first slices (HBM)
    float4 xv[4], wv4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = min(tid + u * kTNT, nx4 - 1) * 4;
        xv[u] = gld(reinterpret_cast<const float4 *>(it.x + min(e, it.K - 4)));
        wv4[u] = gld(reinterpret_cast<const float4 *>(w + min(e, it.K - 4)));
    }
    float bop[4][4];
    slices::load_cb_operands<4>(it.cb, wv, lane, bop);
    const int m = base + tid;
    const int mc = min(m, it.M - 1);
    int j0 = 0, j1 = 0;
    if (outl) {
        j0 = gld(it.rowp + mc);
        j1 = gld(it.rowp + mc + 1);
    }
    const float sc = gld(it.scales + mc);
    const float bs = it.bias ? gld(it.bias + mc) : 0.f;
    int row[1] = {min(m, it.Mp - 1)};                 // rows past M: loaded, never stored
    uint4 ring[kTPF][1];
    slices::ring_start(it.codes, row, it.Mp, 0, S, ring);
    // ---- x * w into LDS and the sum of x^2 (each element once)
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid + u * kTNT;
        if (i < nx4) {
            const bool in = i * 4 < it.K;
            const float4 v = in ? xv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
            ss += fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x)));
            reinterpret_cast<float4 *>(xs)[i] =
                make_float4(v.x * wv4[u].x, v.y * wv4[u].y, v.z * wv4[u].z, v.w * wv4[u].w);
        }
    }
    for (int i = tid + 4 * kTNT; i < nx4; i += kTNT) {   // K > 4096: the rest of x
        const int e = i * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f), g = v;
        if (e < it.K) {
            v = gld(reinterpret_cast<const float4 *>(it.x + e));
            g = gld(reinterpret_cast<const float4 *>(w + e));
        }
        ss += fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, v.x * v.x)));
        reinterpret_cast<float4 *>(xs)[i] = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
    }
    ss = wave_sum_f(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    const float rn = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)it.K + eps);

    float acc[1] = {0.f};
    slices::slice_loop<4, 1, true, kTPF>(xs, L, bop, it.codes, row, it.Mp, 0, S, wv, lane, ring, acc);

    // ---- epilogue: ((r * sum) * s_m + bias) + r * outliers (4 loads in flight)
    if (m >= it.M) return;
    float o = 0.f;
    if (outl) {
        int j = j0;
        for (; j + 4 <= j1; j += 4) {
            int c[4];
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c[u] = gld(it.col + j + u);
                v[u] = gld(it.val + j + u);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) o += v[u] * xs[c[u]];
        }
        for (; j < j1; ++j) o += gld(it.val + j) * xs[gld(it.col + j)];
    }
    float y = (acc[0] * rn) * sc;
    if (it.bias) y += bs;
    it.y[m] = y + o * rn;
}

int launch_tall_rms(const GroupItem &it, const float *w, float eps, hipStream_t st) {
    if ((reinterpret_cast<uintptr_t>(it.x) | reinterpret_cast<uintptr_t>(w)) & 15) {
        set_error("tall linear: 16-byte aligned x and norm weight needed");
        return OJASX_ERR_INVALID;
    }
    const size_t lds = (size_t)it.S * 256 * sizeof(float);
    static size_t granted = 0;
    int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&lut_tall_rms_kernel),
                            lds + slices::lut_bytes(true), &granted);
    if (rc) return rc;
    OJX_LAUNCH(lut_tall_rms_kernel, dim3((it.M + kTNT - 1) / kTNT), dim3(kTNT), lds, st, it, w, eps);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// Per host thread: the staged item array.
struct GroupWork {
    DevBuf items;
    std::vector<GroupItem> host;
    ~GroupWork() { items.release(); }
};
static thread_local GroupWork t_group;

}  // namespace ojx

extern "C" {

OJASX_API int ojasx_linear_forward_grouped_device(const OjasxLinearHandle *handles, int count,
                                                  const float *const *xs, float *const *ys,
                                                  void *stream) {
    using namespace ojx;
    if (!handles || !xs || !ys) return OJASX_ERR_NULL;
    if (count <= 0) return OJASX_OK;
    if (count > 65535) {
        set_error("at most 65535 linears per grouped call (got %d)", count);
        return OJASX_ERR_INVALID;
    }
    GroupWork &gw = t_group;
    gw.host.resize(count);
    int max_blocks = 0;
    size_t lds = 0;
    for (int i = 0; i < count; ++i) {
        if (!handles[i] || !xs[i] || !ys[i]) return OJASX_ERR_NULL;
        GroupItem &it = gw.host[i];
        int rc = linear_items(handles[i], &it);
        if (rc) return rc;
        if (reinterpret_cast<uintptr_t>(xs[i]) & 15) {
            set_error("grouped linear %d: x must be 16-byte aligned", i);
            return OJASX_ERR_INVALID;
        }
        it.x = xs[i];
        it.y = ys[i];
        max_blocks = std::max(max_blocks, (it.M + kGRows - 1) / kGRows);
        lds = std::max(lds, (size_t)it.S * 256 * sizeof(float));
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    int rc = gw.items.ensure(sizeof(GroupItem) * count);
    if (rc) return rc;
    OJX_HIP(hipMemcpyAsync(gw.items.ptr, gw.host.data(), sizeof(GroupItem) * count,
                           hipMemcpyHostToDevice, st));
    // the limit covers the static LUT buffers too (their sum passes 64 KB for K > 7000)
    static size_t granted = 0;
    rc = ensure_dyn_lds(reinterpret_cast<const void *>(&lut_group_kernel),
                        lds + slices::lut_bytes(false), &granted);
    if (rc) return rc;
    OJX_LAUNCH(lut_group_kernel, dim3(max_blocks, count), dim3(kGNT), lds, st,
               gw.items.as<GroupItem>());
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // extern "C"

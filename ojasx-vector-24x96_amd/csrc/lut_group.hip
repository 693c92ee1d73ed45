// lut_group.hip -- the grouped batch-1 LUT-GEMV entry point (its kernel is
// lut_bank_kernel in lut_bank.hip) and the tall RMSNorm linear of the decoder
// (lut_tall_rms_kernel, on the LUT slice loop of lut_slices.h).
#include <algorithm>
#include <vector>

#include "common.h"
#include "lut_slices.h"

namespace ojx {

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

__global__ __launch_bounds__(kTNT) void lut_tall_rms_kernel(GroupItem it, const float *w, float eps,
                                                          float2 *arg_part) {
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
    float o = 0.f;
    if (outl && m < it.M) {
        int j = j0;
        for (; j + 4 <= j1; j += 4) {
            int c[4];
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c[u] = gld(it.col16 + j + u);
                v[u] = gld(it.val + j + u);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) o += v[u] * xs[c[u]];
        }
        for (; j < j1; ++j) o += gld(it.val + j) * xs[gld(it.col16 + j)];
    }
    float y = (acc[0] * rn) * sc;
    if (it.bias) y += bs;
    y += o * rn;
    if (m < it.M) it.y[m] = y;
    if (arg_part) {
        // the workgroup's first maximum: strict > over rows in order, NaN and
        // -inf never taken
        const float v = (m < it.M && y > -INFINITY) ? y : -INFINITY;
        const float wm = wave_max_f(v);
        const int wi = wave_min_i(v > -INFINITY && v == wm ? m : 0x7fffffff);
        __shared__ float2 wpart[kTNT / 64];
        if (lane == 0) wpart[wv] = make_float2(wm, __int_as_float(wi));
        __syncthreads();
        if (tid == 0) {
            float2 b = wpart[0];
            for (int q = 1; q < kTNT / 64; ++q) {
                const float2 c = wpart[q];
                if (c.x > b.x) b = c;   // equal maxima: the lower wave holds the lower row
            }
            arg_part[blockIdx.x] = b;
        }
    }
}

int launch_tall_rms(const GroupItem &it, const float *w, float eps, hipStream_t st,
                    float2 *arg_part) {
    if ((reinterpret_cast<uintptr_t>(it.x) | reinterpret_cast<uintptr_t>(w)) & 15) {
        set_error("tall linear: 16-byte aligned x and norm weight needed");
        return OJASX_ERR_INVALID;
    }
    const size_t lds = (size_t)it.S * 256 * sizeof(float);
    static size_t granted = 0;
    int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&lut_tall_rms_kernel),
                            lds + slices::lut_bytes(true), &granted);
    if (rc) return rc;
    static_assert(kTNT == tall_rows_per_part(), "one argmax partial per workgroup");
    OJX_LAUNCH(lut_tall_rms_kernel, dim3((it.M + kTNT - 1) / kTNT), dim3(kTNT), lds, st, it, w, eps,
               arg_part);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// Per host thread: the item array and the bank kernel's work list ((item,
// first row) per 512-row block) of a call, staged for upload.  A call whose
// arrays equal the last upload (same handles, x and y pointers: the steady
// state of a serving loop) launches on that device copy without a new upload.
struct GroupWork {
    StagingRing ring;
    std::vector<unsigned char> host;
};
static thread_local GroupWork t_group;

// An item runs on the bank kernel when its staged input fits the LDS; the
// kernel reads the 16-bit copy of the outlier columns.
static bool on_bank(const GroupItem &it) { return bank_fits(it.K) && (!it.rowp || it.col16); }

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
    const size_t item_bytes = round_up(sizeof(GroupItem) * count, 16);
    gw.host.assign(item_bytes, 0);                   // padding bytes too, for the comparison
    GroupItem *host = reinterpret_cast<GroupItem *>(gw.host.data());
    int rc = OJASX_OK;
    int max_K = 0;
    std::vector<int> wide;                           // items whose K exceeds the bank kernel's LDS
    for (int i = 0; i < count; ++i) {
        if (!handles[i] || !xs[i] || !ys[i]) return OJASX_ERR_NULL;
        GroupItem &it = host[i];
        rc = linear_items(handles[i], &it);
        if (rc) return rc;
        if (reinterpret_cast<uintptr_t>(xs[i]) & 15) {
            set_error("grouped linear %d: x must be 16-byte aligned", i);
            return OJASX_ERR_INVALID;
        }
        it.x = xs[i];
        it.y = ys[i];
        if (on_bank(it)) max_K = std::max(max_K, it.K);
        else wide.push_back(i);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    // wide items run one by one on the single-linear path (in-place LUT
    // kernel, or the L2-LUT kernels beyond its LDS), on the same stream
    for (int i : wide) {
        rc = linear_forward(handles[i], xs[i], ys[i], 1, OJASX_DTYPE_F32, st);
        if (rc) return rc;
    }
    if (wide.size() == (size_t)count) return OJASX_OK;
    // the bank kernel's work list: every 512-row block of every other item, item-major
    int n_work = 0;
    for (int i = 0; i < count; ++i)
        if (on_bank(host[i])) n_work += (host[i].M + kBankRows - 1) / kBankRows;
    const size_t bytes = item_bytes + sizeof(int2) * (size_t)n_work;
    gw.host.resize(bytes);
    host = reinterpret_cast<GroupItem *>(gw.host.data());
    int2 *wl = reinterpret_cast<int2 *>(gw.host.data() + item_bytes);
    for (int i = 0, t = 0; i < count; ++i)
        if (on_bank(host[i]))
            for (int b = 0; b < host[i].M; b += kBankRows) wl[t++] = make_int2(i, b);
    void *staged = nullptr;
    rc = gw.ring.stage(gw.host.data(), bytes, true, st, &staged);
    if (rc) return rc;
    GroupItem *dev = static_cast<GroupItem *>(staged);
    const int2 *dev_work = reinterpret_cast<const int2 *>(static_cast<unsigned char *>(staged) + item_bytes);
    rc = launch_bank(dev, dev_work, n_work, max_K, st);
    if (rc) return rc;
    return gw.ring.launched(st);
}

}  // extern "C"

// common.h -- shared helpers of the gfx950 LUT engine (host + device).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "ojasx_lut_c_api.h"

namespace ojx {

// Thread-local message of the last failing C-ABI call.
void set_error(const char *fmt, ...);

// Map a HIP status to the C-ABI codes, recording a message.
int hip_fail(hipError_t e, const char *what);

#define OJX_HIP(call)                                           \
    do {                                                        \
        hipError_t _e = (call);                                 \
        if (_e != hipSuccess) return ::ojx::hip_fail(_e, #call); \
    } while (0)

// Device buffer owned by a handle.  Grows on request; never shrinks.
struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
    int ensure(size_t n);  // 0 or an error code
    void release();
    template <typename T> T *as() const { return static_cast<T *>(ptr); }
};

int upload(DevBuf &buf, const void *host, size_t n);  // ensure + memcpy

// The host-pointer entry points (the reference's synchronous C-ABI): a call
// copies its host inputs into this thread's pinned buffer, uploads them with
// one asynchronous copy on this thread's stream, runs its kernels there,
// downloads into the pinned buffer and synchronises that stream once (a
// pageable copy is a synchronous staging pass of its own).
struct HostIO {
    hipStream_t st = nullptr;
    unsigned char *pin = nullptr;
    size_t cap = 0;
    int reserve(size_t bytes);   // creates the stream on first use
    ~HostIO();
};
HostIO &host_io();   // the calling thread's

// Small per-call argument arrays (work lists, descriptors) staged for a
// launch: kSlots slots of pinned host memory and their device copies, so the
// upload is an asynchronous copy (a pageable source would make every call wait
// for it).  A slot is rewritten only after the event recorded behind the last
// launch that read it has completed, whatever stream the calls run on.  With
// reuse, a call whose bytes equal those of a slot uploaded on the same stream
// launches on that device copy without a new upload (callers that rotate over
// a few argument sets keep them resident).  One ring per host thread
// (thread_local).
struct StagingRing {
    static constexpr int kSlots = 4;
    DevBuf dev;                         // [kSlots][cap] bytes
    unsigned char *pinned = nullptr;    // [kSlots][cap] bytes
    size_t cap = 0;
    hipEvent_t ev[kSlots] = {};
    int next = 0, cur = -1;             // the slot of the current call
    size_t bytes_of[kSlots] = {};       // bytes of each slot's upload (0: none)
    hipStream_t stream_of[kSlots] = {}; // the stream each slot was uploaded on
    int reserve(size_t bytes);
    // Uploads bytes from host on st, or with reuse launches on a slot that
    // already holds them, uploaded on st (so the upload precedes the call's
    // launches); *dev_out is the device copy, valid for launches on st until
    // launched() is called.
    int stage(const void *host, size_t bytes, bool reuse, hipStream_t st, void **dev_out);
    // Records the current slot's event on st, behind the launches that read it.
    int launched(hipStream_t st);
    ~StagingRing();
};

// Optional per-kernel timing (ojasx_kernel_timing_*): when enabled, launches
// record start/stop events at the kernel's own begin and end
// (hipExtLaunchKernelGGL), kept per kernel name until the report.
bool timing_on();
void timing_events(const char *name, hipEvent_t *start, hipEvent_t *stop);

#define OJX_LAUNCH(kernel, grid, block, lds, st, ...)                                      \
    do {                                                                                    \
        if (::ojx::timing_on()) {                                                           \
            hipEvent_t _a = nullptr, _b = nullptr;                                          \
            ::ojx::timing_events(#kernel, &_a, &_b);                                        \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, st, _a, _b, 0, __VA_ARGS__);     \
        } else {                                                                            \
            hipLaunchKernelGGL(kernel, grid, block, lds, st, __VA_ARGS__);                  \
        }                                                                                   \
    } while (0)

// Linear handles (lut_linear.hip): shape, and the fused fp32 batch-1 forward
// with a prologue (0 none, 1 RMSNorm with weight w, 2 SwiGLU from a [2K] row)
// and an optional residual added to the output (may alias y).
int linear_shape(const void *h, int *K, int *M, int *D);
// One linear of a grouped launch (lut_group.hip).
struct GroupItem {
    const uint8_t *codes;     // [S][Mp][16]
    const uint8_t *codes_b;   // bank layout [ceil(M/64)][S32][32][64] (lut_bank.hip)
    const float *cb;          // [256][16]
    const void *cb3;          // the codebook split for the bank kernel (split_codebook_bf16x3)
    const float *scales;      // [M]
    const float *bias;        // [M] or null
    const int *rowp;          // [M+1] or null
    const int *col;
    const uint16_t *col16;    // the same columns in 16 bits (in_features <= 65536), or null
    const float *val;
    const float *x;           // [K], 16-byte aligned
    float *y;                 // [M]
    int K, M, Mp, S, S32;     // S32 = ceil(G / 32)
};
// A 256 x 16 fp32 codebook split exactly into three bf16 pieces per value
// (v = v1 + v2 + v3, v1 = bf16(v), v2 = bf16(v - v1), v3 = v - v1 - v2, each
// rounded to nearest even), laid out for the bank kernels' MFMA A operand:
// [centroid][half h][piece][dims 8h .. 8h + 7], 96 bytes per centroid.
constexpr size_t kCb3Bytes = 256 * 2 * 3 * 8 * 2;
void split_codebook_bf16x3(const float *cb, uint16_t *out);
int linear_items(const void *h, GroupItem *it);
// Grouped batch-1 LUT-GEMV with bank-aligned gathers (lut_bank.hip): items
// staged in device memory, work[t] = (item, first row of a 512-row block) in
// item-major order, max_K the largest input length.
constexpr int kBankRows = 512;
int launch_bank(const GroupItem *items_dev, const int2 *work_dev, int n_work, int max_K,
                hipStream_t st);
// Whether the bank kernels' LDS (64 KB of LUT plus the staged input pieces of
// K / 16 groups) fits a workgroup for input length K: K <= 16384.
bool bank_fits(int K);
// Bank layout of [M][G] codes: [row block of 64 rows][group][64 rows], 0 past M.
void pack_bank_codes(const uint8_t *codes, int M, int G, uint8_t *out);
inline size_t bank_codes_bytes(int M, int G) { return (size_t)((M + 63) / 64) * G * 64; }
// Readable bytes allocated after the last block: a partial last slice reads up
// to 31 groups x 64 bytes past its block.
constexpr size_t kBankSlack = 2048;
// MoE stages on the bank kernel (lut_bank.hip): the plan (routed pairs sorted
// by expert into work lists of (pair, 512-row block << 16 | expert); E at
// most 65535), then one launch per stage.
int launch_moe_plan(const int *idx, const float *w, int P, int E, int nb_gu, int nb_dn,
                    int2 *work_gu, int2 *work_dn, int *n_work, hipStream_t st);
struct MoEBankLaunch {
    const uint8_t *codes_b;     // [E][bank layout]
    size_t expert_bytes;
    const void *cb3;            // the split codebook (split_codebook_bf16x3)
    const float *scales;        // [E][M]
    const void *x;              // xs 0: [T][K] fp32, 1: bf16, 2: [P][2K] fp32 gate|up rows
    float *y;                   // [P][M]
    const int *idx;
    const float *w;             // slot weights (read by the direct mapping)
    const int2 *work;           // the plan's work list, or null: workgroup = (pair, row block)
    const int *n_work;          // device count of work entries
    int M, K, k, E, max_work, xs;   // direct mapping: max_work = pairs x row blocks
};
int launch_moe_bank(const MoEBankLaunch &l, hipStream_t st);
// A MoE stage with each group's input LUT built once for all its row blocks
// (lut_bank.hip, moe_resident_kernel): gate/up with groups = tokens and slots
// = k (inputs of at most 2048), down (xs 2) with groups = pairs and slots = 1
// (inputs of at most 1024).
bool moe_resident_fits(int K, int xs);
int launch_moe_resident(const MoEBankLaunch &l, int groups, int slots, hipStream_t st);
// One tall batch-1 fp32 linear with the RMSNorm prologue (lut_group.hip):
// it.x / it.y set, w the norm weight; both 16-byte aligned.  With arg_part
// set, workgroup b also writes arg_part[b] = (max, first row of it as the
// float's bits) over its 256 rows' outputs above -inf (NaN skipped; none: -inf
// and row INT_MAX): tall_rows_per_part() rows per partial.
int launch_tall_rms(const GroupItem &it, const float *w, float eps, hipStream_t st,
                    float2 *arg_part = nullptr);
constexpr int tall_rows_per_part() { return 256; }

// The block_dim-16 linear for many tokens on MFMA (lut_mm.hip): x [B][K] in
// dtype (fp32 16-byte aligned, or bf16), y [B][M] in dtype.
struct MmParams {
    const uint8_t *codes;   // [S][Mp][16]
    const float *cb;        // [256][16]
    const float *scales;    // [M]
    const float *bias;      // [M] or null
    const int *rowp;        // [M + 1] or null
    const int *col;
    const float *val;
    const void *x;
    void *y;
    int K, M, Mp, S, B;
    const void *cb3;        // the codebook's exact bf16 pieces (split_codebook_bf16x3)
};
int launch_mm(const MmParams &p, int dtype, hipStream_t st);
// One linear handle's forward of B tokens (dtype F32 or BF16) on st.
int linear_forward(void *h, const void *x, void *y, int B, int dtype, hipStream_t st);
int linear_forward_fused(void *h, const float *x, float *y, int pro, const float *w, float eps,
                         const float *res, hipStream_t st);
// The RMSNorm linear (prologue 1, no residual) of a decoder's LM head with the
// greedy pick's first stage: when it runs on the tall kernel, arg_part
// [ceil(M / tall_rows_per_part())] receives the per-workgroup maxima and
// *n_part their count; otherwise *n_part = 0 and the pick scans y.
int linear_forward_lm_head(void *h, const float *x, float *y, const float *w, float eps,
                           float2 *arg_part, int *n_part, hipStream_t st);

// Paged code-domain decode (lut_kv.hip) with the context length read on the
// device, *len_dev + len_add <= T_max; head dim 128, block dim 16; chunks of
// 64 * tpl tokens (tpl 1, 2 or 4; 0 picks by T_max); partials part_o
// [Hq][n][128] / part_ml [Hq][n][2], n = kv_device_len_chunks(T_max, tpl).
int kv_device_len_tpl(int T_max);
inline int kv_device_len_chunks(int T_max, int tpl) {
    if (tpl == 0) tpl = kv_device_len_tpl(T_max);
    return (T_max + 64 * tpl - 1) / (64 * tpl);
}
int kv_decode_device_len(const float *q, const uint8_t *kc, const float *ks, const uint8_t *vc,
                         const float *vs, const float *kcb, const float *vcb, const int *bt,
                         const int *len_dev, int len_add, int T_max, int P, int Hq, int Hkv,
                         float sf, float *part_o, float *part_ml, float *out, hipStream_t st,
                         int tpl = 0);
// The log-sum-exp merge of such partials alone (head dim 128): the first
// ceil((*len_dev + len_add) / chunk) chunks of a stride of stride_chunks
// slots, then, with extra set, the partial in the stride's last slot: out
// [Hq][128].
int kv_merge_device_len(const float *part_o, const float *part_ml, int stride_chunks, int chunk,
                        int Hq, const int *len_dev, int len_add, int extra, float *out,
                        hipStream_t st);

// LUT[b][g][k] = <x_b[gD:(g+1)D], C[k]> for g < Gp (0 for g >= G) and all 256
// centroids of the zero-padded codebook cb [256][D]; x [B][K] in dtype.
int launch_lut_build(const void *x, const float *cb, int B, int K, int D, int G, int Gp,
                     float *lut, int dtype, hipStream_t st);

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Raise a kernel's dynamic-LDS limit when a launch needs more than the 64 KB
// default (gfx950 has 160 KB per workgroup).  `granted` caches the last value.
inline int ensure_dyn_lds(const void *fn, size_t bytes, size_t *granted) {
    if (bytes <= 65536 || bytes <= *granted) return OJASX_OK;
    OJX_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    *granted = bytes;
    return OJASX_OK;
}

// ---- device helpers ------------------------------------------------------
// Load through a global-address-space pointer.  Pointers read from device
// memory (not kernel arguments) are otherwise generic, their loads become
// flat loads, and a flat load counts against the LDS counter too: every wait
// for an LDS result would then also wait for the loads still in flight.
template <typename T>
__device__ __forceinline__ T gld(const T *p) {
    typedef __attribute__((address_space(1))) const T global_t;
    return *reinterpret_cast<global_t *>(reinterpret_cast<uintptr_t>(p));
}
// 16-byte vectors: loaded as the compiler's own vector types (HIP's vector
// structs have no copy from the global address space).
__device__ __forceinline__ uint4 gld(const uint4 *p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = gld(reinterpret_cast<const v4u *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gld(const float4 *p) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    const v4f_t v = gld(reinterpret_cast<const v4f_t *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float load_act(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float load_act(const __hip_bfloat16 *p, size_t i) {
    return __bfloat162float(p[i]);
}
__device__ __forceinline__ float load_act(const __half *p, size_t i) { return __half2float(p[i]); }

// One LUT entry for any group width D: sum_{d < D} v[d] * row[d] in d order
// (the reference's scalar LUT loop), for the calling thread's codebook row.
// v (a group of D activations, zeros when !v_ok) is staged through xs, an
// LDS buffer of blockDim.x floats, blockDim.x values at a time; every thread
// of the workgroup must call it (it synchronises).
template <typename T>
__device__ __forceinline__ float staged_group_dot(const T *__restrict__ v, bool v_ok,
                                                  const float *__restrict__ row, int D,
                                                  float *xs) {
    const int nt = blockDim.x, tid = threadIdx.x;
    float dot = 0.f;
    for (int d0 = 0; d0 < D; d0 += nt) {
        const int n = min(nt, D - d0);
        __syncthreads();
        if (tid < n) xs[tid] = v_ok ? load_act(v, (size_t)d0 + tid) : 0.f;
        __syncthreads();
        for (int d = 0; d < n; ++d) dot = fmaf(xs[d], row[d0 + d], dot);
    }
    return dot;
}

// v rounded (to nearest even) to the element type of p and back to fp32:
// the result of a torch elementwise op on tensors of that type.
__device__ __forceinline__ float round_as(const float *, float v) { return v; }
__device__ __forceinline__ float round_as(const __hip_bfloat16 *, float v) {
    return __bfloat162float(__float2bfloat16(v));
}
__device__ __forceinline__ float round_as(const __half *, float v) {
    return __half2float(__float2half_rn(v));
}
// Four consecutive activations as fp32 (p + i must be 16-byte aligned for
// fp32, 8-byte aligned for bf16).
__device__ __forceinline__ float4 load4_act(const float *p, size_t i) {
    return *reinterpret_cast<const float4 *>(p + i);
}
__device__ __forceinline__ float4 load4_act(const __hip_bfloat16 *p, size_t i) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p + i);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                       __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

// Sum over the 4 lanes of a quad (DPP quad permutes, no LDS traffic).
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    return v;
}

// Wave64 reductions with DPP inside each 16-lane row (quad permutes, half
// mirror, mirror) and the 4 row leaders read into scalars; the result is
// uniform across the wave.  No LDS traffic.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, __int_as_float(dpp_i<0xB1>(__float_as_int(v))));   // quad_perm [1,0,3,2]
    v = fmaxf(v, __int_as_float(dpp_i<0x4E>(__float_as_int(v))));   // quad_perm [2,3,0,1]
    v = fmaxf(v, __int_as_float(dpp_i<0x141>(__float_as_int(v))));  // row_half_mirror
    v = fmaxf(v, __int_as_float(dpp_i<0x140>(__float_as_int(v))));  // row_mirror
    const int iv = __float_as_int(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_i<0xB1>(v));
    v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0x141>(v));
    v = min(v, dpp_i<0x140>(v));
    const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return min(min(a, b), min(c, d));
}
// Minima over the wave of N values per lane, the N reductions interleaved
// (independent DPP chains in one straight-line block); every lane gets them.
template <int N>
__device__ __forceinline__ void wave_min_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fminf(v[i], __int_as_float(dpp_i<0xB1>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fminf(v[i], __int_as_float(dpp_i<0x4E>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fminf(v[i], __int_as_float(dpp_i<0x141>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fminf(v[i], __int_as_float(dpp_i<0x140>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int iv = __float_as_int(v[i]);
        const float a = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
        const float b = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
        const float c = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
        const float d = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
        v[i] = fminf(fminf(a, b), fminf(c, d));
    }
}
template <int N>
__device__ __forceinline__ void wave_min_n(int (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = min(v[i], dpp_i<0xB1>(v[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = min(v[i], dpp_i<0x4E>(v[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = min(v[i], dpp_i<0x141>(v[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = min(v[i], dpp_i<0x140>(v[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int a = __builtin_amdgcn_readlane(v[i], 0), b = __builtin_amdgcn_readlane(v[i], 16);
        const int c = __builtin_amdgcn_readlane(v[i], 32), d = __builtin_amdgcn_readlane(v[i], 48);
        v[i] = min(min(a, b), min(c, d));
    }
}

// Maxima / sums over the wave of N values per lane, interleaved as in
// wave_min_n; every lane gets them.
template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<0xB1>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<0x4E>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<0x141>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], __int_as_float(dpp_i<0x140>(__float_as_int(v[i]))));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int iv = __float_as_int(v[i]);
        const float a = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
        const float b = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
        const float c = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
        const float d = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
        v[i] = fmaxf(fmaxf(a, b), fmaxf(c, d));
    }
}
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += __int_as_float(dpp_i<0xB1>(__float_as_int(v[i])));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += __int_as_float(dpp_i<0x4E>(__float_as_int(v[i])));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += __int_as_float(dpp_i<0x141>(__float_as_int(v[i])));
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += __int_as_float(dpp_i<0x140>(__float_as_int(v[i])));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int iv = __float_as_int(v[i]);
        const float a = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
        const float b = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
        const float c = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
        const float d = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
        v[i] = (a + b) + (c + d);
    }
}

// Exact three-way bf16 split of fp32 values and the 32 x 32 x 16 MFMA tile
// over it.  v = v1 + v2 + v3 exactly: v1 = bf16(v), v2 = bf16(v - v1),
// v3 = v - v1 - v2 (an fp32 value has 24 significant bits, each bf16 piece
// takes 8; the remainders are exact in fp32).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ void split3_bf16(const float (&v)[8], bf16x8_t (&p)[3]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const __bf16 h1 = (__bf16)v[i];
        const float r1 = v[i] - (float)h1;
        const __bf16 h2 = (__bf16)r1;
        p[0][i] = h1;
        p[1][i] = h2;
        p[2][i] = (__bf16)(r1 - (float)h2);
    }
}
// A[32 x 16] . B[16 x 32] on v_mfma_f32_32x32x16_bf16 with A = a1 + a2 + a3
// and B = b1 + b2 + b3: the six products a_i b_j with i + j <= 4 (each exact
// in fp32) accumulated in fp32, smallest first; the three left out are below
// 2^-24 of the result.  Lane (h = lane / 32, n = lane % 32) supplies row n of
// A and column n of B, input dimensions 8h .. 8h + 7 of both; its result
// value r is row 8 (r / 4) + 4 h + r % 4 of column n.
__device__ __forceinline__ f32x16_t mfma32_bf16x3(const bf16x8_t (&a)[3], const bf16x8_t (&b)[3]) {
    f32x16_t d = {};
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], d, 0, 0, 0);
    return d;
}

// A 256 x 16 fp32 codebook in LDS as 4 float4 per row, float4 w of row r at
// slot r * 4 + (w ^ ((r >> 1) & 3)).  A row is 16 banks long, so without the
// swizzle float4 w of every row falls in one of two 4-bank groups and lanes
// reading rows at random collide; with it they spread over all eight.
__device__ __forceinline__ int cb_slot(int r, int w) { return r * 4 + (w ^ ((r >> 1) & 3)); }

__device__ __forceinline__ float wave_sum_f(float v) {
    v += __int_as_float(dpp_i<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp_i<0x140>(__float_as_int(v)));
    const int iv = __float_as_int(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(iv, 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(iv, 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(iv, 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(iv, 48));
    return (a + b) + (c + d);
}

__device__ __forceinline__ void store_act(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_act(__hip_bfloat16 *p, size_t i, float v) {
    p[i] = __float2bfloat16(v);
}
__device__ __forceinline__ void store_act(__half *p, size_t i, float v) { p[i] = __float2half_rn(v); }
__device__ __forceinline__ void store_act(double *p, size_t i, float v) { p[i] = (double)v; }

// Copy n activations (converted to fp32) from global memory to LDS with all
// of a thread's loads in flight before the first LDS store: loads and stores
// use clamped indices, so the code is branch-free (out-of-range lanes rewrite
// the last element with its own value) and the loop body is
// one memory round trip for up to NT*4*16 elements (fp32 rows use 16-byte
// loads when 16-byte aligned).  Runtime-trip-count copy loops otherwise
// serialise one round trip per element a thread copies.
template <int NT, int U = 16>
__device__ __forceinline__ void stage_to_lds(float *dst, const float *src, int n) {
    if (((reinterpret_cast<uintptr_t>(src) & 15) == 0) && (n & 3) == 0) {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        const int n4 = n >> 2;
        for (int b = threadIdx.x; b < n4; b += NT * U) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = s4[min(b + u * NT, n4 - 1)];
#pragma unroll
            for (int u = 0; u < U; ++u) reinterpret_cast<float4 *>(dst)[min(b + u * NT, n4 - 1)] = v[u];
        }
        return;
    }
    for (int b = threadIdx.x; b < n; b += NT * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = src[min(b + u * NT, n - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) dst[min(b + u * NT, n - 1)] = v[u];
    }
}

template <int NT, int U = 16>
__device__ __forceinline__ void stage_to_lds(float *dst, const __hip_bfloat16 *src, int n) {
    for (int b = threadIdx.x; b < n; b += NT * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __bfloat162float(src[min(b + u * NT, n - 1)]);
#pragma unroll
        for (int u = 0; u < U; ++u) dst[min(b + u * NT, n - 1)] = v[u];
    }
}

}  // namespace ojx

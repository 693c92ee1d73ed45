// attn_stream.hip -- exact attention over streamed K/V tiles with fp64
// online-softmax state: OnlineSoftmaxBlockAttention.forward_stream
// (ojasx_24x96/long_context.py:92-176) on gfx950, for tiles in fp32, bf16,
// fp16 or fp64, and for the int8 pages of PagedCompressedKVCache (per-token
// fp16 scales, long_context.py:212-267) dequantised in registers.
//
// State per query row (b, h, s) of [B][Hq][Sq], in fp64:
//   [q (D) | acc (D) | m | l]
// the reference's (m_i, l_i, acc_o) (:117-119) plus the query converted once.
// A query row of head h reads kv head h / (Hq / Hkv) (the reference's
// _expand_kv_heads, :80-89); the rows of one kv head, (h, s) in order, are
// contiguous in the state.
//
// One update call folds a list of tiles, in order, into the state:
//  * attn_tile_kernel -- workgroup = (chunk of up to 256 tokens of one tile,
//    batch x kv head, block of RB rows of that kv head's query rows).
//    Scores: thread t owns token t, s_r = (<q_r, k_t> * kscale_t) * scale in
//    fp64 (k_t converted exactly; q_r read at uniform addresses, so scalar
//    operands), -inf where the causal mask hides the key (key position >
//    query position, :133-139).  Chunk maximum m_c, p = exp(s - m_c) with
//    p = 0 for -inf scores (the reference's guard, :144-156), l_c = sum p.
//    Values: thread (4 dims, token phase) accumulates p * vscale_t * v_t of
//    every row over its tokens (int8 v: at head_dim 128 each thread's 32
//    words loaded into registers at the start, otherwise the rows staged in
//    LDS by coalesced loads issued before the scores); the chunk's
//    (acc, m_c, l_c) go to a partial slot.
//  * attn_merge_kernel -- per query row, the state and the partials in chunk
//    order merged as the reference merges tiles (:141-163): m = max of all,
//    each part scaled by exp(m_part - m) (0 for m_part = -inf), l and acc
//    summed in order.
// Finalize: out = acc / l (l = 0 -> 1, :165-166), rounded to the query's type
// as torch's .to() rounds fp64 (through fp32 for bf16 and fp16), and
// lse = m + log(l) per row (:167).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kANT = 256;   // threads per tile workgroup
constexpr int kACH = 256;   // tokens per chunk: one per thread in the score phase
constexpr int kAMaxD = 256;
constexpr size_t kPartCap = size_t(256) << 20;   // partial bytes per launch round

enum { KV_F32 = 0, KV_BF16 = 1, KV_F16 = 2, KV_F64 = 3, KV_INT8 = 4 };

struct AttnTile {           // element strides (k and v share them), scales' strides
    const void *k, *v;
    const __half *ks, *vs;
    long long n, sb, sh, st, ssb, ssh, sst;
};
struct AttnWork {
    int tile, t0, n, pad;
    long long pos;          // stream position of token t0
};
struct AttnParams {
    const AttnTile *tiles;
    const AttnWork *work;   // this round's work items
    const double *state;    // [rows][2D + 2]
    double *part;           // [n_work][rows][D + 2]
    long long qsp;          // query_start_pos
    double scale;
    int Hkv, R, Sq, D, rows, causal;
};

template <int KT> struct Elem;
template <> struct Elem<KV_F32> { typedef float T; };
template <> struct Elem<KV_BF16> { typedef __hip_bfloat16 T; };
template <> struct Elem<KV_F16> { typedef __half T; };
template <> struct Elem<KV_F64> { typedef double T; };
template <> struct Elem<KV_INT8> { typedef int8_t T; };

__device__ __forceinline__ double to_d(float v) { return (double)v; }
__device__ __forceinline__ double to_d(double v) { return v; }
__device__ __forceinline__ double to_d(__hip_bfloat16 v) { return (double)__bfloat162float(v); }
__device__ __forceinline__ double to_d(__half v) { return (double)__half2float(v); }
__device__ __forceinline__ double to_d(int8_t v) { return (double)v; }

// n consecutive elements at p (aligned to n elements, at most 16 bytes) as fp64.
template <typename T, int N>
__device__ __forceinline__ void load_run(const T *p, double (&o)[N]) {
    constexpr int kBytes = N * (int)sizeof(T);
    constexpr int kPiece = kBytes < 16 ? kBytes : 16;   // bytes per load
    constexpr int kPer = kPiece / (int)sizeof(T);       // elements per load
    static_assert(kBytes % kPiece == 0, "whole loads");
#pragma unroll
    for (int u = 0; u < N / kPer; ++u) {
        T e[kPer];
        if constexpr (kPiece == 16) {
            typedef unsigned int v4u __attribute__((ext_vector_type(4)));
            const v4u w = gld(reinterpret_cast<const v4u *>(p + u * kPer));
            __builtin_memcpy(e, &w, 16);
        } else if constexpr (kPiece == 8) {
            typedef unsigned int v2u __attribute__((ext_vector_type(2)));
            const v2u w = gld(reinterpret_cast<const v2u *>(p + u * kPer));
            __builtin_memcpy(e, &w, 8);
        } else {
            static_assert(kPiece == 4, "4, 8 or 16 bytes");
            const uint32_t w = gld(reinterpret_cast<const uint32_t *>(p + u * kPer));
            __builtin_memcpy(e, &w, 4);
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) o[u * kPer + i] = to_d(e[i]);
    }
}

__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
}  // namespace

template <int KT, int RB>
__global__ __launch_bounds__(kANT) void attn_tile_kernel(AttnParams p) {
    typedef typename Elem<KT>::T T;
    constexpr bool kI8 = KT == KV_INT8;
    __shared__ double pv[RB][kACH];           // p * vscale per row and token
    __shared__ double red[kANT][4];           // value-phase partials across token phases
    __shared__ double rm[4][RB], rl[4][RB];   // per-wave maxima and sums
    extern __shared__ uint4 vstage[];         // int8 tiles: the chunk's v rows [n][D] bytes
    const AttnWork wk = p.work[blockIdx.x];
    const AttnTile tl = p.tiles[wk.tile];
    const int bh = blockIdx.y, b = bh / p.Hkv, h = bh - b * p.Hkv;
    const int r0 = blockIdx.z * RB;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = p.D, SW = 2 * D + 2;
    const bool valid = tid < wk.n;
    const long long t = wk.t0 + min(tid, wk.n - 1);
    const T *kp = static_cast<const T *>(tl.k) + b * tl.sb + h * tl.sh + t * tl.st;
    const T *vbase = static_cast<const T *>(tl.v) + b * tl.sb + h * tl.sh + (long long)wk.t0 * tl.st;

    // int8: the chunk's v rows staged through LDS in 16-byte pieces (piece i =
    // bytes 16 i.. of row-major [n][D], D a multiple of 16), loads issued
    // before the scores so they complete under them; 8 per thread per round
    constexpr int kVP = 8;
    const int n_pieces = kI8 ? wk.n * D / 16 : 0;
    uint4 vr[kVP];
    auto v_load = [&](int round) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kVP; ++u) {
            const int i = min(round * kVP * kANT + u * kANT + tid, n_pieces - 1);
            const int row = (16 * i) / D, col = (16 * i) % D;
            vr[u] = gld(reinterpret_cast<const uint4 *>(
                reinterpret_cast<const int8_t *>(vbase) + row * tl.st + col));
        }
    };
    auto v_store = [&](int round) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kVP; ++u) {
            const int i = round * kVP * kANT + u * kANT + tid;
            if (i < n_pieces) vstage[i] = vr[u];
        }
    };
    // int8 with head_dim 128: each value thread (dims 4dq.., phase ts) loads
    // its 32 v words (tokens ts + 8 i) into registers at the start instead --
    // no LDS stage, so more workgroups fit a CU and every load of the chunk is
    // in flight under the scores
    constexpr int kVW = 32;
    const bool vreg = kI8 && D == 128;
    uint32_t vw[kI8 ? kVW : 1];
    if constexpr (kI8) {
        if (vreg) {
            const int dq = tid & 31, ts = tid >> 5;
#pragma unroll
            for (int i = 0; i < kVW; ++i) {
                const int tt = min(ts + 8 * i, wk.n - 1);
                vw[i] = gld(reinterpret_cast<const uint32_t *>(
                    reinterpret_cast<const int8_t *>(vbase) + tt * tl.st + 4 * dq));
            }
        } else {
            v_load(0);
        }
    }

    // ---- scores of the thread's token against the block's rows: the row's
    //      16-byte pieces loaded 8 at a time (all of a 128-dim int8 row at
    //      once), then the FMAs
    double s[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) s[r] = 0.0;
    const double *qb = p.state + (size_t)bh * p.R * SW;
    constexpr int kE = 16 / (int)sizeof(T);           // elements per piece
    for (int d0 = 0; d0 < D; d0 += 8 * kE) {
        uint4 raw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            raw[u] = gld(reinterpret_cast<const uint4 *>(kp + min(d0 + u * kE, D - kE)));
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (d0 + u * kE >= D) break;
            T e[kE];
            __builtin_memcpy(e, &raw[u], 16);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const double *qr = qb + (size_t)min(r0 + r, p.R - 1) * SW + d0 + u * kE;
#pragma unroll
                for (int j = 0; j < kE; ++j) s[r] = fma(qr[j], to_d(e[j]), s[r]);
            }
        }
    }
    double ksc = 1.0, vsc = 1.0;
    if constexpr (kI8) {
        ksc = (double)__half2float(tl.ks[b * tl.ssb + h * tl.ssh + t * tl.sst]);
        vsc = (double)__half2float(tl.vs[b * tl.ssb + h * tl.ssh + t * tl.sst]);
    }
    const long long kpos = wk.pos + tid;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int row = r0 + r;
        const long long qpos = p.qsp + row % p.Sq;
        const bool hide = !valid || row >= p.R || (p.causal && kpos > qpos);
        s[r] = hide ? -INFINITY : (s[r] * ksc) * p.scale;
    }
    // ---- chunk maximum, p = exp(s - m_c), chunk sum
    double mc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const double m = wave_max_d(s[r]);
        if (lane == 0) rm[w][r] = m;
    }
    if constexpr (kI8) {
        if (!vreg) {
            v_store(0);
            for (int round = 1; round * kVP * kANT < n_pieces; ++round) {
                v_load(round);
                v_store(round);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r) mc[r] = fmax(fmax(rm[0][r], rm[1][r]), fmax(rm[2][r], rm[3][r]));
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const double safe = isinf(mc[r]) ? 0.0 : mc[r];
        const double pr = isinf(s[r]) ? 0.0 : exp(s[r] - safe);
        pv[r][tid] = pr * vsc;
        const double l = wave_sum_d(pr);
        if (lane == 0) rl[w][r] = l;
    }
    __syncthreads();

    // ---- values: thread (dims 4dq..4dq+3, token phase ts) accumulates all RB
    //      rows, each v element converted once
    const int NQ = D >> 2, TS = kANT / NQ;
    const int dq = tid % NQ, ts = tid / NQ;
    double a4[RB][4];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) a4[r][j] = 0.0;
    if (vreg) {
        // tokens past n: p = 0 (their v words repeat token n - 1's)
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
            const int tt = ts + 8 * i;
            const uint32_t u = vw[i];
            double v4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v4[j] = (double)(int8_t)(u >> (8 * j));
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const double wgt = pv[r][tt];
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[r][j] = fma(wgt, v4[j], a4[r][j]);
            }
        }
    } else if (ts < TS) {
        const uint32_t *vs32 = reinterpret_cast<const uint32_t *>(vstage) + dq;
        const T *vp = vbase + 4 * dq;
        for (int tt = ts; tt < wk.n; tt += TS) {
            double v4[4];
            if constexpr (kI8) {
                const uint32_t u = vs32[tt * NQ];
#pragma unroll
                for (int j = 0; j < 4; ++j) v4[j] = (double)(int8_t)(u >> (8 * j));
            } else {
                load_run<T, 4>(vp + tt * tl.st, v4);
            }
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const double wgt = pv[r][tt];
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[r][j] = fma(wgt, v4[j], a4[r][j]);
            }
        }
    }
    // the token phases summed in order, one row at a time through LDS
    const size_t slot0 = ((size_t)blockIdx.x * p.rows + (size_t)bh * p.R + r0) * (D + 2);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[tid][j] = a4[r][j];
        __syncthreads();
        if (ts == 0 && r0 + r < p.R) {
            double o[4] = {a4[r][0], a4[r][1], a4[r][2], a4[r][3]};
            for (int u = 1; u < TS; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] += red[tid + u * NQ][j];
#pragma unroll
            for (int j = 0; j < 4; ++j) p.part[slot0 + (size_t)r * (D + 2) + 4 * dq + j] = o[j];
        }
        __syncthreads();
    }
    if (tid < RB && r0 + tid < p.R) {
        const size_t sl = slot0 + (size_t)tid * (D + 2);
        double lsum = 0.0;
        for (int u = 0; u < 4; ++u) lsum += rl[u][tid];
        double m = -INFINITY;
        for (int u = 0; u < 4; ++u) m = fmax(m, rm[u][tid]);
        p.part[sl + D] = m;
        p.part[sl + D + 1] = lsum;
    }
}

// State row `blockIdx.x` <- the state merged with the n partials: the maximum
// over all, then thread (4 dims dq, phase ph) sums f_i * acc_i over partials
// i = ph, ph + PH, ... (f_i = exp(m_i - m), 0 for m_i = -inf), and the phases
// are summed in order -- a fixed order, so results are deterministic.
__global__ __launch_bounds__(kANT) void attn_merge_kernel(double *state, const double *part,
                                                          int n, int rows, int D) {
    __shared__ double red[kANT][4];
    __shared__ double redl[kANT];
    __shared__ double wmax[kANT / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    double *st = state + (size_t)row * (2 * D + 2);
    const double *pp = part + (size_t)row * (D + 2);
    const size_t stride = (size_t)rows * (D + 2);
    const double ms = st[2 * D], ls = st[2 * D + 1];
    double mx = ms;
    for (int i = tid; i < n; i += kANT) mx = fmax(mx, pp[i * stride + D]);
    mx = wave_max_d(mx);
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmax(fmax(wmax[0], wmax[1]), fmax(wmax[2], wmax[3]));
    const double safe = isinf(mx) ? 0.0 : mx;
    const int NQ = D >> 2, PH = kANT / NQ;
    const int dq = tid % NQ, ph = tid / NQ;
    double a4[4] = {0.0, 0.0, 0.0, 0.0}, l = 0.0;
    if (ph < PH) {
        // 4 partials per step, their loads issued together (clamped indices;
        // the repeats past n are not added)
        constexpr int kU = 4;
        for (int i0 = ph; i0 < n; i0 += kU * PH) {
            double mi[kU], li[kU], v[kU][4];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const double *pi = pp + (size_t)min(i0 + u * PH, n - 1) * stride;
                mi[u] = pi[D];
                li[u] = pi[D + 1];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[u][j] = pi[4 * dq + j];
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                if (i0 + u * PH >= n) break;
                const double f = isinf(mi[u]) ? 0.0 : exp(mi[u] - safe);
                l = fma(f, li[u], l);
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[j] = fma(f, v[u][j], a4[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) red[tid][j] = a4[j];
    redl[tid] = l;
    __syncthreads();                          // every thread has read the old state's m and l
    const double alpha = isinf(ms) ? 0.0 : exp(ms - safe);
    if (ph == 0) {
        double acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = alpha * st[D + 4 * dq + j];
        for (int u = 0; u < PH; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] += red[u * NQ + dq][j];
#pragma unroll
        for (int j = 0; j < 4; ++j) st[D + 4 * dq + j] = acc[j];
    }
    if (tid == 0) {
        double lt = alpha * ls;
        for (int u = 0; u < PH; ++u) lt += redl[u * NQ];
        st[2 * D] = mx;
        st[2 * D + 1] = lt;
    }
}

template <typename T>
__global__ __launch_bounds__(kAMaxD) void attn_init_kernel(double *state, const T *q, int D) {
    const int row = blockIdx.x, d = threadIdx.x;
    double *st = state + (size_t)row * (2 * D + 2);
    if (d < D) {
        st[d] = to_d(q[(size_t)row * D + d]);
        st[D + d] = 0.0;
    }
    if (d == 0) {
        st[2 * D] = -INFINITY;
        st[2 * D + 1] = 0.0;
    }
}

__device__ __forceinline__ void store_out(float *o, size_t i, double v) { o[i] = (float)v; }
__device__ __forceinline__ void store_out(double *o, size_t i, double v) { o[i] = v; }
__device__ __forceinline__ void store_out(__hip_bfloat16 *o, size_t i, double v) {
    o[i] = __float2bfloat16((float)v);
}
__device__ __forceinline__ void store_out(__half *o, size_t i, double v) {
    o[i] = __float2half_rn((float)v);
}

template <typename T>
__global__ __launch_bounds__(kAMaxD) void attn_finalize_kernel(const double *state, T *out,
                                                               double *lse, int D) {
    const int row = blockIdx.x, d = threadIdx.x;
    const double *st = state + (size_t)row * (2 * D + 2);
    const double l = st[2 * D + 1];
    const double sl = l > 0.0 ? l : 1.0;
    if (d < D) store_out(out, (size_t)row * D + d, st[D + d] / sl);
    if (d == 0 && lse) lse[row] = st[2 * D] + log(sl);
}

namespace {
struct AttnStage {
    StagingRing ring;
    DevBuf part;
    std::vector<unsigned char> host;
};
thread_local AttnStage t_attn;

int elem_bytes(int kind) {
    switch (kind) {
        case KV_F32: return 4;
        case KV_BF16: case KV_F16: return 2;
        case KV_F64: return 8;
        case KV_INT8: return 1;
    }
    return 0;
}

int check_rows(int rows, int D) {
    if (rows <= 0 || rows > (1 << 30)) {
        set_error("attention stream: %d query rows (1 .. 2^30)", rows);
        return OJASX_ERR_INVALID;
    }
    if (D <= 0 || D > kAMaxD || D % 8) {
        set_error("attention stream: head_dim %d (a multiple of 8, at most %d)", D, kAMaxD);
        return OJASX_ERR_INVALID;
    }
    return OJASX_OK;
}

template <int KT>
int launch_tiles(const AttnParams &p, int n_work, int B, int RB, hipStream_t st) {
    const dim3 grid(n_work, B * p.Hkv, (p.R + RB - 1) / RB);
    // int8 v rows staged in LDS (at most 64 KB), except at head_dim 128 (registers)
    const size_t lds = KT == KV_INT8 && p.D != 128 ? (size_t)kACH * p.D : 0;
    const void *fn = RB == 1   ? reinterpret_cast<const void *>(&attn_tile_kernel<KT, 1>)
                     : RB == 2 ? reinterpret_cast<const void *>(&attn_tile_kernel<KT, 2>)
                     : RB == 4 ? reinterpret_cast<const void *>(&attn_tile_kernel<KT, 4>)
                               : reinterpret_cast<const void *>(&attn_tile_kernel<KT, 8>);
    // The limit bounds the dynamic part; the default admits 64 KB in total
    // with the static arrays, so it is raised whenever the v rows are staged.
    static size_t granted[4] = {};
    size_t &g = granted[RB == 1 ? 0 : RB == 2 ? 1 : RB == 4 ? 2 : 3];
    if (lds > g) {
        OJX_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        g = lds;
    }
    switch (RB) {
        case 1: OJX_LAUNCH((attn_tile_kernel<KT, 1>), grid, dim3(kANT), lds, st, p); break;
        case 2: OJX_LAUNCH((attn_tile_kernel<KT, 2>), grid, dim3(kANT), lds, st, p); break;
        case 4: OJX_LAUNCH((attn_tile_kernel<KT, 4>), grid, dim3(kANT), lds, st, p); break;
        default: OJX_LAUNCH((attn_tile_kernel<KT, 8>), grid, dim3(kANT), lds, st, p); break;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}
}  // namespace

}  // namespace ojx

extern "C" {

OJASX_API int ojasx_attention_stream_init_device(double *state, const void *q, int q_dtype,
                                                 int rows, int head_dim, void *stream) {
    using namespace ojx;
    if (!state || !q) return OJASX_ERR_NULL;
    int rc = check_rows(rows, head_dim);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(rows), block(round_up(head_dim, 64));
    switch (q_dtype) {
        case OJASX_DTYPE_F32:
            OJX_LAUNCH(attn_init_kernel<float>, grid, block, 0, st, state, static_cast<const float *>(q), head_dim);
            break;
        case OJASX_DTYPE_BF16:
            OJX_LAUNCH(attn_init_kernel<__hip_bfloat16>, grid, block, 0, st, state,
                       static_cast<const __hip_bfloat16 *>(q), head_dim);
            break;
        case OJASX_DTYPE_F16:
            OJX_LAUNCH(attn_init_kernel<__half>, grid, block, 0, st, state, static_cast<const __half *>(q), head_dim);
            break;
        case OJASX_DTYPE_F64:
            OJX_LAUNCH(attn_init_kernel<double>, grid, block, 0, st, state, static_cast<const double *>(q), head_dim);
            break;
        default:
            set_error("attention stream: query dtype %d (F32, BF16, F16 or F64)", q_dtype);
            return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API int ojasx_attention_stream_update_device(double *state, int batch, int num_heads,
                                                   int num_kv_heads, int q_len, int head_dim,
                                                   const OjasxAttnTile *tiles, int n_tiles,
                                                   int kv_dtype, int causal,
                                                   long long query_start_pos, long long kv_offset,
                                                   double scale, void *stream) {
    using namespace ojx;
    if (!state || (n_tiles > 0 && !tiles)) return OJASX_ERR_NULL;
    if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || q_len <= 0 ||
        num_heads % num_kv_heads) {
        set_error("attention stream: batch %d, heads %d / kv heads %d, q_len %d", batch, num_heads,
                  num_kv_heads, q_len);
        return OJASX_ERR_INVALID;
    }
    if ((long long)batch * num_kv_heads > 65535) {
        set_error("attention stream: batch x kv heads above 65535");
        return OJASX_ERR_INVALID;
    }
    const long long rows_ll = (long long)batch * num_heads * q_len;
    const int D = head_dim;
    int rc = check_rows(rows_ll > (1 << 30) ? -1 : (int)rows_ll, D);
    if (rc) return rc;
    const int es = elem_bytes(kv_dtype);
    if (!es) {
        set_error("attention stream: kv dtype %d (F32, BF16, F16, F64 or INT8)", kv_dtype);
        return OJASX_ERR_INVALID;
    }
    const int rows = (int)rows_ll, R = num_heads / num_kv_heads * q_len;
    // k rows are read in 16-byte pieces, v rows 4 elements at a time (int8:
    // staged in 16-byte pieces)
    const size_t ak = 16;
    const size_t av = kv_dtype == KV_INT8 ? 16 : std::min(16, 4 * es);
    std::vector<AttnTile> dt;
    std::vector<AttnWork> wl;
    long long pos = kv_offset;
    for (int i = 0; i < n_tiles; ++i) {
        const OjasxAttnTile &s = tiles[i];
        if (s.n_tokens < 0 || s.n_tokens > (1LL << 31) - kACH) {
            set_error("attention stream: tile %d has %lld tokens", i, s.n_tokens);
            return OJASX_ERR_INVALID;
        }
        if (s.n_tokens == 0) continue;
        if (!s.k || !s.v || (kv_dtype == KV_INT8 && (!s.k_scale || !s.v_scale))) return OJASX_ERR_NULL;
        if (kv_dtype == KV_INT8 && D % 16) {
            set_error("attention stream: int8 tiles need head_dim a multiple of 16 (got %d)", D);
            return OJASX_ERR_INVALID;
        }
        const uintptr_t kp = reinterpret_cast<uintptr_t>(s.k), vp = reinterpret_cast<uintptr_t>(s.v);
        const long long strides = s.batch_stride | s.head_stride | s.token_stride;
        if (kp % ak || vp % av || (strides * es) % (long long)ak || s.token_stride < D ||
            s.batch_stride < 0 || s.head_stride < 0) {
            set_error("attention stream: tile %d: k, v and their strides must be aligned to %zu "
                      "bytes (k) and %zu bytes (v), rows of head_dim contiguous elements", i, ak, av);
            return OJASX_ERR_INVALID;
        }
        AttnTile t{};
        t.k = s.k;
        t.v = s.v;
        t.ks = static_cast<const __half *>(s.k_scale);
        t.vs = static_cast<const __half *>(s.v_scale);
        t.n = s.n_tokens;
        t.sb = s.batch_stride;
        t.sh = s.head_stride;
        t.st = s.token_stride;
        t.ssb = s.scale_batch_stride;
        t.ssh = s.scale_head_stride;
        t.sst = s.scale_token_stride;
        const int ti = (int)dt.size();
        dt.push_back(t);
        for (long long t0 = 0; t0 < s.n_tokens; t0 += kACH)
            wl.push_back(AttnWork{ti, (int)t0, (int)std::min<long long>(kACH, s.n_tokens - t0), 0,
                                  pos + t0});
        pos += s.n_tokens;
    }
    if (wl.empty()) return OJASX_OK;
    AttnStage &sg = t_attn;
    const size_t tile_bytes = round_up(sizeof(AttnTile) * dt.size(), 16);
    const size_t bytes = tile_bytes + sizeof(AttnWork) * wl.size();
    sg.host.assign(bytes, 0);
    memcpy(sg.host.data(), dt.data(), sizeof(AttnTile) * dt.size());
    memcpy(sg.host.data() + tile_bytes, wl.data(), sizeof(AttnWork) * wl.size());
    hipStream_t st = static_cast<hipStream_t>(stream);
    void *staged = nullptr;
    rc = sg.ring.stage(sg.host.data(), bytes, true, st, &staged);
    if (rc) return rc;
    const size_t per_work = (size_t)rows * (D + 2) * sizeof(double);
    const int n_work = (int)wl.size();
    const int per_round = (int)std::max<size_t>(1, std::min<size_t>(n_work, kPartCap / per_work));
    rc = sg.part.ensure(per_work * per_round);
    if (rc) return rc;
    int RB = 8;
    while (RB > 1 && RB / 2 >= R) RB /= 2;
    if ((R + RB - 1) / RB > 65535) {
        set_error("attention stream: %d query rows per kv head (at most %d)", R, 65535 * RB);
        return OJASX_ERR_INVALID;
    }
    AttnParams p{};
    p.tiles = static_cast<const AttnTile *>(staged);
    p.state = state;
    p.part = sg.part.as<double>();
    p.qsp = query_start_pos;
    p.scale = scale;
    p.Hkv = num_kv_heads;
    p.R = R;
    p.Sq = q_len;
    p.D = D;
    p.rows = rows;
    p.causal = causal != 0;
    const AttnWork *work_dev = reinterpret_cast<const AttnWork *>(static_cast<unsigned char *>(staged) + tile_bytes);
    for (int w0 = 0; w0 < n_work; w0 += per_round) {
        const int n = std::min(per_round, n_work - w0);
        p.work = work_dev + w0;
        switch (kv_dtype) {
            case KV_F32: rc = launch_tiles<KV_F32>(p, n, batch, RB, st); break;
            case KV_BF16: rc = launch_tiles<KV_BF16>(p, n, batch, RB, st); break;
            case KV_F16: rc = launch_tiles<KV_F16>(p, n, batch, RB, st); break;
            case KV_F64: rc = launch_tiles<KV_F64>(p, n, batch, RB, st); break;
            default: rc = launch_tiles<KV_INT8>(p, n, batch, RB, st); break;
        }
        if (rc) return rc;
        OJX_LAUNCH(attn_merge_kernel, dim3(rows), dim3(kANT), 0, st, state,
                   (const double *)p.part, n, rows, D);
        OJX_HIP(hipGetLastError());
    }
    return sg.ring.launched(st);
}

OJASX_API int ojasx_attention_stream_finalize_device(const double *state, int rows, int head_dim,
                                                     void *out, int out_dtype, double *lse,
                                                     void *stream) {
    using namespace ojx;
    if (!state || !out) return OJASX_ERR_NULL;
    int rc = check_rows(rows, head_dim);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(rows), block(round_up(head_dim, 64));
    switch (out_dtype) {
        case OJASX_DTYPE_F32:
            OJX_LAUNCH(attn_finalize_kernel<float>, grid, block, 0, st, state, static_cast<float *>(out), lse, head_dim);
            break;
        case OJASX_DTYPE_BF16:
            OJX_LAUNCH(attn_finalize_kernel<__hip_bfloat16>, grid, block, 0, st, state,
                       static_cast<__hip_bfloat16 *>(out), lse, head_dim);
            break;
        case OJASX_DTYPE_F16:
            OJX_LAUNCH(attn_finalize_kernel<__half>, grid, block, 0, st, state, static_cast<__half *>(out), lse, head_dim);
            break;
        case OJASX_DTYPE_F64:
            OJX_LAUNCH(attn_finalize_kernel<double>, grid, block, 0, st, state, static_cast<double *>(out), lse, head_dim);
            break;
        default:
            set_error("attention stream: output dtype %d (F32, BF16, F16 or F64)", out_dtype);
            return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // extern "C"

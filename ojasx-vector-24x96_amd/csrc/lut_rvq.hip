// lut_rvq.hip -- multi-stage residual-VQ LUT GEMM (the math engine's
// subspace_lut_rvq_gemm) and the codec's bit packing, on gfx950.
//
//   Y[b, m] = row_scales[m] * sum_{s, g} <X[b, g, :], C_s[code_s[m, g]]> + bias[m]
// with X zero-padded from `columns` to G * block columns, code_s the stage-s
// codes of vector v = m * G + g read from a little-endian bit stream of
// `bits` bits per code (bits in {1, 2, 4, 8}: code v sits at bit v * bits and
// never straddles a 32-bit word), and C_s the stage-s codebook [2^bits][block].
// This is ojasx_24x96/math_engine.py:136-208 with the packing of
// ojasx_24x96/codec.py:176-214; the reference's row_block_size only bounds
// its gather's working memory and has no counterpart here.
//
// lut_rvq_kernel: workgroup = 32 rows x 8 group sets; thread (q, r) owns row
// r and groups q, q+8, ...  Round trip 1 stages, with branch-free batched
// loads, the 32 rows' code words of every stage (one contiguous bit range per
// stage), all stage codebooks (when they fit) and x for up to 4 tokens in
// LDS.  Each thread then unpacks its codes from LDS, computes the dots
// <x_g, C_s[code]> from LDS and the 8 group-set partials are summed in LDS in
// a fixed order.  The epilogue is (scale * sum) + bias, stored in the input
// dtype.
#include <algorithm>
#include <cstring>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;
constexpr int kR = 32;                   // rows per workgroup
constexpr int kQG = kNT / kR;            // group sets per row
constexpr int kMaxBT = 4;                // tokens per workgroup (at most)
constexpr size_t kMaxLds = 160 * 1024;
}  // namespace

struct RvqParams {
    const void *x;            // [B][columns]
    const uint8_t *packed;    // stage s at packed + s * stage_stride
    const float *cb;          // [S][Q][D]
    const float *scales;      // [rows]
    const float *bias;        // [rows] or null
    void *y;                  // [B][rows]
    size_t stage_stride;      // bytes between stages
    size_t stage_bytes;       // packed bytes per stage = ceil(rows * G * bits / 8)
    int B, columns, rows, S, bits, D, Q, G;
    int cb_lds;               // codebooks staged in LDS
    int words;                // LDS words per stage for one workgroup's rows
};

// 32-bit word w of a stage's bit stream, where the stream starts `off` bytes
// into the 4-byte-aligned pointer `base`; bytes at or past `end` (offset from
// base) read as zero.  Loads stay inside [base, base + end).
__device__ __forceinline__ uint32_t stream_word(const uint8_t *base, size_t end, long w) {
    const long b0 = w * 4;
    if (b0 + 4 <= (long)end && b0 >= 0) return *reinterpret_cast<const uint32_t *>(base + b0);
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long b = b0 + i;
        if (b >= 0 && b < (long)end) v |= (uint32_t)base[b] << (8 * i);
    }
    return v;
}

template <typename T, int DT, int kBT>
__global__ __launch_bounds__(kNT) void lut_rvq_kernel(RvqParams p) {
    extern __shared__ float sm[];
    const int D = DT > 0 ? DT : p.D;
    const int GD = p.G * D;
    float *xs = sm;                                        // [kBT][G*D]
    float *cbs = xs + kBT * GD;                            // [S][Q][D] when cb_lds
    uint32_t *cw = reinterpret_cast<uint32_t *>(cbs + (p.cb_lds ? p.S * p.Q * D : 0));  // [S][words]
    __shared__ float red[kQG][kBT][kR];
    const int tid = threadIdx.x;
    const int r = tid % kR, q = tid / kR;
    const int m0 = blockIdx.x * kR;
    const int m = m0 + r;
    const int t0 = blockIdx.y * kBT;
    const int nt = min(kBT, p.B - t0);
    const T *__restrict__ x = static_cast<const T *>(p.x);

    // ---- round trip 1: x (zero past columns), codebooks, code words
    {
        const int n = kBT * GD;
        for (int b = tid; b < n; b += 4 * kNT) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = min(b + u * kNT, n - 1);
                const int t = min(i / GD, nt - 1), c = i - (i / GD) * GD;
                v[u] = c < p.columns ? load_act(x, (size_t)(t0 + t) * p.columns + c) : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) xs[min(b + u * kNT, n - 1)] = v[u];
        }
    }
    if (p.cb_lds) {
        const int n = p.S * p.Q * D;
        for (int b = tid; b < n; b += 4 * kNT) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = p.cb[min(b + u * kNT, n - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u) cbs[min(b + u * kNT, n - 1)] = v[u];
        }
    }
    // stage s: the bits of vectors m0*G .. (m0+32)*G - 1; word 0 of the LDS copy
    // holds the stream's word containing the first bit
    for (int s = 0; s < p.S; ++s) {
        const uint8_t *sp = p.packed + (size_t)s * p.stage_stride;
        const uint8_t *base = reinterpret_cast<const uint8_t *>(reinterpret_cast<uintptr_t>(sp) & ~uintptr_t(3));
        const size_t off = (size_t)(sp - base);
        const size_t end = off + p.stage_bytes;
        const long w0 = (long)((off * 8 + (size_t)m0 * p.G * p.bits) >> 5);
        for (int b = tid; b < p.words; b += 4 * kNT) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = stream_word(base, end, w0 + min(b + u * kNT, p.words - 1));
#pragma unroll
            for (int u = 0; u < 4; ++u) cw[s * p.words + min(b + u * kNT, p.words - 1)] = v[u];
        }
    }
    __syncthreads();

    // ---- dots over this thread's groups and all stages
    float acc[kBT];
#pragma unroll
    for (int t = 0; t < kBT; ++t) acc[t] = 0.f;
    const uint32_t mask = (1u << p.bits) - 1u;
    for (int s = 0; s < p.S; ++s) {
        const uint8_t *sp = p.packed + (size_t)s * p.stage_stride;
        const size_t off = reinterpret_cast<uintptr_t>(sp) & 3;
        const size_t bit0 = off * 8 + (size_t)m0 * p.G * p.bits;   // stream bit of vector m0*G
        const size_t wbase = bit0 >> 5;
        const float *C = p.cb_lds ? cbs + (size_t)s * p.Q * D : p.cb + (size_t)s * p.Q * D;
        for (int g = q; g < p.G; g += kQG) {
            const size_t bit = bit0 + ((size_t)r * p.G + g) * p.bits;
            const uint32_t code = (cw[s * p.words + (int)((bit >> 5) - wbase)] >> (bit & 31)) & mask;
            const float *c = C + (size_t)code * D;
            const float *xg = xs + g * D;
            if (DT > 0) {
                float cr[DT > 0 ? DT : 1];
#pragma unroll
                for (int d = 0; d < D; ++d) cr[d] = c[d];
#pragma unroll
                for (int t = 0; t < kBT; ++t) {
                    float dot = 0.f;
#pragma unroll
                    for (int d = 0; d < D; ++d) dot = fmaf(xg[t * GD + d], cr[d], dot);
                    acc[t] += dot;
                }
            } else {
#pragma unroll
                for (int t = 0; t < kBT; ++t) {
                    float dot = 0.f;
                    for (int d = 0; d < D; ++d) dot = fmaf(xg[t * GD + d], c[d], dot);
                    acc[t] += dot;
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kBT; ++t) red[q][t][r] = acc[t];
    __syncthreads();
    if (q != 0 || m >= p.rows) return;
    const float sc = p.scales[m];
    const float bs = p.bias ? p.bias[m] : 0.f;
    T *y = static_cast<T *>(p.y);
#pragma unroll
    for (int t = 0; t < kBT; ++t) {
        if (t >= nt) break;
        float a = red[0][t][r];
#pragma unroll
        for (int k = 1; k < kQG; ++k) a += red[k][t][r];
        float v = a * sc;
        if (p.bias) v += bs;
        store_act(y, (size_t)(t0 + t) * p.rows + m, v);
    }
}

// codes[i] (uint8, < 2^bits) -> little-endian bit stream, one output byte per thread.
__global__ __launch_bounds__(kNT) void pack_codes_kernel(const uint8_t *codes, long count, int bits,
                                                         uint8_t *packed, long nbytes) {
    const long i = (long)blockIdx.x * kNT + threadIdx.x;
    if (i >= nbytes) return;
    const int per = 8 / bits;
    uint32_t v = 0;
    for (int k = 0; k < per; ++k) {
        const long c = i * per + k;
        if (c < count) v |= ((uint32_t)codes[c] & ((1u << bits) - 1u)) << (k * bits);
    }
    packed[i] = (uint8_t)v;
}

__global__ __launch_bounds__(kNT) void unpack_codes_kernel(const uint8_t *packed, long count, int bits,
                                                           uint8_t *codes) {
    const long i = (long)blockIdx.x * kNT + threadIdx.x;
    if (i >= count) return;
    const long bit = i * bits;
    codes[i] = (uint8_t)((packed[bit >> 3] >> (bit & 7)) & ((1u << bits) - 1u));
}

namespace {

bool valid_bits(int bits) { return bits == 1 || bits == 2 || bits == 4 || bits == 8; }

template <typename T, int DT, int BT>
int launch_rvq_bt(RvqParams &p, size_t lds, hipStream_t st) {
    static size_t granted = 0;
    const void *fn = reinterpret_cast<const void *>(&lut_rvq_kernel<T, DT, BT>);
    int rc = ensure_dyn_lds(fn, lds, &granted);
    if (rc) return rc;
    dim3 grid((p.rows + kR - 1) / kR, (p.B + BT - 1) / BT);
    OJX_LAUNCH((lut_rvq_kernel<T, DT, BT>), grid, dim3(kNT), lds, st, p);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

template <typename T, int DT>
int launch_rvq_d(RvqParams &p, int bt, size_t lds, hipStream_t st) {
    if (bt == 4) return launch_rvq_bt<T, DT, 4>(p, lds, st);
    if (bt == 2) return launch_rvq_bt<T, DT, 2>(p, lds, st);
    return launch_rvq_bt<T, DT, 1>(p, lds, st);
}

template <typename T>
int launch_rvq(RvqParams &p, int bt, size_t lds, hipStream_t st) {
    switch (p.D) {
        case 4: return launch_rvq_d<T, 4>(p, bt, lds, st);
        case 8: return launch_rvq_d<T, 8>(p, bt, lds, st);
        case 16: return launch_rvq_d<T, 16>(p, bt, lds, st);
        default: return launch_rvq_d<T, 0>(p, bt, lds, st);
    }
}

}  // namespace
}  // namespace ojx

extern "C" {

OJASX_API int ojasx_subspace_lut_gemm_device(const void *x, int batch, int columns, int rows,
                                             const uint8_t *packed_codes, size_t stage_stride_bytes,
                                             int stages, int bits, int block_size,
                                             const float *codebooks, const float *row_scales,
                                             const float *bias, void *y, int dtype, void *stream) {
    using namespace ojx;
    if (!x || !packed_codes || !codebooks || !row_scales || !y) return OJASX_ERR_NULL;
    if (batch <= 0 || rows <= 0) return OJASX_OK;
    if (columns <= 0 || stages <= 0 || !valid_bits(bits) || block_size <= 0 || block_size > 64) {
        set_error("invalid LUT GEMM shape: columns=%d stages=%d bits=%d block=%d", columns, stages,
                  bits, block_size);
        return OJASX_ERR_INVALID;
    }
    if (dtype != OJASX_DTYPE_F32 && dtype != OJASX_DTYPE_BF16) {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    if ((long)batch > 65535L) {
        set_error("batch %d too large for one call", batch);
        return OJASX_ERR_INVALID;
    }
    RvqParams p{};
    p.x = x;
    p.packed = packed_codes;
    p.cb = codebooks;
    p.scales = row_scales;
    p.bias = bias;
    p.y = y;
    p.B = batch;
    p.columns = columns;
    p.rows = rows;
    p.S = stages;
    p.bits = bits;
    p.D = block_size;
    p.Q = 1 << bits;
    p.G = (columns + block_size - 1) / block_size;
    p.stage_stride = stage_stride_bytes;
    p.stage_bytes = ((size_t)rows * p.G * bits + 7) / 8;
    if (stages > 1 && stage_stride_bytes < p.stage_bytes) {
        set_error("stage stride %zu below the %zu packed bytes of a stage", stage_stride_bytes,
                  p.stage_bytes);
        return OJASX_ERR_INVALID;
    }
    // code words of kR rows per stage, plus one for the unaligned start
    p.words = (int)(((size_t)kR * p.G * bits + 31) / 32 + 2);
    // tokens per workgroup: 4, or fewer when x of 4 tokens and the code words
    // do not fit the LDS; codebooks are staged when they still fit
    const size_t xrow = (size_t)p.G * block_size * sizeof(float);
    const size_t cwb = (size_t)stages * p.words * sizeof(uint32_t);
    const size_t cbb = (size_t)stages * p.Q * block_size * sizeof(float);
    int bt = std::min(batch, kMaxBT) >= 3 ? 4 : std::min(batch, kMaxBT);
    while (bt > 1 && bt * xrow + cwb > kMaxLds) bt /= 2;
    if (bt * xrow + cwb > kMaxLds) {
        set_error("LUT GEMM of %d columns x %d stages does not fit the 160 KB LDS", columns, stages);
        return OJASX_ERR_INVALID;
    }
    p.cb_lds = bt * xrow + cwb + cbb <= kMaxLds;
    const size_t lds = bt * xrow + cwb + (p.cb_lds ? cbb : 0);
    hipStream_t st = static_cast<hipStream_t>(stream);
    return dtype == OJASX_DTYPE_F32 ? launch_rvq<float>(p, bt, lds, st)
                                    : launch_rvq<__hip_bfloat16>(p, bt, lds, st);
}

OJASX_API int ojasx_pack_codes_device(const uint8_t *codes, long count, int bits, uint8_t *packed,
                                      void *stream) {
    using namespace ojx;
    if (!codes || !packed) return OJASX_ERR_NULL;
    if (!valid_bits(bits) || count < 0) {
        set_error("bits must be 1, 2, 4 or 8");
        return OJASX_ERR_INVALID;
    }
    const long nbytes = (count * bits + 7) / 8;
    if (nbytes == 0) return OJASX_OK;
    OJX_LAUNCH(pack_codes_kernel, dim3((nbytes + kNT - 1) / kNT), dim3(kNT), 0,
               static_cast<hipStream_t>(stream), codes, count, bits, packed, nbytes);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API int ojasx_unpack_codes_device(const uint8_t *packed, long count, int bits, uint8_t *codes,
                                        void *stream) {
    using namespace ojx;
    if (!codes || !packed) return OJASX_ERR_NULL;
    if (!valid_bits(bits) || count < 0) {
        set_error("bits must be 1, 2, 4 or 8");
        return OJASX_ERR_INVALID;
    }
    if (count == 0) return OJASX_OK;
    OJX_LAUNCH(unpack_codes_kernel, dim3((count + kNT - 1) / kNT), dim3(kNT), 0,
               static_cast<hipStream_t>(stream), packed, count, bits, codes);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // extern "C"

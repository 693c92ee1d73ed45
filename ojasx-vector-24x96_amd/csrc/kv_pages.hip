// kv_pages.hip -- the KV cache's write side on gfx950: int8 page quantisation
// for PagedCompressedKVCache and codebook encode-and-append into the paged
// code layout that the decode kernels read.
//
//  * quantize_int8 (ojasx_24x96/long_context.py:234-240), per token row of D
//    values, in the arithmetic torch applies to a tensor of the input type
//    (every elementwise result rounded to that type):
//      a = max(max_d |t_d|, T(1e-8)),  s = T(a / 127),
//      q_d = clamp(round_half_even(T(t_d / s)), -127, 127) as int8,
//    s stored as fp16.  For fp32 input every T() is the identity; fp64 rows
//    run the same steps in fp64 (quantize_int8_f64_kernel).  One wave
//    per row: abs-max by DPP wave reduction, then each lane writes its
//    elements.  Rows are addressed as (group, row) with strides, so a slice
//    of a [B, H, S, D] tensor quantises straight into a page buffer.
//  * dequantize_int8 (long_context.py:242-244): float(q) * float(s) in fp32,
//    stored in the output type (round to nearest even).
//  * kv_encode_append: token i, kv head h, for K and V alike:
//      s = max(1e-8, max_d |k_d|) / 127   (ojasx_lut_kv_cache.cpp:29-34),
//      x_d = k_d / s,
//    then per group g of D coordinates either
//      - with a codebook: code = argmin_c sum_d (x[gD+d] - C_h[c][d])^2 over
//        the 256 centroids, the sum accumulated with fmaf in d order from 0,
//        ties to the lower index; or
//      - without one (NULL): the reference quantiser, code =
//        clamp(round_half_away(x[gD]), -128, 127) + 128 from coordinate gD
//        only (ojasx_lut_kv_cache.cpp:36-45).
//    Codes and scales land at slot_mapping[i] = page * page_size + offset in
//    the paged layout [page][h][offset][G] / [page][h][offset]; a slot that
//    is negative or past num_pages pages skips the token.  Workgroup =
//    (token, kv head), thread = centroid, which holds its K and V centroid
//    rows in registers across the groups.
#include <cmath>

#include "common.h"
#include "kv_encode.h"

namespace ojx {

namespace {
constexpr int kNT = kEncNT;
constexpr int kNW = kNT / 64;
}  // namespace

struct QuantParams {
    const void *x;
    int8_t *q;
    __half *scale;
    long groups;
    int rows, dim;
    long x_gs, q_gs, s_gs;      // group strides, elements
};

template <typename T>
__global__ __launch_bounds__(kNT) void quantize_int8_kernel(QuantParams p) {
    const int lane = threadIdx.x & 63;
    const long r = (long)blockIdx.x * kNW + (threadIdx.x >> 6);
    if (r >= p.groups * p.rows) return;          // wave-uniform
    const long g = r / p.rows;
    const int row = (int)(r - g * p.rows);
    const T *xr = static_cast<const T *>(p.x) + g * p.x_gs + (long)row * p.dim;
    float am = 0.f;
    for (int d = lane; d < p.dim; d += 64) am = fmaxf(am, fabsf(load_act(xr, d)));
    am = wave_max_f(am);
    const float s = round_as(xr, fmaxf(am, round_as(xr, 1e-8f)) / 127.0f);
    int8_t *qr = p.q + g * p.q_gs + (long)row * p.dim;
    for (int d = lane; d < p.dim; d += 64) {
        const float v = rintf(round_as(xr, load_act(xr, d) / s));
        // v is NaN only for an all-zero fp16 row (s rounds to 0 there); the
        // reference's int8 cast of that NaN has no defined value: write 0.
        qr[d] = (v != v) ? (int8_t)0 : (int8_t)fminf(127.f, fmaxf(-127.f, v));
    }
    if (lane == 0) p.scale[g * p.s_gs + row] = __float2half_rn(s);
}

// fp32 -> fp16 bits, round to nearest even, in integer steps: the compiler
// otherwise merges (half)(float)d into one fp64 -> fp16 rounding, while torch
// rounds a float64 scale to float32 first and then to float16.
__device__ __forceinline__ unsigned short f32_to_f16_bits_rne(float f) {
    const unsigned int b = __float_as_uint(f);
    const unsigned int sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xffu);
    unsigned int m = b & 0x7fffffu;
    if (e == 0xff) return (unsigned short)(sign | 0x7c00u | (m ? 0x200u : 0u));
    const int he = e - 127 + 15;                 // biased half exponent
    if (he >= 31) return (unsigned short)(sign | 0x7c00u);
    if (he >= 1) {                               // normal half: 10 of 23 mantissa bits
        const unsigned int hm = m >> 13, rem = m & 0x1fffu;
        unsigned int v = ((unsigned int)he << 10) | hm;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++v;   // a carry may reach inf
        return (unsigned short)(sign | v);
    }
    if (he < -10) return (unsigned short)sign;   // below half the smallest subnormal
    m |= 0x800000u;                              // subnormal half: units of 2^-24
    const int shift = 14 - he;                   // 14 .. 24
    unsigned int hm = m >> shift;
    const unsigned int rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return (unsigned short)(sign | hm);
}

// fp64 rows: the same steps in fp64 (torch's arithmetic on a float64 tensor),
// the scale stored as torch casts float64 to float16 (through fp32: two
// roundings to nearest even).
__global__ __launch_bounds__(kNT) void quantize_int8_f64_kernel(QuantParams p) {
    const int lane = threadIdx.x & 63;
    const long r = (long)blockIdx.x * kNW + (threadIdx.x >> 6);
    if (r >= p.groups * p.rows) return;          // wave-uniform
    const long g = r / p.rows;
    const int row = (int)(r - g * p.rows);
    const double *xr = static_cast<const double *>(p.x) + g * p.x_gs + (long)row * p.dim;
    double am = 0.0;
    for (int d = lane; d < p.dim; d += 64) am = fmax(am, fabs(xr[d]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) am = fmax(am, __shfl_xor(am, o, 64));
    const double s = fmax(am, 1e-8) / 127.0;
    int8_t *qr = p.q + g * p.q_gs + (long)row * p.dim;
    for (int d = lane; d < p.dim; d += 64)
        qr[d] = (int8_t)fmin(127.0, fmax(-127.0, rint(xr[d] / s)));
    if (lane == 0)
        reinterpret_cast<unsigned short *>(p.scale)[g * p.s_gs + row] =
            f32_to_f16_bits_rne((float)s);
}

template <typename T>
__global__ __launch_bounds__(kNT) void dequantize_int8_kernel(const int8_t *__restrict__ q,
                                                              const __half *__restrict__ scale,
                                                              long groups, int rows, int dim,
                                                              long q_gs, long s_gs, T *out) {
    const long i = (long)blockIdx.x * kNT + threadIdx.x;
    const long per_group = (long)rows * dim;
    if (i >= groups * per_group) return;
    const long g = i / per_group;
    const long e = i - g * per_group;
    const int row = (int)(e / dim);
    const float s = __half2float(scale[g * s_gs + row]);
    store_act(out, i, (float)q[g * q_gs + e] * s);
}

struct EncodeParams {
    const float *k, *v;         // [n][Hkv][hd]
    const float *kcb, *vcb;     // [Hkv][256][D], or both NULL
    const int *slots;           // [n]
    uint8_t *kc, *vc;           // [pages][Hkv][P][G]
    float *ks, *vs;             // [pages][Hkv][P]
    int Hkv, hd, D, G, P, num_pages;
};

// Workgroup (token i, kv head h, z): z = 0 encodes the token's K row, z = 1
// its V row (two workgroups per token and head: each runs half the nearest-
// centroid work, and the two chains run side by side).
template <int DT>
__global__ __launch_bounds__(kNT) void kv_encode_append_kernel(EncodeParams p) {
    extern __shared__ float xs[];                // [hd]: the row / its scale
    const int i = blockIdx.x, h = blockIdx.y, kv = blockIdx.z;
    float creg[DT > 0 ? DT : 1];
    const float *cb = kv ? p.vcb : p.kcb;
    if (cb) {
        cb += (size_t)h * 256 * p.D;
        enc_load_centroid<DT>(cb, creg);
    }
    const int slot = p.slots[i];
    if (slot < 0 || slot / p.P >= p.num_pages) return;   // skipped slot; workgroup-uniform
    const int page = slot / p.P;
    const size_t row = ((size_t)page * p.Hkv + h) * p.P + (slot - page * p.P);
    encode_row<DT>((kv ? p.v : p.k) + ((size_t)i * p.Hkv + h) * p.hd, cb, creg, p.hd, p.D, p.G,
                   (kv ? p.vc : p.kc) + row * p.G, (kv ? p.vs : p.ks) + row, xs);
}

}  // namespace ojx

extern "C" {

OJASX_API int ojasx_quantize_int8_device(const void *x, long groups, int rows, int dim,
                                         long x_group_stride, int dtype, int8_t *q,
                                         long q_group_stride, void *scale_f16,
                                         long scale_group_stride, void *stream) {
    using namespace ojx;
    if (!x || !q || !scale_f16) return OJASX_ERR_NULL;
    if (groups < 0 || rows < 0 || dim <= 0 || x_group_stride < 0 || q_group_stride < 0 ||
        scale_group_stride < 0) {
        set_error("invalid int8 quantisation shape");
        return OJASX_ERR_INVALID;
    }
    if (groups == 0 || rows == 0) return OJASX_OK;
    const long total = groups * rows;
    if ((total + kNW - 1) / kNW > 0x7fffffffL) {
        set_error("too many rows: %ld", total);
        return OJASX_ERR_INVALID;
    }
    QuantParams p{x, q, static_cast<__half *>(scale_f16), groups, rows, dim,
                  x_group_stride, q_group_stride, scale_group_stride};
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)((total + kNW - 1) / kNW));
    if (dtype == OJASX_DTYPE_F32)
        OJX_LAUNCH(quantize_int8_kernel<float>, grid, dim3(kNT), 0, st, p);
    else if (dtype == OJASX_DTYPE_BF16)
        OJX_LAUNCH(quantize_int8_kernel<__hip_bfloat16>, grid, dim3(kNT), 0, st, p);
    else if (dtype == OJASX_DTYPE_F16)
        OJX_LAUNCH(quantize_int8_kernel<__half>, grid, dim3(kNT), 0, st, p);
    else if (dtype == OJASX_DTYPE_F64)
        OJX_LAUNCH(quantize_int8_f64_kernel, grid, dim3(kNT), 0, st, p);
    else {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API int ojasx_dequantize_int8_device(const int8_t *q, const void *scale_f16, long groups,
                                           int rows, int dim, long q_group_stride,
                                           long scale_group_stride, void *out, int dtype,
                                           void *stream) {
    using namespace ojx;
    if (!q || !scale_f16 || !out) return OJASX_ERR_NULL;
    if (groups < 0 || rows < 0 || dim <= 0 || q_group_stride < 0 || scale_group_stride < 0) {
        set_error("invalid int8 dequantisation shape");
        return OJASX_ERR_INVALID;
    }
    const long total = groups * rows * (long)dim;
    if (total == 0) return OJASX_OK;
    if ((total + kNT - 1) / kNT > 0x7fffffffL) {
        set_error("too many elements: %ld", total);
        return OJASX_ERR_INVALID;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const __half *s = static_cast<const __half *>(scale_f16);
    const dim3 grid((unsigned)((total + kNT - 1) / kNT));
    if (dtype == OJASX_DTYPE_F32)
        OJX_LAUNCH(dequantize_int8_kernel<float>, grid, dim3(kNT), 0, st, q, s, groups, rows, dim,
                   q_group_stride, scale_group_stride, static_cast<float *>(out));
    else if (dtype == OJASX_DTYPE_BF16)
        OJX_LAUNCH(dequantize_int8_kernel<__hip_bfloat16>, grid, dim3(kNT), 0, st, q, s, groups,
                   rows, dim, q_group_stride, scale_group_stride,
                   static_cast<__hip_bfloat16 *>(out));
    else if (dtype == OJASX_DTYPE_F16)
        OJX_LAUNCH(dequantize_int8_kernel<__half>, grid, dim3(kNT), 0, st, q, s, groups, rows, dim,
                   q_group_stride, scale_group_stride, static_cast<__half *>(out));
    else if (dtype == OJASX_DTYPE_F64)
        OJX_LAUNCH(dequantize_int8_kernel<double>, grid, dim3(kNT), 0, st, q, s, groups, rows, dim,
                   q_group_stride, scale_group_stride, static_cast<double *>(out));
    else {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API int ojasx_kv_encode_append_device(const float *k, const float *v, int num_tokens,
                                            int num_kv_heads, int head_dim, int block_dim,
                                            const float *k_codebook, const float *v_codebook,
                                            const int *slot_mapping, int page_size,
                                            int num_pages, uint8_t *k_codes, float *k_scales, uint8_t *v_codes,
                                            float *v_scales, void *stream) {
    using namespace ojx;
    if (!k || !v || !slot_mapping || !k_codes || !k_scales || !v_codes || !v_scales)
        return OJASX_ERR_NULL;
    if ((k_codebook == nullptr) != (v_codebook == nullptr)) {
        set_error("k_codebook and v_codebook must both be given or both be NULL");
        return OJASX_ERR_NULL;
    }
    if (num_tokens < 0 || num_kv_heads <= 0 || num_kv_heads > 65535 || head_dim <= 0 ||
        block_dim <= 0 || head_dim % block_dim || head_dim / block_dim > kMaxEncGroups ||
        head_dim > 16384 || page_size <= 0 || num_pages <= 0) {
        set_error("invalid KV append shape (head_dim %d, block_dim %d: at most %d groups)",
                  head_dim, block_dim, kMaxEncGroups);
        return OJASX_ERR_INVALID;
    }
    if (num_tokens == 0) return OJASX_OK;
    EncodeParams p{k, v, k_codebook, v_codebook, slot_mapping, k_codes, v_codes, k_scales,
                   v_scales, num_kv_heads, head_dim, block_dim, head_dim / block_dim, page_size,
                   num_pages};
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t lds = (size_t)head_dim * sizeof(float);
    const dim3 grid(num_tokens, num_kv_heads, 2);   // z: K, then V
    const bool reg16 = block_dim == 16 && k_codebook &&
                       (reinterpret_cast<uintptr_t>(k_codebook) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(v_codebook) & 15) == 0;
    if (reg16) {
        static size_t granted = 0;
        int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_encode_append_kernel<16>), lds,
                                &granted);
        if (rc) return rc;
        OJX_LAUNCH(kv_encode_append_kernel<16>, grid, dim3(kNT), lds, st, p);
    } else {
        static size_t granted = 0;
        int rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_encode_append_kernel<0>), lds,
                                &granted);
        if (rc) return rc;
        OJX_LAUNCH(kv_encode_append_kernel<0>, grid, dim3(kNT), lds, st, p);
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // extern "C"

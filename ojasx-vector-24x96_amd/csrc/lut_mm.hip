// lut_mm.hip -- the LUT linear (block_dim 16, 256 centroids) for many tokens
// as x . W^T on fp32 MFMA.
//
// y[b][m] = (s_m * sum_g LUT_b[g, codes[m, g]] + bias_m) + sum_j val_j x_b[col_j]
// with LUT_b[g, k] = <x_b[16g..16g+16), C[k]> (ojasx_lut_cpu.cpp:132-206).  By
// the identity LUT-gather = x . W^T, with W[m][16g + d] = C[codes[m, g]][d],
// the sum over groups is a GEMM against W decoded from the codes: the
// per-token LUTs grow with the batch (1 KB per group and token), W does not
// (64 bytes per group and row, decoded in registers from the codebook in
// LDS).
//
// A wave computes one 16-row x 16-token tile over part of the input: the kQ
// waves of a row tile split every 256-wide input slice (16 groups), wave q
// taking groups GPW q .. GPW q + GPW - 1 (GPW = 16 / kQ; kQ = 8 with one tile
// per workgroup, 4 otherwise), 4 MFMAs (v_mfma_f32_16x16x4f32) per group with
//   A[m][k] = C[code(m, g)][4k + ks]   (one 16-byte LDS read of the codebook row),
//   B[k][n] = x_n[16g + 4k + ks]       (one 16-byte LDS read of the staged x),
// for ks = 0..3: MFMA ks covers dims 4k + ks of the group, so a lane's four
// values are contiguous in both the codebook row and x.  Two accumulators
// (even and odd groups) keep the MFMA chains independent.  The partial sums
// of a tile meet in LDS at the end, added in wave order.  Splitting the input
// gives kQ times the waves of a one-wave-per-tile layout.  A workgroup holds
// RT row tiles (kQ RT waves) of the same 16 tokens, sharing the codebook and
// the staged x slices: two LDS buffers, and the x loads kept Sh::kPX slices
// ahead in a register ring (a slice's MFMAs per wave are far shorter than a
// load's round trip); codes Sh::kPF slices ahead.
//
// The CSR outliers of the workgroup's rows are staged in LDS; wave q < 4 of a
// tile adds those of row 4 (lane / 16) + q whose columns fall in the current
// slice from the staged x (a row's entries are sorted by column), so no x is
// read at random from memory; the outlier sums meet in LDS with the partial
// sums.  The epilogue applies the scale and the bias:
// (s_m * sum + bias) + outliers.
//
// MFMA 16x16x4 fp32 operand layout: lane l supplies A[m = l % 16][k = l / 16]
// and B[k = l / 16][n = l % 16]; the result's value v of lane l is
// D[m = 4 (l / 16) + v][n = l % 16].
#include "common.h"

namespace ojx {

namespace {
constexpr int kMmTok = 16;       // tokens per workgroup
constexpr int kXStride = 260;    // floats per staged x row (256 + pad)
constexpr int kOutPass = 3;      // outlier candidates per row per pass
typedef float v4f __attribute__((ext_vector_type(4)));

// RT row tiles per workgroup, each split over kQ waves (16 / kQ groups of
// every slice per wave): 8 with one tile per workgroup (small batches, where
// the waves are few), 4 otherwise.
template <int RT>
struct MmShape {
    static constexpr int kQ = RT == 1 ? 8 : 4;
    static constexpr int kGPW = 16 / kQ;            // groups per wave per slice
    static constexpr int kNT = 64 * kQ * RT;        // threads
    static constexpr int kRows = 16 * RT;           // rows
    static constexpr int kXF = kMmTok * 256 / kNT;  // x floats staged per thread per slice
    // slices of x and of codes in flight (kPX divides kPF and the kernel's
    // reduced depth): deeper where the registers allow, since few waves per
    // SIMD leave a slice short
    static constexpr int kPX = 2;
    static constexpr int kPF = 4;
    // CSR entries of the workgroup's rows staged in LDS (columns as 16-bit:
    // in_features <= 65535 on this path): 16 per row, against 9.7 on average
    // at 0.38 % of 2560 inputs; a denser block takes its outliers from memory
    static constexpr int kCsr = kNT;
    // waves per SIMD the register budget is cut for: 3 workgroups per CU
    // (LDS) up to 2 row tiles, 2 at 4 row tiles
    static constexpr int kWaves = RT == 1 ? 5 : RT == 2 ? 6 : 8;
};
}  // namespace

// x of tokens n0..n0+15, inputs 256 s .. 256 s + 255: thread t loads floats
// t XF .. t XF + XF - 1 of the 16 x 256 slice, from clamped addresses (always
// in bounds); mm_store_x zeroes them past K and past B.  The loads are not
// touched until the store, so a prefetch is not waited for early.
template <typename T, int XF>
__device__ __forceinline__ void mm_load_x(const MmParams &p, int n0, int s, float (&r)[XF]) {
    const int e = threadIdx.x * XF;
    const int n = n0 + (e >> 8), k = s * 256 + (e & 255);
    const T *src = static_cast<const T *>(p.x) + (size_t)min(n, p.B - 1) * p.K + min(k, p.K - XF);
    if constexpr (sizeof(T) == 4) {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
#pragma unroll
        for (int u = 0; u < XF / 4; ++u) {
            const float4 f = gld(s4 + u);
            r[4 * u] = f.x;
            r[4 * u + 1] = f.y;
            r[4 * u + 2] = f.z;
            r[4 * u + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < XF; ++u) r[u] = load_act(src, u);
    }
}

// Store slice s's loaded x into an LDS buffer, zero past K and past B.
template <int XF>
__device__ __forceinline__ void mm_store_x(const MmParams &p, int n0, int s, float *xs, const float (&r)[XF]) {
    const int e = threadIdx.x * XF;
    const bool ok = n0 + (e >> 8) < p.B && s * 256 + (e & 255) < p.K;   // K is a multiple of 16, XF divides 16
    float4 *d = reinterpret_cast<float4 *>(xs + (e >> 8) * kXStride + (e & 255));
#pragma unroll
    for (int u = 0; u < XF / 4; ++u)
        d[u] = ok ? make_float4(r[4 * u], r[4 * u + 1], r[4 * u + 2], r[4 * u + 3])
                  : make_float4(0.f, 0.f, 0.f, 0.f);
}

// Codes of groups GPW q .. GPW q + GPW - 1 of slice s for a row, as one word.
template <int GPW>
__device__ __forceinline__ uint32_t mm_codes(const MmParams &p, int s, int row, int q) {
    const uint8_t *src = p.codes + ((size_t)s * p.Mp + row) * 16 + GPW * q;
    if constexpr (GPW == 4) return gld(reinterpret_cast<const uint32_t *>(src));
    else return gld(reinterpret_cast<const unsigned short *>(src));
}

template <typename T, int RT>
__global__ __launch_bounds__(MmShape<RT>::kNT) __attribute__((amdgpu_waves_per_eu(MmShape<RT>::kWaves))) void lut_mm_kernel(MmParams p) {
    using Sh = MmShape<RT>;
    // two code slices in flight where four spill at the register budget
    // (fp32 at 4 row tiles, bf16 at 2 and 4): 2-2.5 % faster there
    constexpr int PF = (RT == 4 || (RT == 2 && !std::is_same<T, float>::value)) ? 2 : Sh::kPF;
    constexpr int NT = Sh::kNT, XF = Sh::kXF, NC = Sh::kCsr, PX = Sh::kPX;
    constexpr int kQ = Sh::kQ, GPW = Sh::kGPW;
    static_assert(PF % PX == 0, "the unrolled slice body covers both rings");
    __shared__ float4 cb4[256 * 4];                 // codebook [256][16]
    __shared__ __align__(16) float xs[2][kMmTok * kXStride];   // staged x slices; the quarter sums at the end
    __shared__ unsigned short lcol[NC];             // the workgroup's CSR outliers
    __shared__ float lval[NC];
    static_assert(RT * ((kQ - 1) * 64 * 4 + 4 * 64) <= 2 * kMmTok * kXStride,
                  "partial and outlier sums fit the x buffers");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rt = w / kQ, q = w % kQ;              // row tile, input part
    const int ml = lane & 15, kk = lane >> 4;
    const int mb = blockIdx.x * Sh::kRows;
    const int m0 = mb + rt * 16;
    const int n0 = blockIdx.y * kMmTok;
    const int row = min(m0 + ml, p.M - 1);          // rows past M: computed, never stored
    const int mo = m0 + 4 * kk + q;                 // the lane's outlier row (waves q < 4)
    const bool outw = q < 4;

    // ---- round trip 1: codebook, x slices 0 .. PX, the CSR range of the rows, codes
    static_assert(1024 % NT == 0, "the codebook is staged in whole float4 rounds");
    float4 c4[1024 / NT];
    const float4 *gcb = reinterpret_cast<const float4 *>(p.cb);
#pragma unroll
    for (int u = 0; u < 1024 / NT; ++u) c4[u] = gld(gcb + tid + u * NT);
    float x0[XF];
    mm_load_x<T, XF>(p, n0, 0, x0);
    float xr[PX][XF];   // x of slices s + 1 .. s + PX, slot (slice % PX)
#pragma unroll
    for (int t = 1; t <= PX; ++t) mm_load_x<T, XF>(p, n0, min(t, p.S - 1), xr[t % PX]);
    int e_lo = 0, e_hi = 0, j = 0, je = 0;
    if (p.rowp) {
        e_lo = gld(p.rowp + mb);
        e_hi = gld(p.rowp + min(mb + Sh::kRows, p.M));
        j = gld(p.rowp + min(mo, p.M - 1));
        je = outw && mo < p.M ? gld(p.rowp + mo + 1) : j;
    }
    uint32_t cr[PF];   // codes of slices s .. s + PF - 1, slot (s % PF)
#pragma unroll
    for (int u = 0; u < PF; ++u) cr[u] = mm_codes<GPW>(p, min(u, p.S - 1), row, q);
    // ---- round trip 2: the CSR entries of the workgroup's rows into LDS when
    // they fit (the usual case: each row's entries sorted by column are then
    // added slice by slice from the staged x), else from memory at the end
    const bool staged = e_hi - e_lo <= NC;
    if (p.rowp && staged && e_hi > e_lo) {
        const int e = min(e_lo + tid, e_hi - 1);    // an entry of these rows
        const int c = gld(p.col + e);
        const float v = gld(p.val + e);
        if (e_lo + tid < e_hi) {
            lcol[tid] = (unsigned short)c;
            lval[tid] = v;
        }
    }
#pragma unroll
    for (int u = 0; u < 1024 / NT; ++u) cb4[tid + u * NT] = c4[u];
    mm_store_x<XF>(p, n0, 0, xs[0], x0);
    __syncthreads();

    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float o = 0.f;
    j -= e_lo;
    je -= e_lo;
    // Slice s uses code slot s % PF, and stores x slot (s + 1) % PX for the
    // next slice: constants in the unrolled body (no register moves of loads
    // in flight).  The slots are refilled with slices s + PF and s + 1 + PX,
    // unconditionally (clamped to the last slice).  The main loop runs whole
    // groups of PF slices with no branch in its body other than the
    // outlier pass, so the wait counts for the rings stay exact across its
    // back edge (a merge of differing paths makes the compiler wait for every
    // load in flight); the last S % PF slices follow it.
    auto slice = [&](const int s, const int u) __attribute__((always_inline)) {
        const float *xt = xs[s & 1] + ml * kXStride;
        const float *xb = xt + 4 * kk + 16 * GPW * q;
        const uint32_t cw = cr[u];
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const uint32_t code = (cw >> (8 * i)) & 0xffu;
            const float4 a = cb4[code * 4 + kk];
            const float4 b = *reinterpret_cast<const float4 *>(xb + 16 * i);
            v4f &acc = (i & 1) ? acc1 : acc0;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
        }
        // outliers of the lane's row mo whose columns fall in this slice:
        // kOutPass candidates per pass, the reads of a pass in flight together
        // (one pass covers a slice unless the row has more than kOutPass
        // entries in it); added in column order
        if (outw && p.rowp && staged) {
            const int lim = (s + 1) * 256;
            bool more = true;
            while (more) {
                int c[kOutPass];
                float vv[kOutPass];
#pragma unroll
                for (int k = 0; k < kOutPass; ++k) {
                    const int e = min(j + k, NC - 1);
                    c[k] = lcol[e];
                    vv[k] = lval[e];
                }
                bool in = true;
                int took = 0;
#pragma unroll
                for (int k = 0; k < kOutPass; ++k) {
                    in = in && j + k < je && c[k] < lim;
                    const float xv = xt[in ? c[k] - s * 256 : 0];
                    if (in) o += vv[k] * xv;
                    took += in ? 1 : 0;
                }
                j += took;
                more = took == kOutPass;
            }
        }
        // slice s + 1 into the other buffer (past the last slice: a clamped
        // reload, never read), then the freed ring slots refilled
        const int slot = (u + 1) % PX;
        mm_store_x<XF>(p, n0, min(s + 1, p.S - 1), xs[(s + 1) & 1], xr[slot]);
        mm_load_x<T, XF>(p, n0, min(s + 1 + PX, p.S - 1), xr[slot]);
        cr[u] = mm_codes<GPW>(p, min(s + PF, p.S - 1), row, q);
        __syncthreads();   // slice s + 1 staged; slice s's reads done before it is overwritten
    };
    int s0 = 0;
    for (; s0 + PF <= p.S; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) slice(s0 + u, u);
    }
#pragma unroll
    for (int u = 0; u < PF - 1; ++u)
        if (s0 + u < p.S) slice(s0 + u, u);

    // ---- a dense-outlier block: the row's entries and x from memory
    const int n = n0 + ml;
    const T *xn = static_cast<const T *>(p.x) + (size_t)min(n, p.B - 1) * p.K;
    if (p.rowp && !staged && n < p.B && outw)
        for (int e = j; e < je; ++e) o += gld(p.val + e_lo + e) * load_act(xn, gld(p.col + e_lo + e));

    // ---- the partial sums and outlier sums of each tile through LDS (the x
    // buffers are free: the last slice ended with a barrier); wave 0 of the
    // tile adds the partial sums in wave order
    float4 *red = reinterpret_cast<float4 *>(&xs[0][0]);                 // [RT][kQ - 1][64]
    float *ored = &xs[0][0] + RT * (kQ - 1) * 64 * 4;                    // [RT][4][64]
    const v4f part = acc0 + acc1;
    if (q > 0) red[(rt * (kQ - 1) + q - 1) * 64 + lane] = make_float4(part[0], part[1], part[2], part[3]);
    if (outw) ored[(rt * 4 + q) * 64 + lane] = o;
    __syncthreads();
    if (q > 0) return;
    float sum[4] = {part[0], part[1], part[2], part[3]};
#pragma unroll
    for (int r = 0; r < kQ - 1; ++r) {
        const float4 t = red[(rt * (kQ - 1) + r) * 64 + lane];
        sum[0] += t.x;
        sum[1] += t.y;
        sum[2] += t.z;
        sum[3] += t.w;
    }

    // ---- epilogue: lane holds rows m0 + 4 kk + v of token n
    if (n >= p.B) return;
    T *yn = static_cast<T *>(p.y) + (size_t)n * p.M;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int m = m0 + 4 * kk + v;
        if (m >= p.M) continue;
        float yv = sum[v] * gld(p.scales + m);
        if (p.bias) yv += gld(p.bias + m);
        store_act(yn, (size_t)m, yv + ored[(rt * 4 + v) * 64 + lane]);
    }
}

// ---- 32-row x 32-token tiles on bf16 MFMA
//
// lut_mm32_kernel: workgroup = 32 RT rows x 32 TT tokens (RT TT <= 2), 8 waves:
// wave q computes the RT x TT 32 x 32 tiles over groups 2q, 2q + 1 of every
// 16-group input slice (each A operand serves every token tile, each B operand
// every row tile), on v_mfma_f32_32x32x16_bf16 (one 16-dimension group per
// MFMA):
//   A[m][k] = C[code(m, g)][k]  (the codebook's exact bf16 pieces, staged in LDS),
//   B[k][n] = x_n[16 g + k]     (x staged per slice in LDS as fp32, split into
//                                exact bf16 pieces at use; bf16 activations are
//                                one piece already),
// with the six products a_i b_j, i + j <= 4, of fp32 inputs (x split by
// truncation, split3_trunc: the three left out are below 2^-22 of |a b|) or
// the three a_i b of bf16 inputs, all accumulated in fp32 (mfma32_bf16x3's
// operand layout).  A 32 x 32 tile reads 3 KB of A and 1-3 KB of B per group
// for 16384 multiply-adds, against 2 KB per 4096 for the 16 x 16 fp32 tiles
// of lut_mm_kernel.  Every workgroup splits the x of its tokens for itself: two
// row tiles per workgroup halve that work per row.  The x slices are staged
// through a register ring one slice ahead; codes kM32PF slices ahead.
//
// The 8 waves' partial tiles meet in LDS at the end, added in wave order; wave
// q then finishes the values r = 2q, 2q + 1 of its lanes in every tile (rows
// 8 (r / 4) + 4 h + r % 4 of token n, h = lane / 32, n = lane % 32).  The CSR
// outliers are added slice by slice from the staged x (entries in LDS, sorted
// by column; thread tid takes row tid / TPR for tokens tid % TPR + TPR k), or
// from memory when the workgroup's rows hold more than the staging holds;
// their sums reach the epilogue through LDS.  Epilogue
// (s_m * sum + bias) + outliers.
namespace {
constexpr int kM32XS = 260;      // floats per staged x row (256 + pad: conflict-free b128 reads)
constexpr int kM32PF = 4;        // slices of codes in flight
constexpr int kM32NT = 512;      // threads: 8 waves
// above 32 tokens: two row tiles per workgroup (else two token tiles)
template <typename T> constexpr bool kM32RowPairs = std::is_same<T, float>::value;
}  // namespace

// Exact three-way bf16 split of 8 fp32 values by truncation: v = p0 + p1 + p2,
// p0 = v with its low 16 bits cleared, p1 the same of v - p0, p2 = v - p0 - p1
// (the remainders are exact in fp32; p2 has at most 8 significant bits, a
// bf16 value).  |p1| < 2^-7 |v|, |p2| < 2^-15 |v|.  About five operations per
// value (1.5 of them packing).
__device__ __forceinline__ void split3_trunc(const float (&v)[8], bf16x8_t (&p)[3]) {
    uint32_t w[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t ua = __float_as_uint(v[2 * i]), ub = __float_as_uint(v[2 * i + 1]);
        const float ra = v[2 * i] - __uint_as_float(ua & 0xffff0000u);
        const float rb = v[2 * i + 1] - __uint_as_float(ub & 0xffff0000u);
        const uint32_t ura = __float_as_uint(ra), urb = __float_as_uint(rb);
        const float sa = ra - __uint_as_float(ura & 0xffff0000u);
        const float sb = rb - __uint_as_float(urb & 0xffff0000u);
        // high halves of (a, b) into one word, element 2i in its low half
        w[0][i] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
        w[1][i] = __builtin_amdgcn_perm(urb, ura, 0x07060302u);
        w[2][i] = __builtin_amdgcn_perm(__float_as_uint(sb), __float_as_uint(sa), 0x07060302u);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) __builtin_memcpy(&p[k], w[k], sizeof(bf16x8_t));
}

template <typename T, int RT, int TT>
__global__ __launch_bounds__(kM32NT) void lut_mm32_kernel(MmParams p) {
    constexpr int KP = kM32NT / 64;               // input parts, one wave each
    constexpr int GPS = 16 / KP;                  // groups per slice per wave
    constexpr int RV = 16 / KP;                   // tile values a wave finishes
    constexpr int NROW = 32 * RT, NTOK = 32 * TT;
    constexpr int XU = NTOK * 64 / kM32NT;        // float4 of a slice's x per thread
    constexpr int NC = 512 * RT;                  // CSR entries staged per workgroup
    constexpr int TPR = kM32NT / NROW;            // outlier threads per row
    constexpr int NOT = NTOK / TPR;               // tokens per outlier thread
    constexpr bool BF = !std::is_same<T, float>::value;
    static_assert(RT * TT <= 2 && GPS == 2, "tile shapes");
    // [centroid][half][piece], 16-byte units: 7 per centroid where the LDS
    // allows (112-byte rows put 16 lanes' random rows over all 16 four-bank
    // groups instead of 8: 16.9 -> 16.2 us for bf16 x at 16 tokens), else 6;
    // the outlier sums at the end
    constexpr int CBS = TT == 2 ? 6 : 7;
    __shared__ bf16x8_t cb3s[256 * CBS];
    __shared__ __align__(16) float xs[2][NTOK * kM32XS];   // x slices; the partial tiles at the end
    __shared__ unsigned short lcol[NC];
    __shared__ float lval[NC];
    static_assert(RT * TT * KP * 16 * 64 <= 2 * NTOK * kM32XS &&
                      NROW * NTOK * sizeof(float) <= sizeof(cb3s),
                  "partial tiles and outlier sums fit the staging buffers");
    const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
    const int h = lane >> 5, n = lane & 31;
    const int m0 = blockIdx.x * NROW;
    const int n0 = blockIdx.y * NTOK;
    int arow[RT];                                 // the lane's A rows (rows past M: never stored)
#pragma unroll
    for (int r = 0; r < RT; ++r) arow[r] = min(m0 + 32 * r + n, p.Mp - 1);
    auto row_of = [&](int v) { return 8 * (v >> 2) + 4 * h + (v & 3); };   // tile row of value v

    // ---- round trip 1: the codebook pieces, x slices 0 and 1, the CSR ranges, codes
    constexpr int CBU = 256 * 2 * 3 / kM32NT;
    const bf16x8_t *gcb = static_cast<const bf16x8_t *>(p.cb3);
    bf16x8_t c3[CBU];
#pragma unroll
    for (int u = 0; u < CBU; ++u) c3[u] = gcb[tid + u * kM32NT];
    // x staging: thread tid holds float4 tid % 64 (dims 4 (tid % 64) ..) of
    // tokens tid / 64 + 8 u, u < XU.  Tokens past B read the last token and
    // feed only outputs that are never stored; dims past K (a last partial
    // slice) are clamped on load and zeroed before the store.
    const int xd = 4 * (tid & 63);
    size_t xrow[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) xrow[u] = (size_t)min(n0 + (tid >> 6) + 8 * u, p.B - 1) * p.K;
    auto load_x = [&](int s, float4 (&r)[XU]) __attribute__((always_inline)) {
        const T *xs0 = static_cast<const T *>(p.x) + min(s * 256 + xd, p.K - 4);
#pragma unroll
        for (int u = 0; u < XU; ++u) r[u] = load4_act(xs0, xrow[u]);
    };
    auto store_x = [&](int s, float *dst, float4 (&r)[XU]) __attribute__((always_inline)) {
        if (s * 256 + xd >= p.K)                  // K % 16 == 0: a float4 is in or out
#pragma unroll
            for (int u = 0; u < XU; ++u) r[u] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < XU; ++u)
            reinterpret_cast<float4 *>(dst + ((tid >> 6) + 8 * u) * kM32XS)[tid & 63] = r[u];
    };
    float4 x0[XU], xr[XU];
    load_x(0, x0);
    load_x(min(1, p.S - 1), xr);
    // outliers: thread tid adds those of row ro = tid / TPR for tokens
    // tid % TPR + TPR k, k < NOT
    const int ro = tid / TPR, to = tid % TPR;
    int e_lo = 0, e_hi = 0, j = 0, je = 0;
    if (p.rowp) {
        e_lo = gld(p.rowp + m0);
        e_hi = gld(p.rowp + min(m0 + NROW, p.M));
        j = gld(p.rowp + min(m0 + ro, p.M - 1));
        je = m0 + ro < p.M ? gld(p.rowp + m0 + ro + 1) : j;
    }
    uint32_t cr[kM32PF][RT];   // codes of slices s .. s + kM32PF - 1, slot s % kM32PF
    auto load_codes = [&](int s, int r) __attribute__((always_inline)) {
        return (uint32_t)gld(reinterpret_cast<const unsigned short *>(
            p.codes + ((size_t)s * p.Mp + arow[r]) * 16 + GPS * q));
    };
#pragma unroll
    for (int u = 0; u < kM32PF; ++u)
#pragma unroll
        for (int r = 0; r < RT; ++r) cr[u][r] = load_codes(min(u, p.S - 1), r);
    // ---- round trip 2: the CSR entries of the workgroup's rows into LDS when they fit
    const bool staged = e_hi - e_lo <= NC;
    if (p.rowp && staged && e_hi > e_lo) {
#pragma unroll
        for (int u = 0; u < NC / kM32NT; ++u) {
            const int i = tid + u * kM32NT;
            const int e = min(e_lo + i, e_hi - 1);
            const int c = gld(p.col + e);
            const float v = gld(p.val + e);
            if (e_lo + i < e_hi) {
                lcol[i] = (unsigned short)c;
                lval[i] = v;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < CBU; ++u) {
        const int i = tid + u * kM32NT;
        cb3s[(i / 6) * CBS + i % 6] = c3[u];
    }
    store_x(0, xs[0], x0);
    __syncthreads();

    f32x16_t acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x16_t{};
    float o[NOT];
#pragma unroll
    for (int k = 0; k < NOT; ++k) o[k] = 0.f;
    j -= e_lo;
    je -= e_lo;
    const bool outl = p.rowp && staged;
    // Slice s: code slot s % kM32PF, a constant in the unrolled body; the
    // slot is refilled with slice s + kM32PF, and the x ring with slice s + 2,
    // unconditionally (clamped to the last slice), so the loop body has one
    // path and the wait counts of the rings stay exact across its back edge.
    auto slice = [&](const int s, const int u) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < GPS; ++i) {
            const int g = GPS * q + i;
            bf16x8_t a[RT][3];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const uint32_t code = (cr[u][r] >> (8 * i)) & 0xffu;
                const bf16x8_t *ap = cb3s + code * CBS + h * 3;
                a[r][0] = ap[0];
                a[r][1] = ap[1];
                a[r][2] = ap[2];
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float *xt = xs[s & 1] + (32 * t + n) * kM32XS + 16 * g + 8 * h;
                const float4 xa = *reinterpret_cast<const float4 *>(xt);
                const float4 xb = *reinterpret_cast<const float4 *>(xt + 4);
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                if constexpr (BF) {
                    bf16x8_t b;
#pragma unroll
                    for (int e = 0; e < 8; ++e) b[e] = (__bf16)xv[e];   // exact: bf16 values
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][2], b, acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][1], b, acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][0], b, acc[r][t], 0, 0, 0);
                    }
                } else {
                    bf16x8_t b[3];
                    split3_trunc(xv, b);
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][0], b[2], acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][1], b[1], acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][2], b[0], acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][0], b[1], acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][1], b[0], acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r][0], b[0], acc[r][t], 0, 0, 0);
                    }
                }
            }
        }
        // the thread's outliers whose columns fall in this slice, in column
        // order (a row's entries are sorted by column): kOutPass candidates
        // per pass, the reads of a pass in flight together (one pass covers a
        // slice unless the row has more entries in it)
        if (outl) {
            const float *xsl = xs[s & 1] + to * kM32XS - s * 256;
            const int lim = (s + 1) * 256;
            bool more = true;
            while (more) {
                int c[kOutPass];
                float vv[kOutPass];
#pragma unroll
                for (int k = 0; k < kOutPass; ++k) {
                    const int e = min(j + k, NC - 1);
                    c[k] = lcol[e];
                    vv[k] = lval[e];
                }
                bool in = true;
                int took = 0;
#pragma unroll
                for (int k = 0; k < kOutPass; ++k) {
                    in = in && j + k < je && c[k] < lim;
                    const int cc = in ? c[k] : s * 256;
#pragma unroll
                    for (int v = 0; v < NOT; ++v) {
                        const float xv = xsl[TPR * v * kM32XS + cc];
                        if (in) o[v] += vv[k] * xv;
                    }
                    took += in ? 1 : 0;
                }
                j += took;
                more = took == kOutPass;
            }
        }
        // slice s + 1 into the other buffer (past the last slice: a clamped
        // reload, never read), then the rings refilled
        store_x(min(s + 1, p.S - 1), xs[(s + 1) & 1], xr);
        load_x(min(s + 2, p.S - 1), xr);
#pragma unroll
        for (int r = 0; r < RT; ++r) cr[u][r] = load_codes(min(s + kM32PF, p.S - 1), r);
        __syncthreads();   // slice s + 1 staged; slice s's reads done before it is overwritten
    };
    int s0 = 0;
    for (; s0 + kM32PF <= p.S; s0 += kM32PF) {
#pragma unroll
        for (int u = 0; u < kM32PF; ++u) slice(s0 + u, u);
    }
#pragma unroll
    for (int u = 0; u < kM32PF - 1; ++u)
        if (s0 + u < p.S) slice(s0 + u, u);

    // ---- a dense-outlier block: the row's entries and x from memory
    if (p.rowp && !staged && m0 + ro < p.M)
#pragma unroll
        for (int v = 0; v < NOT; ++v) {
            const int nn = n0 + to + TPR * v;
            if (nn >= p.B) continue;
            const T *xn = static_cast<const T *>(p.x) + (size_t)nn * p.K;
            for (int e = j; e < je; ++e) o[v] += gld(p.val + e_lo + e) * load_act(xn, gld(p.col + e_lo + e));
        }
    // ---- the waves' partial tiles and the outlier sums through LDS (the
    // staging buffers are free: the last slice ended with a barrier); the
    // partial tiles are summed in wave order
    float *red = &xs[0][0];                       // [RT][TT][KP][16][64]
    float *osum = reinterpret_cast<float *>(cb3s);   // [NROW][NTOK]
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) red[(((r * TT + t) * KP + q) * 16 + v) * 64 + lane] = acc[r][t][v];
#pragma unroll
    for (int v = 0; v < NOT; ++v) osum[ro * NTOK + to + TPR * v] = o[v];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int i = 0; i < RV; ++i) {
            const int v = RV * q + i;
            const int mr = 32 * r + row_of(v);            // row within the workgroup
            const int m = m0 + mr;
            if (m >= p.M) continue;
            const float sc = gld(p.scales + m);
            const float bs = p.bias ? gld(p.bias + m) : 0.f;
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int nn = n0 + 32 * t + n;
                if (nn >= p.B) continue;
                const float *rt = red + ((r * TT + t) * KP * 16 + v) * 64 + lane;
                float sum = rt[0];
#pragma unroll
                for (int qq = 1; qq < KP; ++qq) sum += rt[qq * 16 * 64];
                float yv = sum * sc;
                if (p.bias) yv += bs;
                store_act(static_cast<T *>(p.y) + (size_t)nn * p.M, (size_t)m,
                          yv + osum[mr * NTOK + 32 * t + n]);
            }
        }
}

// Tile shape by batch: one 32 x 32 tile per workgroup up to 32 tokens; above,
// two tiles per workgroup: two row tiles for fp32 x (each workgroup splits
// half as much x per row), two token tiles for bf16 x (no split: each A
// operand serves both).
template <typename T>
static void launch_mm32_t(const MmParams &p, hipStream_t st) {
    const int gx1 = (p.M + 31) / 32, gx2 = (p.M + 63) / 64;
    if (p.B <= 32)
        OJX_LAUNCH((lut_mm32_kernel<T, 1, 1>), dim3(gx1, (p.B + 31) / 32), dim3(kM32NT), 0, st, p);
    else if (kM32RowPairs<T>)
        OJX_LAUNCH((lut_mm32_kernel<T, 2, 1>), dim3(gx2, (p.B + 31) / 32), dim3(kM32NT), 0, st, p);
    else
        OJX_LAUNCH((lut_mm32_kernel<T, 1, 2>), dim3(gx1, (p.B + 63) / 64), dim3(kM32NT), 0, st, p);
}

// Row tiles per workgroup by batch: small batches take one tile per
// workgroup for the most workgroups, larger ones share the staged x among
// more tiles.
static int mm_row_tiles(int B) { return B <= 16 ? 1 : B <= 32 ? 2 : 4; }

template <typename T>
static void launch_mm_t(const MmParams &p, int rt, int gy, hipStream_t st) {
    if (rt == 1)
        OJX_LAUNCH((lut_mm_kernel<T, 1>), dim3((p.M + 15) / 16, gy), dim3(MmShape<1>::kNT), 0, st, p);
    else if (rt == 2)
        OJX_LAUNCH((lut_mm_kernel<T, 2>), dim3((p.M + 31) / 32, gy), dim3(MmShape<2>::kNT), 0, st, p);
    else
        OJX_LAUNCH((lut_mm_kernel<T, 4>), dim3((p.M + 63) / 64, gy), dim3(MmShape<4>::kNT), 0, st, p);
}

// From this many tokens the 32 x 32 bf16-MFMA tiles run (lut_mm32_kernel):
// fp32 x from 17 (at 9-16 the 16 x 16 fp32 tiles are faster: 17.6-18.0 vs
// 18.4-18.7 us at 2560->6912), bf16 x from 9 (16.9-17.0 vs 17.4-17.9 us).
constexpr int kMm32MinBatchF32 = 17;
constexpr int kMm32MinBatchBF16 = 9;

int launch_mm(const MmParams &p, int dtype, hipStream_t st) {
    const int gy = (p.B + kMmTok - 1) / kMmTok;
    if (gy > 65535) {
        set_error("batch %d too large for the MFMA path", p.B);
        return OJASX_ERR_INVALID;
    }
    if (p.cb3 && (dtype == OJASX_DTYPE_F32 ? p.B >= kMm32MinBatchF32
                                           : p.B >= kMm32MinBatchBF16 &&
                                                 reinterpret_cast<uintptr_t>(p.x) % 8 == 0)) {
        if (dtype == OJASX_DTYPE_F32)
            launch_mm32_t<float>(p, st);
        else
            launch_mm32_t<__hip_bfloat16>(p, st);
        OJX_HIP(hipGetLastError());
        return OJASX_OK;
    }
    const int rt = mm_row_tiles(p.B);
    if (dtype == OJASX_DTYPE_F32)
        launch_mm_t<float>(p, rt, gy, st);
    else
        launch_mm_t<__hip_bfloat16>(p, rt, gy, st);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // namespace ojx

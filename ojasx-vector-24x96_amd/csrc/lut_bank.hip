// lut_bank.hip -- many independent batch-1 LUT linears (block_dim 16, 256
// centroids, fp32) in one launch, with gathers that never conflict in LDS.
//
// y_i[m] = (s_m * sum_g LUT_i[g, codes_i[m, g]] + bias_i[m]) + sum_j val_j x_i[col_j]
// with LUT_i[g, k] = <x_i[16g .. 16g + 16), C_i[k]> (ojasx_lut_cpu.cpp:18-206).
//
// The LDS has 32 banks of 4 bytes; a wave's 4-byte reads run as two halves
// of 32 lanes, and each half takes as many cycles as the most requests any
// one bank receives.  A lane-per-row gather reads LUT[g][code] at random
// banks (measured on gfx950: 7.5 cycles per wave read against 2.4 when every
// lane of a half reads its own bank).  Here a lane owns a GROUP instead:
//  * the LUT of a slice of 32 groups is stored code-major, word
//    code * 64 + 32 * buffer + g, so group g lives in bank g whatever the code
//    and the 32 lanes of a half-wave (groups 0..31) never share a bank;
//  * lane (h, g) of a wave gathers group g of 32 rows (half h of the wave's 64
//    rows), one accumulator per row, over the slices in order;
//  * after the last slice a butterfly across the 32 lanes of each half
//    (v_permlane16_swap, then DPP row mirror, half mirror and quad permutes;
//    at each stage a lane keeps the half of its rows its lane bit selects)
//    leaves row r's sum in lane r.
// The byte address of an entry, code * 256 + 4 g + 128 * buffer, is one
// v_perm_b32 of the code word and a per-lane constant.
//
// LUT build: per slice, LUT^T[256 x 32] = C[256 x 16] . X_s^T[16 x 32], wave
// w computing centroids 32w .. 32w + 31 on v_mfma_f32_32x32x16_bf16 over an
// exact three-way bf16 split of both operands (six products, fp32 sums:
// fp32 accuracy at 2.7x fewer matrix cycles than eight fp32 32x32x2 steps).
// Its output lane (h, n) holds rows 8(r/4) + 4h + r%4 of column n, so the
// stores of each half-wave hit 32 distinct banks.  Lane half h supplies input
// dimensions 8h .. 8h + 7 of both operands: 8 contiguous floats of x and of
// its codebook row.  The codebook is split once when the handle is made (its
// pieces loaded as they are), x once per workgroup when it is staged (its
// three pieces side by side in LDS, zero rows up to the last slice's end, so
// groups past G give zero LUT columns).
// Two LUT buffers in the 64-word rows: slice s + 1 is built while slice s is
// gathered, one barrier per slice.
//
// Codes come from the handle's bank layout [row block of 64][slice][group]
// [64 rows]: a lane's 32 codes of a slice are 32 contiguous bytes, a wave's
// 2 KB contiguous; kBPF slices are in flight in a register ring.
// Outliers: the workgroup's CSR range (its rows are contiguous) is loaded
// coalesced (most of it before the slice loop), the products val * x[col]
// staged in the then free LUT space, and each lane adds its row's products in
// CSR order.
#include <algorithm>

#include "common.h"

namespace ojx {

namespace {
constexpr int kBW = 8;                  // waves per workgroup
constexpr int kBNT = kBW * 64;          // threads per workgroup
constexpr int kBRows = kBW * 64;        // rows per workgroup: 32 per half-wave
constexpr int kBPF = 2;                 // slices of codes in flight
constexpr int kLutRow = 64;             // words per code in the LUT: two buffers of 32 groups
constexpr int kStagePT = 12;            // CSR entries staged per thread
constexpr int kEarlyPT = 10;            // of which loaded before the slice loop
constexpr int kStage = kStagePT * kBNT; // per workgroup (4 B each, in the 64 KB LUT space)
typedef f32x16_t v16f;

// Codes of slice s for lane (h, g) from the block's bank layout [G][64 rows]:
// cp points at group g, rows 32h...  In a partial last slice the lanes past G
// read the bytes after the block (the next block's, or the kBankSlack bytes
// allocated after the last one): their LUT column is 0, so any code adds 0.
// (A clamp here would cost the loop its immediate load offsets.)
__device__ __forceinline__ void bank_codes(const uint8_t *cp, int s, uint4 (&c)[2]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(cp + 2048 * s);
    c[0] = gld(p);
    c[1] = gld(p + 1);
}

// x staged in LDS once per workgroup, already split into its three bf16
// pieces (x = x1 + x2 + x3 exactly, see split3_bf16): a row of kXRow words per
// group, piece p in words 8p .. 8p + 7 (16 bf16), no padding (two
// workgroups per CU up to K = 2560: 64 KB of LUT + 96 B per group each).  x
// itself is (x1 + x2) + x3 in fp32, exact (24 significant bits).
constexpr int kXRow = 24;

typedef bf16x8_t v8bf;

// MFMA B operand of slice s: the three pieces of x[16 (32 s + g) + 8 h .. + 8)
// from the staged x (zero rows for the groups past G up to the slice's end,
// so their LUT columns come out 0).
__device__ __forceinline__ void bank_xop(const float *xs, int s, int g, int h, v8bf (&b)[3]) {
    const v8bf *p = reinterpret_cast<const v8bf *>(xs + (32 * s + g) * kXRow + 4 * h);
    b[0] = p[0];
    b[1] = p[2];
    b[2] = p[4];
}

// x[k] from its staged pieces.
__device__ __forceinline__ float xs_value(const float *xs, int k) {
    const __bf16 *r = reinterpret_cast<const __bf16 *>(xs + (k >> 4) * kXRow) + (k & 15);
    return ((float)r[0] + (float)r[16]) + (float)r[32];
}

// LUT tile = C_tile . X_s^T on v_mfma_f32_32x32x16_bf16 (16 input dims in one
// step) over the exact bf16 splits of C and x (mfma32_bf16x3: fp32 accuracy).
// A lane's 8 values are dimensions 8h .. 8h + 7 in both operands.
__device__ __forceinline__ v16f bank_build(const v8bf (&a)[3], const v8bf (&b)[3]) {
    return mfma32_bf16x3(a, b);
}

// LUT[32 w + m][g] of buffer buf <- column g of the wave's tile.
__device__ __forceinline__ void bank_store(float *L, int buf, int w, int g, int h, const v16f &d) {
    float *p = L + (32 * w + 4 * h) * kLutRow + 32 * buf + g;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[(8 * (r / 4) + (r % 4)) * kLutRow] = d[r];
}

// acc[j] += LUT[code of row j][g] for the 32 rows of the lane's half.  gsel
// byte 0 = 4 g + 128 buffer, byte 2 = bits 16-23 of the LUT's byte offset
// from L (so a LUT 64 KB above L costs no address add per read).
__device__ __forceinline__ void bank_gather(const float *L, uint32_t gsel, const uint4 (&c)[2],
                                            float (&acc)[32]) {
    const uint32_t wd[8] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w};
    const char *Lb = reinterpret_cast<const char *>(L);
    // eight reads in flight at a time: addresses, then the reads, then the adds
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // byte 1 <- the code (byte i % 4 of its word), bytes 0 and 2 <- gsel's
            const uint32_t a = __builtin_amdgcn_perm(wd[2 * q2 + i / 4], gsel,
                                                     0x0c020400u + ((i % 4) << 8));
            v[i] = *reinterpret_cast<const float *>(Lb + a);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[8 * q2 + i] += v[i];
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum of acc[r] over the 32 lanes of each half-wave, returned in lane r.
__device__ __forceinline__ float bank_reduce(const float (&acc)[32], int lane) {
    float a16[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {   // lanes 16..31 <-> 0..15: rows j (low lanes), j + 16 (high)
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[j]),
                                                        __float_as_uint(acc[j + 16]), false, false);
        a16[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2, b0 = lane & 1;
    float a8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {    // row mirror: lane i <-> 15 - i (bit 3 flips)
        const float lo = a16[j] + dpp_f<0x140>(a16[j]);
        const float hi = a16[j + 8] + dpp_f<0x140>(a16[j + 8]);
        a8[j] = b3 ? hi : lo;
    }
    float a4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {    // half mirror: lane i <-> 7 - i within 8 (bit 2 flips)
        const float lo = a8[j] + dpp_f<0x141>(a8[j]);
        const float hi = a8[j + 4] + dpp_f<0x141>(a8[j + 4]);
        a4[j] = b2 ? hi : lo;
    }
    float a2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {    // quad_perm [2,3,0,1]: bit 1 flips
        const float lo = a4[j] + dpp_f<0x4E>(a4[j]);
        const float hi = a4[j + 2] + dpp_f<0x4E>(a4[j + 2]);
        a2[j] = b1 ? hi : lo;
    }
    const float lo = a2[0] + dpp_f<0xB1>(a2[0]);    // quad_perm [1,0,3,2]: bit 0 flips
    const float hi = a2[1] + dpp_f<0xB1>(a2[1]);
    return b0 ? hi : lo;
}
}  // namespace

// One 512-row block of one matrix: its bank-layout codes, codebook, scales,
// optional bias and CSR outliers, input and output.
struct BankBlock {
    const uint8_t *codes_b;     // the matrix's bank layout [ceil(M/64)][G][64]
    const v8bf *cb3;            // [256][2][3] the codebook's bf16 pieces (split_codebook_bf16x3)
    const float *scales;        // [M]
    const float *bias;          // [M] or null
    const int *rowp;            // [M + 1] or null
    const uint16_t *col;        // [nnz] 16-bit columns (K <= 16384 here)
    const float *val;
    const void *x;              // XS_F32: [K] fp32; XS_BF16: [K] bf16; XS_SWIGLU: [2K] fp32
    float *y;                   // [M]
    int K, M, base;
};
enum { XS_F32 = 0, XS_BF16 = 1, XS_SWIGLU = 2 };

// x (or silu(gate) * up, silu(v) = v / (1 + exp(-v))) into LDS, float4 i
// holding dims 4(i%4).. of group i/4; two loads in flight per thread.
// Dims 4 (i % 4) .. + 3 of group i / 4 into the staged rows, as three pieces.
__device__ __forceinline__ void bank_put_x(float *xs, int i, float4 v) {
    const float f[4] = {v.x, v.y, v.z, v.w};
    __bf16 pc[3][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const __bf16 h1 = (__bf16)f[k];
        const float r1 = f[k] - (float)h1;
        const __bf16 h2 = (__bf16)r1;
        pc[0][k] = h1;
        pc[1][k] = h2;
        pc[2][k] = (__bf16)(r1 - (float)h2);
    }
    uint2 *row = reinterpret_cast<uint2 *>(xs + (i >> 2) * kXRow) + (i & 3);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        uint2 w;
        __builtin_memcpy(&w, pc[p], 8);
        row[4 * p] = w;
    }
}

template <int XS>
__device__ __forceinline__ void bank_stage_x(const void *x, int K, float *xs, int tid) {
    for (int i = tid; i < K / 4; i += 2 * kBNT) {
        const int i2 = min(i + kBNT, K / 4 - 1);
        float4 u, v;
        if constexpr (XS == XS_F32) {
            const float4 *x4 = static_cast<const float4 *>(x);
            u = gld(x4 + i);
            v = gld(x4 + i2);
        } else if constexpr (XS == XS_BF16) {
            const __hip_bfloat16 *xb = static_cast<const __hip_bfloat16 *>(x);
            u = load4_act(xb, (size_t)4 * i);
            v = load4_act(xb, (size_t)4 * i2);
        } else {
            const float4 *g4 = static_cast<const float4 *>(x), *u4 = g4 + K / 4;
            const float4 ga = gld(g4 + i), ua = gld(u4 + i), gb = gld(g4 + i2), ub = gld(u4 + i2);
            auto sw = [](float gg, float uu) { return gg / (1.f + expf(-gg)) * uu; };
            u = make_float4(sw(ga.x, ua.x), sw(ga.y, ua.y), sw(ga.z, ua.z), sw(ga.w, ua.w));
            v = make_float4(sw(gb.x, ub.x), sw(gb.y, ub.y), sw(gb.z, ub.z), sw(gb.w, ub.w));
        }
        bank_put_x(xs, i, u);
        bank_put_x(xs, i2, v);
    }
    // zero rows for groups G .. 32 S - 1 (the last slice's missing groups)
    const int G = K >> 4, GS = ((G + 31) >> 5) << 5;
    float4 *z = reinterpret_cast<float4 *>(xs + G * kXRow);
    for (int i = tid; i < (GS - G) * (kXRow / 4); i += kBNT) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int XS>
__device__ __forceinline__ void bank_block(const BankBlock &bb, float *L, float *xs) {
    const int base = bb.base;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, g = lane & 31;
    const int K = bb.K, G = K >> 4, S = (G + 31) >> 5;
    const int rb = min((base >> 6) + w, ((bb.M + 63) >> 6) - 1);   // past M: a real block, unused
    const uint8_t *cp = bb.codes_b + ((size_t)rb * G + g) * 64 + 32 * h;
    const int m = base + 64 * w + 32 * h + g;        // the row this lane finishes
    const int mc = min(m, bb.M - 1);
    const bool outl = bb.rowp != nullptr;

    // ---- round trip 1: L2-resident operands first, then the HBM codes
    // MFMA A operand: centroid 32 w + g, dims 8 h .. 8 h + 7, three bf16 pieces
    v8bf a[3];
    {
        const v8bf *p = bb.cb3 + ((32 * w + g) * 2 + h) * 3;
        a[0] = gld(p);
        a[1] = gld(p + 1);
        a[2] = gld(p + 2);
    }
    const float sc = gld(bb.scales + mc);
    const float bs = bb.bias ? gld(bb.bias + mc) : 0.f;
    int j0 = 0, j1 = 0, e0 = 0, e1 = 0;
    if (outl) {
        j0 = gld(bb.rowp + mc);
        j1 = m < bb.M ? gld(bb.rowp + mc + 1) : j0;
        e0 = gld(bb.rowp + base);
        e1 = gld(bb.rowp + min(base + kBRows, bb.M));
    }
    uint4 ring[kBPF][2];
#pragma unroll
    for (int q = 0; q < kBPF; ++q) bank_codes(cp, min(q, S - 1), ring[q]);
    bank_stage_x<XS>(bb.x, K, xs, tid);
    const uint32_t gsel0 = 4u * g, gsel1 = 4u * g + 128u;
    __syncthreads();

    // ---- slice 0 into buffer 0
    v8bf b[3];
    bank_xop(xs, 0, g, h, b);
    {
        const v16f d = bank_build(a, b);
        bank_store(L, 0, w, g, h, d);
    }
    bank_xop(xs, min(1, S - 1), g, h, b);
    __syncthreads();

    // The outliers' loads (the workgroup's CSR range, coalesced): the first
    // kEarlyPT per thread go out now, under the slices; the rest, needed only
    // by ranges longer than kEarlyPT * 512 entries, before the last slice
    // (all of them here would hold 24 registers across the slice loop).
    const int ne = min(e1 - e0, kStage);
    int cl[kStagePT];
    float vl[kStagePT];
    if (ne > 0) {
#pragma unroll
        for (int i = 0; i < kEarlyPT; ++i) {
            const int e = e0 + min(tid + i * kBNT, ne - 1);
            cl[i] = gld(bb.col + e);
            vl[i] = gld(bb.val + e);
        }
    }
    float acc[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) acc[j] = 0.f;
    // Slice s uses ring slot q = s % kBPF, a constant in the unrolled body (no
    // register moves of loads in flight); refills run unconditionally, clamped
    // to the last slice (past it: a reload), so the loop body has no branch
    // and the wait counts for the ring stay exact.  Slices 0 .. S-2 build the
    // next slice's LUT beside their gathers; the last slice builds nothing.
    auto one = [&](const int s, const int q) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        const v16f d = bank_build(a, b);                         // slice s + 1
        bank_gather(L, (s & 1) ? gsel1 : gsel0, ring[q], acc);   // slice s
        bank_codes(cp, min(s + kBPF, S - 1), ring[q]);
        __builtin_amdgcn_sched_barrier(0);                       // b is read by the build above
        bank_xop(xs, min(s + 2, S - 1), g, h, b);
        bank_store(L, (s + 1) & 1, w, g, h, d);
        __syncthreads();
    };
    int sb = 0;
    for (; sb + kBPF <= S - 1; sb += kBPF) {
#pragma unroll
        for (int q = 0; q < kBPF; ++q) one(sb + q, q);
    }
#pragma unroll
    for (int q = 0; q < kBPF - 1; ++q)
        if (sb + q < S - 1) one(sb + q, q);
    if (ne > kEarlyPT * kBNT) {
#pragma unroll
        for (int i = kEarlyPT; i < kStagePT; ++i) {
            const int e = e0 + min(tid + i * kBNT, ne - 1);
            cl[i] = gld(bb.col + e);
            vl[i] = gld(bb.val + e);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if ((S - 1) % kBPF == 0)                                     // the last slice
        bank_gather(L, ((S - 1) & 1) ? gsel1 : gsel0, ring[0], acc);
    else
        bank_gather(L, ((S - 1) & 1) ? gsel1 : gsel0, ring[1], acc);
    static_assert(kBPF == 2, "the last slice's ring slot is picked from two");
    __syncthreads();

    // ---- outliers: each staged entry's product val * x[col] goes to the LUT
    //      space, then every lane sums its row's products in CSR order (the
    //      entries past the stage from memory)
    float *sp = L;
    const float tot = bank_reduce(acc, lane);
    if (ne > 0) {
#pragma unroll
        for (int i = 0; i < kStagePT; ++i)
            if (tid + i * kBNT < ne) sp[tid + i * kBNT] = vl[i] * xs_value(xs, cl[i]);
        __syncthreads();
    }
    float o = 0.f;
    const int js = max(j0, min(j1, e0 + ne));
    int j = j0;
    for (; j + 4 <= js; j += 4) {
        float pr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) pr[u] = sp[j + u - e0];
#pragma unroll
        for (int u = 0; u < 4; ++u) o += pr[u];
    }
    for (; j < js; ++j) o += sp[j - e0];
    for (; j < j1; ++j) o += gld(bb.val + j) * xs_value(xs, gld(bb.col + j));
    float y = tot * sc;
    if (bb.bias) y += bs;
    if (m < bb.M) bb.y[m] = y + o;
}

// The grouped linear call: workgroup i takes work[i] = (item, first row).
__global__ __launch_bounds__(kBNT) void lut_bank_kernel(const GroupItem *__restrict__ items,
                                                        const int2 *__restrict__ work) {
    __shared__ float L[256 * kLutRow];               // two LUT buffers; then the products
    extern __shared__ float xs[];                    // [32 S][kXRow]: x pieces (B operands, outliers)
    const int2 wk = work[blockIdx.x];
    const GroupItem it = items[wk.x];
    const BankBlock bb{it.codes_b, static_cast<const v8bf *>(it.cb3), it.scales, it.bias, it.rowp, it.col16, it.val,
                       it.x, it.y, it.K, it.M, wk.y};
    bank_block<XS_F32>(bb, L, xs);
}

// MoE stages on the routed pairs (no outliers, no bias): gate/up (x = the
// pair's token row, M = 2I gate then up rows) or down (x = silu(gate) * up of
// the pair's gate/up row, M = H).  work[] = (pair, 512-row block << 16 |
// expert) comes from the plan kernel, sorted by expert; workgroup i takes position
// (i % 8) * ceil(n / 8) + i / 8, so each of the 8 XCDs (workgroups go to XCD
// i % 8) walks a contiguous stretch of the sorted list and the pairs of one
// expert read its codes back to back through one L2.
struct MoEBankParams {
    const uint8_t *codes_b;     // [E][bank layout of M x G]
    size_t expert_bytes;
    const v8bf *cb3;            // [256][2][3] the codebook's bf16 pieces
    const float *scales;        // [E][M]
    const void *x;              // gate/up: [T][K]; down: [P][2K] fp32
    float *y;                   // [P][M]
    const int *idx;             // [P] expert of each pair
    const float *w;             // [P] slot weights (direct mapping: the skip rule)
    const int2 *work;           // [n] (pair, block << 16 | expert), or null: direct mapping
    const int *n_work;          // n
    int M, K, k, E, nb;         // rows, inputs, slots per token, experts, row blocks per pair
};

template <int XS>
__global__ __launch_bounds__(kBNT) void moe_bank_kernel(MoEBankParams p) {
    __shared__ float L[256 * kLutRow];
    extern __shared__ float xs[];
    int pr, e, blk;
    if (p.work) {
        const int n = *p.n_work;
        const int q = (n + 7) >> 3;
        const int pos = (int)(blockIdx.x & 7) * q + (int)(blockIdx.x >> 3);
        if (pos >= n || (int)(blockIdx.x >> 3) >= q) return;
        const int2 wk = p.work[pos];
        pr = wk.x;
        e = wk.y & 0xffff;                            // the expert travels with the entry
        blk = wk.y >> 16;
    } else {
        // direct mapping, no plan: workgroup = (pair, row block) in pair
        // order; skipped pairs (ojasx_lut_cpu.cpp:284-286) exit at once
        pr = (int)blockIdx.x / p.nb;
        blk = (int)blockIdx.x - pr * p.nb;
        e = p.idx[pr];
        if (e < 0 || e >= p.E || fabsf(p.w[pr]) < 1e-8f) return;
    }
    const void *x;
    if constexpr (XS == XS_SWIGLU)
        x = static_cast<const float *>(p.x) + (size_t)pr * 2 * p.K;
    else if constexpr (XS == XS_BF16)
        x = static_cast<const __hip_bfloat16 *>(p.x) + (size_t)(pr / p.k) * p.K;
    else
        x = static_cast<const float *>(p.x) + (size_t)(pr / p.k) * p.K;
    const BankBlock bb{p.codes_b + (size_t)e * p.expert_bytes, p.cb3,
                       p.scales + (size_t)e * p.M, nullptr, nullptr, nullptr, nullptr,
                       x, p.y + (size_t)pr * p.M, p.K, p.M, blk * kBRows};
    bank_block<XS>(bb, L, xs);
}

// MoE stages with a group's input LUT resident over many row blocks.  Gate/up
// (XS_F32, XS_BF16; inputs of at most 4 slices, K <= 2048) runs token-major:
// the input codebook is shared by all experts, so a token's LUT serves every
// slot the token is routed to (group = token, k slots).  Down (XS_SWIGLU;
// at most 2 slices, K <= 1024) runs pair-major: group = one routed pair, its
// input silu(gate) * up of the pair's gate/up row, one slot.  Workgroup =
// (group, up to R consecutive units), unit u = (slot u / nb, 512-row block
// u % nb) of the group: all slices of the group's LUT are built once (the
// [256][64]-word buffer pairs of bank_block: slices 0-1, and 2-3 above them),
// one barrier, then the units' codes stream through the gathers with no
// barrier at all, unit i + 1's codes and scales in flight while unit i
// gathers.  Skipped slots (expert outside [0, E) or |w| < 1e-8,
// ojasx_lut_cpu.cpp:284-286) are passed over.  Each row sees the same LUT
// entries in the same order as in moe_bank_kernel: identical results.
struct MoEResParams {
    const uint8_t *codes_b;     // [E][bank layout of M x G]
    size_t expert_bytes;
    const v8bf *cb3;            // [256][2][3] the codebook's bf16 pieces
    const float *scales;        // [E][M]
    const void *x;              // gate/up: [T][K] fp32 or bf16; down: [P][2K] fp32
    float *y;                   // [P][M]
    const int *idx;             // [P]
    const float *w;             // [P]
    int M, K, k, E, nb, R, cpt; // rows, inputs, slots per group, experts, blocks per pair, units per workgroup, workgroups per group
};
constexpr int kResMaxUnits = 8;

// TEAMS teams of 8 waves share the LUT.  Gate/up: two teams (16 waves, 128 KB
// of LUT, one workgroup per CU); team q builds the slices q, q + 2 and runs
// the units i = q, q + 2, ... of the workgroup's list (one team of 8 waves,
// two per SIMD, measured 6-7 % slower there).  Down: one team, 64 KB of LUT,
// two workgroups per CU (two teams in one workgroup per CU measured slower).
template <int XS, int TEAMS>
__global__ __launch_bounds__(TEAMS * kBNT) void moe_resident_kernel(MoEResParams p) {
    constexpr int NSL = 2 * TEAMS;                   // slices the LUT holds
    // the LUT at a fixed LDS address (static), so the gathers' addresses need
    // no base add; the staged x (dynamic) after it
    __shared__ float Ls[TEAMS * 256 * kLutRow];
    extern __shared__ float xs[];
    const int K = p.K, G = K >> 4, S = (G + 31) >> 5, M = p.M;
    const int tid = threadIdx.x, lane = tid & 63, wt_ = tid >> 6, h = lane >> 5, g = lane & 31;
    const int w = wt_ & 7, team = TEAMS == 2 ? wt_ >> 3 : 0;
    const int t = (int)blockIdx.x / p.cpt, c = (int)blockIdx.x - t * p.cpt;
    const int u0 = c * p.R, u1 = min(u0 + p.R, p.k * p.nb);
    const int rb_last = ((M + 63) >> 6) - 1;

    // ---- the units' slots (L2), then the first valid unit's codes (HBM)
    unsigned mask = 0;
#pragma unroll
    for (int i = 0; i < kResMaxUnits; ++i) {
        const int u = min(u0 + i, u1 - 1);
        const int pr = t * p.k + u / p.nb;
        const int e = gld(p.idx + pr);
        const float wt = gld(p.w + pr);
        if (u0 + i < u1 && e >= 0 && e < p.E && fabsf(wt) >= 1e-8f) mask |= 1u << i;
    }
    if (!mask) return;                               // the same for every wave
    if (TEAMS == 2) mask &= team ? 0xaaaaaaaau : 0x55555555u;   // this team's units
    // codes of unit i (all slices, clamped to the last) and its rows' scale;
    // the unit's expert id is read again here (a cached load) rather than kept
    // in an array indexed at run time, which would live in scratch
    auto load_unit = [&](int i, uint4 (&cc)[NSL][2], float &sc) {
        const int u = u0 + i, b = u % p.nb;
        const int e = gld(p.idx + t * p.k + u / p.nb);
        const int rb = min(b * (kBRows / 64) + w, rb_last);
        const uint8_t *cp = p.codes_b + (size_t)e * p.expert_bytes + ((size_t)rb * G + g) * 64 + 32 * h;
#pragma unroll
        for (int s4 = 0; s4 < NSL; ++s4) bank_codes(cp, min(s4, S - 1), cc[s4]);
        const int m = b * kBRows + 64 * w + 32 * h + g;
        sc = gld(p.scales + (size_t)e * M + min(m, M - 1));
    };
    v8bf a[3];
    {
        const v8bf *ap = p.cb3 + ((32 * w + g) * 2 + h) * 3;
        a[0] = gld(ap);
        a[1] = gld(ap + 1);
        a[2] = gld(ap + 2);
    }
    uint4 cA[NSL][2], cB[NSL][2];
    float sA = 0.f, sB = 0.f;
    int iA = mask ? __builtin_ctz(mask) : kResMaxUnits;
    if (mask) load_unit(iA, cA, sA);
    mask &= mask - 1;

    // ---- the group's input staged as bf16 pieces, then every slice of its LUT
    const void *x;
    if constexpr (XS == XS_SWIGLU)
        x = static_cast<const float *>(p.x) + (size_t)t * 2 * K;
    else if constexpr (XS == XS_BF16)
        x = static_cast<const __hip_bfloat16 *>(p.x) + (size_t)t * K;
    else
        x = static_cast<const float *>(p.x) + (size_t)t * K;
    if (tid < kBNT) bank_stage_x<XS>(x, K, xs, tid);
    __syncthreads();
#pragma unroll
    for (int s4 = 0; s4 < NSL; ++s4) {
        if (s4 < S && (TEAMS == 1 || (s4 & 1) == team)) {
            v8bf b[3];
            bank_xop(xs, s4, g, h, b);
            const v16f d = bank_build(a, b);
            bank_store(Ls + (s4 >> 1) * 256 * kLutRow, s4 & 1, w, g, h, d);
        }
    }
    __syncthreads();

    // ---- the units: gathers from the resident LUT, the next unit's loads in flight
    // slice s4 at byte 65536 (s4 >> 1) + 128 (s4 & 1) + 4 g + 256 code of Ls
    static_assert(256 * kLutRow * sizeof(float) == 65536, "slices 2-3 start 64 KB above Ls");
    auto run = [&](int i, const uint4 (&cc)[NSL][2], float sc) __attribute__((always_inline)) {
        float acc[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) acc[j] = 0.f;
#pragma unroll
        for (int s4 = 0; s4 < NSL; ++s4)
            if (s4 < S) bank_gather(Ls, 4u * g + 128u * (s4 & 1) + ((uint32_t)(s4 >> 1) << 16), cc[s4], acc);
        const float tot = bank_reduce(acc, lane);
        const int u = u0 + i, b = u % p.nb;
        const int m = b * kBRows + 64 * w + 32 * h + g;
        if (m < M) p.y[(size_t)(t * p.k + u / p.nb) * M + m] = tot * sc;
    };
    while (iA < kResMaxUnits) {
        const int iB = mask ? __builtin_ctz(mask) : kResMaxUnits;
        mask &= mask - 1;
        if (iB < kResMaxUnits) load_unit(iB, cB, sB);
        run(iA, cA, sA);
        if (iB >= kResMaxUnits) break;
        iA = mask ? __builtin_ctz(mask) : kResMaxUnits;
        mask &= mask - 1;
        if (iA < kResMaxUnits) load_unit(iA, cA, sA);
        run(iB, cB, sB);
    }
}

// The MoE plan, one workgroup: the valid routed pairs (expert id in [0, E),
// |w| >= 1e-8) sorted by expert (counting sort; the order within an expert
// does not change any result), expanded into the gate/up and down work lists
// ordered (expert, row block, pair); n_work[0] / n_work[1] = their lengths.
__global__ __launch_bounds__(1024) void moe_plan_kernel(const int *idx, const float *w, int P, int E,
                                                        int nb_gu, int nb_dn, int2 *work_gu,
                                                        int2 *work_dn, int *n_work) {
    extern __shared__ int sh[];
    int *cnt = sh, *start = sh + E, *cur = sh + 2 * E, *sorted = sh + 3 * E;
    __shared__ int wsum[16], total;
    const int tid = threadIdx.x, NT = blockDim.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < E; e += NT) cnt[e] = 0;
    __syncthreads();
    for (int q = tid; q < P; q += NT) {
        const int e = idx[q];
        if (e >= 0 && e < E && fabsf(w[q]) >= 1e-8f) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive prefix over the experts: thread tid owns a run of per experts;
    // run sums scanned within each wave (shuffles), then across the waves
    const int per = (E + NT - 1) / NT, e0 = min(E, tid * per), e1 = min(E, e0 + per);
    int s = 0;
    for (int e = e0; e < e1; ++e) s += cnt[e];
    int incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < NT / 64; ++i) {
            const int v = wsum[i];
            wsum[i] = run;
            run += v;
        }
        total = run;
        n_work[0] = run * nb_gu;
        n_work[1] = run * nb_dn;
    }
    __syncthreads();
    int run = wsum[wv] + incl - s;
    for (int e = e0; e < e1; ++e) {
        start[e] = run;
        cur[e] = run;
        run += cnt[e];
    }
    __syncthreads();
    for (int q = tid; q < P; q += NT) {
        const int e = idx[q];
        if (e >= 0 && e < E && fabsf(w[q]) >= 1e-8f) sorted[atomicAdd(&cur[e], 1)] = q;
    }
    __syncthreads();
    const int nv = total;
    for (int i = tid; i < nv * nb_gu; i += NT) {
        const int kk = i / nb_gu, b = i % nb_gu;
        const int pr = sorted[kk], e = idx[pr];
        work_gu[nb_gu * start[e] + b * cnt[e] + (kk - start[e])] = make_int2(pr, (b << 16) | e);
    }
    for (int i = tid; i < nv * nb_dn; i += NT) {
        const int kk = i / nb_dn, b = i % nb_dn;
        const int pr = sorted[kk], e = idx[pr];
        work_dn[nb_dn * start[e] + b * cnt[e] + (kk - start[e])] = make_int2(pr, (b << 16) | e);
    }
}

namespace {
template <typename F>
int set_dyn_lds(F *fn, size_t lds, size_t *granted) {
    // The attribute bounds the dynamic part; with the 64 KB of static LUT the
    // total passes the 64 KB default for any input.
    if (lds > *granted) {
        OJX_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        *granted = lds;
    }
    return OJASX_OK;
}
}  // namespace

bool bank_fits(int K) {
    return 64 * 1024 + round_up((size_t)(K / 16), 32) * kXRow * sizeof(float) <= 160 * 1024;
}

int launch_bank(const GroupItem *items_dev, const int2 *work_dev, int n_work, int max_K,
                hipStream_t st) {
    const size_t lds = round_up((size_t)(max_K / 16), 32) * kXRow * sizeof(float);
    static size_t granted = 0;
    int rc = set_dyn_lds(&lut_bank_kernel, lds, &granted);
    if (rc) return rc;
    OJX_LAUNCH(lut_bank_kernel, dim3(n_work), dim3(kBNT), lds, st, items_dev, work_dev);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

int launch_moe_plan(const int *idx, const float *w, int P, int E, int nb_gu, int nb_dn,
                    int2 *work_gu, int2 *work_dn, int *n_work, hipStream_t st) {
    const size_t lds = (size_t)(3 * E + P) * sizeof(int);
    static size_t granted = 0;
    if (lds > 65536 && lds > granted) {
        OJX_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&moe_plan_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    OJX_LAUNCH(moe_plan_kernel, dim3(1), dim3(1024), lds, st, idx, w, P, E, nb_gu, nb_dn, work_gu,
               work_dn, n_work);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

int launch_moe_bank(const MoEBankLaunch &l, hipStream_t st) {
    const int nb = (l.M + kBRows - 1) / kBRows;
    MoEBankParams p{l.codes_b, l.expert_bytes, static_cast<const v8bf *>(l.cb3), l.scales, l.x, l.y, l.idx,
                    l.w, l.work, l.n_work, l.M, l.K, l.k, l.E, nb};
    const size_t lds = round_up((size_t)(l.K / 16), 32) * kXRow * sizeof(float);
    const int grid = l.work ? 8 * ((l.max_work + 7) / 8) : l.max_work;
    int rc = OJASX_OK;
    if (l.xs == XS_SWIGLU) {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_bank_kernel<XS_SWIGLU>, lds, &gr);
        if (!rc) OJX_LAUNCH(moe_bank_kernel<XS_SWIGLU>, dim3(grid), dim3(kBNT), lds, st, p);
    } else if (l.xs == XS_BF16) {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_bank_kernel<XS_BF16>, lds, &gr);
        if (!rc) OJX_LAUNCH(moe_bank_kernel<XS_BF16>, dim3(grid), dim3(kBNT), lds, st, p);
    } else {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_bank_kernel<XS_F32>, lds, &gr);
        if (!rc) OJX_LAUNCH(moe_bank_kernel<XS_F32>, dim3(grid), dim3(kBNT), lds, st, p);
    }
    if (rc) return rc;
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

bool moe_resident_fits(int K, int xs) {
    return K % 16 == 0 && K / 16 <= (xs == XS_SWIGLU ? 2 : 4) * 32;
}

int launch_moe_resident(const MoEBankLaunch &l, int groups, int slots, hipStream_t st) {
    if (!moe_resident_fits(l.K, l.xs)) {
        set_error("resident-LUT MoE stage: too many inputs (%d)", l.K);
        return OJASX_ERR_INVALID;
    }
    const int teams = l.xs == XS_SWIGLU ? 1 : 2;
    const int nb = (l.M + kBRows - 1) / kBRows;
    const int units = slots * nb;
    // about one round of workgroups (2 / teams per CU), at least one unit
    // per team and at most kResMaxUnits units per workgroup
    const long total = (long)groups * units, round = 512 / teams;
    const int R = (int)std::min<long>({(long)kResMaxUnits, (long)std::max(units, teams),
                                       std::max<long>(teams, (total + round - 1) / round)});
    const int cpt = (units + R - 1) / R;
    if ((long)groups * cpt > 0x7fffffffL) {
        set_error("resident-LUT MoE stage: too many workgroups");
        return OJASX_ERR_INVALID;
    }
    MoEResParams p{l.codes_b, l.expert_bytes, static_cast<const v8bf *>(l.cb3), l.scales, l.x, l.y,
                   l.idx, l.w, l.M, l.K, slots, l.E, nb, R, cpt};
    const size_t lds = round_up((size_t)(l.K / 16), 32) * kXRow * sizeof(float);   // + the static LUT
    const dim3 grid(groups * cpt), block(teams * kBNT);
    int rc = OJASX_OK;
    if (l.xs == XS_SWIGLU) {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_resident_kernel<XS_SWIGLU, 1>, lds, &gr);
        if (!rc) OJX_LAUNCH((moe_resident_kernel<XS_SWIGLU, 1>), grid, block, lds, st, p);
    } else if (l.xs == XS_BF16) {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_resident_kernel<XS_BF16, 2>, lds, &gr);
        if (!rc) OJX_LAUNCH((moe_resident_kernel<XS_BF16, 2>), grid, block, lds, st, p);
    } else {
        static size_t gr = 0;
        rc = set_dyn_lds(&moe_resident_kernel<XS_F32, 2>, lds, &gr);
        if (!rc) OJX_LAUNCH((moe_resident_kernel<XS_F32, 2>), grid, block, lds, st, p);
    }
    if (rc) return rc;
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

void pack_bank_codes(const uint8_t *codes, int M, int G, uint8_t *out) {
    for (int m = 0; m < M; ++m) {
        const uint8_t *row = codes + (size_t)m * G;
        const size_t rb = (size_t)(m / 64), r = (size_t)(m % 64);
        for (int gg = 0; gg < G; ++gg) out[(rb * G + gg) * 64 + r] = row[gg];
    }
}

}  // namespace ojx

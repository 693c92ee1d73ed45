// lut_moe.hip -- top-k split-manifold MoE layer and router on gfx950.
//
// Per token t and routed slot j (expert e = idx[t][j], weight w = w[t][j]):
//   gate_i = sg_e[i]   * sum_g LUT_in[g, gu_codes[e][i][g]]
//   up_i   = sg_e[I+i] * sum_g LUT_in[g, gu_codes[e][I+i][g]]
//   inter_i = silu(gate_i) * up_i,             silu(v) = v / (1 + exp(-v))
//   y[t][h] = sum_j w * (sd_e[h] * sum_g LUT_down[g, dn_codes[e][h][g]])   (j ascending)
// the computation of split_manifold_lut_experiment/native/src/
// ojasx_lut_cpu.cpp:213-365, including its skip rule (:284-286: e outside
// [0,E) or |w| < 1e-8 contributes nothing) and output rule (:220-223: y is
// zeroed when k_active > 0, untouched otherwise).  Only routed experts' codes
// are ever read.
//
// Four paths, none with cross-workgroup synchronisation inside a kernel (a
// "pair" is one routed (token, slot)):
//  * block_dim 16, fewer than kGroupMinTokens tokens (latency-bound): two
//    launches that compute LUT entries where they are used, <v_g, C[code]>,
//    from the codebook and the input vector staged in LDS -- moe_up_dec
//    (gate/up + SwiGLU per (pair, 32 intermediate rows)) and moe_down_dec
//    (down + combine per (token, hidden rows), slots summed in slot order).
//  * block_dim 16, kGroupMinTokens up to kBankMinTokens tokens: the pairs as
//    grouped LUT GEMVs in slot order, each workgroup building its 16-group
//    LUT slices with MFMA -- moe_gu_group (gate/up + SwiGLU), moe_dn_group
//    (down, scaled), moe_combine.
//  * block_dim 16, more tokens, aligned activations: the pairs on the
//    bank-layout LUT-GEMV of lut_bank.hip -- moe_bank (gate/up), moe_bank
//    (SwiGLU input, down), moe_combine -- from 128 tokens grouped by expert
//    first (moe_plan, a counting sort), so each distinct expert's codes
//    stream from HBM once.
//  * other block sizes (any divisor of H and I): LUT_in build, moe_gateup
//    (gathers from the L2-resident LUT, SwiGLU), moe_lut_down (the pair's
//    LUT_down rows), moe_down, moe_combine.
// Every path sums slots in slot order, so results are deterministic.
//  Router: moe_route, one workgroup per token.
#include <algorithm>
#include <cstring>
#include <type_traits>
#include <vector>

#include "common.h"
#include "lut_slices.h"

namespace ojx {

namespace {
constexpr int kNT = 256;
constexpr int kGS = 16;
constexpr int kCB = 256;
constexpr int kRowAlign = 256;
constexpr int kRG = 32;   // intermediate rows per gate/up workgroup
constexpr int kRD = 64;   // hidden rows per down workgroup
}  // namespace

struct MoE {
    int E = 0, H = 0, I = 0, top_k = 0, D = 0;
    int Gin = 0, Gi = 0, Sin = 0, Si = 0, Ip = 0, Hp = 0;
    DevBuf cb_in, cb_dn, gu, dn, gus, dns;
    DevBuf cb3_in, cb3_dn;              // bank path: the codebooks' bf16 pieces
    DevBuf gub, dnb;                    // bank layouts per expert (block_dim 16)
    size_t gub_bytes = 0, dnb_bytes = 0;
    DevBuf lut_in, lut_dn, dout, inter, gu_part, xstage, ystage;
    DevBuf work, nwork, gu_out;         // bank path: plan output, gate/up rows per pair
    ~MoE() {
        for (DevBuf *b : {&cb_in, &cb_dn, &cb3_in, &cb3_dn, &gu, &dn, &gus, &dns, &gub, &dnb, &lut_in, &lut_dn,
                          &dout, &inter, &gu_part, &xstage, &ystage, &work,
                          &nwork, &gu_out})
            b->release();
    }
};

struct MoEParams {
    const uint8_t *gu;      // [E][Sin][2][Ip][16]
    const uint8_t *dn;      // [E][Si][Hp][16]
    const float *gus;       // [E][2I]
    const float *dns;       // [E][H]
    const float *cb_dn;     // [256][D]
    const float *lut_in;    // [T][Sin*16][256]
    float *lut_dn;          // [P][Si*16][256]
    float *dout;            // [P][H]
    float *inter;           // [P][I]: silu(gate) * up
    const int *idx;         // [T][k]
    const float *w;         // [T][k]
    void *y;                // [T][H]
    int E, H, I, D, Sin, Si, Ip, Hp, T, k;
};

__device__ __forceinline__ bool pair_active(const MoEParams &p, int pr, int *e_out) {
    const int e = p.idx[pr];
    const float w = p.w[pr];
    *e_out = e;
    return e >= 0 && e < p.E && fabsf(w) >= 1e-8f;
}

__device__ __forceinline__ uint4 ld_codes(const uint8_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}

// Sum of the 16 LUT entries selected by 16 codes from 16 consecutive LUT rows.
__device__ __forceinline__ float gather16(const float *__restrict__ L, uint4 c) {
    const uint32_t w4[4] = {c.x, c.y, c.z, c.w};
    float v[kGS];
#pragma unroll
    for (int g = 0; g < kGS; ++g) v[g] = L[g * kCB + ((w4[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
    float a = 0.f;
#pragma unroll
    for (int g = 0; g < kGS; ++g) a += v[g];
    return a;
}

__global__ __launch_bounds__(kNT) void moe_gateup_kernel(MoEParams p) {
    constexpr int QG = kNT / kRG;  // 8 slice groups
    __shared__ float red[2][QG][kRG];
    const int tid = threadIdx.x;
    const int r = tid % kRG, q = tid / kRG;
    const int nrb = (p.I + kRG - 1) / kRG;
    const int pr = blockIdx.x / nrb;
    const int rb = blockIdx.x - pr * nrb;
    int e;
    if (!pair_active(p, pr, &e)) return;
    const int t = pr / p.k;
    const int i = rb * kRG + r;                   // < Ip (multiple of 256)
    const uint8_t *eg = p.gu + (size_t)e * p.Sin * 2 * p.Ip * kGS;
    const float *L = p.lut_in + (size_t)t * p.Sin * kGS * kCB;

    float ag = 0.f, au = 0.f;
    for (int s = q; s < p.Sin; s += QG) {  // one step when Sin <= 8 (H <= 2048 at D = 16)
        const uint4 cg = ld_codes(eg + (((size_t)s * 2 + 0) * p.Ip + i) * kGS);
        const uint4 cu = ld_codes(eg + (((size_t)s * 2 + 1) * p.Ip + i) * kGS);
        ag += gather16(L + (size_t)s * kGS * kCB, cg);
        au += gather16(L + (size_t)s * kGS * kCB, cu);
    }
    red[0][q][r] = ag;
    red[1][q][r] = au;
    __syncthreads();
    if (q != 0 || i >= p.I) return;
    float g = red[0][0][r], u = red[1][0][r];
#pragma unroll
    for (int k = 1; k < QG; ++k) {
        g += red[0][k][r];
        u += red[1][k][r];
    }
    g *= p.gus[(size_t)e * 2 * p.I + i];
    u *= p.gus[(size_t)e * 2 * p.I + p.I + i];
    p.inter[(size_t)pr * p.I + i] = g / (1.f + expf(-g)) * u;
}

// LUT_down of one active pair: row g (blockIdx.y, all Si * 16 rows of the
// slices, zero past Gi) = <inter[pair][gD : gD + D], C_down[k]> for thread
// k, any block size D (the group is staged 256 values at a time).  Every
// row the down gathers can read is written here, so the workspace needs no
// clearing.
__global__ __launch_bounds__(kNT) void moe_lut_down_kernel(MoEParams p) {
    __shared__ float xs[kNT];
    const int pr = blockIdx.x, g = blockIdx.y, k = threadIdx.x;
    int e;
    if (!pair_active(p, pr, &e)) return;
    const int Gi = p.I / p.D;
    const float dot = staged_group_dot(p.inter + (size_t)pr * p.I + (size_t)min(g, Gi - 1) * p.D,
                                       g < Gi, p.cb_dn + (size_t)k * p.D, p.D, xs);
    p.lut_dn[((size_t)pr * p.Si * kGS + g) * kCB + k] = dot;
}

__global__ __launch_bounds__(kNT) void moe_down_kernel(MoEParams p) {
    constexpr int QG = kNT / kRD;  // 4 slice groups
    __shared__ float red[QG][kRD];
    const int tid = threadIdx.x;
    const int r = tid % kRD, q = tid / kRD;
    const int nrb = (p.H + kRD - 1) / kRD;
    const int pr = blockIdx.x / nrb;
    const int rb = blockIdx.x - pr * nrb;
    int e;
    if (!pair_active(p, pr, &e)) return;
    const int h = rb * kRD + r;                   // < Hp
    const uint8_t *ed = p.dn + (size_t)e * p.Si * p.Hp * kGS;
    const float *L = p.lut_dn + (size_t)pr * p.Si * kGS * kCB;
    float a = 0.f;
    for (int s = q; s < p.Si; s += QG)  // one step when Si <= 4 (I <= 1024 at D = 16)
        a += gather16(L + (size_t)s * kGS * kCB, ld_codes(ed + ((size_t)s * p.Hp + h) * kGS));
    red[q][r] = a;
    __syncthreads();
    if (q != 0 || h >= p.H) return;
    float s = red[0][r];
#pragma unroll
    for (int k = 1; k < QG; ++k) s += red[k][r];
    p.dout[(size_t)pr * p.H + h] = s * p.dns[(size_t)e * p.H + h];
}

// ---------------------------------------------------------------------------
// block_dim 16: two launches.  LUT entries are computed where they are used,
// <v_g, C[code]>, from the codebook and the input vector staged in LDS, with
// lane (r, j) owning quarter j of every 16-float dot (as in lut_linear.hip).

struct MoEDecParams {
    const uint8_t *gu;      // [E][Sin][2][Ip][16]
    const uint8_t *dn;      // [E][Si][Hp][16]
    const float *gus;       // [E][2I]
    const float *dns;       // [E][H]
    const float *cb_in;     // [256][16]
    const float *cb_dn;     // [256][16]
    const void *x;          // [T][H]
    float *inter;           // [P][I]
    const int *idx;         // [T][k]
    const float *w;         // [T][k]
    void *y;                // [T][H]
    int E, H, I, Sin, Si, Ip, Hp, T, k, NW;
};

__device__ __forceinline__ bool slot_active(const int *idx, const float *w, int pr, int E, int *e) {
    *e = idx[pr];
    return *e >= 0 && *e < E && fabsf(w[pr]) >= 1e-8f;
}

// Gate/up + SwiGLU.  Workgroup = (pair, 16*NI intermediate rows); wave w owns
// input slices w, w+NW, ...; lane (r, j) owns gate and up rows i = base + r +
// 16n (n < NI).  Writes inter[pair][i] = silu(s_g * gate_i) * (s_u * up_i).
// Loads are issued codebook and x first (L2), then codes (HBM), so the LDS
// stores wait only for the L2 loads.
template <typename T, int NI>
__global__ __launch_bounds__(1024) void moe_up_dec_kernel(MoEDecParams p) {
    constexpr int R = 16 * NI;
    extern __shared__ float sm[];
    float *cbs = sm;                       // [256][16]
    float *xs = sm + kCB * 16;             // [Sin*256], zero past H
    __shared__ float part[2][16][R];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, w = tid >> 6;
    const int r = lane >> 2, j = lane & 3;
    const int nib = (p.I + R - 1) / R;
    const int pr = blockIdx.x / nib;
    const int base = (blockIdx.x - pr * nib) * R;   // base + R <= Ip
    int e;
    if (!slot_active(p.idx, p.w, pr, p.E, &e)) return;
    const int t = pr / p.k;
    const int KS = p.Sin * 256, nx4 = KS / 4;
    const T *__restrict__ x = static_cast<const T *>(p.x) + (size_t)t * p.H;

    float4 cv4[2], xv4[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) cv4[u] = reinterpret_cast<const float4 *>(p.cb_in)[min(tid + u * nthr, 1023)];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int el = min(tid + u * nthr, nx4 - 1) * 4;
        xv4[u] = load4_act(x, min(el, p.H - 4));
        if (el >= p.H) xv4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const uint8_t *eg = p.gu + (size_t)e * p.Sin * 2 * p.Ip * kGS;
    uint4 cw[NI][2];
#pragma unroll
    for (int n = 0; n < NI; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            cw[n][h] = ld_codes(eg + (((size_t)w * 2 + h) * p.Ip + base + r + 16 * n) * kGS);
    float sg = 0.f, su = 0.f;
    if (tid < R) {
        const int i = min(base + tid, p.I - 1);
        sg = p.gus[(size_t)e * 2 * p.I + i];
        su = p.gus[(size_t)e * 2 * p.I + p.I + i];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) reinterpret_cast<float4 *>(cbs)[min(tid + u * nthr, 1023)] = cv4[u];
#pragma unroll
    for (int u = 0; u < 2; ++u) reinterpret_cast<float4 *>(xs)[min(tid + u * nthr, nx4 - 1)] = xv4[u];
    for (int b = tid + 2 * nthr; b < 1024; b += nthr)     // fewer than 512 threads
        reinterpret_cast<float4 *>(cbs)[b] = reinterpret_cast<const float4 *>(p.cb_in)[b];
    for (int b = tid + 2 * nthr; b < nx4; b += nthr) {    // H > 8 * threads
        const int el = b * 4;
        reinterpret_cast<float4 *>(xs)[b] = el < p.H ? load4_act(x, el) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();

    float acc[NI][2][2];
#pragma unroll
    for (int n = 0; n < NI; ++n)
        acc[n][0][0] = acc[n][0][1] = acc[n][1][0] = acc[n][1][1] = 0.f;
    const float *cbj = cbs + 4 * j;
    for (int s = w; s < p.Sin; s += p.NW) {
        uint32_t wd[NI][2][4];
#pragma unroll
        for (int n = 0; n < NI; ++n)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                wd[n][h][0] = cw[n][h].x;
                wd[n][h][1] = cw[n][h].y;
                wd[n][h][2] = cw[n][h].z;
                wd[n][h][3] = cw[n][h].w;
            }
        if (s + p.NW < p.Sin) {
#pragma unroll
            for (int n = 0; n < NI; ++n)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    cw[n][h] = ld_codes(eg + (((size_t)(s + p.NW) * 2 + h) * p.Ip + base + r + 16 * n) * kGS);
        }
        const float *xsj = xs + s * 256 + 4 * j;
#pragma unroll
        for (int g = 0; g < kGS; ++g) {
            const float4 xv = *reinterpret_cast<const float4 *>(xsj + g * 16);
#pragma unroll
            for (int n = 0; n < NI; ++n)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int code = (wd[n][h][g >> 2] >> ((g & 3) * 8)) & 0xffu;
                    const float4 c = *reinterpret_cast<const float4 *>(cbj + code * 16);
                    float a = acc[n][h][g & 1];
                    a = fmaf(xv.x, c.x, a);
                    a = fmaf(xv.y, c.y, a);
                    a = fmaf(xv.z, c.z, a);
                    a = fmaf(xv.w, c.w, a);
                    acc[n][h][g & 1] = a;
                }
        }
    }
#pragma unroll
    for (int n = 0; n < NI; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float v = quad_sum(acc[n][h][0] + acc[n][h][1]);
            if (j == 0) part[h][w][r + 16 * n] = v;
        }
    __syncthreads();
    if (tid >= R) return;
    const int i = base + tid;
    if (i >= p.I) return;
    float g = 0.f, u = 0.f;
    for (int k = 0; k < p.NW; ++k) {
        g += part[0][k][tid];
        u += part[1][k][tid];
    }
    g *= sg;
    u *= su;
    p.inter[(size_t)pr * p.I + i] = g / (1.f + expf(-g)) * u;
}

// Down projection + combine.  Workgroup = (token, 16*RPL hidden rows); wave w
// owns slots w, w+NW, ...; lane (r, j) owns rows h = base + r + 16n.  The
// token's k intermediate vectors and the down codebook are staged in LDS.
// part[j][h] = s_dn[e_j][h] * dot_j(h), then y[t][h] = sum_j w_j * part[j][h]
// over active slots in slot order (the reference's w * (s * sum) order).  A
// wave's first slot, its codes (up to kDS slices) and its row scales are
// loaded before the staging stores, so the kernel has one dependent round
// trip (slot id -> codes) besides the staging.
constexpr int kDS = 4;
template <typename T, int RPL>
__global__ __launch_bounds__(1024) void moe_down_dec_kernel(MoEDecParams p) {
    constexpr int R = 16 * RPL;
    extern __shared__ float sm[];
    float *cbs = sm;                       // [256][16]
    float *is = sm + kCB * 16;             // [k][Si*256], zero past I
    __shared__ float part[32][R];
    __shared__ float wsl[32];
    __shared__ int onl[32];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, w = tid >> 6;
    const int r = lane >> 2, j = lane & 3;
    const int t = blockIdx.y;
    const int base = blockIdx.x * R;       // base + R <= Hp
    const int IS = p.Si * 256, i4 = IS / 4, n4 = p.k * i4;

    float4 cv4[2], iv4[4];
#pragma unroll
    for (int u = 0; u < 2; ++u) cv4[u] = reinterpret_cast<const float4 *>(p.cb_dn)[min(tid + u * nthr, 1023)];
    const float *it = p.inter + (size_t)t * p.k * p.I;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        // rows of inactive slots are stale and never used
        const int b = min(tid + u * nthr, n4 - 1);
        const int jj = b / i4, el = (b - jj * i4) * 4;
        iv4[u] = *reinterpret_cast<const float4 *>(it + (size_t)jj * p.I + min(el, p.I - 4));
        if (el >= p.I) iv4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    int e0 = 0;
    const bool on0 = w < p.k && slot_active(p.idx, p.w, t * p.k + min(w, p.k - 1), p.E, &e0);
    uint4 cw[kDS][RPL];
    float dsc[RPL];
    {
        const int ee = on0 ? e0 : 0;
        const uint8_t *ed = p.dn + (size_t)ee * p.Si * p.Hp * kGS;
#pragma unroll
        for (int s = 0; s < kDS; ++s)
#pragma unroll
            for (int n = 0; n < RPL; ++n)
                cw[s][n] = ld_codes(ed + ((size_t)min(s, p.Si - 1) * p.Hp + base + r + 16 * n) * kGS);
#pragma unroll
        for (int n = 0; n < RPL; ++n) dsc[n] = p.dns[(size_t)ee * p.H + min(base + r + 16 * n, p.H - 1)];
    }
    if (tid < p.k) {
        int e;
        onl[tid] = slot_active(p.idx, p.w, t * p.k + tid, p.E, &e) ? 1 : 0;
        wsl[tid] = p.w[t * p.k + tid];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) reinterpret_cast<float4 *>(cbs)[min(tid + u * nthr, 1023)] = cv4[u];
#pragma unroll
    for (int u = 0; u < 4; ++u) reinterpret_cast<float4 *>(is)[min(tid + u * nthr, n4 - 1)] = iv4[u];
    for (int b = tid + 2 * nthr; b < 1024; b += nthr)      // fewer than 512 threads
        reinterpret_cast<float4 *>(cbs)[b] = reinterpret_cast<const float4 *>(p.cb_dn)[b];
    for (int b = tid + 4 * nthr; b < n4; b += nthr) {      // k*I > 16 * threads
        const int jj = b / i4, el = (b - jj * i4) * 4;
        reinterpret_cast<float4 *>(is)[b] = el < p.I
            ? *reinterpret_cast<const float4 *>(it + (size_t)jj * p.I + el) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    const float *cbj = cbs + 4 * j;
    for (int js = w; js < p.k; js += p.NW) {
        int e = e0;
        bool on = on0;
        if (js != w) {                             // later slots of this wave (k > NW)
            on = slot_active(p.idx, p.w, t * p.k + js, p.E, &e);
            const int ee = on ? e : 0;
            const uint8_t *ed = p.dn + (size_t)ee * p.Si * p.Hp * kGS;
#pragma unroll
            for (int s = 0; s < kDS; ++s)
#pragma unroll
                for (int n = 0; n < RPL; ++n)
                    cw[s][n] = ld_codes(ed + ((size_t)min(s, p.Si - 1) * p.Hp + base + r + 16 * n) * kGS);
#pragma unroll
            for (int n = 0; n < RPL; ++n) dsc[n] = p.dns[(size_t)ee * p.H + min(base + r + 16 * n, p.H - 1)];
        }
        if (!on) continue;                         // wave-uniform
        const uint8_t *ed = p.dn + (size_t)e * p.Si * p.Hp * kGS;
        float acc[RPL][2];
#pragma unroll
        for (int n = 0; n < RPL; ++n) acc[n][0] = acc[n][1] = 0.f;
        for (int s = 0; s < p.Si; ++s) {
            uint4 cs[RPL];
#pragma unroll
            for (int n = 0; n < RPL; ++n) {
                cs[n] = cw[0][n];
#pragma unroll
                for (int q = 1; q < kDS; ++q)
                    if (s == q) cs[n] = cw[q][n];
                if (s >= kDS) cs[n] = ld_codes(ed + ((size_t)s * p.Hp + base + r + 16 * n) * kGS);
            }
            const float *ij = is + js * IS + s * 256 + 4 * j;
#pragma unroll
            for (int g = 0; g < kGS; ++g) {
                const float4 iv = *reinterpret_cast<const float4 *>(ij + g * 16);
#pragma unroll
                for (int n = 0; n < RPL; ++n) {
                    const uint32_t wd = g < 4 ? cs[n].x : g < 8 ? cs[n].y : g < 12 ? cs[n].z : cs[n].w;
                    const int code = (wd >> ((g & 3) * 8)) & 0xffu;
                    const float4 c = *reinterpret_cast<const float4 *>(cbj + code * 16);
                    float a = acc[n][g & 1];
                    a = fmaf(iv.x, c.x, a);
                    a = fmaf(iv.y, c.y, a);
                    a = fmaf(iv.z, c.z, a);
                    a = fmaf(iv.w, c.w, a);
                    acc[n][g & 1] = a;
                }
            }
        }
#pragma unroll
        for (int n = 0; n < RPL; ++n) {
            const float v = quad_sum(acc[n][0] + acc[n][1]);
            if (j == 0) part[js][r + 16 * n] = dsc[n] * v;
        }
    }
    __syncthreads();
    if (tid >= R) return;
    const int h = base + tid;
    if (h >= p.H) return;
    float y = 0.f;
    for (int js = 0; js < p.k; ++js)
        if (onl[js]) y += wsl[js] * part[js][tid];
    store_act(static_cast<T *>(p.y), (size_t)t * p.H + h, y);
}

// ---------------------------------------------------------------------------
// Many tokens (block_dim 16): the routed pairs as grouped LUT GEMVs.  Each
// workgroup builds the LUT slices it gathers from with MFMA (lut_slices.h),
// so no LUT goes through memory.  A "pair" is one routed (token, slot).
//  moe_gu_group: workgroup = (256 IPT intermediate indices, pair, slice part):
//    x_t staged in LDS, each thread holds the gate row i and the up row Ip + i
//    of IPT indices i of the pair's expert (one [Sin][2 Ip][16] code tile).
//    With the input slices in one part it writes inter[pair][i] =
//    silu(s_g * gate_i) * (s_u * up_i); with NS parts, part ps of slices
//    [ps Sin / NS, (ps + 1) Sin / NS) writes its raw sums to
//    gu_part[pair][ps][2 Ip] and moe_dn_group sums the parts in order.
//  moe_dn_group: workgroup = (256 R hidden rows, pair): inter[pair] staged in
//    LDS -> dout[pair][h] = s_dn[e][h] * down_h.
//  moe_combine: y[t][h] = sum_j w_j dout[pair (t, j)][h], active slots in
//    slot order.
// Inactive pairs (expert outside [0, E) or |w| < 1e-8) exit at once: their
// codes are never read.
struct MoEGroupParams {
    const uint8_t *gu;      // [E][Sin][2][Ip][16]
    const uint8_t *dn;      // [E][Si][Hp][16]
    const float *gus;       // [E][2I]
    const float *dns;       // [E][H]
    const float *cb_in;     // [256][16]
    const float *cb_dn;     // [256][16]
    const void *x;          // [T][H]
    float *inter;           // [P][Ip]
    float *gu_part;         // [P][NS][2 Ip]
    float *dout;            // [P][H]
    const int *idx;         // [T][k]
    const float *w;         // [T][k]
    int E, H, I, Sin, Si, Ip, Hp, k, NS;
};

// Staging of an input vector into xs[0 .. S*256) (zeros past n): XR values per
// thread are loaded into registers by stage_load before the caller issues
// its code loads, and stored by stage_store with the rest.
template <int NT>
constexpr int stage_regs() { return NT >= 2048 ? 1 : 2048 / NT; }

template <int NT, typename T>
__device__ __forceinline__ void stage_load(const T *v, int n, float (&r)[stage_regs<NT>()]) {
#pragma unroll
    for (int u = 0; u < stage_regs<NT>(); ++u) {
        const int i = threadIdx.x + u * NT;
        r[u] = load_act(v, min(i, n - 1));
        if (i >= n) r[u] = 0.f;
    }
}

template <int NT, typename T>
__device__ __forceinline__ void stage_store(const T *v, int n, int S, const float (&r)[stage_regs<NT>()],
                                            float *xs) {
#pragma unroll
    for (int u = 0; u < stage_regs<NT>(); ++u) {
        const int i = threadIdx.x + u * NT;
        if (i < S * 256) xs[i] = r[u];
    }
    for (int i = threadIdx.x + stage_regs<NT>() * NT; i < S * 256; i += NT)
        xs[i] = i < n ? load_act(v, i) : 0.f;
}

__device__ __forceinline__ float swiglu_scaled(float g, float u, float sg, float su) {
    g *= sg;
    u *= su;
    return g / (1.f + expf(-g)) * u;
}

template <typename T, int NW, int IPT, bool DB, int PF>
__global__ __launch_bounds__(64 * NW) void moe_gu_group_kernel(MoEGroupParams p) {
    constexpr int NT = 64 * NW;
    __shared__ float L[DB ? 2 * slices::kLutFloats : slices::kLutFloats];
    extern __shared__ float xs[];                   // [Sin * 256]
    const int pr = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ps = blockIdx.z;
    const int s0 = ps * p.Sin / p.NS, s1 = (ps + 1) * p.Sin / p.NS;
    // the slot, x of its token and the codebook operands (none depends on the
    // expert id), then the expert's codes and scales
    const int e = p.idx[pr];
    const float wgt = p.w[pr];
    const T *xr = static_cast<const T *>(p.x) + (size_t)(pr / p.k) * p.H;
    float xv[stage_regs<NT>()];
    stage_load<NT>(xr, p.H, xv);
    float bop[16 / NW][4];
    slices::load_cb_operands<NW>(p.cb_in, w, lane, bop);
    if (!(e >= 0 && e < p.E && fabsf(wgt) >= 1e-8f)) return;   // whole workgroup
    // rows 2r, 2r + 1: gate and up of index i_r (clamped: loaded, never stored)
    const int i0 = (int)blockIdx.x * (NT * IPT) + tid;
    int row[2 * IPT];
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
        const int i = min(i0 + NT * r, p.I - 1);
        row[2 * r] = i;
        row[2 * r + 1] = p.Ip + i;
    }
    const uint8_t *codes = p.gu + (size_t)e * p.Sin * 2 * p.Ip * kGS;
    uint4 ring[PF][2 * IPT];
    slices::ring_start(codes, row, 2 * p.Ip, s0, s1, ring);
    float sg[IPT], su[IPT];
    if (p.NS == 1) {
        const float *sc = p.gus + (size_t)e * 2 * p.I;
#pragma unroll
        for (int r = 0; r < IPT; ++r) {
            sg[r] = sc[row[2 * r]];
            su[r] = sc[p.I + row[2 * r]];
        }
    }
    stage_store<NT>(xr, p.H, p.Sin, xv, xs);
    __syncthreads();
    float acc[2 * IPT] = {};
    slices::slice_loop<NW, 2 * IPT, DB, PF>(xs, L, bop, codes, row, 2 * p.Ip, s0, s1, w, lane, ring, acc);
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
        const int i = i0 + NT * r;
        if (i >= p.I) continue;
        if (p.NS == 1) {
            p.inter[(size_t)pr * p.Ip + i] = swiglu_scaled(acc[2 * r], acc[2 * r + 1], sg[r], su[r]);
        } else {
            float *o = p.gu_part + ((size_t)pr * p.NS + ps) * 2 * p.Ip;
            o[i] = acc[2 * r];
            o[p.Ip + i] = acc[2 * r + 1];
        }
    }
}

// NS: gate/up parts to sum (1: the intermediate vector is ready in inter).
template <int NW, int R, bool DB, int PF, int NS>
__global__ __launch_bounds__(64 * NW) void moe_dn_group_kernel(MoEGroupParams p) {
    constexpr int NT = 64 * NW, XR = stage_regs<NT>();
    __shared__ float L[DB ? 2 * slices::kLutFloats : slices::kLutFloats];
    extern __shared__ float xs[];                   // [Si * 256]
    const int pr = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int e = p.idx[pr];
    const float wgt = p.w[pr];
    // the pair's intermediate vector (or its gate/up part sums, in part
    // order) and the codebook operands, then the expert's codes and scales
    float gv[XR], uv[XR];
    if constexpr (NS == 1) {
        stage_load<NT>(p.inter + (size_t)pr * p.Ip, p.I, gv);
    } else {
        const float *gp = p.gu_part + (size_t)pr * NS * 2 * p.Ip;
#pragma unroll
        for (int u = 0; u < XR; ++u) {
            const int i = min(tid + u * NT, p.I - 1);
            float g = 0.f, v = 0.f;
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                g += gp[(size_t)q * 2 * p.Ip + i];
                v += gp[(size_t)q * 2 * p.Ip + p.Ip + i];
            }
            gv[u] = g;
            uv[u] = v;
        }
    }
    float bop[16 / NW][4];
    slices::load_cb_operands<NW>(p.cb_dn, w, lane, bop);
    if (!(e >= 0 && e < p.E && fabsf(wgt) >= 1e-8f)) return;
    const int h0 = (int)blockIdx.x * (NT * R) + tid;
    int row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row[r] = min(h0 + NT * r, p.H - 1);
    const uint8_t *codes = p.dn + (size_t)e * p.Si * p.Hp * kGS;
    uint4 ring[PF][R];
    slices::ring_start(codes, row, p.Hp, 0, p.Si, ring);
    float scl[R];
#pragma unroll
    for (int r = 0; r < R; ++r) scl[r] = p.dns[(size_t)e * p.H + row[r]];
    if constexpr (NS == 1) {
        stage_store<NT>(p.inter + (size_t)pr * p.Ip, p.I, p.Si, gv, xs);
    } else {
        const float *sc = p.gus + (size_t)e * 2 * p.I;
        const float *gp = p.gu_part + (size_t)pr * NS * 2 * p.Ip;
#pragma unroll
        for (int u = 0; u < XR; ++u) {
            const int i = tid + u * NT;
            const int ic = min(i, p.I - 1);
            const float v = swiglu_scaled(gv[u], uv[u], sc[ic], sc[p.I + ic]);
            if (i < p.Si * 256) xs[i] = i < p.I ? v : 0.f;
        }
        for (int i = tid + XR * NT; i < p.Si * 256; i += NT) {   // I > 256 XR
            float v = 0.f;
            if (i < p.I) {
                float g = 0.f, u = 0.f;
                for (int q = 0; q < NS; ++q) {
                    g += gp[(size_t)q * 2 * p.Ip + i];
                    u += gp[(size_t)q * 2 * p.Ip + p.Ip + i];
                }
                v = swiglu_scaled(g, u, sc[i], sc[p.I + i]);
            }
            xs[i] = v;
        }
    }
    __syncthreads();
    float acc[R] = {};
    slices::slice_loop<NW, R, DB, PF>(xs, L, bop, codes, row, p.Hp, 0, p.Si, w, lane, ring, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int h = h0 + NT * r;
        if (h < p.H) p.dout[(size_t)pr * p.H + h] = scl[r] * acc[r];
    }
}

template <typename T>
__global__ __launch_bounds__(kNT) void moe_combine_kernel(MoEParams p) {
    // Slot weights (0 for skipped slots) and all per-pair outputs are loaded
    // before the ordered sum, so the whole combine is one round trip.
    constexpr int KB = 16;
    const int t = blockIdx.y;
    const int h = min((int)(blockIdx.x * kNT + threadIdx.x), p.H - 1);
    float y = 0.f;
    for (int j0 = 0; j0 < p.k; j0 += KB) {
        float wj[KB], v[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int j = min(j0 + u, p.k - 1);
            const int pr = t * p.k + j;
            int e;
            wj[u] = (j0 + u < p.k && pair_active(p, pr, &e)) ? p.w[pr] : 0.f;
            v[u] = p.dout[(size_t)pr * p.H + h];
        }
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (wj[u] != 0.f) y += v[u] * wj[u];
    }
    if ((int)(blockIdx.x * kNT + threadIdx.x) < p.H) store_act(static_cast<T *>(p.y), (size_t)t * p.H + h, y);
}

// Router: top-k of the logits (descending, ties to the lower index) and the
// softmax probability of each selected expert, optionally renormalised.  One
// wave per token: lane l holds logits l + 64*i (E <= 1024).  Each of the k
// rounds is a local argmax over the lane's 16 values, a DPP max over the wave
// (quad permutes and row mirrors inside each 16-lane row, then the 4 row
// leaders read into scalars), and a DPP min over the expert ids of the lanes
// that hold that maximum -- no LDS round trips, no barriers.
__global__ __launch_bounds__(kNT) void moe_route_kernel(const float *logits, int T, int E, int k,
                                                       int renorm, int *idx, float *w) {
    constexpr int NV = 16;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t_raw = blockIdx.x * (kNT / 64) + wv;
    const int t = min(t_raw, T - 1);
    const float *l = logits + (size_t)t * E;
    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = lane + 64 * i;
        const float x = l[min(e, E - 1)];
        v[i] = e < E ? x : -INFINITY;
    }
    uint32_t taken = 0;
    float myv = 0.f;   // lane j < k keeps the j-th selection
    int myi = 0;
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e = lane + 64 * i;
            if (e < E && !((taken >> i) & 1u) && (v[i] > bv || bi == 0x7fffffff)) {
                bv = v[i];
                bi = e;
            }
        }
        const float m = wave_max_f(bv);
        const int wi = wave_min_i(bi != 0x7fffffff && bv == m ? bi : 0x7fffffff);
        if ((wi & 63) == lane) taken |= 1u << (wi >> 6);
        if (lane == j) {
            myv = m;
            myi = wi;
        }
    }
    // softmax statistics over all E logits
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) mx = fmaxf(mx, v[i]);
    mx = wave_max_f(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (lane + 64 * i < E) sum += expf(v[i] - mx);
    sum = wave_sum_f(sum);
    float wj = lane < k ? expf(myv - mx) / sum : 0.f;
    if (renorm) wj = wj / wave_sum_f(wj);
    if (lane < k && t_raw < T) {
        idx[(size_t)t * k + lane] = myi;
        w[(size_t)t * k + lane] = wj;
    }
}

namespace {

constexpr size_t kMaxLds = 160 * 1024;
// From this many tokens the grouped path beats computing LUT entries in place:
// measured 18.4 vs 21.6 us at 3 tokens, 16.9 vs 18.2 us at 2 (the 512-expert
// H 2048 / I 768 top-10 layer).
constexpr int kGroupMinTokens = 3;
// From this many tokens the routed pairs run grouped by expert on the bank
// kernel (up to kBankMaxPairs pairs per call: the plan's LDS).  Measured on
// the 512-expert H 2048 / I 768 top-10 layer, per call, two alternating
// 151 MB banks: 33.4 vs 34.2 us at 16 tokens, 48.2 vs 51.9 at 32, 85.4 vs
// 87.1 at 64, 264 vs 286 at 256 (bank vs grouped per slot); 27.1 vs 26.7 at 8.
constexpr int kBankMinTokens = 16;
constexpr size_t kBankMaxPairs = 16384;   // sorted by expert: the plan's LDS
// From this many tokens a plan launch sorts the pairs by expert first; below
// it workgroups map straight to (pair, row block): a repeated expert's codes
// are read once per pair (about 15 % more code bytes at 16 tokens) but the
// plan's dependent launch leaves the chain.  Measured per call (same box,
// sorted vs direct): 29.6 vs 26.5 us at 16 tokens, 44.0 vs 41.6 at 32, 75.3
// vs 72.9 at 64, 104.7 vs 104.0 at 96, 132.5 vs 131.4 at 128, 237.3 vs
// 240.3 at 256: the gathers and LUT builds per pair, not the code stream,
// set the time.
constexpr int kBankSortMinTokens = 128;
// From this many tokens (and at most 2048 inputs) gate/up runs token-major:
// each token's LUT is built once for all its routed slots instead of once per
// (pair, row block).  Measured gate/up kernel per call (same box, bank vs
// token-major, 512 experts, H 2048, I 768, top-10): 11.4 vs 12.6 us at 16
// tokens, 15.8 vs 15.2 at 24, 19.7 vs 18.7 at 32, 27.2 vs 23.0 at 48, 35.3
// vs 27.8 at 64, 111.5 vs 94.3 at 256.  Down (at most 1024 intermediate
// values) always runs pair-major, each pair's LUT built once for all its row
// blocks: per call 26.3 vs 25.3 us at 16 tokens, 32.8 vs 29.6 at 24, 63.0 vs
// 55.0 at 64, 213.6 vs 175 at 256 (bank vs pair-major down).  With both
// stages resident no work list is read, so no plan runs.
constexpr int kTokGateUpMinTokens = 24;

template <typename T>
int moe_forward_dec(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_, int k,
                    hipStream_t st) {
    const size_t P = (size_t)T_ * k;
    int rc = m->inter.ensure(P * m->I * sizeof(float));
    if (rc) return rc;
    MoEDecParams p{};
    p.gu = m->gu.as<uint8_t>();
    p.dn = m->dn.as<uint8_t>();
    p.gus = m->gus.as<float>();
    p.dns = m->dns.as<float>();
    p.cb_in = m->cb_in.as<float>();
    p.cb_dn = m->cb_dn.as<float>();
    p.x = x;
    p.inter = m->inter.as<float>();
    p.idx = idx;
    p.w = w;
    p.y = y;
    p.E = m->E;
    p.H = m->H;
    p.I = m->I;
    p.Sin = m->Sin;
    p.Si = m->Si;
    p.Ip = m->Ip;
    p.Hp = m->Hp;
    p.T = T_;
    p.k = k;
    // gate/up + SwiGLU: 32 intermediate rows per workgroup
    {
        constexpr int NI = 2;
        p.NW = std::min(m->Sin, 16);
        const size_t lds = (size_t)(kCB * 16 + m->Sin * 256) * sizeof(float);
        static size_t granted = 0;
        const void *fn = reinterpret_cast<const void *>(&moe_up_dec_kernel<T, NI>);
        rc = ensure_dyn_lds(fn, lds, &granted);
        if (rc) return rc;
        const int nib = (m->I + 16 * NI - 1) / (16 * NI);
        OJX_LAUNCH((moe_up_dec_kernel<T, NI>), dim3(P * nib), dim3(64 * p.NW), lds, st, p);
    }
    // down + combine: 16 or 32 hidden rows per workgroup
    {
        p.NW = std::min(k, 16);
        const size_t lds = (size_t)(kCB * 16 + (size_t)k * m->Si * 256) * sizeof(float);
        const bool r2 = (long)T_ * ((m->H + 31) / 32) >= 192;
        const void *fn = r2 ? reinterpret_cast<const void *>(&moe_down_dec_kernel<T, 2>)
                            : reinterpret_cast<const void *>(&moe_down_dec_kernel<T, 1>);
        static size_t granted1 = 0, granted2 = 0;
        rc = ensure_dyn_lds(fn, lds, r2 ? &granted2 : &granted1);
        if (rc) return rc;
        if (r2)
            OJX_LAUNCH((moe_down_dec_kernel<T, 2>), dim3((m->H + 31) / 32, T_), dim3(64 * p.NW),
                               lds, st, p);
        else
            OJX_LAUNCH((moe_down_dec_kernel<T, 1>), dim3((m->H + 15) / 16, T_), dim3(64 * p.NW),
                               lds, st, p);
    }
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// Launch shapes of the grouped path (the 512-expert H 2048 / I 768 top-10
// layer, 3-16 tokens): gate/up workgroups of 4 waves with one intermediate
// index per thread, down workgroups of 8 waves with one hidden row per
// thread, both with two LUT buffers and two slices of codes in flight; the
// gate/up input slices split in two parts below 128 routed slots, where
// there are too few workgroups to fill the CUs.
constexpr int kGuWaves = 4, kGuIdx = 1, kDnWaves = 8, kDnRows = 1, kGroupPF = 2;
constexpr bool kGroupDB = true;
constexpr size_t kGroupSplitBelow = 128;

template <int NS>
int launch_dn(const MoEGroupParams &p, size_t P, size_t lds, hipStream_t st) {
    const void *fn = reinterpret_cast<const void *>(
        &moe_dn_group_kernel<kDnWaves, kDnRows, kGroupDB, kGroupPF, NS>);
    static size_t granted = 0;
    int rc = ensure_dyn_lds(fn, lds + slices::lut_bytes(kGroupDB), &granted);
    if (rc) return rc;
    const int nb = (p.H + 64 * kDnWaves * kDnRows - 1) / (64 * kDnWaves * kDnRows);
    OJX_LAUNCH((moe_dn_group_kernel<kDnWaves, kDnRows, kGroupDB, kGroupPF, NS>), dim3(nb, P),
               dim3(64 * kDnWaves), lds, st, p);
    return OJASX_OK;
}

template <typename T>
int moe_forward_group(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_, int k,
                      hipStream_t st) {
    const size_t P = (size_t)T_ * k;
    if (P > 65535) {
        set_error("at most 65535 routed slots per call (got %zu)", P);
        return OJASX_ERR_INVALID;
    }
    const int ns = P < kGroupSplitBelow && m->Sin >= 2 ? 2 : 1;
    int rc = m->inter.ensure(P * m->Ip * sizeof(float));
    if (!rc) rc = m->dout.ensure(P * m->H * sizeof(float));
    if (!rc && ns > 1) rc = m->gu_part.ensure(P * ns * 2 * m->Ip * sizeof(float));
    if (rc) return rc;
    MoEGroupParams p{};
    p.gu = m->gu.as<uint8_t>();
    p.dn = m->dn.as<uint8_t>();
    p.gus = m->gus.as<float>();
    p.dns = m->dns.as<float>();
    p.cb_in = m->cb_in.as<float>();
    p.cb_dn = m->cb_dn.as<float>();
    p.x = x;
    p.inter = m->inter.as<float>();
    p.gu_part = m->gu_part.as<float>();
    p.dout = m->dout.as<float>();
    p.idx = idx;
    p.w = w;
    p.E = m->E;
    p.H = m->H;
    p.I = m->I;
    p.Sin = m->Sin;
    p.Si = m->Si;
    p.Ip = m->Ip;
    p.Hp = m->Hp;
    p.k = k;
    p.NS = ns;
    {
        const void *fn = reinterpret_cast<const void *>(
            &moe_gu_group_kernel<T, kGuWaves, kGuIdx, kGroupDB, kGroupPF>);
        const size_t lds = (size_t)m->Sin * 256 * sizeof(float);
        static size_t granted = 0;
        rc = ensure_dyn_lds(fn, lds + slices::lut_bytes(kGroupDB), &granted);
        if (rc) return rc;
        const int nb = (m->I + 64 * kGuWaves * kGuIdx - 1) / (64 * kGuWaves * kGuIdx);
        OJX_LAUNCH((moe_gu_group_kernel<T, kGuWaves, kGuIdx, kGroupDB, kGroupPF>), dim3(nb, P, ns),
                   dim3(64 * kGuWaves), lds, st, p);
    }
    rc = ns == 1 ? launch_dn<1>(p, P, (size_t)m->Si * 256 * sizeof(float), st)
                 : launch_dn<2>(p, P, (size_t)m->Si * 256 * sizeof(float), st);
    if (rc) return rc;
    MoEParams cp{};
    cp.dout = m->dout.as<float>();
    cp.idx = idx;
    cp.w = w;
    cp.y = y;
    cp.E = m->E;
    cp.H = m->H;
    cp.T = T_;
    cp.k = k;
    OJX_LAUNCH((moe_combine_kernel<T>), dim3((m->H + kNT - 1) / kNT, T_), dim3(kNT), 0, st, cp);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// Routed pairs on the bank kernel (lut_bank.hip): from kBankSortMinTokens
// tokens a plan launch sorts the valid pairs by expert into work lists of
// (pair, 512-row block), so the pairs of one expert run back to back on one
// XCD and its codes stream through one L2; below it workgroups map straight
// to (pair, row block).  From kTokGateUpMinTokens tokens gate/up runs on the
// token-major resident-LUT kernel instead, and down on the pair-major one
// whenever its input fits (their rows are the same sums in the same order).
// Gate/up writes s_m * (gate | up) rows per pair, down
// stages silu(gate) * up as its input and writes s_dn * down per pair, and
// the ordered combine sums w_j * down_j over the slots.
template <typename T>
int moe_forward_bank(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_, int k,
                     bool sorted, hipStream_t st) {
    const size_t P = (size_t)T_ * k;
    const int nb_gu = (2 * m->I + kBankRows - 1) / kBankRows, nb_dn = (m->H + kBankRows - 1) / kBankRows;
    int rc = m->gu_out.ensure(P * 2 * m->I * sizeof(float));
    if (!rc) rc = m->dout.ensure(P * m->H * sizeof(float));
    if (!rc && sorted) rc = m->work.ensure(P * (nb_gu + nb_dn) * sizeof(int2));
    if (!rc && sorted) rc = m->nwork.ensure(2 * sizeof(int));
    if (rc) return rc;
    int2 *work_gu = nullptr, *work_dn = nullptr;
    if (sorted) {
        work_gu = m->work.as<int2>();
        work_dn = work_gu + P * nb_gu;
        rc = launch_moe_plan(idx, w, (int)P, m->E, nb_gu, nb_dn, work_gu, work_dn,
                             m->nwork.as<int>(), st);
        if (rc) return rc;
    }
    MoEBankLaunch l{};
    l.codes_b = m->gub.as<uint8_t>();
    l.expert_bytes = m->gub_bytes;
    l.cb3 = m->cb3_in.ptr;
    l.scales = m->gus.as<float>();
    l.x = x;
    l.y = m->gu_out.as<float>();
    l.idx = idx;
    l.w = w;
    l.work = work_gu;
    l.n_work = m->nwork.as<int>();
    l.M = 2 * m->I;
    l.K = m->H;
    l.k = k;
    l.E = m->E;
    l.max_work = (int)(P * nb_gu);
    l.xs = std::is_same<T, float>::value ? 0 : 1;
    rc = T_ >= kTokGateUpMinTokens && moe_resident_fits(m->H, l.xs) ? launch_moe_resident(l, T_, k, st)
                                                                     : launch_moe_bank(l, st);
    if (rc) return rc;
    l.codes_b = m->dnb.as<uint8_t>();
    l.expert_bytes = m->dnb_bytes;
    l.cb3 = m->cb3_dn.ptr;
    l.scales = m->dns.as<float>();
    l.x = m->gu_out.as<float>();
    l.y = m->dout.as<float>();
    l.work = work_dn;
    l.n_work = sorted ? m->nwork.as<int>() + 1 : nullptr;
    l.M = m->H;
    l.K = m->I;
    l.max_work = (int)(P * nb_dn);
    l.xs = 2;
    rc = moe_resident_fits(m->I, l.xs) ? launch_moe_resident(l, (int)P, 1, st) : launch_moe_bank(l, st);
    if (rc) return rc;
    MoEParams cp{};
    cp.dout = m->dout.as<float>();
    cp.idx = idx;
    cp.w = w;
    cp.y = y;
    cp.E = m->E;
    cp.H = m->H;
    cp.T = T_;
    cp.k = k;
    OJX_LAUNCH((moe_combine_kernel<T>), dim3((m->H + kNT - 1) / kNT, T_), dim3(kNT), 0, st, cp);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

int moe_forward(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_, int k,
                int dtype, hipStream_t st) {
    if (k <= 0 || T_ <= 0) return OJASX_OK;
    if (dtype != OJASX_DTYPE_F32 && dtype != OJASX_DTYPE_BF16) {
        set_error("unsupported dtype %d", dtype);
        return OJASX_ERR_INVALID;
    }
    if (T_ > 65535) {
        set_error("too many tokens in one call");
        return OJASX_ERR_INVALID;
    }
    {
        // single-kernel-per-stage path: block_dim 16, aligned activations,
        // the staged vectors fit LDS
        const size_t align = dtype == OJASX_DTYPE_F32 ? 16 : 8;
        const bool aligned = m->H % 4 == 0 && m->I % 4 == 0 &&
                             reinterpret_cast<uintptr_t>(x) % align == 0;
        // (the dynamic LDS plus the kernels' static partial sums, <= 4.3 KB)
        constexpr size_t kDecStatic = 8 * 1024;
        const bool ok = m->D == 16 && k <= 32 && aligned &&
                        (size_t)(kCB * 16 + (size_t)k * m->Si * 256) * 4 + kDecStatic <= kMaxLds &&
                        (size_t)(kCB * 16 + m->Sin * 256) * 4 + kDecStatic <= kMaxLds;
        // on the bank kernel; sorted by expert, the expert ids must fit the
        // work entries' 16 bits and the plan kernel's LDS hold 3 E + P ints
        const size_t P = (size_t)T_ * k;
        const bool resident = T_ >= kTokGateUpMinTokens && moe_resident_fits(m->H, 0) &&
                              moe_resident_fits(m->I, 2);
        const bool sorted = T_ >= kBankSortMinTokens && !resident;
        const bool plan_fits = P <= kBankMaxPairs && m->E <= 65535 &&
                               (3 * (size_t)m->E + P) * sizeof(int) <= kMaxLds;
        const int nb = (std::max(2 * m->I, m->H) + kBankRows - 1) / kBankRows;
        if (m->D == 16 && aligned && T_ >= kBankMinTokens && m->gub.ptr && bank_fits(m->H) &&
            bank_fits(m->I) && (sorted ? plan_fits : P * nb <= 0x7fffffff))
            return dtype == OJASX_DTYPE_F32
                       ? moe_forward_bank<float>(m, x, idx, w, y, T_, k, sorted, st)
                       : moe_forward_bank<__hip_bfloat16>(m, x, idx, w, y, T_, k, sorted, st);
        // grouped per slot: the staged input and two LUT buffers fit the LDS
        const bool group_fits =
            (size_t)std::max(m->Sin, m->Si) * 256 * sizeof(float) + slices::lut_bytes(kGroupDB) <=
            kMaxLds;
        if (m->D == 16 && T_ >= kGroupMinTokens && group_fits)
            return dtype == OJASX_DTYPE_F32 ? moe_forward_group<float>(m, x, idx, w, y, T_, k, st)
                                            : moe_forward_group<__hip_bfloat16>(m, x, idx, w, y, T_, k, st);
        if (ok)
            return dtype == OJASX_DTYPE_F32 ? moe_forward_dec<float>(m, x, idx, w, y, T_, k, st)
                                            : moe_forward_dec<__hip_bfloat16>(m, x, idx, w, y, T_, k, st);
    }
    const size_t P = (size_t)T_ * k;
    const int Gp_in = m->Sin * kGS;
    int rc = m->lut_in.ensure((size_t)T_ * Gp_in * kCB * sizeof(float));
    if (!rc) rc = m->dout.ensure(P * m->H * sizeof(float));
    if (!rc) rc = m->inter.ensure(P * m->I * sizeof(float));
    if (!rc) rc = m->lut_dn.ensure(P * m->Si * kGS * kCB * sizeof(float));
    if (rc) return rc;
    rc = launch_lut_build(x, m->cb_in.as<float>(), T_, m->H, m->D, m->Gin, Gp_in,
                          m->lut_in.as<float>(), dtype, st);
    if (rc) return rc;
    MoEParams p{};
    p.gu = m->gu.as<uint8_t>();
    p.dn = m->dn.as<uint8_t>();
    p.gus = m->gus.as<float>();
    p.dns = m->dns.as<float>();
    p.cb_dn = m->cb_dn.as<float>();
    p.lut_in = m->lut_in.as<float>();
    p.lut_dn = m->lut_dn.as<float>();
    p.dout = m->dout.as<float>();
    p.inter = m->inter.as<float>();
    p.idx = idx;
    p.w = w;
    p.y = y;
    p.E = m->E;
    p.H = m->H;
    p.I = m->I;
    p.D = m->D;
    p.Sin = m->Sin;
    p.Si = m->Si;
    p.Ip = m->Ip;
    p.Hp = m->Hp;
    p.T = T_;
    p.k = k;
    const int nrb_g = (m->I + kRG - 1) / kRG;
    const int nrb_d = (m->H + kRD - 1) / kRD;
    OJX_LAUNCH(moe_gateup_kernel, dim3(P * nrb_g), dim3(kNT), 0, st, p);
    OJX_LAUNCH(moe_lut_down_kernel, dim3(P, m->Si * kGS), dim3(kNT), 0, st, p);
    OJX_LAUNCH(moe_down_kernel, dim3(P * nrb_d), dim3(kNT), 0, st, p);
    dim3 gc((m->H + kNT - 1) / kNT, T_);
    if (dtype == OJASX_DTYPE_F32)
        OJX_LAUNCH(moe_combine_kernel<float>, gc, dim3(kNT), 0, st, p);
    else
        OJX_LAUNCH(moe_combine_kernel<__hip_bfloat16>, gc, dim3(kNT), 0, st, p);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

}  // namespace
}  // namespace ojx

using ojx::MoE;

extern "C" {

OJASX_API OjasxMoEHandle ojasx_create_moe(int num_experts, int hidden_dim, int intermediate_dim,
                                          int top_k, int block_dim, const float *codebook_in,
                                          const float *codebook_down,
                                          const uint8_t *gate_up_codes,
                                          const float *gate_up_scales, const uint8_t *down_codes,
                                          const float *down_scales) {
    using namespace ojx;
    if (num_experts <= 0 || hidden_dim <= 0 || intermediate_dim <= 0 || block_dim <= 0 ||
        hidden_dim % block_dim || intermediate_dim % block_dim) {
        set_error("invalid MoE shape E=%d H=%d I=%d block=%d (block must divide 32)", num_experts, hidden_dim,
                  intermediate_dim, block_dim);
        return nullptr;
    }
    MoE *m = new (std::nothrow) MoE;
    if (!m) return nullptr;
    m->E = num_experts;
    m->H = hidden_dim;
    m->I = intermediate_dim;
    m->top_k = top_k;
    m->D = block_dim;
    m->Gin = hidden_dim / block_dim;
    m->Gi = intermediate_dim / block_dim;
    m->Sin = (m->Gin + kGS - 1) / kGS;
    m->Si = (m->Gi + kGS - 1) / kGS;
    m->Ip = (int)round_up(intermediate_dim, kRowAlign);
    m->Hp = (int)round_up(hidden_dim, kRowAlign);
    const size_t E = num_experts, I = intermediate_dim, H = hidden_dim;
    // gate/up: [E][Sin][2][Ip][16], gate rows in half 0, up rows in half 1
    std::vector<uint8_t> gu(E * m->Sin * 2 * m->Ip * kGS, 0);
    if (gate_up_codes)
        for (size_t e = 0; e < E; ++e)
            for (size_t r = 0; r < 2 * I; ++r) {
                const size_t half = r / I, i = r % I;
                const uint8_t *row = gate_up_codes + (e * 2 * I + r) * m->Gin;
                for (int g = 0; g < m->Gin; ++g)
                    gu[(((e * m->Sin + g / kGS) * 2 + half) * m->Ip + i) * kGS + g % kGS] = row[g];
            }
    std::vector<uint8_t> dn(E * m->Si * m->Hp * kGS, 0);
    if (down_codes)
        for (size_t e = 0; e < E; ++e)
            for (size_t h = 0; h < H; ++h) {
                const uint8_t *row = down_codes + (e * H + h) * m->Gi;
                for (int g = 0; g < m->Gi; ++g)
                    dn[((e * m->Si + g / kGS) * m->Hp + h) * kGS + g % kGS] = row[g];
            }
    std::vector<float> cbi((size_t)kCB * block_dim, 0.f), cbd((size_t)kCB * block_dim, 0.f);
    if (codebook_in) memcpy(cbi.data(), codebook_in, sizeof(float) * kCB * block_dim);
    if (codebook_down) memcpy(cbd.data(), codebook_down, sizeof(float) * kCB * block_dim);
    std::vector<float> gus(E * 2 * I, 1.f), dns(E * H, 1.f);
    if (gate_up_scales) memcpy(gus.data(), gate_up_scales, sizeof(float) * gus.size());
    if (down_scales) memcpy(dns.data(), down_scales, sizeof(float) * dns.size());
    int rc = upload(m->gu, gu.data(), gu.size());
    if (!rc) rc = upload(m->dn, dn.data(), dn.size());
    if (!rc && block_dim == 16) {   // the bank kernel's layouts, expert after expert
        m->gub_bytes = bank_codes_bytes(2 * intermediate_dim, m->Gin);
        m->dnb_bytes = bank_codes_bytes(hidden_dim, m->Gi);
        std::vector<uint8_t> gb(E * m->gub_bytes + kBankSlack, 0), db(E * m->dnb_bytes + kBankSlack, 0);
        if (gate_up_codes)
            for (size_t e = 0; e < E; ++e)
                pack_bank_codes(gate_up_codes + e * 2 * I * m->Gin, 2 * intermediate_dim, m->Gin,
                                gb.data() + e * m->gub_bytes);
        if (down_codes)
            for (size_t e = 0; e < E; ++e)
                pack_bank_codes(down_codes + e * H * m->Gi, hidden_dim, m->Gi,
                                db.data() + e * m->dnb_bytes);
        rc = upload(m->gub, gb.data(), gb.size());
        if (!rc) rc = upload(m->dnb, db.data(), db.size());
        std::vector<uint16_t> c3(kCb3Bytes / 2);
        split_codebook_bf16x3(cbi.data(), c3.data());
        if (!rc) rc = upload(m->cb3_in, c3.data(), kCb3Bytes);
        split_codebook_bf16x3(cbd.data(), c3.data());
        if (!rc) rc = upload(m->cb3_dn, c3.data(), kCb3Bytes);
    }
    if (!rc) rc = upload(m->cb_in, cbi.data(), cbi.size() * 4);
    if (!rc) rc = upload(m->cb_dn, cbd.data(), cbd.size() * 4);
    if (!rc) rc = upload(m->gus, gus.data(), gus.size() * 4);
    if (!rc) rc = upload(m->dns, dns.data(), dns.size() * 4);
    if (rc) {
        delete m;
        return nullptr;
    }
    return m;
}

OJASX_API int ojasx_moe_forward_device(OjasxMoEHandle handle, const void *x, const int *idx,
                                       const float *w, void *y, int num_tokens, int k_active,
                                       int dtype, void *stream) {
    if (!handle || !x || !idx || !w || !y) return OJASX_ERR_NULL;
    return ojx::moe_forward(static_cast<MoE *>(handle), x, idx, w, y, num_tokens, k_active, dtype,
                            static_cast<hipStream_t>(stream));
}

OJASX_API int ojasx_moe_forward(OjasxMoEHandle handle, const float *x, const int *top_k_indices,
                                const float *top_k_weights, float *y_out, int k_active) {
    using namespace ojx;
    if (!handle || !x || !top_k_indices || !top_k_weights || !y_out) return OJASX_ERR_NULL;
    if (k_active <= 0) return OJASX_OK;
    MoE *m = static_cast<MoE *>(handle);
    // one upload: x [H] | indices [k] | weights [k], 256-byte aligned parts
    const size_t xb = (size_t)m->H * 4, kb = (size_t)k_active * 4;
    const size_t io_i = round_up(xb, 256), io_w = io_i + round_up(kb, 256);
    const size_t in_bytes = io_w + kb, yo = round_up(in_bytes, 256);
    int rc = m->xstage.ensure(in_bytes);
    if (!rc) rc = m->ystage.ensure(xb);
    HostIO &io = host_io();
    if (!rc) rc = io.reserve(yo + xb);
    if (rc) return rc;
    memcpy(io.pin, x, xb);
    memcpy(io.pin + io_i, top_k_indices, kb);
    memcpy(io.pin + io_w, top_k_weights, kb);
    unsigned char *d = m->xstage.as<unsigned char>();
    OJX_HIP(hipMemcpyAsync(d, io.pin, in_bytes, hipMemcpyHostToDevice, io.st));
    rc = moe_forward(m, d, reinterpret_cast<const int *>(d + io_i),
                     reinterpret_cast<const float *>(d + io_w), m->ystage.ptr, 1, k_active,
                     OJASX_DTYPE_F32, io.st);
    if (!rc) OJX_HIP(hipMemcpyAsync(io.pin + yo, m->ystage.ptr, xb, hipMemcpyDeviceToHost, io.st));
    OJX_HIP(hipStreamSynchronize(io.st));
    if (rc) return rc;
    memcpy(y_out, io.pin + yo, xb);
    return OJASX_OK;
}

OJASX_API int ojasx_moe_route_device(const float *logits, int num_tokens, int num_experts, int k,
                                     int renormalize, int *idx, float *w, void *stream) {
    using namespace ojx;
    if (!logits || !idx || !w) return OJASX_ERR_NULL;
    if (num_tokens <= 0) return OJASX_OK;
    if (num_experts <= 0 || num_experts > 1024 || k <= 0 || k > 32 || k > num_experts) {
        set_error("router supports 1 <= k <= min(32, E), E <= 1024");
        return OJASX_ERR_INVALID;
    }
    OJX_LAUNCH(moe_route_kernel, dim3((num_tokens + kNT / 64 - 1) / (kNT / 64)), dim3(kNT), 0,
                       static_cast<hipStream_t>(stream), logits, num_tokens, num_experts, k,
                       renormalize, idx, w);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

OJASX_API size_t ojasx_moe_get_compressed_size(OjasxMoEHandle handle) {
    if (!handle) return 0;
    const MoE *m = static_cast<const MoE *>(handle);
    const size_t E = m->E;
    return E * 2 * m->I * m->Gin + E * 2 * m->I * 4 + E * m->H * m->Gi + E * m->H * 4 +
           (size_t)2 * 256 * m->D * 4;
}

OJASX_API float ojasx_moe_get_compression_ratio(OjasxMoEHandle handle) {
    if (!handle) return 0.f;
    const MoE *m = static_cast<const MoE *>(handle);
    const double dense = (double)m->E * 3 * m->H * m->I * 4;
    const size_t c = ojasx_moe_get_compressed_size(handle);
    return (float)(dense / (double)(c ? c : 1));
}

OJASX_API void ojasx_destroy_moe(OjasxMoEHandle handle) { delete static_cast<MoE *>(handle); }

}  // extern "C"

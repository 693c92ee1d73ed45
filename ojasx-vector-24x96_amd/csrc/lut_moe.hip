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
// Four launches per call, no cross-workgroup synchronisation inside a kernel
// (a "pair" is one routed (token, slot)):
//  1. LUT_in of every token (the linear layer's LUT-build kernel).
//  2. moe_gateup: workgroup = (pair, 32 intermediate rows) x 8 slice groups;
//     thread (q, r) gathers gate row i and up row i for its slices, the slice
//     partials are reduced in LDS in a fixed order, then SwiGLU gives 32
//     intermediate values -- two 16-wide groups -- from which the same
//     workgroup builds those groups' LUT_down rows (256 centroids each).
//  3. moe_down: workgroup = (pair, 64 hidden rows) x 4 slice groups: gather
//     from the pair's LUT_down, reduce, scale -> per-pair output [P][H].
//  4. moe_combine: y[t][h] = sum_j w_j * out[t,j][h] in slot order -- a fixed
//     order, so results are deterministic.
//  Router: moe_route, one workgroup per token.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

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
    DevBuf lut_in, lut_dn, dout, xstage, ystage, istage, wstage;
    size_t lut_dn_pairs = 0;
    ~MoE() {
        for (DevBuf *b : {&cb_in, &cb_dn, &gu, &dn, &gus, &dns, &lut_in, &lut_dn, &dout, &xstage,
                          &ystage, &istage, &wstage})
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

template <int DT>
__global__ __launch_bounds__(kNT) void moe_gateup_kernel(MoEParams p) {
    constexpr int QG = kNT / kRG;  // 8 slice groups
    __shared__ float red[2][QG][kRG];
    __shared__ float inter_s[kRG];
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
    if (q == 0) {
        float g = red[0][0][r], u = red[1][0][r];
#pragma unroll
        for (int k = 1; k < QG; ++k) {
            g += red[0][k][r];
            u += red[1][k][r];
        }
        float v = 0.f;
        if (i < p.I) {
            g *= p.gus[(size_t)e * 2 * p.I + i];
            u *= p.gus[(size_t)e * 2 * p.I + p.I + i];
            v = g / (1.f + expf(-g)) * u;
        }
        inter_s[r] = v;
    }
    __syncthreads();
    // LUT_down rows of the kRG / D groups this workgroup produced.
    constexpr int DMAX = DT > 0 ? DT : 32;
    const int D = DT > 0 ? DT : p.D;
    const int ng = kRG / D;
    const int g0 = rb * ng;
    float c[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) c[d] = d < D ? p.cb_dn[tid * D + d] : 0.f;
    float *Ld = p.lut_dn + (size_t)pr * p.Si * kGS * kCB;
    for (int gl = 0; gl < ng; ++gl) {
        const int g = g0 + gl;
        if (g * D >= p.I) break;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) dot = fmaf(inter_s[gl * D + d], c[d], dot);
        Ld[(size_t)g * kCB + tid] = dot;
    }
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
// wave per token: lane l holds logits l + 64*i (E <= 1024); each of the k
// rounds is a local argmax plus a 6-step shuffle reduction, no barriers.
__global__ __launch_bounds__(kNT) void moe_route_kernel(const float *logits, int T, int E, int k,
                                                       int renorm, int *idx, float *w) {
    constexpr int NV = 16;
    __shared__ float selv[kNT / 64][32];
    __shared__ int seli[kNT / 64][32];
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
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e = lane + 64 * i;
            if (e < E && !((taken >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) {
                bv = v[i];
                bi = e;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == 0) {
            selv[wv][j] = bv;
            seli[wv][j] = bi;
        }
    }
    // softmax statistics over all E logits
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) m = fmaxf(m, v[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (lane + 64 * i < E) sum += expf(v[i] - m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    __syncthreads();
    float wj = 0.f;
    int ij = 0;
    if (lane < k) {
        ij = seli[wv][lane];
        wj = expf(selv[wv][lane] - m) / sum;
    }
    if (renorm) {
        float tot = wj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off);
        wj = wj / tot;
    }
    if (lane < k && t_raw < T) {
        idx[(size_t)t * k + lane] = ij;
        w[(size_t)t * k + lane] = wj;
    }
}

namespace {

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
    const size_t P = (size_t)T_ * k;
    const int Gp_in = m->Sin * kGS;
    int rc = m->lut_in.ensure((size_t)T_ * Gp_in * kCB * sizeof(float));
    if (!rc) rc = m->dout.ensure(P * m->H * sizeof(float));
    if (rc) return rc;
    const size_t ldn = (size_t)m->Si * kGS * kCB * sizeof(float);
    if (P > m->lut_dn_pairs) {
        // LUT_down rows of padded groups (>= Gi) stay zero: written only here.
        rc = m->lut_dn.ensure(P * ldn);
        if (rc) return rc;
        OJX_HIP(hipMemsetAsync(m->lut_dn.ptr, 0, P * ldn, st));
        m->lut_dn_pairs = P;
    }
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
    if (m->D == 16)
        hipLaunchKernelGGL(moe_gateup_kernel<16>, dim3(P * nrb_g), dim3(kNT), 0, st, p);
    else
        hipLaunchKernelGGL(moe_gateup_kernel<0>, dim3(P * nrb_g), dim3(kNT), 0, st, p);
    hipLaunchKernelGGL(moe_down_kernel, dim3(P * nrb_d), dim3(kNT), 0, st, p);
    dim3 gc((m->H + kNT - 1) / kNT, T_);
    if (dtype == OJASX_DTYPE_F32)
        hipLaunchKernelGGL(moe_combine_kernel<float>, gc, dim3(kNT), 0, st, p);
    else
        hipLaunchKernelGGL(moe_combine_kernel<__hip_bfloat16>, gc, dim3(kNT), 0, st, p);
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
        block_dim > 32 || hidden_dim % block_dim || intermediate_dim % block_dim ||
        kRG % block_dim) {
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
    int rc = m->xstage.ensure((size_t)m->H * 4);
    if (!rc) rc = m->ystage.ensure((size_t)m->H * 4);
    if (!rc) rc = m->istage.ensure((size_t)k_active * 4);
    if (!rc) rc = m->wstage.ensure((size_t)k_active * 4);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(m->xstage.ptr, x, (size_t)m->H * 4, hipMemcpyHostToDevice));
    OJX_HIP(hipMemcpy(m->istage.ptr, top_k_indices, (size_t)k_active * 4, hipMemcpyHostToDevice));
    OJX_HIP(hipMemcpy(m->wstage.ptr, top_k_weights, (size_t)k_active * 4, hipMemcpyHostToDevice));
    rc = moe_forward(m, m->xstage.ptr, m->istage.as<int>(), m->wstage.as<float>(), m->ystage.ptr,
                     1, k_active, OJASX_DTYPE_F32, nullptr);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(y_out, m->ystage.ptr, (size_t)m->H * 4, hipMemcpyDeviceToHost));
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
    hipLaunchKernelGGL(moe_route_kernel, dim3((num_tokens + kNT / 64 - 1) / (kNT / 64)), dim3(kNT), 0,
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

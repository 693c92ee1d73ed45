// lut_moe.hip -- top-k split-manifold MoE layer and router on gfx950.
//
// Per token t and routed slot j (expert e = idx[t][j], weight w = w[t][j]):
//   gate_i = sg_e[i]   * sum_g LUT_in[g, gu_codes[e][i][g]]
//   up_i   = sg_e[I+i] * sum_g LUT_in[g, gu_codes[e][I+i][g]]
//   inter_i = silu(gate_i) * up_i,             silu(v) = v / (1 + exp(-v))
//   y[t][h] += w * sd_e[h] * sum_g LUT_down[g, dn_codes[e][h][g]]   (j ascending)
// the computation of split_manifold_lut_experiment/native/src/
// ojasx_lut_cpu.cpp:213-365, including its skip rule (:284-286: e outside
// [0,E) or |w| < 1e-8 contributes nothing) and output rule (:220-223: y is
// zeroed when k_active > 0, untouched otherwise).  Only routed experts' codes
// are ever read.
//
// Kernels (one stream, four launches per call):
//  1. moe_gateup: workgroup = (pair, run of 16-group slices of H).  Builds the
//     token's LUT_in slice in LDS, gathers gate row i and up row i for
//     i = tid + 256*j in the same thread; partial sums go to the workspace
//     and the last workgroup of the pair (ticket) reduces them in slice
//     order and applies scales and SwiGLU -> inter[pair][I] (fp32).
//  2. moe_down: workgroup = (pair, 16-group slice of I, row block of H).
//     Builds LUT_down for the slice from inter, gathers, writes unscaled
//     partials [pair][slice][H].
//  3. moe_combine: y[t][h] = sum_j w_j * (sd_e[h] * sum_s partial[s]) in
//     slot order -- a fixed order, so results are deterministic.
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
constexpr int kMaxJ = 4;  // I <= 1024 (gate/up rows per thread)
}  // namespace

struct MoE {
    int E = 0, H = 0, I = 0, top_k = 0, D = 0;
    int Gin = 0, Gi = 0, Sin = 0, Si = 0, Ip = 0, Hp = 0;
    DevBuf cb_in, cb_dn, gu, dn, gus, dns;
    DevBuf part1, ctr, inter, part2, xstage, ystage, istage, wstage;
    size_t ctr_n = 0;
    ~MoE() {
        for (DevBuf *b : {&cb_in, &cb_dn, &gu, &dn, &gus, &dns, &part1, &ctr, &inter, &part2,
                          &xstage, &ystage, &istage, &wstage})
            b->release();
    }
};

struct MoEParams {
    const uint8_t *gu;      // [E][Sin][2][Ip][16]
    const uint8_t *dn;      // [E][Si][Hp][16]
    const float *gus;       // [E][2I]
    const float *dns;       // [E][H]
    const float *cb_in;     // [256][D]
    const float *cb_dn;     // [256][D]
    const void *x;          // [T][H]
    const int *idx;         // [T][k]
    const float *w;         // [T][k]
    void *y;                // [T][H]
    float *part1;           // [P][n_split1][2][Ip]
    unsigned *ctr;          // [P]
    float *inter;           // [P][I]
    float *part2;           // [P][Si][Hp]
    int E, H, I, D, Sin, Si, Ip, Hp, T, k, spw1, n_split1, rpb2;
};

__device__ __forceinline__ bool pair_active(const MoEParams &p, int pr, int *e_out) {
    const int e = p.idx[pr];
    const float w = p.w[pr];
    *e_out = e;
    return e >= 0 && e < p.E && fabsf(w) >= 1e-8f;
}

// LUT[g][k = tid] for 16 groups from xs[16*D] (LDS) and centroid k in registers.
template <int DMAX>
__device__ __forceinline__ void build_slice(const float *xs, const float *cb, int D, float *lut) {
    const int tid = threadIdx.x;
#pragma unroll 4
    for (int g = 0; g < kGS; ++g) {
        const float *xg = xs + g * D;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) dot = fmaf(xg[d], cb[d], dot);
        lut[g * kCB + tid] = dot;
    }
}

__device__ __forceinline__ float gather16(const float *lut, uint4 c) {
    const uint32_t w4[4] = {c.x, c.y, c.z, c.w};
    float a = 0.f;
#pragma unroll
    for (int g = 0; g < kGS; ++g) a += lut[g * kCB + ((w4[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
    return a;
}

template <int DT, typename T>
__global__ __launch_bounds__(kNT) void moe_gateup_kernel(MoEParams p) {
    constexpr int DMAX = DT > 0 ? DT : 32;
    const int D = DT > 0 ? DT : p.D;
    const int sc = kGS * D;
    __shared__ float lut[kGS * kCB];
    __shared__ float xs[kGS * 32];
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int pr = blockIdx.x / p.n_split1;
    const int sp = blockIdx.x - pr * p.n_split1;
    int e;
    if (!pair_active(p, pr, &e)) return;
    const int t = pr / p.k;
    const T *x = static_cast<const T *>(p.x);
    const int nj = (p.I + kNT - 1) / kNT;

    float cb[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) cb[d] = (d < D) ? p.cb_in[tid * D + d] : 0.f;
    float ag[kMaxJ], au[kMaxJ];
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j) ag[j] = au[j] = 0.f;

    const int s0 = sp * p.spw1, s1 = min(p.Sin, s0 + p.spw1);
    const uint8_t *eg = p.gu + (size_t)e * p.Sin * 2 * p.Ip * kGS;
    for (int s = s0; s < s1; ++s) {
        uint4 cg[kMaxJ], cu[kMaxJ];
        const uint8_t *gs = eg + (size_t)s * 2 * p.Ip * kGS;
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j)
            if (j < nj) {
                const int i = j * kNT + tid;
                cg[j] = *reinterpret_cast<const uint4 *>(gs + (size_t)i * kGS);
                cu[j] = *reinterpret_cast<const uint4 *>(gs + ((size_t)p.Ip + i) * kGS);
            }
        for (int i = tid; i < sc; i += kNT) {
            const int col = s * sc + i;
            xs[i] = col < p.H ? load_act(x, (size_t)t * p.H + col) : 0.f;
        }
        __syncthreads();
        build_slice<DMAX>(xs, cb, D, lut);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j)
            if (j < nj) {
                ag[j] += gather16(lut, cg[j]);
                au[j] += gather16(lut, cu[j]);
            }
        __syncthreads();
    }

    const float *gsc = p.gus + (size_t)e * 2 * p.I;
    if (p.n_split1 == 1) {
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j) {
            const int i = j * kNT + tid;
            if (j < nj && i < p.I) {
                const float g = ag[j] * gsc[i], u = au[j] * gsc[p.I + i];
                p.inter[(size_t)pr * p.I + i] = g / (1.f + expf(-g)) * u;
            }
        }
        return;
    }
    float *pp = p.part1 + ((size_t)pr * p.n_split1 + sp) * 2 * p.Ip;
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j)
        if (j < nj) {
            const int i = j * kNT + tid;
            pp[i] = ag[j];
            pp[p.Ip + i] = au[j];
        }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned old = atomicAdd(p.ctr + pr, 1u);
        s_last = (old == (unsigned)(p.n_split1 - 1));
        if (s_last) atomicExch(p.ctr + pr, 0u);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float *pb = p.part1 + (size_t)pr * p.n_split1 * 2 * p.Ip;
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j) {
        const int i = j * kNT + tid;
        if (j < nj && i < p.I) {
            float g = 0.f, u = 0.f;
            for (int q = 0; q < p.n_split1; ++q) {
                g += pb[(size_t)q * 2 * p.Ip + i];
                u += pb[(size_t)q * 2 * p.Ip + p.Ip + i];
            }
            g *= gsc[i];
            u *= gsc[p.I + i];
            p.inter[(size_t)pr * p.I + i] = g / (1.f + expf(-g)) * u;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kNT) void moe_down_kernel(MoEParams p) {
    constexpr int DMAX = DT > 0 ? DT : 32;
    const int D = DT > 0 ? DT : p.D;
    const int sc = kGS * D;
    __shared__ float lut[kGS * kCB];
    __shared__ float xs[kGS * 32];
    const int tid = threadIdx.x;
    const int n_rb = (p.H + kNT * p.rpb2 - 1) / (kNT * p.rpb2);
    int b = blockIdx.x;
    const int rb = b % n_rb;
    b /= n_rb;
    const int s = b % p.Si;
    const int pr = b / p.Si;
    int e;
    if (!pair_active(p, pr, &e)) return;

    float cb[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) cb[d] = (d < D) ? p.cb_dn[tid * D + d] : 0.f;
    for (int i = tid; i < sc; i += kNT) {
        const int col = s * sc + i;
        xs[i] = col < p.I ? p.inter[(size_t)pr * p.I + col] : 0.f;
    }
    const uint8_t *es = p.dn + ((size_t)e * p.Si + s) * p.Hp * kGS;
    __syncthreads();
    build_slice<DMAX>(xs, cb, D, lut);
    __syncthreads();
    float *out = p.part2 + ((size_t)pr * p.Si + s) * p.Hp;
    for (int j = 0; j < p.rpb2; ++j) {
        const int h = (rb * p.rpb2 + j) * kNT + tid;
        if (h < p.Hp) out[h] = gather16(lut, *reinterpret_cast<const uint4 *>(es + (size_t)h * kGS));
    }
}

template <typename T>
__global__ __launch_bounds__(kNT) void moe_combine_kernel(MoEParams p) {
    const int t = blockIdx.y;
    const int h = blockIdx.x * kNT + threadIdx.x;
    if (h >= p.H) return;
    float y = 0.f;
    for (int j = 0; j < p.k; ++j) {
        const int pr = t * p.k + j;
        int e;
        if (!pair_active(p, pr, &e)) continue;
        const float *pp = p.part2 + (size_t)pr * p.Si * p.Hp + h;
        float s = 0.f;
        for (int q = 0; q < p.Si; ++q) s += pp[(size_t)q * p.Hp];
        y += (s * p.dns[(size_t)e * p.H + h]) * p.w[pr];
    }
    store_act(static_cast<T *>(p.y), (size_t)t * p.H + h, y);
}

// Router: top-k of the logits (descending, ties to the lower index) and the
// softmax probability of each selected expert, optionally renormalised.
__global__ __launch_bounds__(kNT) void moe_route_kernel(const float *logits, int E, int k,
                                                       int renorm, int *idx, float *w) {
    __shared__ float lg[1024];
    __shared__ unsigned char taken[1024];
    __shared__ float rv[kNT];
    __shared__ int ri[kNT];
    __shared__ float s_max, s_sum;
    __shared__ int sel[32];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *l = logits + (size_t)t * E;
    for (int i = tid; i < E; i += kNT) {
        lg[i] = l[i];
        taken[i] = 0;
    }
    __syncthreads();
    for (int j = 0; j < k; ++j) {
        float bv = 0.f;
        int bi = -1;
        for (int i = tid; i < E; i += kNT)
            if (!taken[i] && (bi < 0 || lg[i] > bv)) {
                bv = lg[i];
                bi = i;
            }
        rv[tid] = bv;
        ri[tid] = bi;
        __syncthreads();
        for (int st = kNT / 2; st > 0; st >>= 1) {
            if (tid < st) {
                const float ov = rv[tid + st];
                const int oi = ri[tid + st];
                const int mi = ri[tid];
                if (oi >= 0 && (mi < 0 || ov > rv[tid] || (ov == rv[tid] && oi < mi))) {
                    rv[tid] = ov;
                    ri[tid] = oi;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            sel[j] = ri[0];
            taken[ri[0]] = 1;
        }
        __syncthreads();
    }
    // softmax statistics over all experts
    float m = -INFINITY;
    for (int i = tid; i < E; i += kNT) m = fmaxf(m, lg[i]);
    rv[tid] = m;
    __syncthreads();
    for (int st = kNT / 2; st > 0; st >>= 1) {
        if (tid < st) rv[tid] = fmaxf(rv[tid], rv[tid + st]);
        __syncthreads();
    }
    if (tid == 0) s_max = rv[0];
    __syncthreads();
    float s = 0.f;
    for (int i = tid; i < E; i += kNT) s += expf(lg[i] - s_max);
    rv[tid] = s;
    __syncthreads();
    for (int st = kNT / 2; st > 0; st >>= 1) {
        if (tid < st) rv[tid] += rv[tid + st];
        __syncthreads();
    }
    if (tid == 0) s_sum = rv[0];
    __syncthreads();
    if (tid == 0) {
        float tot = 0.f;
        float ww[32];
        for (int j = 0; j < k; ++j) {
            ww[j] = expf(lg[sel[j]] - s_max) / s_sum;
            tot += ww[j];
        }
        for (int j = 0; j < k; ++j) {
            idx[(size_t)t * k + j] = sel[j];
            w[(size_t)t * k + j] = renorm ? ww[j] / tot : ww[j];
        }
    }
}

namespace {

template <typename T>
int moe_launch(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_,
               int k, hipStream_t st) {
    const int P = T_ * k;
    // Slices of the gate/up pass per workgroup: enough workgroups to fill the chip.
    const int want = std::max(1, std::min(m->Sin, (512 + P - 1) / P));
    const int spw1 = (m->Sin + want - 1) / want;
    const int n_split1 = (m->Sin + spw1 - 1) / spw1;
    int rc = m->inter.ensure((size_t)P * m->I * sizeof(float));
    if (!rc) rc = m->part2.ensure((size_t)P * m->Si * m->Hp * sizeof(float));
    if (!rc && n_split1 > 1) rc = m->part1.ensure((size_t)P * n_split1 * 2 * m->Ip * sizeof(float));
    if (rc) return rc;
    if ((size_t)P > m->ctr_n) {
        rc = m->ctr.ensure((size_t)P * sizeof(unsigned));
        if (rc) return rc;
        OJX_HIP(hipMemset(m->ctr.ptr, 0, (size_t)P * sizeof(unsigned)));
        m->ctr_n = P;
    }
    MoEParams p{};
    p.gu = m->gu.as<uint8_t>();
    p.dn = m->dn.as<uint8_t>();
    p.gus = m->gus.as<float>();
    p.dns = m->dns.as<float>();
    p.cb_in = m->cb_in.as<float>();
    p.cb_dn = m->cb_dn.as<float>();
    p.x = x;
    p.idx = idx;
    p.w = w;
    p.y = y;
    p.part1 = m->part1.as<float>();
    p.ctr = m->ctr.as<unsigned>();
    p.inter = m->inter.as<float>();
    p.part2 = m->part2.as<float>();
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
    p.spw1 = spw1;
    p.n_split1 = n_split1;
    // down pass: row blocks of 256*rpb2 rows, enough workgroups to fill the chip
    const int per_pair = m->Si;
    int rpb2 = std::max(1, m->Hp / kNT);
    while (rpb2 > 1 && (size_t)P * per_pair * ((m->Hp / kNT + rpb2 - 1) / rpb2) < 512) rpb2 = (rpb2 + 1) / 2;
    p.rpb2 = rpb2;
    const int n_rb2 = (m->H + kNT * rpb2 - 1) / (kNT * rpb2);
    if (m->D == 16) {
        hipLaunchKernelGGL((moe_gateup_kernel<16, T>), dim3(P * n_split1), dim3(kNT), 0, st, p);
        hipLaunchKernelGGL((moe_down_kernel<16>), dim3(P * m->Si * n_rb2), dim3(kNT), 0, st, p);
    } else {
        hipLaunchKernelGGL((moe_gateup_kernel<0, T>), dim3(P * n_split1), dim3(kNT), 0, st, p);
        hipLaunchKernelGGL((moe_down_kernel<0>), dim3(P * m->Si * n_rb2), dim3(kNT), 0, st, p);
    }
    hipLaunchKernelGGL((moe_combine_kernel<T>), dim3((m->H + kNT - 1) / kNT, T_), dim3(kNT), 0,
                       st, p);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

int moe_forward(MoE *m, const void *x, const int *idx, const float *w, void *y, int T_, int k,
                int dtype, hipStream_t st) {
    if (k <= 0 || T_ <= 0) return OJASX_OK;
    if (T_ > 65535) {
        set_error("too many tokens in one call");
        return OJASX_ERR_INVALID;
    }
    if (dtype == OJASX_DTYPE_F32) return moe_launch<float>(m, x, idx, w, y, T_, k, st);
    if (dtype == OJASX_DTYPE_BF16) return moe_launch<__hip_bfloat16>(m, x, idx, w, y, T_, k, st);
    set_error("unsupported dtype %d", dtype);
    return OJASX_ERR_INVALID;
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
        intermediate_dim > kMaxJ * kNT) {
        set_error("invalid MoE shape E=%d H=%d I=%d block=%d", num_experts, hidden_dim,
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
    m->Ip = (int)round_up(intermediate_dim, kNT);
    m->Hp = (int)round_up(hidden_dim, kNT);
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
    hipLaunchKernelGGL(moe_route_kernel, dim3(num_tokens), dim3(kNT), 0,
                       static_cast<hipStream_t>(stream), logits, num_experts, k, renormalize, idx, w);
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

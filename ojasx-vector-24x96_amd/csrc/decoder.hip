// decoder.hip -- a Qwen3-4B-shaped decoder whose every linear layer is a
// split-manifold LUT linear (d = 16, 256 centroids, CSR outliers) and whose
// KV cache is the paged code-domain cache, greedy batch-1 decode on gfx950.
//
// One token step, all state on the device (position, step, token), so the
// step is a fixed launch sequence that a HIP graph replays:
//   per layer
//     1. qkv  = LUT(Wqkv, RMSNorm(x, w_in))           lut_dec_kernel, RMSNorm prologue
//     2. q    = RoPE(RMSNorm_head(q, w_qn));  k = RoPE(RMSNorm_head(k, w_kn));
//        k, v encoded into the layer's paged code cache at `pos`;
//        attn = softmax(q K^T / sqrt(hd)) V over pos + 1 tokens  attn_decode_kernel + merge
//        (partials per 64-token chunk of the cached tokens and one for the new token)
//     3. x   += LUT(Wo, attn)                          residual epilogue
//     4. h    = silu(gate) * up, [gate; up] = LUT(Wgu, RMSNorm(x, w_post))
//                                                     RMSNorm prologue, SwiGLU epilogue (a
//                                                     workgroup owns gate rows and their up rows)
//     5. x   += LUT(Wdown, h)                          residual epilogue
//   head: logits = LUT(Wlm, RMSNorm(x, w_final)); argmax_embed_kernel picks the
//   token (ties to the lower id), stores it, loads its embedding row into x
//   and advances the position.
// RMSNorm is x * (1 / sqrt(mean(x^2) + eps)) * w; RoPE rotates dimension i
// with i + hd/2 by the angle fp32(pos) * inv_freq[i], inv_freq[i] =
// fp32(1 / theta^(2i / hd)), through cos / sin tables computed on the host.
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kHd = 128;          // head dim of the decode kernels
constexpr int kBd = 16;           // block dim of every LUT linear and of the KV codebooks
constexpr int kG = kHd / kBd;     // KV code groups per head
constexpr int kArgNT = 1024;
constexpr int kArgBatch = 8;      // float4 loads in flight per thread in the logit scan
}  // namespace

struct AttnParams {
    const float *qkv;             // [Hq*hd | Hkv*hd (k) | Hkv*hd (v)]
    const float *qn_w, *kn_w;     // [hd]
    const float *cos_t, *sin_t;   // [max_ctx][hd/2]
    const int *state;             // state[0] = position of the new token
    const int *bt;                // block table, ceil(max_ctx / P) entries
    const float *kcb, *vcb;       // [Hkv][256][16]
    uint8_t *kc, *vc;             // [pages][Hkv][P][G]
    float *ks, *vs;               // [pages][Hkv][P]
    float *part_o, *part_ml;      // [Hq][n_chunks + 1][hd], [Hq][n_chunks + 1][2]
    int Hq, Hkv, P, max_ctx, n_chunks;
    float eps, sf;
};

constexpr int kAttnNT = 256;
constexpr int kAttnC = 64;        // tokens per chunk, one per lane

// Attention of the new token at pos = state[0] over the pos + 1 tokens of the
// cache, prologue included, as partials (o, max, sum) per query head: one per
// 64-token chunk of the tokens before pos, and the new token's own in the
// last slot (index n_chunks); kv_merge_kernel combines them.
// Workgroup (x, kv head h, slice z of up to 4 of its query heads); wave j < nj
// owns query head h*R + 4z + j, whose q it normalises (RMSNorm by a wave sum)
// and rotates itself: lane l holds dimensions l and l + 64, a RoPE pair.
//   x < n_chunks: chunk x of the tokens before pos.  Lane (token 16 j + l / 4,
//     quarter l % 4) of wave j reads its token's K codebook quarter once per
//     group for all the workgroup's query heads (a quad sum completes each
//     score); wave j then takes head j's softmax over the chunk (wave
//     reductions); for V, lane l of wave j accumulates output dimensions 2l,
//     2l + 1 of every head over tokens 16 j .. 16 j + 15 (each V codebook row
//     read once), and the four waves' sums are added in wave order.
//   x = n_chunks, n_chunks + 1: the new token's K and V.  Wave 2 of the first
//     normalises and rotates k, wave 3 of the second takes v as is, each
//     scaled by max|.| / 127; thread t holds centroid t of the head's K (V)
//     codebook for the nearest-centroid search of each 16-dimension group
//     (ties to the lower index); slice z = 0 stores codes and scales into the
//     cache.  Its partial (slot n_chunks): max = its score and sum = 1 from the
//     K workgroup, o = v_scale * Cv[code] from the V workgroup.  No workgroup
//     reads the slot being written, and the encoder's chains run beside the
//     chunks' instead of inside one.
__global__ __launch_bounds__(kAttnNT) void attn_decode_kernel(AttnParams p) {
    __shared__ float4 ck4[256 * 4];      // K codebook [256][16], rows swizzled (cb_slot)
    __shared__ float4 cv4[256 * 4];      // V codebook [256][16]
    __shared__ float4 q4s[4 * 32];       // rotated q [4][128]
    __shared__ __align__(16) float xs[kHd];       // new token: k / s_k or v / s_v
    __shared__ float nscale[2];          // its scales
    __shared__ float wd[1][kG][4];       // per-wave nearest distance
    __shared__ int wi[1][kG][4];         // and its lowest centroid
    __shared__ uint2 ncode[2];           // its K and V codes
    __shared__ uint2 kcw[kAttnC], vcw[kAttnC];
    __shared__ float wsc[4][kAttnC];     // K scale * sf and V scale, then p_jt * vs_t
    __shared__ float ssc[4][kAttnC];     // scores of the chunk's tokens per head
    __shared__ float2 ored[4][4][64];    // V sums per wave, head and dim pair
    const int tid = threadIdx.x, lane = tid & 63, j = tid >> 6;
    const int R = p.Hq / p.Hkv;
    const int h = blockIdx.y;
    const int j0 = h * R + blockIdx.z * 4;
    const int nj = min(4, R - (int)blockIdx.z * 4);
    const int c = blockIdx.x;
    const bool fresh = c >= p.n_chunks;          // the new token's workgroups: K, then V
    const int kvf = c - p.n_chunks;              // 0: K, 1: V (fresh)
    const int stride = p.n_chunks + 1;           // partial slots per query head
    // the new token's workgroup has the longest chain (norms, RoPE, the
    // nearest-centroid searches): its waves issue first on their SIMDs
    if (fresh) __builtin_amdgcn_s_setprio(3);
    // ---- round trip 1: the position, codebooks, q rows and norm weights, the
    // new token's k / v rows (its workgroup), wave 0's block-table entry
    const int pos = min(p.state[0], p.max_ctx - 1);
    const float4 *gk = reinterpret_cast<const float4 *>(p.kcb + (size_t)h * 256 * 16);
    const float4 *gv = reinterpret_cast<const float4 *>(p.vcb + (size_t)h * 256 * 16);
    float4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        a[u] = gk[tid + u * kAttnNT];
        b[u] = gv[tid + u * kAttnNT];
    }
    float r0 = 0.f, r1 = 0.f, w0 = 0.f, w1 = 0.f;   // q row and q_norm weights
    if (j < nj) {
        const float *src = p.qkv + (size_t)(j0 + j) * kHd;
        r0 = src[lane];
        r1 = src[lane + 64];
        w0 = p.qn_w[lane];
        w1 = p.qn_w[lane + 64];
    }
    float e0 = 0.f, e1 = 0.f, u0 = 0.f, u1 = 0.f;   // k (wave 2, k_norm weights) / v (wave 3)
    if (fresh && j == 2 + kvf) {
        const float *src = p.qkv + (size_t)(p.Hq + (j - 2) * p.Hkv + h) * kHd;
        e0 = src[lane];
        e1 = src[lane + 64];
        if (j == 2) {
            u0 = p.kn_w[lane];
            u1 = p.kn_w[lane + 64];
        }
    }
    const int tw = c * kAttnC + lane;            // wave 0's token (a chunk)
    const int pg = (!fresh && j == 0) ? p.bt[min(tw, p.max_ctx - 1) / p.P] : 0;
    if (!fresh && c * kAttnC >= pos) return;     // whole workgroup: a chunk past the cached tokens
    // ---- round trip 2: cos / sin at pos; the chunk's codes and scales, or
    // the new token's page
    const float cs = p.cos_t[(size_t)pos * (kHd / 2) + lane];
    const float sn = p.sin_t[(size_t)pos * (kHd / 2) + lane];
    uint2 kw = make_uint2(0, 0), vw = make_uint2(0, 0);
    float ksv = 0.f, vsv = 0.f;
    if (!fresh && j == 0 && tw < pos) {
        const size_t slot = ((size_t)pg * p.Hkv + h) * p.P + (tw % p.P);
        kw = *reinterpret_cast<const uint2 *>(p.kc + slot * kG);
        vw = *reinterpret_cast<const uint2 *>(p.vc + slot * kG);
        ksv = p.ks[slot];
        vsv = p.vs[slot];
    }
    const int npage = fresh ? p.bt[pos / p.P] : 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid + u * kAttnNT;
        ck4[cb_slot(i >> 2, i & 3)] = a[u];
        cv4[tid + u * kAttnNT] = b[u];
    }
    if (j < nj) {
        const float rn = 1.0f / sqrtf(wave_sum_f(r0 * r0 + r1 * r1) / (float)kHd + p.eps);
        const float x0 = (r0 * rn) * w0, x1 = (r1 * rn) * w1;
        float *qf = reinterpret_cast<float *>(q4s) + j * kHd;
        qf[lane] = x0 * cs - x1 * sn;
        qf[lane + 64] = x1 * cs + x0 * sn;
    }

    if (fresh) {
        // kvf = 0: wave 2 normalises and rotates k; kvf = 1: wave 3 takes v
        if (j == 2 && kvf == 0) {
            const float rn = 1.0f / sqrtf(wave_sum_f(e0 * e0 + e1 * e1) / (float)kHd + p.eps);
            const float x0 = (e0 * rn) * u0, x1 = (e1 * rn) * u1;
            e0 = x0 * cs - x1 * sn;
            e1 = x1 * cs + x0 * sn;
        }
        if (j == 2 + kvf) {
            const float s = fmaxf(1e-8f, wave_max_f(fmaxf(fabsf(e0), fabsf(e1)))) / 127.0f;
            xs[lane] = e0 / s;
            xs[lane + 64] = e1 / s;
            if (lane == 0) nscale[kvf] = s;
        }
        __syncthreads();
        const float4 *cb4 = kvf ? cv4 : ck4;
        float cc[kBd];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 ka = cb4[kvf ? tid * 4 + u : cb_slot(tid, u)];
            cc[4 * u] = ka.x, cc[4 * u + 1] = ka.y, cc[4 * u + 2] = ka.z, cc[4 * u + 3] = ka.w;
        }
        // squared distances of centroid tid to the 8 groups, then the 8 wave
        // minima and their lowest centroids, interleaved
        float dd[kG];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const float4 *xg = reinterpret_cast<const float4 *>(xs + g * kBd);
            float dk = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float4 a4 = xg[w];
                const float ak[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float fk = ak[e] - cc[4 * w + e];
                    dk = fmaf(fk, fk, dk);
                }
            }
            dd[g] = dk;
        }
        float mn[kG];
        int id[kG];
#pragma unroll
        for (int i = 0; i < kG; ++i) mn[i] = dd[i];
        wave_min_n(mn);
#pragma unroll
        for (int i = 0; i < kG; ++i) id[i] = dd[i] == mn[i] ? tid : 0x7fffffff;
        wave_min_n(id);
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                wd[0][g][j] = mn[g];
                wi[0][g][j] = id[g];
            }
        }
        __syncthreads();
        if (tid < kG) {
            const int g = tid;
            float bm = wd[0][g][0];
            int bi = wi[0][g][0];
#pragma unroll
            for (int q = 1; q < 4; ++q)
                if (wd[0][g][q] < bm) {   // strictly smaller: earlier waves hold lower indices
                    bm = wd[0][g][q];
                    bi = wi[0][g][q];
                }
            reinterpret_cast<uint8_t *>(ncode)[kvf * kG + g] = (uint8_t)bi;
            if (blockIdx.z == 0) {
                const size_t row = ((size_t)npage * p.Hkv + h) * p.P + (pos % p.P);
                (kvf ? p.vc : p.kc)[row * kG + g] = (uint8_t)bi;
                if (g == 0) (kvf ? p.vs : p.ks)[row] = nscale[kvf];
            }
        }
        __syncthreads();
        // the new token's partial for head j (slot n_chunks): the K workgroup
        // writes its score (the chunk arithmetic for one token) as the max and
        // 1 as the sum, the V workgroup o = v_scale * Cv[code]
        if (j < nj && kvf == 0) {
            const uint2 kn = ncode[0];
            const uint32_t kd[2] = {kn.x, kn.y};
            float acc = 0.f;
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                const uint32_t code = (kd[g >> 2] >> ((g & 3) * 8)) & 0xffu;
                const float4 *qr = q4s + j * 32 + g * 4;
                float dot = 0.f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float4 cq = ck4[cb_slot(code, w)], qq = qr[w];
                    dot = fmaf(qq.x, cq.x, dot);
                    dot = fmaf(qq.y, cq.y, dot);
                    dot = fmaf(qq.z, cq.z, dot);
                    dot = fmaf(qq.w, cq.w, dot);
                }
                acc += dot;
            }
            if (lane == 0) {
                float *ml = p.part_ml + ((size_t)(j0 + j) * stride + p.n_chunks) * 2;
                ml[0] = acc * (nscale[0] * p.sf);
                ml[1] = 1.0f;
            }
        }
        if (j < nj && kvf == 1) {
            const uint2 vn = ncode[1];
            const int g = lane >> 3, d0 = (lane & 7) * 2;
            const uint32_t code = ((g < 4 ? vn.x : vn.y) >> ((g & 3) * 8)) & 0xffu;
            const float2 cvv =
                *reinterpret_cast<const float2 *>(reinterpret_cast<const float *>(cv4) + code * 16 + d0);
            const float wv = nscale[1];
            float *po = p.part_o + ((size_t)(j0 + j) * stride + p.n_chunks) * kHd + lane * 2;
            po[0] = wv * cvv.x;
            po[1] = wv * cvv.y;
        }
        return;
    }

    // ---- a chunk of the tokens before pos
    const int T = pos;
    if (j == 0) {
        kcw[lane] = kw;
        vcw[lane] = vw;
        wsc[0][lane] = tw < T ? ksv * p.sf : 0.f;
        wsc[1][lane] = tw < T ? vsv : 0.f;
    }
    __syncthreads();

    // scores: lane (token tq = 16 j + lane / 4, quarter k4 = lane % 4) reads
    // its token's codebook quarter once per group for every head; the quarters
    // are summed across the lane quad
    const int tq = 16 * j + (lane >> 2), k4 = lane & 3;
    float pq[4] = {0.f, 0.f, 0.f, 0.f};
    {
        const uint2 kq = kcw[tq];
        const uint32_t kd[2] = {kq.x, kq.y};
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const uint32_t code = (kd[g >> 2] >> ((g & 3) * 8)) & 0xffu;
            const float4 cq = ck4[cb_slot(code, k4)];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                if (jj >= nj) break;
                const float4 qq = q4s[jj * 32 + g * 4 + k4];
                float dot = pq[jj];
                dot = fmaf(qq.x, cq.x, dot);
                dot = fmaf(qq.y, cq.y, dot);
                dot = fmaf(qq.z, cq.z, dot);
                dot = fmaf(qq.w, cq.w, dot);
                pq[jj] = dot;
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        pq[jj] += __shfl_xor(pq[jj], 1);
        pq[jj] += __shfl_xor(pq[jj], 2);
    }
    const float kfq = wsc[0][tq], vf = wsc[1][lane];
    if (k4 == 0) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            ssc[jj][tq] = c * kAttnC + tq < T ? pq[jj] * kfq : -INFINITY;
    }
    __syncthreads();   // the scores are in; wsc is rewritten with the weights below

    // softmax of head j over the chunk (lane = token)
    const float sc = j < nj ? ssc[j][lane] : -INFINITY;
    const float m = wave_max_f(sc);
    const float e = (sc == -INFINITY) ? 0.f : expf(sc - m);
    wsc[j][lane] = e * vf;
    const float l = wave_sum_f(e);
    __syncthreads();

    // V: lane owns dims 2 lane, 2 lane + 1 (group g = lane / 8) of every head;
    // wave j takes tokens 16 j .. 16 j + 15; the waves' sums meet in LDS
    {
        const int g = lane >> 3, d0 = (lane & 7) * 2;
        const float *cvf = reinterpret_cast<const float *>(cv4);
        float o[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
#pragma unroll 4
        for (int tl = 16 * j; tl < 16 * j + 16; ++tl) {
            const uint2 cw = vcw[tl];
            const uint32_t code = ((g < 4 ? cw.x : cw.y) >> ((g & 3) * 8)) & 0xffu;
            const float2 cvv = *reinterpret_cast<const float2 *>(cvf + code * 16 + d0);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const float wgt = wsc[jj][tl];
                o[jj][0] = fmaf(wgt, cvv.x, o[jj][0]);
                o[jj][1] = fmaf(wgt, cvv.y, o[jj][1]);
            }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) ored[j][jj][lane] = make_float2(o[jj][0], o[jj][1]);
    }
    __syncthreads();
    if (j < nj) {
        float2 o = ored[0][j][lane];
#pragma unroll
        for (int u = 1; u < 4; ++u) {
            const float2 t = ored[u][j][lane];
            o.x += t.x;
            o.y += t.y;
        }
        float *po = p.part_o + ((size_t)(j0 + j) * stride + c) * kHd + lane * 2;
        po[0] = o.x;
        po[1] = o.y;
        if (lane == 0) {
            float *ml = p.part_ml + ((size_t)(j0 + j) * stride + c) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
}

// Greedy pick over V logits (first maximum above -inf; none: token 0), from
// the n_part per-workgroup maxima of the LM head when n_part > 0, else from
// the logits; then the picked token's embedding row into x; thread 0 records
// the token and advances state = {position, step, token}.
__global__ __launch_bounds__(kArgNT) void argmax_embed_kernel(const float *logits, int V,
                                                             const float2 *part, int n_part,
                                                             const float *emb, int hidden,
                                                             float *x, int *state, int *tokens,
                                                             int max_steps) {
    __shared__ float wm[kArgNT / 64];
    __shared__ int wi[kArgNT / 64];
    __shared__ int pick;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    // partials of the LM head's workgroups (first maximum of each, in row
    // order): strict > keeps the first, equal maxima go to the lower row below
    for (int i = tid; i < n_part; i += kArgNT) {
        const float2 c = part[i];
        if (c.x > best || (c.x == best && __float_as_int(c.y) < bi)) {
            best = c.x;
            bi = __float_as_int(c.y);
        }
    }
    // no partials: each thread visits its logits in increasing order,
    // kArgBatch float4 loads in flight per batch; strict > keeps the first
    // maximum
    const int n4 = n_part ? 0 : V / 4;
    const float4 *l4 = reinterpret_cast<const float4 *>(logits);
    for (int b = tid; b < n4; b += kArgNT * kArgBatch) {
        float4 v[kArgBatch];
#pragma unroll
        for (int u = 0; u < kArgBatch; ++u) {
            const int i4 = min(b + u * kArgNT, n4 - 1);
            v[u] = l4[i4];
            if (b + u * kArgNT >= n4) v[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int u = 0; u < kArgBatch; ++u) {
            const int i = (b + u * kArgNT) * 4;
            if (v[u].x > best) { best = v[u].x; bi = i; }
            if (v[u].y > best) { best = v[u].y; bi = i + 1; }
            if (v[u].z > best) { best = v[u].z; bi = i + 2; }
            if (v[u].w > best) { best = v[u].w; bi = i + 3; }
        }
    }
    for (int i = n4 * 4 + tid; i < (n_part ? 0 : V); i += kArgNT) {
        const float v = logits[i];
        if (v > best) {
            best = v;
            bi = i;
        }
    }
    const float m = wave_max_f(best);
    const int mi = wave_min_i(best == m ? bi : 0x7fffffff);
    if (lane == 0) {
        wm[w] = m;
        wi[w] = mi;
    }
    __syncthreads();
    if (tid == 0) {
        float bm = wm[0];
        int b = wi[0];
        for (int q = 1; q < kArgNT / 64; ++q)
            if (wm[q] > bm || (wm[q] == bm && wi[q] < b)) {
                bm = wm[q];
                b = wi[q];
            }
        pick = b < V ? b : 0;                     // no logit above -inf (all NaN): token 0
    }
    __syncthreads();
    const int tok = pick;
    for (int d = tid; d < hidden; d += kArgNT) x[d] = emb[(size_t)tok * hidden + d];
    if (tid == 0) {
        const int step = state[1];
        if (step >= 0 && step < max_steps) tokens[step] = tok;
        state[0] += 1;
        state[1] = step + 1;
        state[2] = tok;
    }
}

// x = embedding row of state[2].
__global__ __launch_bounds__(kArgNT) void embed_kernel(const float *emb, int hidden, int V,
                                                      const int *state, float *x) {
    const int tok = min(max(state[2], 0), V - 1);
    for (int d = threadIdx.x; d < hidden; d += kArgNT) x[d] = emb[(size_t)tok * hidden + d];
}

struct DecoderLayer {
    void *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;   // Linear handles (not owned)
    DevBuf in_norm, post_norm, q_norm, k_norm, kcb, vcb, kc, ks, vc, vs;
};

struct Decoder {
    int hidden = 0, layers = 0, Hq = 0, Hkv = 0, inter = 0, vocab = 0, max_ctx = 0, P = 0,
        pages = 0, max_steps = 0;
    float eps = 0.f, theta = 0.f;
    std::vector<DecoderLayer> L;
    void *lm = nullptr;
    DevBuf final_norm, emb, cos_t, sin_t, bt, x, qkv, attn, gu, logits, arg_part, part_o, part_ml,
        state, tokens;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool ready_layers = false, ready_head = false;

    // The captured step holds the device pointers of every linear handle and
    // buffer it launched on; replacing a handle makes it stale, so the next
    // generate with use_graph captures again.
    void drop_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }

    ~Decoder() {
        drop_graph();
        if (stream) (void)hipStreamDestroy(stream);
        for (DecoderLayer &l : L)
            for (DevBuf *b : {&l.in_norm, &l.post_norm, &l.q_norm, &l.k_norm, &l.kcb, &l.vcb, &l.kc,
                              &l.ks, &l.vc, &l.vs})
                b->release();
        for (DevBuf *b : {&final_norm, &emb, &cos_t, &sin_t, &bt, &x, &qkv, &attn, &gu, &logits,
                          &arg_part, &part_o, &part_ml, &state, &tokens})
            b->release();
    }

    int n_chunks() const { return (max_ctx + kAttnC - 1) / kAttnC; }

    // One token step on `st` (device-resident position and token).
    int step(hipStream_t st) {
        int rc;
        const int *pos = state.as<int>();
        const float sf = 1.0f / sqrtf((float)kHd);
        for (int l = 0; l < layers; ++l) {
            DecoderLayer &ly = L[l];
            rc = linear_forward_fused(ly.qkv, x.as<float>(), qkv.as<float>(), 1,
                                      ly.in_norm.as<float>(), eps, nullptr, st);
            if (rc) return rc;
            AttnParams ap{qkv.as<float>(), ly.q_norm.as<float>(), ly.k_norm.as<float>(),
                          cos_t.as<float>(), sin_t.as<float>(), pos, bt.as<int>(),
                          ly.kcb.as<float>(), ly.vcb.as<float>(), ly.kc.as<uint8_t>(),
                          ly.vc.as<uint8_t>(), ly.ks.as<float>(), ly.vs.as<float>(),
                          part_o.as<float>(), part_ml.as<float>(), Hq, Hkv, P, max_ctx,
                          n_chunks(), eps, sf};
            OJX_LAUNCH(attn_decode_kernel, dim3(n_chunks() + 2, Hkv, (Hq / Hkv + 3) / 4),
                       dim3(kAttnNT), 0, st, ap);
            rc = kv_merge_device_len(part_o.as<float>(), part_ml.as<float>(), n_chunks() + 1,
                                     kAttnC, Hq, pos, 0, 1, attn.as<float>(), st);
            if (rc) return rc;
            rc = linear_forward_fused(ly.o, attn.as<float>(), x.as<float>(), 0, nullptr, 0.f,
                                      x.as<float>(), st);
            if (rc) return rc;
            // gate/up with the SwiGLU epilogue: gu holds silu(gate) * up (I floats)
            rc = linear_forward_fused(ly.gu, x.as<float>(), gu.as<float>(), 3,
                                      ly.post_norm.as<float>(), eps, nullptr, st);
            if (rc) return rc;
            rc = linear_forward_fused(ly.down, gu.as<float>(), x.as<float>(), 0, nullptr, 0.f,
                                      x.as<float>(), st);
            if (rc) return rc;
        }
        int n_part = 0;
        rc = linear_forward_lm_head(lm, x.as<float>(), logits.as<float>(), final_norm.as<float>(),
                                    eps, arg_part.as<float2>(), &n_part, st);
        if (rc) return rc;
        OJX_LAUNCH(argmax_embed_kernel, dim3(1), dim3(kArgNT), 0, st, logits.as<float>(), vocab,
                   arg_part.as<float2>(), n_part, emb.as<float>(), hidden, x.as<float>(),
                   state.as<int>(), tokens.as<int>(), max_steps);
        OJX_HIP(hipGetLastError());
        return OJASX_OK;
    }
};

namespace {

int check_linear(void *h, int K, int M, const char *what) {
    if (!h) {
        set_error("decoder: %s linear handle is NULL", what);
        return OJASX_ERR_NULL;
    }
    int k, m, d;
    linear_shape(h, &k, &m, &d);
    if (k != K || m != M || d != kBd) {
        set_error("decoder: %s linear is %d -> %d (block %d); expected %d -> %d (block 16)", what, k,
                  m, d, K, M);
        return OJASX_ERR_INVALID;
    }
    return OJASX_OK;
}

int copy_d2d(DevBuf &dst, const void *src, size_t n) {
    int rc = dst.ensure(n);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(dst.ptr, src, n, hipMemcpyDeviceToDevice));
    return OJASX_OK;
}

}  // namespace
}  // namespace ojx

using ojx::Decoder;

extern "C" {

OJASX_API OjasxDecoderHandle ojasx_create_decoder(int hidden, int layers, int q_heads,
                                                  int kv_heads, int head_dim, int intermediate,
                                                  int vocab, int max_context, int page_size,
                                                  int max_steps, float rms_eps, float rope_theta) {
    using namespace ojx;
    if (hidden <= 0 || hidden % kBd || layers <= 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads || head_dim != kHd || intermediate <= 0 || intermediate % kBd ||
        vocab <= 0 || max_context <= 0 || page_size <= 0 || max_steps <= 0 || kv_heads > 65535 ||
        q_heads + kv_heads > 65535 || !(rms_eps > 0.f) || !(rope_theta > 0.f)) {
        set_error("invalid decoder shape (head_dim must be %d)", kHd);
        return nullptr;
    }
    Decoder *d = new (std::nothrow) Decoder;
    if (!d) return nullptr;
    d->hidden = hidden;
    d->layers = layers;
    d->Hq = q_heads;
    d->Hkv = kv_heads;
    d->inter = intermediate;
    d->vocab = vocab;
    d->max_ctx = max_context;
    d->P = page_size;
    d->pages = (max_context + page_size - 1) / page_size;
    d->max_steps = max_steps;
    d->eps = rms_eps;
    d->theta = rope_theta;
    d->L.resize(layers);
    int rc = OJASX_OK;
    const size_t kv_rows = (size_t)d->pages * kv_heads * page_size;
    for (auto &ly : d->L) {
        if (!rc) rc = ly.kc.ensure(kv_rows * kG);
        if (!rc) rc = ly.vc.ensure(kv_rows * kG);
        if (!rc) rc = ly.ks.ensure(kv_rows * 4);
        if (!rc) rc = ly.vs.ensure(kv_rows * 4);
    }
    // RoPE tables: angle = fp32(pos) * fp32 inv_freq, cos / sin rounded to fp32.
    const int half = kHd / 2;
    std::vector<float> inv(half), ct((size_t)max_context * half), stb((size_t)max_context * half);
    for (int i = 0; i < half; ++i)
        inv[i] = (float)(1.0 / std::pow((double)rope_theta, (double)(2 * i) / kHd));
    for (int pos = 0; pos < max_context; ++pos)
        for (int i = 0; i < half; ++i) {
            const float ang = (float)pos * inv[i];
            ct[(size_t)pos * half + i] = (float)std::cos((double)ang);
            stb[(size_t)pos * half + i] = (float)std::sin((double)ang);
        }
    if (!rc) rc = upload(d->cos_t, ct.data(), ct.size() * 4);
    if (!rc) rc = upload(d->sin_t, stb.data(), stb.size() * 4);
    std::vector<int> bt(d->pages);
    for (int i = 0; i < d->pages; ++i) bt[i] = i;
    if (!rc) rc = upload(d->bt, bt.data(), bt.size() * 4);
    const size_t qkv_n = (size_t)(q_heads + 2 * kv_heads) * kHd;
    if (!rc) rc = d->x.ensure((size_t)hidden * 4);
    if (!rc) rc = d->qkv.ensure(qkv_n * 4);
    if (!rc) rc = d->attn.ensure((size_t)q_heads * kHd * 4);
    if (!rc) rc = d->gu.ensure((size_t)2 * intermediate * 4);
    if (!rc) rc = d->logits.ensure((size_t)vocab * 4);
    if (!rc)   // the LM head's per-workgroup argmax partials
        rc = d->arg_part.ensure((size_t)(vocab + tall_rows_per_part() - 1) / tall_rows_per_part() *
                                sizeof(float2));
    if (!rc) rc = d->part_o.ensure((size_t)q_heads * (d->n_chunks() + 1) * kHd * 4);
    if (!rc) rc = d->part_ml.ensure((size_t)q_heads * (d->n_chunks() + 1) * 2 * 4);
    const int st0[4] = {0, 0, 0, 0};
    if (!rc) rc = upload(d->state, st0, sizeof(st0));
    if (!rc) rc = d->tokens.ensure((size_t)max_steps * 4);
    if (!rc && hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("decoder: hipStreamCreateWithFlags failed");
        rc = OJASX_ERR_HIP;
    }
    if (rc) {
        delete d;
        return nullptr;
    }
    return d;
}

OJASX_API void ojasx_destroy_decoder(OjasxDecoderHandle handle) {
    if (!handle) return;
    Decoder *d = static_cast<Decoder *>(handle);
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    delete d;
}

OJASX_API int ojasx_decoder_set_layer(OjasxDecoderHandle handle, int layer,
                                      OjasxLinearHandle qkv, OjasxLinearHandle o,
                                      OjasxLinearHandle gate_up, OjasxLinearHandle down,
                                      const float *input_norm, const float *post_norm,
                                      const float *q_norm, const float *k_norm,
                                      const float *k_codebook, const float *v_codebook) {
    using namespace ojx;
    if (!handle || !input_norm || !post_norm || !q_norm || !k_norm || !k_codebook || !v_codebook)
        return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    if (layer < 0 || layer >= d->layers) return OJASX_ERR_HEAD;
    OJX_HIP(hipStreamSynchronize(d->stream));
    d->drop_graph();
    const int qd = d->Hq * kHd, kvd = d->Hkv * kHd;
    int rc = check_linear(qkv, d->hidden, qd + 2 * kvd, "qkv");
    if (!rc) rc = check_linear(o, qd, d->hidden, "o");
    if (!rc) rc = check_linear(gate_up, d->hidden, 2 * d->inter, "gate_up");
    if (!rc) rc = check_linear(down, d->inter, d->hidden, "down");
    if (rc) return rc;
    DecoderLayer &ly = d->L[layer];
    ly.qkv = qkv;
    ly.o = o;
    ly.gu = gate_up;
    ly.down = down;
    rc = copy_d2d(ly.in_norm, input_norm, (size_t)d->hidden * 4);
    if (!rc) rc = copy_d2d(ly.post_norm, post_norm, (size_t)d->hidden * 4);
    if (!rc) rc = copy_d2d(ly.q_norm, q_norm, kHd * 4);
    if (!rc) rc = copy_d2d(ly.k_norm, k_norm, kHd * 4);
    if (!rc) rc = copy_d2d(ly.kcb, k_codebook, (size_t)d->Hkv * 256 * kBd * 4);
    if (!rc) rc = copy_d2d(ly.vcb, v_codebook, (size_t)d->Hkv * 256 * kBd * 4);
    if (rc) return rc;
    bool all = true;
    for (auto &l : d->L) all = all && l.qkv;
    d->ready_layers = all;
    return OJASX_OK;
}

OJASX_API int ojasx_decoder_set_head(OjasxDecoderHandle handle, OjasxLinearHandle lm_head,
                                     const float *final_norm, const float *embedding) {
    using namespace ojx;
    if (!handle || !final_norm || !embedding) return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    int rc = check_linear(lm_head, d->hidden, d->vocab, "lm_head");
    if (rc) return rc;
    OJX_HIP(hipStreamSynchronize(d->stream));
    d->drop_graph();
    d->lm = lm_head;
    rc = copy_d2d(d->final_norm, final_norm, (size_t)d->hidden * 4);
    if (!rc) rc = copy_d2d(d->emb, embedding, (size_t)d->vocab * d->hidden * 4);
    if (rc) return rc;
    d->ready_head = true;
    return OJASX_OK;
}

OJASX_API int ojasx_decoder_set_context(OjasxDecoderHandle handle, int layer,
                                        const uint8_t *k_codes, const float *k_scales,
                                        const uint8_t *v_codes, const float *v_scales,
                                        int num_tokens) {
    using namespace ojx;
    if (!handle || !k_codes || !k_scales || !v_codes || !v_scales) return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    if (layer < 0 || layer >= d->layers) return OJASX_ERR_HEAD;
    if (num_tokens < 0 || num_tokens > d->max_ctx) {
        set_error("decoder: context of %d tokens exceeds max_context %d", num_tokens, d->max_ctx);
        return OJASX_ERR_INVALID;
    }
    DecoderLayer &ly = d->L[layer];
    const size_t rows = (size_t)((num_tokens + d->P - 1) / d->P) * d->Hkv * d->P;
    OJX_HIP(hipMemcpy(ly.kc.ptr, k_codes, rows * kG, hipMemcpyDeviceToDevice));
    OJX_HIP(hipMemcpy(ly.vc.ptr, v_codes, rows * kG, hipMemcpyDeviceToDevice));
    OJX_HIP(hipMemcpy(ly.ks.ptr, k_scales, rows * 4, hipMemcpyDeviceToDevice));
    OJX_HIP(hipMemcpy(ly.vs.ptr, v_scales, rows * 4, hipMemcpyDeviceToDevice));
    return OJASX_OK;
}

OJASX_API int ojasx_decoder_reset(OjasxDecoderHandle handle, int position) {
    using namespace ojx;
    if (!handle) return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    if (position < 0 || position >= d->max_ctx) {
        set_error("decoder: position %d outside [0, %d)", position, d->max_ctx);
        return OJASX_ERR_INVALID;
    }
    const int st[3] = {position, 0, 0};
    OJX_HIP(hipStreamSynchronize(d->stream));
    OJX_HIP(hipMemcpy(d->state.ptr, st, sizeof(st), hipMemcpyHostToDevice));
    return OJASX_OK;
}

OJASX_API int ojasx_decoder_generate(OjasxDecoderHandle handle, int first_token, int num_tokens,
                                     int use_graph, int *tokens_out, float *last_logits) {
    using namespace ojx;
    if (!handle || !tokens_out) return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    if (!d->ready_layers || !d->ready_head) {
        set_error("decoder: set every layer and the head first");
        return OJASX_ERR_INVALID;
    }
    if (num_tokens <= 0) return OJASX_OK;
    if (num_tokens > d->max_steps || first_token < 0 || first_token >= d->vocab) {
        set_error("decoder: %d tokens (max_steps %d), first token %d", num_tokens, d->max_steps,
                  first_token);
        return OJASX_ERR_INVALID;
    }
    hipStream_t st = d->stream;
    int state[3];
    OJX_HIP(hipStreamSynchronize(st));
    OJX_HIP(hipMemcpy(state, d->state.ptr, sizeof(state), hipMemcpyDeviceToHost));
    if (state[0] + num_tokens > d->max_ctx) {
        set_error("decoder: position %d + %d tokens exceeds max_context %d", state[0], num_tokens,
                  d->max_ctx);
        return OJASX_ERR_INVALID;
    }
    state[1] = 0;
    state[2] = first_token;
    OJX_HIP(hipMemcpy(d->state.ptr, state, sizeof(state), hipMemcpyHostToDevice));
    OJX_LAUNCH(embed_kernel, dim3(1), dim3(kArgNT), 0, st, d->emb.as<float>(), d->hidden, d->vocab,
               d->state.as<int>(), d->x.as<float>());
    int rc = OJASX_OK;
    int done = 0;
    if (use_graph && !d->exec) {
        // One eager step first: it sets every kernel attribute, so capture
        // records launches only.
        rc = d->step(st);
        if (rc) return rc;
        done = 1;
        if (timing_on()) {
            set_error("decoder: graph capture with kernel timing enabled");
            return OJASX_ERR_INVALID;
        }
        OJX_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        rc = d->step(st);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        OJX_HIP(e);
        d->graph = g;
        OJX_HIP(hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0));
    }
    for (int i = done; i < num_tokens; ++i) {
        if (use_graph) {
            OJX_HIP(hipGraphLaunch(d->exec, st));
        } else {
            rc = d->step(st);
            if (rc) return rc;
        }
    }
    OJX_HIP(hipMemcpyAsync(tokens_out, d->tokens.ptr, (size_t)num_tokens * 4,
                           hipMemcpyDeviceToHost, st));
    if (last_logits)
        OJX_HIP(hipMemcpyAsync(last_logits, d->logits.ptr, (size_t)d->vocab * 4,
                               hipMemcpyDeviceToHost, st));
    OJX_HIP(hipStreamSynchronize(st));
    return OJASX_OK;
}

OJASX_API int ojasx_decoder_read_kv(OjasxDecoderHandle handle, int layer, int first_token,
                                    int num_tokens, uint8_t *k_codes, float *k_scales,
                                    uint8_t *v_codes, float *v_scales) {
    using namespace ojx;
    if (!handle || !k_codes || !k_scales || !v_codes || !v_scales) return OJASX_ERR_NULL;
    Decoder *d = static_cast<Decoder *>(handle);
    if (layer < 0 || layer >= d->layers) return OJASX_ERR_HEAD;
    if (first_token < 0 || num_tokens < 0 || first_token + num_tokens > d->max_ctx ||
        first_token % d->P) {
        set_error("decoder: KV range [%d, +%d) (must start on a page)", first_token, num_tokens);
        return OJASX_ERR_INVALID;
    }
    OJX_HIP(hipStreamSynchronize(d->stream));
    DecoderLayer &ly = d->L[layer];
    const size_t r0 = (size_t)(first_token / d->P) * d->Hkv * d->P;
    const size_t rows = (size_t)((num_tokens + d->P - 1) / d->P) * d->Hkv * d->P;
    OJX_HIP(hipMemcpy(k_codes, ly.kc.as<uint8_t>() + r0 * kG, rows * kG, hipMemcpyDeviceToHost));
    OJX_HIP(hipMemcpy(v_codes, ly.vc.as<uint8_t>() + r0 * kG, rows * kG, hipMemcpyDeviceToHost));
    OJX_HIP(hipMemcpy(k_scales, ly.ks.as<float>() + r0, rows * 4, hipMemcpyDeviceToHost));
    OJX_HIP(hipMemcpy(v_scales, ly.vs.as<float>() + r0, rows * 4, hipMemcpyDeviceToHost));
    return OJASX_OK;
}

}  // extern "C"

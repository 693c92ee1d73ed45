// lut_kv.hip -- code-domain paged KV decode attention on gfx950.
//
// For query head j (kv head h = j / (Hq/Hkv)) over tokens t < T:
//   LUT_q[g][c] = <q_j[gD:(g+1)D], Ck_h[c]>
//   l_t = sf * s_t * sum_g LUT_q[g, kcode_t[g]]
//   p = softmax(l)
//   o[gD+d] = sum_t p_t * vs_t * Cv_h[vcode_t[g]][d]
// This is the computation of split_manifold_lut_experiment/native/src/
// ojasx_lut_kv_cache.cpp:67-132 with ojasx_lut_c_api.cpp:160-196 (two-pass
// softmax), generalised from the reference's implicit codebook
// C[c] = (c - 128) e_0 to a per-kv-head 256 x D codebook; the reference
// C-ABI (ojasx_kv_cache_*) runs on the same kernels with that special
// codebook, which reproduces its arithmetic exactly (the other coordinates
// contribute exact zeros).
//
// Kernels:
//  * kv_append: the reference quantiser (ojasx_lut_kv_cache.cpp:16-65) for one
//    token of one head: s = max(1e-8, max|k|) / 127, code[g] =
//    clamp(round(k[gD] / s), -128, 127) + 128 (round half away from zero).
//  * kv_decode_chunk: workgroup = (chunk of Tc tokens, kv head, group of
//    query heads).  Builds LUT_q for its query heads in LDS, computes the
//    chunk's logits from the K codes (page table indirection), the chunk max
//    and exp, then accumulates V in the code domain: a histogram
//    W[j][g][c] += p_t * vs_t over the chunk (LDS atomics) followed by one
//    [heads*groups x 256] x [256 x D] contraction with the V codebook.
//    Writes (max, sum, o) per chunk.
//  * kv_merge: log-sum-exp merge of the chunks in chunk order (the online
//    softmax combine of ojasx_24x96/long_context.py:133-166).
// Cache layout (device): codes [pages][Hkv][page][G] uint8, scales
// [pages][Hkv][page] fp32, so a page of one kv head is contiguous.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.h"

namespace ojx {

namespace {
constexpr int kNT = 256;
constexpr int kMaxRG = 32;   // query heads per workgroup x groups per head
constexpr int kMaxD = 32;
}  // namespace

__global__ __launch_bounds__(128) void kv_append_kernel(const float *__restrict__ k,
                                                       const float *__restrict__ v, int hd, int D,
                                                       uint8_t *kc, uint8_t *vc, float *ks,
                                                       float *vs) {
    __shared__ float red[2][128];
    const int tid = threadIdx.x;
    float mk = 0.f, mv = 0.f;
    for (int d = tid; d < hd; d += 128) {
        mk = fmaxf(mk, fabsf(k[d]));
        mv = fmaxf(mv, fabsf(v[d]));
    }
    red[0][tid] = mk;
    red[1][tid] = mv;
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
        if (tid < st) {
            red[0][tid] = fmaxf(red[0][tid], red[0][tid + st]);
            red[1][tid] = fmaxf(red[1][tid], red[1][tid + st]);
        }
        __syncthreads();
    }
    const float sk = fmaxf(1e-8f, red[0][0]) / 127.0f;
    const float sv = fmaxf(1e-8f, red[1][0]) / 127.0f;
    const int G = hd / D;
    for (int g = tid; g < G; g += 128) {
        int qk = (int)roundf(k[g * D] / sk);
        int qv = (int)roundf(v[g * D] / sv);
        kc[g] = (uint8_t)(min(127, max(-128, qk)) + 128);
        vc[g] = (uint8_t)(min(127, max(-128, qv)) + 128);
    }
    if (tid == 0) {
        *ks = sk;
        *vs = sv;
    }
}

struct KVParams {
    const float *q;
    const uint8_t *kc, *vc;
    const float *ks, *vs, *kcb, *vcb;
    const int *bt;
    float *part_o;   // [Hq][n_chunks][hd]
    float *part_ml;  // [Hq][n_chunks][2]
    int T, P, Hq, Hkv, hd, D, G, Tc, RS, n_chunks;
    float sf;
};

__global__ __launch_bounds__(kNT) void kv_decode_chunk_kernel(KVParams p) {
    extern __shared__ float sm[];
    const int R = p.Hq / p.Hkv;
    const int h = blockIdx.y;
    const int j0 = h * R + blockIdx.z * p.RS;
    const int nj = min(p.RS, R - blockIdx.z * p.RS);
    const int G = p.G, D = p.D, Tc = p.Tc;
    float *lutq = sm;                               // [RS][G][256]
    float *hist = lutq + p.RS * G * 256;            // [RS][G][256]
    float *cv = hist + p.RS * G * 256;              // [256][D]
    float *pb = cv + 256 * D;                       // [RS][Tc]
    float *red = pb + p.RS * Tc;                    // [kNT]
    __shared__ float s_m[8], s_l[8];
    const int tid = threadIdx.x;
    const int c = blockIdx.x;
    const int t_begin = c * Tc;

    // V codebook of this head, LUT_q of the query heads, zero histogram
    const float *vcb = p.vcb + (size_t)h * 256 * D;
    for (int i = tid; i < 256 * D; i += kNT) cv[i] = vcb[i];
    const float *kcb = p.kcb + (size_t)h * 256 * D;
    for (int i = tid; i < nj * G * 256; i += kNT) {
        const int cc = i & 255;
        const int jg = i >> 8;
        const int j = jg / G, g = jg - j * G;
        const float *qv = p.q + (size_t)(j0 + j) * p.hd + g * D;
        const float *cvec = kcb + (size_t)cc * D;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot = fmaf(qv[d], cvec[d], dot);
        lutq[i] = dot;
        hist[i] = 0.f;
    }
    __syncthreads();

    // logits of the chunk
    for (int tl = tid; tl < Tc; tl += kNT) {
        const int t = t_begin + tl;
        if (t < p.T) {
            const int page = p.bt[t / p.P];
            const size_t slot = ((size_t)page * p.Hkv + h) * p.P + (t % p.P);
            const uint8_t *code = p.kc + slot * G;
            const float s = p.ks[slot] * p.sf;
            for (int j = 0; j < nj; ++j) {
                const float *L = lutq + j * G * 256;
                float a = 0.f;
                for (int g = 0; g < G; ++g) a += L[g * 256 + code[g]];
                pb[j * Tc + tl] = a * s;
            }
        } else {
            for (int j = 0; j < nj; ++j) pb[j * Tc + tl] = -INFINITY;
        }
    }
    __syncthreads();
    // chunk max and sum of exp per query head
    for (int j = 0; j < nj; ++j) {
        float m = -INFINITY;
        for (int tl = tid; tl < Tc; tl += kNT) m = fmaxf(m, pb[j * Tc + tl]);
        red[tid] = m;
        __syncthreads();
        for (int st = kNT / 2; st > 0; st >>= 1) {
            if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
            __syncthreads();
        }
        m = red[0];
        __syncthreads();
        float l = 0.f;
        for (int tl = tid; tl < Tc; tl += kNT) {
            const float v = pb[j * Tc + tl];
            const float e = v == -INFINITY ? 0.f : expf(v - m);
            pb[j * Tc + tl] = e;
            l += e;
        }
        red[tid] = l;
        __syncthreads();
        for (int st = kNT / 2; st > 0; st >>= 1) {
            if (tid < st) red[tid] += red[tid + st];
            __syncthreads();
        }
        if (tid == 0) {
            s_m[j] = m;
            s_l[j] = red[0];
        }
        __syncthreads();
    }
    // V histogram in the code domain
    for (int tl = tid; tl < Tc; tl += kNT) {
        const int t = t_begin + tl;
        if (t >= p.T) continue;
        const int page = p.bt[t / p.P];
        const size_t slot = ((size_t)page * p.Hkv + h) * p.P + (t % p.P);
        const uint8_t *code = p.vc + slot * G;
        const float vs = p.vs[slot];
        for (int j = 0; j < nj; ++j) {
            const float w = pb[j * Tc + tl] * vs;
            if (w == 0.f) continue;
            float *H = hist + j * G * 256;
            for (int g = 0; g < G; ++g) atomicAdd(&H[g * 256 + code[g]], w);
        }
    }
    __syncthreads();
    // o[j][g*D + d] = sum_c hist[j][g][c] * Cv[c][d]
    for (int i = tid; i < nj * p.hd; i += kNT) {
        const int j = i / p.hd;
        const int od = i - j * p.hd;
        const int g = od / D, d = od - g * D;
        const float *H = hist + (j * G + g) * 256;
        float a = 0.f;
        for (int cc = 0; cc < 256; ++cc) a = fmaf(H[cc], cv[cc * D + d], a);
        p.part_o[((size_t)(j0 + j) * p.n_chunks + c) * p.hd + od] = a;
    }
    if (tid < nj) {
        float *ml = p.part_ml + ((size_t)(j0 + tid) * p.n_chunks + c) * 2;
        ml[0] = s_m[tid];
        ml[1] = s_l[tid];
    }
}

__global__ void kv_merge_kernel(const float *part_o, const float *part_ml, int n_chunks, int hd,
                                float *out) {
    const int j = blockIdx.x;
    const float *ml = part_ml + (size_t)j * n_chunks * 2;
    float m = -INFINITY;
    for (int c = 0; c < n_chunks; ++c) m = fmaxf(m, ml[2 * c]);
    float l = 0.f;
    for (int c = 0; c < n_chunks; ++c)
        if (ml[2 * c] != -INFINITY) l += ml[2 * c + 1] * expf(ml[2 * c] - m);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.f;
        for (int c = 0; c < n_chunks; ++c)
            if (ml[2 * c] != -INFINITY)
                o += part_o[((size_t)j * n_chunks + c) * hd + d] * expf(ml[2 * c] - m);
        out[(size_t)j * hd + d] = o / l;
    }
}

// Workspace for the decode partials, one per thread of the host (device
// entry points called from several host threads each get their own).
struct KVWork {
    DevBuf o, ml;
    ~KVWork() {
        o.release();
        ml.release();
    }
};
static thread_local KVWork t_work;

int kv_decode(const float *q, const uint8_t *kc, const float *ks, const uint8_t *vc,
              const float *vs, const float *kcb, const float *vcb, const int *bt, int T, int P,
              int Hq, int Hkv, int hd, int D, float sf, float *out, hipStream_t st,
              KVWork &wk) {
    if (T <= 0) return OJASX_OK;
    if (Hkv <= 0 || Hq <= 0 || Hq % Hkv || D <= 0 || D > kMaxD || hd <= 0 || hd % D || P <= 0 ||
        hd > 1024) {
        set_error("invalid KV decode shape Hq=%d Hkv=%d hd=%d D=%d page=%d", Hq, Hkv, hd, D, P);
        return OJASX_ERR_INVALID;
    }
    if (sf <= 0.f) sf = 1.0f / sqrtf((float)hd);
    const int G = hd / D;
    const int R = Hq / Hkv;
    if (G > kMaxRG) {
        set_error("head_dim / block_dim must be <= %d", kMaxRG);
        return OJASX_ERR_INVALID;
    }
    // Query heads per workgroup: LUT_q and histogram take RS*G KB each.
    int RS = std::max(1, std::min({R, kMaxRG / G, 8}));
    const int nz = (R + RS - 1) / RS;
    // Chunk length: enough workgroups to fill the chip, a multiple of 256,
    // and the LDS footprint within 150 KB.
    long want = (long)T * Hkv * nz / 512;
    int Tc = (int)std::max<long>(256, ((want + 255) / 256) * 256);
    Tc = std::min(Tc, 2048);
    const long lds_fixed = (long)RS * G * 256 * 2 + 256L * D + kNT;
    while (Tc > 256 && (lds_fixed + (long)RS * Tc) * 4 > 150 * 1024) Tc -= 256;
    const int n_chunks = (T + Tc - 1) / Tc;
    int rc = wk.o.ensure((size_t)Hq * n_chunks * hd * 4);
    if (!rc) rc = wk.ml.ensure((size_t)Hq * n_chunks * 2 * 4);
    if (rc) return rc;
    KVParams p{q, kc, vc, ks, vs, kcb, vcb, bt, wk.o.as<float>(), wk.ml.as<float>(), T, P, Hq,
               Hkv, hd, D, G, Tc, RS, n_chunks, sf};
    const size_t lds = ((size_t)RS * G * 256 * 2 + 256 * D + (size_t)RS * Tc + kNT) * 4;
    static size_t granted = 0;
    rc = ensure_dyn_lds(reinterpret_cast<const void *>(&kv_decode_chunk_kernel), lds, &granted);
    if (rc) return rc;
    hipLaunchKernelGGL(kv_decode_chunk_kernel, dim3(n_chunks, Hkv, nz), dim3(kNT), lds, st, p);
    hipLaunchKernelGGL(kv_merge_kernel, dim3(Hq), dim3(128), 0, st, wk.o.as<float>(),
                       wk.ml.as<float>(), n_chunks, hd, out);
    OJX_HIP(hipGetLastError());
    return OJASX_OK;
}

// ---- reference-API KV cache: one code stream per head ---------------------
struct KVHead {
    DevBuf kc, vc, ks, vs;
    int len = 0, cap = 0;
};

struct KVCache {
    int heads = 0, hd = 0, D = 0, G = 0, max_seq = 0;
    std::vector<KVHead> h;
    DevBuf cb, bt, kstage, vstage, qstage, ostage;
    int bt_pages = 0;
    KVWork work;
    ~KVCache() {
        for (auto &x : h)
            for (DevBuf *b : {&x.kc, &x.vc, &x.ks, &x.vs}) b->release();
        for (DevBuf *b : {&cb, &bt, &kstage, &vstage, &qstage, &ostage}) b->release();
    }
};

static int grow(DevBuf &b, size_t old_bytes, size_t new_bytes) {
    DevBuf nb;
    int rc = nb.ensure(new_bytes);
    if (rc) return rc;
    OJX_HIP(hipMemset(nb.ptr, 0, new_bytes));
    if (old_bytes) OJX_HIP(hipMemcpy(nb.ptr, b.ptr, old_bytes, hipMemcpyDeviceToDevice));
    b.release();
    b = nb;
    nb.ptr = nullptr;
    return OJASX_OK;
}

static int ensure_pages(KVCache *c, int pages) {
    if (pages <= c->bt_pages) return OJASX_OK;
    std::vector<int> id(pages);
    for (int i = 0; i < pages; ++i) id[i] = i;
    int rc = upload(c->bt, id.data(), id.size() * 4);
    if (rc) return rc;
    c->bt_pages = pages;
    return OJASX_OK;
}

}  // namespace ojx

using ojx::KVCache;

extern "C" {

OJASX_API OjasxKVHandle ojasx_create_kv_cache(int num_heads, int head_dim, int max_seq_len,
                                              int block_dim) {
    using namespace ojx;
    if (num_heads <= 0 || head_dim <= 0 || block_dim <= 0 || block_dim > kMaxD ||
        head_dim % block_dim || head_dim / block_dim > kMaxRG || max_seq_len < 0 ||
        head_dim > 1024) {
        set_error("invalid KV cache shape");
        return nullptr;
    }
    KVCache *c = new (std::nothrow) KVCache;
    if (!c) return nullptr;
    c->heads = num_heads;
    c->hd = head_dim;
    c->D = block_dim;
    c->G = head_dim / block_dim;
    c->max_seq = max_seq_len;
    c->h.resize(num_heads);
    // The reference's implicit codebook: C[c] = (c - 128) e_0.
    std::vector<float> cb((size_t)256 * block_dim, 0.f);
    for (int i = 0; i < 256; ++i) cb[(size_t)i * block_dim] = (float)(i - 128);
    int rc = upload(c->cb, cb.data(), cb.size() * 4);
    for (auto &hh : c->h) {
        if (rc) break;
        const int cap = (int)round_up(std::max(max_seq_len, 1), 16);
        rc = grow(hh.kc, 0, (size_t)cap * c->G);
        if (!rc) rc = grow(hh.vc, 0, (size_t)cap * c->G);
        if (!rc) rc = grow(hh.ks, 0, (size_t)cap * 4);
        if (!rc) rc = grow(hh.vs, 0, (size_t)cap * 4);
        hh.cap = cap;
    }
    if (!rc) rc = c->kstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->vstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->qstage.ensure((size_t)head_dim * 4);
    if (!rc) rc = c->ostage.ensure((size_t)head_dim * 4);
    if (rc) {
        delete c;
        return nullptr;
    }
    return c;
}

OJASX_API int ojasx_kv_cache_append(OjasxKVHandle handle, int head_idx, const float *k,
                                    const float *v) {
    using namespace ojx;
    if (!handle || !k || !v) return OJASX_ERR_NULL;
    KVCache *c = static_cast<KVCache *>(handle);
    if (head_idx < 0 || head_idx >= c->heads) return OJASX_ERR_HEAD;
    KVHead &hh = c->h[head_idx];
    if (hh.len >= hh.cap) {  // ojasx_lut_kv_cache.cpp:17-25: grow to max(1024, 2 * cap)
        const int nc = (int)round_up(std::max(1024, hh.cap * 2), 16);
        int rc = grow(hh.kc, (size_t)hh.cap * c->G, (size_t)nc * c->G);
        if (!rc) rc = grow(hh.vc, (size_t)hh.cap * c->G, (size_t)nc * c->G);
        if (!rc) rc = grow(hh.ks, (size_t)hh.cap * 4, (size_t)nc * 4);
        if (!rc) rc = grow(hh.vs, (size_t)hh.cap * 4, (size_t)nc * 4);
        if (rc) return rc;
        hh.cap = nc;
    }
    OJX_HIP(hipMemcpy(c->kstage.ptr, k, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    OJX_HIP(hipMemcpy(c->vstage.ptr, v, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(kv_append_kernel, dim3(1), dim3(128), 0, nullptr, c->kstage.as<float>(),
                       c->vstage.as<float>(), c->hd, c->D, hh.kc.as<uint8_t>() + (size_t)hh.len * c->G,
                       hh.vc.as<uint8_t>() + (size_t)hh.len * c->G, hh.ks.as<float>() + hh.len,
                       hh.vs.as<float>() + hh.len);
    OJX_HIP(hipGetLastError());
    OJX_HIP(hipDeviceSynchronize());
    hh.len++;
    return OJASX_OK;
}

OJASX_API int ojasx_kv_cache_attention(OjasxKVHandle handle, int head_idx, const float *q,
                                       float *out_context, float scale_factor) {
    using namespace ojx;
    if (!handle || !q || !out_context) return OJASX_ERR_NULL;
    KVCache *c = static_cast<KVCache *>(handle);
    if (head_idx < 0 || head_idx >= c->heads) return OJASX_ERR_HEAD;
    KVHead &hh = c->h[head_idx];
    if (hh.len == 0) return OJASX_OK;
    int rc = ensure_pages(c, hh.cap / 16);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(c->qstage.ptr, q, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    rc = kv_decode(c->qstage.as<float>(), hh.kc.as<uint8_t>(), hh.ks.as<float>(),
                   hh.vc.as<uint8_t>(), hh.vs.as<float>(), c->cb.as<float>(), c->cb.as<float>(),
                   c->bt.as<int>(), hh.len, 16, 1, 1, c->hd, c->D, scale_factor,
                   c->ostage.as<float>(), nullptr, c->work);
    if (rc) return rc;
    OJX_HIP(hipMemcpy(out_context, c->ostage.ptr, (size_t)c->hd * 4, hipMemcpyDeviceToHost));
    return OJASX_OK;
}

OJASX_API size_t ojasx_kv_cache_get_memory_size(OjasxKVHandle handle) {
    if (!handle) return 0;
    const KVCache *c = static_cast<const KVCache *>(handle);
    size_t b = 0;
    for (const auto &hh : c->h)  // ojasx_lut_kv_cache.h:40-44 accounting
        b += (size_t)hh.cap * c->G * 2 + (size_t)hh.cap * 4 * 2 + (size_t)256 * c->D * 4 * 2;
    return b;
}

OJASX_API float ojasx_kv_cache_get_compression_ratio(OjasxKVHandle handle) {
    if (!handle) return 0.f;
    const KVCache *c = static_cast<const KVCache *>(handle);
    if (c->heads == 0) return 0.f;
    const size_t len = c->h[0].len;
    const size_t dense = 2 * (size_t)c->hd * len * 4;
    const size_t comp = len * (c->G * 2 + 2 * 4);
    return (float)dense / (float)(comp ? comp : 1);
}

OJASX_API void ojasx_destroy_kv_cache(OjasxKVHandle handle) {
    delete static_cast<KVCache *>(handle);
}

OJASX_API int ojasx_kv_decode_paged_device(const float *q, const uint8_t *k_codes,
                                           const float *k_scales, const uint8_t *v_codes,
                                           const float *v_scales, const float *k_cb,
                                           const float *v_cb, const int *block_table, int seq_len,
                                           int page_size, int num_q_heads, int num_kv_heads,
                                           int head_dim, int block_dim, float scale_factor,
                                           float *out, void *stream) {
    using namespace ojx;
    if (!q || !k_codes || !k_scales || !v_codes || !v_scales || !k_cb || !v_cb || !block_table ||
        !out)
        return OJASX_ERR_NULL;
    return kv_decode(q, k_codes, k_scales, v_codes, v_scales, k_cb, v_cb, block_table, seq_len,
                     page_size, num_q_heads, num_kv_heads, head_dim, block_dim, scale_factor, out,
                     static_cast<hipStream_t>(stream), t_work);
}

}  // extern "C"

// decoder.hip -- a Qwen3-4B-shaped decoder whose every linear layer is a
// split-manifold LUT linear (d = 16, 256 centroids, CSR outliers) and whose
// KV cache is the paged code-domain cache, greedy batch-1 decode on gfx950.
//
// One token step, all state on the device (position, step, token), so the
// step is a fixed launch sequence that a HIP graph replays:
//   per layer
//     1. qkv  = LUT(Wqkv, RMSNorm(x, w_in))           lut_dec_kernel, RMSNorm prologue
//     2. q    = RoPE(RMSNorm_head(q, w_qn));  k = RoPE(RMSNorm_head(k, w_kn));
//        k, v encoded into the layer's paged code cache at `pos`   attn_prep_kernel
//     3. attn = softmax(q K^T / sqrt(hd)) V over pos + 1 tokens   kv_decode_small_kernel + merge
//     4. x   += LUT(Wo, attn)                          residual epilogue
//     5. gu   = LUT(Wgu, RMSNorm(x, w_post))           RMSNorm prologue (gate rows, then up rows)
//     6. x   += LUT(Wdown, silu(gate) * up)            SwiGLU prologue, residual epilogue
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
#include "kv_encode.h"

namespace ojx {

namespace {
constexpr int kHd = 128;          // head dim of the decode kernels
constexpr int kBd = 16;           // block dim of every LUT linear and of the KV codebooks
constexpr int kG = kHd / kBd;     // KV code groups per head
constexpr int kArgNT = 1024;
}  // namespace

struct AttnPrepParams {
    const float *qkv;             // [Hq*hd | Hkv*hd (k) | Hkv*hd (v)]
    const float *qn_w, *kn_w;     // [hd]
    const float *cos_t, *sin_t;   // [max_ctx][hd/2]
    const int *state;             // state[0] = position of the new token
    const int *bt;                // block table
    const float *kcb, *vcb;       // [Hkv][256][16]
    float *q_out;                 // [Hq][hd]
    uint8_t *kc, *vc;             // [pages][Hkv][P][G]
    float *ks, *vs;               // [pages][Hkv][P]
    int Hq, Hkv, P, max_ctx;
    float eps;
};

// Workgroup b < Hq: query head b; otherwise kv head b - Hq.  Thread d < hd
// owns dimension d: the per-head RMSNorm (wave sums), then RoPE with the
// partner dimension from LDS.  Query heads store q; kv heads encode the
// rotated k and the raw v into the cache (all 256 threads, kv_encode.h).
__global__ __launch_bounds__(kEncNT) void attn_prep_kernel(AttnPrepParams p) {
    __shared__ float xs[2 * kHd];    // encoder scratch
    __shared__ float xn[kHd];        // normalised row
    __shared__ float kr[kHd];        // rotated k
    __shared__ float red[kEncNW];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const bool is_q = b < p.Hq;
    const int h = is_q ? b : b - p.Hq;
    float kreg[kBd], vreg[kBd];
    const float *kcb = (!is_q && p.kcb) ? p.kcb + (size_t)h * 256 * kBd : nullptr;
    const float *vcb = (!is_q && p.vcb) ? p.vcb + (size_t)h * 256 * kBd : nullptr;
    if (kcb) enc_load_centroids<kBd>(kcb, vcb, kreg, vreg);
    const int pos = min(p.state[0], p.max_ctx - 1);
    const float *src = p.qkv + (is_q ? (size_t)h * kHd : (size_t)(p.Hq + h) * kHd);
    const float *wn = is_q ? p.qn_w : p.kn_w;
    const float v = tid < kHd ? src[tid] : 0.f;
    const float wv = tid < kHd ? wn[tid] : 0.f;
    constexpr int half = kHd / 2;
    const float c = tid < kHd ? p.cos_t[(size_t)pos * half + (tid % half)] : 0.f;
    const float s = tid < kHd ? p.sin_t[(size_t)pos * half + (tid % half)] : 0.f;
    const int page = is_q ? 0 : p.bt[pos / p.P];   // with the row loads, not after the rotation
    const float ss = wave_sum_f(v * v);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    const float var = ((red[0] + red[1]) + (red[2] + red[3])) / (float)kHd;
    const float rn = 1.0f / sqrtf(var + p.eps);
    const float xv = (v * rn) * wv;
    if (tid < kHd) xn[tid] = xv;
    __syncthreads();
    float out = 0.f;
    if (tid < kHd) out = tid < half ? xv * c - xn[tid + half] * s : xv * c + xn[tid - half] * s;
    if (is_q) {
        if (tid < kHd) p.q_out[(size_t)h * kHd + tid] = out;
        return;                                  // whole workgroup
    }
    if (tid < kHd) kr[tid] = out;
    __syncthreads();
    const size_t row = ((size_t)page * p.Hkv + h) * p.P + (pos % p.P);
    const float *vr = p.qkv + (size_t)(p.Hq + p.Hkv + h) * kHd;
    encode_kv_token<kBd>(kr, vr, kcb, vcb, kreg, vreg, kHd, kBd, kG, p.kc + row * kG,
                         p.vc + row * kG, p.ks + row, p.vs + row, xs);
}

// Greedy pick over V logits (first maximum), then the picked token's
// embedding row into x; thread 0 records the token and advances
// state = {position, step, token}.
__global__ __launch_bounds__(kArgNT) void argmax_embed_kernel(const float *logits, int V,
                                                             const float *emb, int hidden,
                                                             float *x, int *state, int *tokens,
                                                             int max_steps) {
    __shared__ float wm[kArgNT / 64];
    __shared__ int wi[kArgNT / 64];
    __shared__ int pick;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // each thread visits its indices in increasing order, 8 float4 loads in
    // flight per batch; strict > keeps the first maximum
    float best = -INFINITY;
    int bi = 0x7fffffff;
    const int n4 = V / 4;
    const float4 *l4 = reinterpret_cast<const float4 *>(logits);
    for (int b = tid; b < n4; b += kArgNT * 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i4 = b + u * kArgNT;
            v[u] = i4 < n4 ? l4[i4] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = (b + u * kArgNT) * 4;
            if (v[u].x > best) { best = v[u].x; bi = i; }
            if (v[u].y > best) { best = v[u].y; bi = i + 1; }
            if (v[u].z > best) { best = v[u].z; bi = i + 2; }
            if (v[u].w > best) { best = v[u].w; bi = i + 3; }
        }
    }
    for (int i = n4 * 4 + tid; i < V; i += kArgNT) {
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
        pick = min(max(b, 0), V - 1);            // all-NaN logits: token 0
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
    DevBuf final_norm, emb, cos_t, sin_t, bt, x, qkv, q, attn, gu, logits, part_o, part_ml,
        state, tokens;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool ready_layers = false, ready_head = false;

    ~Decoder() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (stream) (void)hipStreamDestroy(stream);
        for (DecoderLayer &l : L)
            for (DevBuf *b : {&l.in_norm, &l.post_norm, &l.q_norm, &l.k_norm, &l.kcb, &l.vcb, &l.kc,
                              &l.ks, &l.vc, &l.vs})
                b->release();
        for (DevBuf *b : {&final_norm, &emb, &cos_t, &sin_t, &bt, &x, &qkv, &q, &attn, &gu, &logits,
                          &part_o, &part_ml, &state, &tokens})
            b->release();
    }

    int n_chunks() const { return (max_ctx + 63) / 64; }

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
            AttnPrepParams ap{qkv.as<float>(), ly.q_norm.as<float>(), ly.k_norm.as<float>(),
                              cos_t.as<float>(), sin_t.as<float>(), pos, bt.as<int>(),
                              ly.kcb.as<float>(), ly.vcb.as<float>(), q.as<float>(),
                              ly.kc.as<uint8_t>(), ly.vc.as<uint8_t>(), ly.ks.as<float>(),
                              ly.vs.as<float>(), Hq, Hkv, P, max_ctx, eps};
            OJX_LAUNCH(attn_prep_kernel, dim3(Hq + Hkv), dim3(kEncNT), 0, st, ap);
            rc = kv_decode_device_len(q.as<float>(), ly.kc.as<uint8_t>(), ly.ks.as<float>(),
                                      ly.vc.as<uint8_t>(), ly.vs.as<float>(), ly.kcb.as<float>(),
                                      ly.vcb.as<float>(), bt.as<int>(), pos, 1, max_ctx, P, Hq,
                                      Hkv, sf, part_o.as<float>(), part_ml.as<float>(),
                                      attn.as<float>(), st);
            if (rc) return rc;
            rc = linear_forward_fused(ly.o, attn.as<float>(), x.as<float>(), 0, nullptr, 0.f,
                                      x.as<float>(), st);
            if (rc) return rc;
            rc = linear_forward_fused(ly.gu, x.as<float>(), gu.as<float>(), 1,
                                      ly.post_norm.as<float>(), eps, nullptr, st);
            if (rc) return rc;
            rc = linear_forward_fused(ly.down, gu.as<float>(), x.as<float>(), 2, nullptr, 0.f,
                                      x.as<float>(), st);
            if (rc) return rc;
        }
        rc = linear_forward_fused(lm, x.as<float>(), logits.as<float>(), 1, final_norm.as<float>(),
                                  eps, nullptr, st);
        if (rc) return rc;
        OJX_LAUNCH(argmax_embed_kernel, dim3(1), dim3(kArgNT), 0, st, logits.as<float>(), vocab,
                   emb.as<float>(), hidden, x.as<float>(), state.as<int>(), tokens.as<int>(),
                   max_steps);
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
    if (!rc) rc = d->q.ensure((size_t)q_heads * kHd * 4);
    if (!rc) rc = d->attn.ensure((size_t)q_heads * kHd * 4);
    if (!rc) rc = d->gu.ensure((size_t)2 * intermediate * 4);
    if (!rc) rc = d->logits.ensure((size_t)vocab * 4);
    if (!rc) rc = d->part_o.ensure((size_t)q_heads * d->n_chunks() * kHd * 4);
    if (!rc) rc = d->part_ml.ensure((size_t)q_heads * d->n_chunks() * 2 * 4);
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

/*
 * ojasx_lut_c_api.h -- C-ABI of the MI355X (gfx950) split-manifold LUT engine.
 *
 * Drop-in for the reference C-ABI (split_manifold_lut_experiment/native/
 * include/ojasx_lut_c_api.h, cited below as "ref.h:<line>"), implemented with
 * hand-written HIP kernels in libojasx_lut_hip.so.
 *
 * Two faces:
 *  1. The reference's 21 symbols, same names and signatures, same semantics:
 *     host pointers, synchronous, create_* deep-copies every array (here: into
 *     device memory, repacked into the kernels' tiled layout), NULL data means
 *     zeros (scales default to 1), int status 0 = OK, -1 = null handle or
 *     pointer, -2 = head index out of range, create_* returns NULL on failure.
 *  2. Device variants (no counterpart in the reference, whose GPU code is
 *     never built): device pointers, an activation dtype tag and a hipStream_t
 *     passed as void*.  They enqueue work and return without synchronising.
 *
 * Extra status codes: -3 invalid argument (shape, dtype, CSR structure, an
 * expert id is validated by the skip rule instead), -4 HIP runtime error,
 * -5 device out of memory.  ojasx_get_last_error() returns a message for the
 * last failing call on the calling thread.
 *
 * Concurrency: calls on one handle must be serialised by the caller (the
 * reference's mutators are unlocked too); forward calls on one handle share
 * that handle's workspace.
 */
#ifndef OJASX_LUT_C_API_H
#define OJASX_LUT_C_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OJASX_API __attribute__((visibility("default")))

typedef void *OjasxLinearHandle; /* ref.h:35 */
typedef void *OjasxKVHandle;     /* ref.h:36 */
typedef void *OjasxMoEHandle;    /* ref.h:37 */
typedef void *OjasxDecoderHandle; /* no reference counterpart (the decoder below) */

enum {
    OJASX_OK = 0,
    OJASX_ERR_NULL = -1,
    OJASX_ERR_HEAD = -2,
    OJASX_ERR_INVALID = -3,
    OJASX_ERR_HIP = -4,
    OJASX_ERR_OOM = -5
};

/* Activation / output element types of the device entry points (F64 and
 * INT8 only where an entry point says so). */
enum {
    OJASX_DTYPE_F32 = 0,
    OJASX_DTYPE_BF16 = 1,
    OJASX_DTYPE_F16 = 2,
    OJASX_DTYPE_F64 = 3,
    OJASX_DTYPE_INT8 = 4
};

/* ---- metadata (ref.h:40-41) ------------------------------------------- */
OJASX_API const char *ojasx_get_version(void);
OJASX_API const char *ojasx_get_backend_name(void);
/* No reference counterpart: message of the last failing call (thread-local). */
OJASX_API const char *ojasx_get_last_error(void);
/* No reference counterpart (measurement): while enabled, every kernel the
 * library launches records events at its own start and end; the report
 * synchronises the device, writes {"kernel": {"calls": n, "avg_us": t}, ...,
 * "_dropped": d} (at most 65536 launches are kept) into buf, clears the
 * records and returns the length needed including the terminating NUL.
 * Not thread-safe; timing changes launch overhead, so time throughput with
 * it disabled. */
OJASX_API int ojasx_kernel_timing_enable(int enable);
OJASX_API int ojasx_kernel_timing_report(char *buf, size_t buf_size);

/* ---- linear (ref.h:46-91) --------------------------------------------- */
/* ref.h:46-55.  codes_data is [out_features][in_features/block_dim] uint8,
 * codebook_data [codebook_size][block_dim] fp32.  Any block_dim dividing
 * in_features, codebook_size <= 256 (block_dim 16 runs the single-kernel and
 * MFMA paths, other sizes the LUT-build + gather path). */
OJASX_API OjasxLinearHandle ojasx_create_linear(int in_features, int out_features,
                                                int block_dim, int codebook_size,
                                                const float *codebook_data,
                                                const uint8_t *codes_data,
                                                const float *scales_data,
                                                const float *bias_data);
/* ref.h:60-66.  CSR over [out_features][in_features]; replaces any previous
 * outliers; nnz == 0 clears them.  Validated: row_ptrs monotone from 0 to
 * nnz, columns in range (-3 otherwise).  Each row's entries are stored sorted
 * by column (stable), so a row's outlier sum is formed in column order. */
OJASX_API int ojasx_set_linear_outliers(OjasxLinearHandle handle, int nnz,
                                        const int *row_ptrs, const int *col_indices,
                                        const float *values);
/* ref.h:72-78.  Host x [batch][in], y [batch][out], fp32; synchronous.
 * num_threads is accepted for compatibility and ignored (the GPU runs it). */
OJASX_API int ojasx_linear_forward(OjasxLinearHandle handle, const float *x, float *y,
                                   int batch_size, int num_threads);
/* ref.h:83-86: sizes of the reference's own representation (codes + codebook
 * + scales + bias + int32/int32/fp32 CSR) so callers' accounting is unchanged. */
OJASX_API size_t ojasx_get_compressed_size(OjasxLinearHandle handle);
OJASX_API size_t ojasx_get_dense_size(OjasxLinearHandle handle);
OJASX_API size_t ojasx_get_lut_sram_size(OjasxLinearHandle handle);
OJASX_API float ojasx_get_compression_ratio(OjasxLinearHandle handle);
/* ref.h:91 */
OJASX_API void ojasx_destroy_linear(OjasxLinearHandle handle);

/* Device variant of ref.h:72-78 (no reference counterpart): x [batch][in],
 * y [batch][out] in HBM, dtype OJASX_DTYPE_F32 or _BF16 for both, enqueued on
 * stream (a hipStream_t; NULL = default stream).  block_dim 16: below 9
 * tokens one in-place LUT kernel; from 9 tokens (in_features <= 65535, fp32
 * x 16-byte aligned) x . W^T on fp32 MFMA with W decoded from the codes. */
OJASX_API int ojasx_linear_forward_device(OjasxLinearHandle handle, const void *x, void *y,
                                          int batch_size, int dtype, void *stream);
/* Many independent linears in one launch (no reference counterpart; the
 * sustained-throughput form of ref.h:72-78): y_i = handles[i](x_i) for i <
 * count, batch 1, fp32 device pointers (x_i 16-byte aligned), block_dim 16.
 * Each 16-group LUT slice is built with MFMA and gathered per row.  Calls from
 * one host thread share a staging buffer: order them on one stream. */
OJASX_API int ojasx_linear_forward_grouped_device(const OjasxLinearHandle *handles, int count,
                                                  const float *const *xs, float *const *ys,
                                                  void *stream);
/* LUT[b][g][k] = <x_b[g*D:(g+1)*D], C[k]> for k < codebook_size (fp32 out,
 * [batch][groups][codebook_size]); the standalone LUT build of
 * split_manifold_engine.py:185-200 / ojasx_lut_cpu.cpp:18-102 (no reference
 * C-ABI counterpart).  x [batch][groups*block_dim] in dtype, codebook fp32. */
OJASX_API int ojasx_build_lut_device(const void *x, const float *codebook, int batch_size,
                                     int groups, int block_dim, int codebook_size, float *lut,
                                     int dtype, void *stream);
/* Bytes the batch-1 forward reads per call that are weights: packed codes,
 * outlier stream (16-bit columns and fp32 values, 6 bytes per entry, where
 * in_features <= 65536; plus the row pointers), codebook, scales, bias (no
 * reference counterpart; for roofline accounting).  The batched kernels (9
 * tokens and more) read 32-bit columns: 2 more bytes per outlier. */
OJASX_API size_t ojasx_linear_device_weight_bytes(OjasxLinearHandle handle);

/* ---- KV cache (ref.h:96-120) ------------------------------------------ */
OJASX_API OjasxKVHandle ojasx_create_kv_cache(int num_heads, int head_dim, int max_seq_len,
                                              int block_dim);
/* ref.h:103-108: quantise and append one token of one head (host k, v). */
OJASX_API int ojasx_kv_cache_append(OjasxKVHandle handle, int head_idx, const float *k,
                                    const float *v);
/* ref.h:110-116: softmax(q.K^T * sf) . V for one head; sf <= 0 means
 * 1/sqrt(head_dim); an empty head returns 0 and leaves out_context untouched. */
OJASX_API int ojasx_kv_cache_attention(OjasxKVHandle handle, int head_idx, const float *q,
                                       float *out_context, float scale_factor);
OJASX_API size_t ojasx_kv_cache_get_memory_size(OjasxKVHandle handle);
OJASX_API float ojasx_kv_cache_get_compression_ratio(OjasxKVHandle handle);
OJASX_API void ojasx_destroy_kv_cache(OjasxKVHandle handle);

/* Paged code-domain decode attention over device memory (no reference
 * counterpart; generalises ref.h:110-116 to a per-kv-head 256 x block_dim
 * codebook, GQA and a block table).
 *   q        [num_q_heads][head_dim] fp32
 *   k_codes  [num_pages][num_kv_heads][page_size][head_dim/block_dim] uint8
 *   k_scales [num_pages][num_kv_heads][page_size] fp32 (same for v_*)
 *   k_cb     [num_kv_heads][256][block_dim] fp32 (same for v_cb)
 *   block_table [ceil(seq_len/page_size)] int32 physical page of each logical page
 *   out      [num_q_heads][head_dim] fp32
 * q head j attends with kv head j / (num_q_heads / num_kv_heads);
 * head_dim / block_dim <= 32, block_dim <= 32; sf <= 0 means 1/sqrt(head_dim);
 * seq_len == 0 leaves out untouched.  Calls from one host thread share a
 * workspace and must be ordered on one stream. */
OJASX_API int ojasx_kv_decode_paged_device(const float *q, const uint8_t *k_codes,
                                           const float *k_scales, const uint8_t *v_codes,
                                           const float *v_scales, const float *k_cb,
                                           const float *v_cb, const int *block_table,
                                           int seq_len, int page_size, int num_q_heads,
                                           int num_kv_heads, int head_dim, int block_dim,
                                           float scale_factor, float *out, void *stream);

/* No counterpart in the reference: ojasx_kv_decode_paged_device for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels
 * and results; the decode partials live in a fixed library scratch of
 * 4 MiB + 64 KiB per GPU (held until the process ends) instead of a growable
 * workspace: partial outputs (num_q_heads x chunks x head_dim fp32) in the
 * 4 MiB, partial maxima and sums (num_q_heads x chunks x 2 fp32) in the
 * 64 KiB, so num_q_heads x chunks <= min(4 MiB / (head_dim * 4), 8192):
 * 8192 at head_dim 128 and at 64.  Chunks per call: the GQA-4, head_dim 128,
 * block_dim 16 path takes ceil(seq_len / 64) up to 4096 tokens, then
 * ceil(seq_len / C) with C = 64 .. 1024 tokens (about one workgroup per CU;
 * 1024 from 65536 tokens at 8 kv heads); other shapes take
 * ceil(seq_len / 256).  A single chunk needs no scratch.  Larger calls return
 * OJASX_ERR_INVALID with a message.  All calls on one GPU share the scratch:
 * calls that overlap in time on one GPU (other streams, other host threads)
 * race. */
OJASX_API int ojasx_kv_decode_paged_device_noalloc(const float *q, const uint8_t *k_codes,
                                                   const float *k_scales, const uint8_t *v_codes,
                                                   const float *v_scales, const float *k_cb,
                                                   const float *v_cb, const int *block_table,
                                                   int seq_len, int page_size, int num_q_heads,
                                                   int num_kv_heads, int head_dim, int block_dim,
                                                   float scale_factor, float *out, void *stream);

/* Device append into the paged code layout above; replaces
 * HeadKVCache::append_token (ojasx_lut_kv_cache.cpp:16-65, ref.h:103-108) for
 * num_tokens tokens and all kv heads in one call.
 *   k, v [num_tokens][num_kv_heads][head_dim] fp32
 *   s = max(1e-8, max_d |k_d|) / 127 per token and head, x = k / s;
 *   with codebooks ([num_kv_heads][256][block_dim] fp32): code[g] = the
 *     centroid nearest x[g*block_dim ..) in squared distance (fmaf in d order,
 *     ties to the lower index);
 *   with both codebooks NULL: the reference quantiser,
 *     clamp(round_half_away(x[g*block_dim]), -128, 127) + 128.
 *   slot_mapping [num_tokens] int32: page * page_size + offset of each token
 *     (negative or >= num_pages * page_size: token skipped).
 * head_dim / block_dim <= 64, head_dim <= 16384. */
OJASX_API int ojasx_kv_encode_append_device(const float *k, const float *v, int num_tokens,
                                            int num_kv_heads, int head_dim, int block_dim,
                                            const float *k_codebook, const float *v_codebook,
                                            const int *slot_mapping, int page_size,
                                            int num_pages, uint8_t *k_codes, float *k_scales,
                                            uint8_t *v_codes, float *v_scales, void *stream);

/* PagedCompressedKVCache._quantize_int8 (ojasx_24x96/long_context.py:234-240)
 * on device: rows of dim elements of x (dtype F32, BF16, F16 or F64), row r of
 * group g at x + g*x_group_stride + r*dim (elements), int8 codes to
 * q + g*q_group_stride + r*dim and the fp16 scale to scale + g*scale_group_stride + r.
 * Arithmetic as torch on a tensor of x's dtype: s = T(max(max|x|, T(1e-8)) / 127),
 * q = clamp(round_half_even(T(x / s)), -127, 127); an F64 scale is stored as
 * torch casts float64 to float16 (through float32). */
OJASX_API int ojasx_quantize_int8_device(const void *x, long groups, int rows, int dim,
                                         long x_group_stride, int dtype, int8_t *q,
                                         long q_group_stride, void *scale_f16,
                                         long scale_group_stride, void *stream);
/* long_context.py:242-244 _dequantize_int8: out[g][r][d] = dtype(float(q) * float(s))
 * into a contiguous [groups][rows][dim] out (F32, BF16, F16 or F64); q and scale
 * addressed as in ojasx_quantize_int8_device. */
OJASX_API int ojasx_dequantize_int8_device(const int8_t *q, const void *scale_f16, long groups,
                                           int rows, int dim, long q_group_stride,
                                           long scale_group_stride, void *out, int dtype,
                                           void *stream);

/* ojasx_kv_decode_paged_device with the context length read on the device
 * (*seq_len_dev, clamped to max_seq_len; 0 leaves out untouched), so a captured
 * HIP graph can replay the call as the context grows: the launch covers
 * max_seq_len (block_table holds ceil(max_seq_len / page_size) entries).  head_dim 128, block_dim 16, 16-byte aligned q and codebooks.
 * Chunks of 64 * tokens_per_lane tokens (1, 2 or 4; 0 picks by max_seq_len).
 * Workspace as ojasx_kv_decode_paged_device: call once outside a capture with
 * the same max_seq_len before capturing.  A later call that needs a larger
 * workspace moves to a new one and keeps the old until the host thread exits,
 * so graphs captured before stay valid; calls from one host thread on several
 * streams share the workspace and must not overlap in time. */
OJASX_API int ojasx_kv_decode_paged_device_len(const float *q, const uint8_t *k_codes,
                                               const float *k_scales, const uint8_t *v_codes,
                                               const float *v_scales, const float *k_cb,
                                               const float *v_cb, const int *block_table,
                                               const int *seq_len_dev, int max_seq_len,
                                               int page_size, int num_q_heads, int num_kv_heads,
                                               int head_dim, int block_dim, float scale_factor,
                                               int tokens_per_lane, float *out, void *stream);

/* ---- streamed exact attention (ojasx_24x96/long_context.py:92-176) ------ */
/* OnlineSoftmaxBlockAttention.forward_stream on device, fp64 state, in three
 * calls: init (state <- query), update (fold tiles in), finalize (output).
 * Query rows are [batch][num_heads][q_len] (row = (b * num_heads + h) * q_len
 * + s), each of head_dim elements; head h attends kv head
 * h / (num_heads / num_kv_heads).  state: [rows][2 * head_dim + 2] fp64 =
 * (query, acc, m, l) per row; head_dim a multiple of 8, at most 256. */
typedef struct OjasxAttnTile {
    const void *k, *v;            /* [batch][kv heads][n_tokens][head_dim], strided */
    const void *k_scale, *v_scale; /* OJASX_DTYPE_INT8 tiles: fp16 per-token scales */
    long long n_tokens;
    long long batch_stride, head_stride, token_stride;       /* elements, k and v */
    long long scale_batch_stride, scale_head_stride, scale_token_stride;
} OjasxAttnTile;
/* long_context.py:117-127: state <- (q as fp64, acc 0, m -inf, l 0); q
 * [rows][head_dim] contiguous, q_dtype F32, BF16, F16 or F64. */
OJASX_API int ojasx_attention_stream_init_device(double *state, const void *q, int q_dtype,
                                                 int rows, int head_dim, void *stream);
/* long_context.py:129-163 for n_tiles tiles in order (the tiles' device
 * descriptors are staged by the library; the host array may be reused on
 * return).  Token t of the stream (kv_offset + tokens of earlier tiles + t)
 * is hidden from query s when causal != 0 and t > query_start_pos + s.
 * kv_dtype F32, BF16, F16, F64, or INT8 (the paged cache's pages: value =
 * int8 * fp16 scale of its token, exact; head_dim a multiple of 16).  Scores
 * (q . k) * scale, in fp64.  k and v 16-byte aligned with strides that keep
 * every row 16-byte aligned (float v: 4-element aligned), rows contiguous.
 * Calls from one host thread share a workspace: serialise them (one stream). */
OJASX_API int ojasx_attention_stream_update_device(double *state, int batch, int num_heads,
                                                   int num_kv_heads, int q_len, int head_dim,
                                                   const OjasxAttnTile *tiles, int n_tiles,
                                                   int kv_dtype, int causal,
                                                   long long query_start_pos, long long kv_offset,
                                                   double scale, void *stream);
/* long_context.py:165-167: out [rows][head_dim] = acc / l (l = 0 -> 1) in
 * out_dtype (F32, BF16, F16 or F64; bf16 and fp16 rounded through fp32 as
 * torch's .to() from fp64), lse [rows] = m + log(l) (NULL: not written). */
OJASX_API int ojasx_attention_stream_finalize_device(const double *state, int rows, int head_dim,
                                                     void *out, int out_dtype, double *lse,
                                                     void *stream);

/* ---- MoE (ref.h:125-150) ---------------------------------------------- */
OJASX_API OjasxMoEHandle ojasx_create_moe(int num_experts, int hidden_dim,
                                          int intermediate_dim, int top_k, int block_dim,
                                          const float *codebook_in, const float *codebook_down,
                                          const uint8_t *gate_up_codes,
                                          const float *gate_up_scales,
                                          const uint8_t *down_codes, const float *down_scales);
/* ref.h:139-146: one token; k_active <= 0 leaves y_out untouched. */
OJASX_API int ojasx_moe_forward(OjasxMoEHandle handle, const float *x, const int *top_k_indices,
                                const float *top_k_weights, float *y_out, int k_active);
OJASX_API size_t ojasx_moe_get_compressed_size(OjasxMoEHandle handle);
OJASX_API float ojasx_moe_get_compression_ratio(OjasxMoEHandle handle);
OJASX_API void ojasx_destroy_moe(OjasxMoEHandle handle);

/* Device variant of ref.h:139-146 for a batch of tokens (no reference
 * counterpart): x [num_tokens][hidden], idx/w [num_tokens][k_active],
 * y [num_tokens][hidden] fully overwritten (k_active <= 0: untouched).
 * Calls on one handle share its workspaces, grown as larger batches arrive:
 * serialise them per handle.  Once a call with a given (num_tokens,
 * k_active) has run, later calls with those values neither allocate nor
 * record a memset, so they can be captured in a HIP graph and replayed. */
OJASX_API int ojasx_moe_forward_device(OjasxMoEHandle handle, const void *x, const int *idx,
                                       const float *w, void *y, int num_tokens, int k_active,
                                       int dtype, void *stream);
/* Router (absent from the reference; its callers pass indices and weights):
 * logits [num_tokens][num_experts] fp32 -> idx [num_tokens][k] int32 (the k
 * largest logits, descending, ties to the lower index) and w [num_tokens][k]
 * = softmax over all experts at those indices, divided by their sum when
 * renormalize != 0.  num_experts <= 1024, k <= 32. */
OJASX_API int ojasx_moe_route_device(const float *logits, int num_tokens, int num_experts, int k,
                                     int renormalize, int *idx, float *w, void *stream);

/* ---- math engine (ojasx_24x96/math_engine.py, codec.py) ------------------ */
/* math_engine.py:136-208 subspace_lut_rvq_gemm, device pointers on `stream`:
 * y[b][m] = row_scales[m] * sum_{s,g} <x[b][g*block .. +block), C_s[code_s(m,g)]>
 * (+ bias[m]), x zero-padded to G = ceil(columns/block) blocks.  packed_codes
 * holds `stages` little-endian bit streams (codec.py:176-195) of
 * rows * G codes of `bits` in {1,2,4,8} bits, stage s at packed_codes +
 * s * stage_stride_bytes (no alignment required); codebooks fp32
 * [stages][2^bits][block]; row_scales fp32 [rows]; bias fp32 [rows] or NULL.
 * x and y are fp32 or bf16 per dtype (y in x's dtype).  block <= 64. */
OJASX_API int ojasx_subspace_lut_gemm_device(const void *x, int batch, int columns, int rows,
                                             const uint8_t *packed_codes, size_t stage_stride_bytes,
                                             int stages, int bits, int block_size,
                                             const float *codebooks, const float *row_scales,
                                             const float *bias, void *y, int dtype, void *stream);
/* codec.py:176-195 pack_codes: count codes (uint8, < 2^bits) -> ceil(count*bits/8)
 * packed bytes, little-endian within each byte. */
OJASX_API int ojasx_pack_codes_device(const uint8_t *codes, long count, int bits, uint8_t *packed,
                                      void *stream);
/* codec.py:198-214 unpack_codes: inverse of pack_codes for `count` codes. */
OJASX_API int ojasx_unpack_codes_device(const uint8_t *packed, long count, int bits, uint8_t *codes,
                                        void *stream);

/* ---- decoder (no reference counterpart) ---------------------------------- */
/* A decoder stack whose linears are LUT linears and whose KV cache is the paged
 * code cache, greedy batch-1 decode: the reference's 4B-shaped configuration
 * (hidden 2560, 36 layers, 32 q / 8 kv heads, MLP 9728).  Each layer:
 *   qkv = Wqkv RMSNorm(x; input_norm); q, k per-head RMSNorm (q_norm, k_norm)
 *   and RoPE (theta); k, v encoded into the layer's KV cache (256 x 16
 *   codebooks per kv head); attention over the cache; x += Wo attn;
 *   x += Wdown (silu(gate) * up) with [gate; up] = Wgate_up RMSNorm(x; post_norm).
 * Head: logits = Wlm RMSNorm(x; final_norm); next token = first argmax.
 * head_dim must be 128; every linear block_dim 16. */
OJASX_API OjasxDecoderHandle ojasx_create_decoder(int hidden, int layers, int q_heads,
                                                  int kv_heads, int head_dim, int intermediate,
                                                  int vocab, int max_context, int page_size,
                                                  int max_steps, float rms_eps, float rope_theta);
OJASX_API void ojasx_destroy_decoder(OjasxDecoderHandle handle);
/* Linear handles (ojasx_create_linear) are referenced, not copied, and must
 * outlive the decoder: qkv hidden -> (q_heads + 2 kv_heads) * 128 (q rows,
 * then k, then v), o q_heads*128 -> hidden, gate_up hidden -> 2*intermediate
 * (gate rows, then up rows), down intermediate -> hidden.  The other arrays
 * are device pointers, copied: norms [hidden] / [128], codebooks
 * [kv_heads][256][16] fp32. */
OJASX_API int ojasx_decoder_set_layer(OjasxDecoderHandle handle, int layer,
                                      OjasxLinearHandle qkv, OjasxLinearHandle o,
                                      OjasxLinearHandle gate_up, OjasxLinearHandle down,
                                      const float *input_norm, const float *post_norm,
                                      const float *q_norm, const float *k_norm,
                                      const float *k_codebook, const float *v_codebook);
/* lm_head hidden -> vocab (referenced); final_norm [hidden] and embedding
 * [vocab][hidden] fp32 device pointers, copied. */
OJASX_API int ojasx_decoder_set_head(OjasxDecoderHandle handle, OjasxLinearHandle lm_head,
                                     const float *final_norm, const float *embedding);
/* Prefilled context of one layer, device pointers in the paged layout of
 * ojasx_kv_decode_paged_device with the identity block table. */
OJASX_API int ojasx_decoder_set_context(OjasxDecoderHandle handle, int layer,
                                        const uint8_t *k_codes, const float *k_scales,
                                        const uint8_t *v_codes, const float *v_scales,
                                        int num_tokens);
/* Position of the next token (= context length). */
OJASX_API int ojasx_decoder_reset(OjasxDecoderHandle handle, int position);
/* Greedy decode of num_tokens tokens starting from first_token at the current
 * position: tokens_out [num_tokens] (host), last_logits [vocab] (host, or
 * NULL) = logits of the last step.  use_graph != 0 replays one captured HIP
 * graph per token (captured on the first such call).  Synchronous. */
OJASX_API int ojasx_decoder_generate(OjasxDecoderHandle handle, int first_token, int num_tokens,
                                     int use_graph, int *tokens_out, float *last_logits);
/* Host copy of one layer's KV cache rows for tokens [first_token,
 * first_token + num_tokens), first_token a multiple of page_size: codes
 * [pages][kv_heads][page_size][8], scales [pages][kv_heads][page_size]. */
OJASX_API int ojasx_decoder_read_kv(OjasxDecoderHandle handle, int layer, int first_token,
                                    int num_tokens, uint8_t *k_codes, float *k_scales,
                                    uint8_t *v_codes, float *v_scales);
/* Fused fp32 batch-1 LUT linear of the decoder: prologue 0 = none, 1 =
 * RMSNorm(x; norm_weight, eps), 2 = silu(x[:K]) * x[K:] from a 2K row; y =
 * residual + (...) when residual != NULL (residual may equal y).  Prologue 3
 * = RMSNorm as 1 with a SwiGLU epilogue: out_features = 2I (gate rows, then up
 * rows) and y [I] = silu(z[:I]) * z[I:] of the linear's output z, the input
 * prologue 2 computes from z; no residual. */
OJASX_API int ojasx_linear_forward_fused_device(OjasxLinearHandle handle, const float *x,
                                                float *y, int prologue, const float *norm_weight,
                                                float eps, const float *residual, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OJASX_LUT_C_API_H */

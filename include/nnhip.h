/*
 * nnhip.h -- C ABI of libnnhip.so, the MI355X (gfx950) HIP backend for the
 * speculative-decoding path of islhkafaa/neural-network.
 *
 * Conventions: plain pointers and sizes only; every function returns 0 or a
 * negative status (NNHIP_E*) and leaves a message for nnhip_last_error() on
 * the calling thread (the reference throws std::runtime_error with the same
 * text, e.g. tensor.cpp:393-402, layer.cpp:1176-1179).  A context owns one HIP
 * stream; calls are ordered on it; functions that take host buffers return
 * with the result in them.  A context is used by one host thread at a time.
 *
 * Host buffers are marked "host", device buffers (from nnhip_malloc) "dev".
 * Token ids are int32 (the reference carries them as fp32, layer.cpp:1402).
 */
#ifndef NNHIP_H
#define NNHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NNHIP_OK 0
#define NNHIP_EARG (-1)          /* bad argument or shape                   */
#define NNHIP_ECAPACITY (-2)     /* sequence would exceed max_seq_len        */
#define NNHIP_EHIP (-3)          /* HIP runtime failure                      */
#define NNHIP_EUNSUPPORTED (-4)  /* option the device path does not provide  */
#define NNHIP_EIO (-5)           /* a file could not be opened or written    */

typedef struct nnhip_ctx nnhip_ctx;
typedef struct nnhip_model nnhip_model;
typedef struct nnhip_kvcache nnhip_kvcache;

typedef struct {
  int64_t cycles;     /* speculative cycles after the first token         */
  int64_t drafted;    /* sum over cycles of M = min(k, tokens remaining)   */
  int64_t accepted;   /* accepted draft tokens                             */
  int64_t ties;       /* accept tests with |r - p/q| < 1e-6                */
  int64_t resampled;  /* cycles ending in a residual resample              */
  int64_t bonus;      /* cycles ending in a bonus sample                   */
} nnhip_spec_stats;

typedef struct {
  double prefill_ms;        /* prompt forward of target + draft, first token */
  double decode_ms;         /* the cycle loop                                 */
  int64_t cycles_launched;  /* cycles enqueued (one may run after the end)    */
} nnhip_spec_timing;

/* ---- errors, lifecycle, memory -------------------------------------------
 * Replace the device side of ExecutionBackend (include/backend/backend.hpp:
 * 20-33): allocate, copy_host_to_device, copy_to_device,
 * copy_device_to_host; DeviceBuffer (backend.hpp:9-18) is a dev pointer. */
const char *nnhip_last_error(void);
/* nnhip_init makes `device` the calling thread's current device and gives
 * the context its own stream on it.  Calls on a context launch on that
 * stream; the scratch some of them allocate (grown on demand) is allocated
 * on the current device, so a thread that switches devices makes the
 * context's device current again before calling on it (nnhip_malloc,
 * nnhip_decoder_create and nnhip_destroy select it themselves). */
int nnhip_init(int device, nnhip_ctx **out);
int nnhip_destroy(nnhip_ctx *ctx);
/* "graphs": 1 = replay each speculative cycle as one HIP graph (default).
 * "rng": uniforms of nnhip_generate_speculative(_batch) and
 * nnhip_generate_advanced(_batch) on this context: 0 = the Philox stream
 * (default), 1 = the reference's std::mt19937 (layer.cpp:1249, 1394), one
 * engine per sequence seeded (uint32_t)(seed + seq0 + b) -- for one
 * sequence exactly std::mt19937 gen(seed) -- drawn in the reference's
 * order with libstdc++'s float and double draws.
 * "gemm_wide": 1 = the int8 MFMA GEMM may use 32x64 tiles on large grids
 * (default: the prompt prefill's 8192-row down projection), 0 = always
 * 32x32 tiles (process-wide).
 * "attn_waves": number of (key split) waves an attention launch aims for;
 * the key range of each sequence is split accordingly (default 4096;
 * process-wide).
 * "attn_short_q": queries per workgroup of an attention launch of fewer
 * than 64 (sequence, head) pairs (one sequence's verify step): 1 (default),
 * 2, 4, or 8 = one workgroup for up to 8 queries (process-wide).
 * "attn_w4": attention rows of 4+ queries run in workgroups of 4 key
 * splits (two per CU) instead of 8: 1 = when a launch has 128 or more
 * workgroups (default), 2 = always, 0 = never (process-wide).
 * "kv_stream": fp32 KV rows read with non-temporal loads: 0 never, 1 when
 * one attention launch reads more rows than the L2 caches hold (default),
 * 2 always (process-wide).
 * "lds_min_rows": the LDS-resident GEMM serves projections from this many
 * rows on (default 128; process-wide).
 * "limb_k8": the digit-plane GEMM splits K over 8 waves from this K on
 * (default 512; process-wide).
 * "o_head_digits": 1 = for 64-wide heads the merged attention writes the
 * output projection's digit planes itself, one exponent per (row, head),
 * and the digit-plane GEMM scales each head's exact total by its own
 * exponent (default); 0 = act_quant digitises the context rows with one
 * exponent per row (process-wide).
 * "o_limb_rows": after the merged attention, the output projection of up
 * to this many rows runs as act_quant + digit-plane GEMM, taller inputs on
 * the LDS GEMM digitising the context rows (default 256; process-wide).
 * "gemv_down_rows": the down projection of up to this many rows runs on the
 * GEMV over the fp32 SwiGLU rows (default 64; process-wide).
 * "gemv_ln": Linear layers on the GEMV (short rows) over a LayerNorm's
 * output form the LayerNorm in the GEMV's prologue up to this many rows
 * (default 2); more rows get a LayerNorm launch of their own before the
 * GEMV (process-wide).
 * "ln_split": 1 = LayerNorm rows of 512 / 1024 spread over 2 / 4 waves
 * (default), 0 = one wave per row (process-wide).
 * No option changes results beyond fp32 rounding order. */
int nnhip_set_option(nnhip_ctx *ctx, const char *key, int value);
int nnhip_sync(nnhip_ctx *ctx);
int nnhip_malloc(nnhip_ctx *ctx, size_t bytes, void **out);
int nnhip_free(nnhip_ctx *ctx, void *dev);
int nnhip_h2d(nnhip_ctx *ctx, void *dev_dst, const void *host_src,
              size_t bytes);
int nnhip_d2h(nnhip_ctx *ctx, void *host_dst, const void *dev_src,
              size_t bytes);
/* Stream-ordered timer: begin records an event, end records a second one,
 * waits for it and returns the elapsed milliseconds. */
int nnhip_timer_begin(nnhip_ctx *ctx);
int nnhip_timer_end(nnhip_ctx *ctx, float *ms);

/* ---- decoder --------------------------------------------------------------
 * TransformerDecoder(vocab_size, embed_dim, num_heads, dim_feedforward,
 * num_layers, max_seq_len) (include/nn/layer.hpp:300-302): post-LN layers of
 * RoPE multi-head attention and SwiGLU, lm_head; weights resident on the
 * device. */
int nnhip_decoder_create(nnhip_ctx *ctx, int vocab, int d_model, int n_heads,
                         int d_ff, int n_layers, int max_seq_len,
                         nnhip_model **out);
int nnhip_decoder_free(nnhip_model *m);
/* TransformerDecoder::parameters() order (layer.cpp:1140-1154): token_emb;
 * per layer q.w q.b k.w k.b v.w v.b o.w o.b gate.w gate.b up.w up.b down.w
 * down.b ln1.g ln1.b ln2.g ln2.b; lm_head.w lm_head.b.  Dense weights are
 * [in][out] row-major as in the reference (layer.cpp:151-160). */
int nnhip_decoder_num_params(const nnhip_model *m, int *n);
int nnhip_decoder_param_shape(const nnhip_model *m, int idx, int64_t *rows,
                              int64_t *cols);
/* Tensor::copy_from_host / to_host on parameters()[idx] (host buffers). */
int nnhip_decoder_set_param(nnhip_model *m, int idx, const float *host);
int nnhip_decoder_get_param(const nnhip_model *m, int idx, float *host);
/* Seeded initialisation on the device: Dense weights and the embedding
 * N(0, std) from Philox4x32-10 + Box-Muller, biases 0, LayerNorm gamma 1 and
 * beta 0.  Replaces the random_device initialisers
 * (include/nn/initialization.hpp:13-66), which are not reproducible. */
int nnhip_decoder_init_normal(nnhip_model *m, uint64_t seed, float stdv);
/* quantize_model + MultiHeadAttention::quantize + QuantizedDense ctor
 * (quantization.cpp:7-87, 156-171; layer.cpp:545-558) applied to every Dense
 * of the decoder (q, k, v, o, gate, up, down, lm_head); the embedding stays
 * fp32.  bits: 8 (INT8) or 4 (INT4: scale max|w| / 7, codes in [-7, 7],
 * held one per byte on the device, so the INT8 kernels serve both). */
int nnhip_decoder_quantize(nnhip_model *m, int bits);
/* QuantizedDense::packed_weights / scales (quantization.hpp:31-33) of one
 * Dense: which 0..6 = q,k,v,o,gate,up,down of `layer`, 7 = lm_head.  codes
 * [in][out] int8 (host), scales [out] (host). */
int nnhip_decoder_get_quantized(const nnhip_model *m, int layer, int which,
                                int8_t *codes, float *scales);
/* Layer::save_weights / load_weights (layer.cpp:463-470) over parameters():
 * the NETW v1 file of serialization::save_parameters / load_parameters
 * (serialization.cpp:8-111): "NETW", uint16 version 1, uint32 count, per
 * tensor uint32 rank, uint64 extents, uint64 element count, fp32 data, in
 * the reference's shapes (embedding [V][d], Dense weight [in][out], bias
 * [1][out], LayerNorm gamma / beta [d]).  load rejects a file whose count,
 * ranks or extents differ from the model's with the reference's messages
 * (NNHIP_EARG) and re-quantises a quantised model's Dense layers from the
 * loaded fp32 weights; a file that cannot be opened is NNHIP_EIO. */
int nnhip_decoder_save_weights(const nnhip_model *m, const char *path);
int nnhip_decoder_load_weights(nnhip_model *m, const char *path);
/* TransformerDecoder::forward(x, caches) (layer.cpp:1161-1193) for B
 * sequences of S ids each: ids [B][S] (host), logits [B][S][V] (host).
 * cache may be NULL (no cache: attention over the S ids only).  With a
 * cache, sequence b continues at its own length, which grows by S. */
int nnhip_decoder_forward(nnhip_model *m, nnhip_kvcache *cache,
                          const int32_t *ids, int B, int S, float *logits);

/* ---- KV cache --------------------------------------------------------------
 * KVCache (layer.hpp:212-230) for `batch` sequences with one length each,
 * capacity max_seq_len.  quantized != 0 is KVCache(true): every appended
 * k / v row of one head is stored as int8 codes with one fp32 scale
 * (quantize_kv, layer.cpp:635-657) and attention reads code * scale
 * (layer.cpp:878-890, 925-938); head dim even and <= 64. */
int nnhip_kvcache_create(nnhip_model *m, int batch, int quantized,
                         nnhip_kvcache **out);
/* KVCache::quantized_k / quantized_v / k_scales / v_scales (layer.hpp:
 * 216-220) of one layer and sequence of an int8 cache, its first
 * length(b) positions: codes [H][len][D] and scales [H][len] (host). */
int nnhip_kvcache_read_q8(const nnhip_kvcache *c, int layer, int b,
                          int8_t *kcodes, float *kscales, int8_t *vcodes,
                          float *vscales);
/* KVCache::k / KVCache::v (layer.hpp:213-214) of one layer and sequence of
 * an fp32 cache, its first length(b) positions: [H][len][D] each (host);
 * k after RoPE, as the reference stores it. */
int nnhip_kvcache_read(const nnhip_kvcache *c, int layer, int b, float *k,
                       float *v);
int nnhip_kvcache_free(nnhip_kvcache *c);
int nnhip_kvcache_length(const nnhip_kvcache *c, int b, int *len);
/* KVCache::truncate(len) (layer.cpp:67-149) for sequence b: an O(1) length
 * update; a longer len leaves the cache unchanged. */
int nnhip_kvcache_truncate(nnhip_kvcache *c, int b, int len);

/* ---- generation -----------------------------------------------------------
 * TransformerDecoder::generate_speculative(draft, prompt, max_new_tokens,
 * lookahead, temperature, top_k, top_p, seed, quantized_cache)
 * (layer.hpp:318-323, layer.cpp:1382-1661).  out [P + max(max_new, 1)]
 * (host) receives the prompt and the generated ids.  Uniforms come from the
 * Philox stream u[seq][cycle][slot] (slot j < k: draft sample j, k + j:
 * accept test j, 2k: resample or bonus; cycle 0 slot 2k: first token), or
 * with the context option "rng" 1 from std::mt19937 as the reference draws
 * them.  temperature <= 0 is greedy.  top_k / top_p
 * filter every get_probs as nnhip_sample_rows describes.  quantized_cache
 * != 0 gives both models int8 KV caches (KVCache(true), layer.cpp:
 * 1396-1398).  A vocabulary above 32768 returns NNHIP_EUNSUPPORTED. */
int nnhip_generate_speculative(nnhip_model *target, nnhip_model *draft,
                               const int32_t *prompt, int P, int max_new,
                               int lookahead, float temperature, int top_k,
                               float top_p, uint64_t seed,
                               int quantized_cache, int32_t *out,
                               nnhip_spec_stats *stats);
/* The same for B independent sequences of equal prompt length P (the
 * reference is batch-1; this runs B of its loops in lockstep on one GPU
 * with per-sequence cache lengths).  prompts [B][P], out
 * [B][P + max(max_new, 1)], stats [B] (or NULL), timing (or NULL).
 * Sequence b uses Philox sequence index seq0 + b (or the mt19937 engine
 * seeded seed + seq0 + b). */
int nnhip_generate_speculative_batch(nnhip_model *target, nnhip_model *draft,
                                     int B, const int32_t *prompts, int P,
                                     int max_new, int lookahead,
                                     float temperature, int top_k, float top_p,
                                     uint64_t seed, uint32_t seq0,
                                     int quantized_cache, int32_t *out,
                                     nnhip_spec_stats *stats,
                                     nnhip_spec_timing *timing);
/* TransformerDecoder::generate_advanced(prompt, max_new_tokens, temperature,
 * top_k, top_p, seed, use_kv_cache) (layer.hpp:310-316, layer.cpp:
 * 1240-1380); sampled mode draws u[seq][step][0] (or, with "rng" 1, the
 * next double of the sequence's std::mt19937). */
int nnhip_generate_advanced(nnhip_model *m, const int32_t *prompt, int P,
                            int max_new, float temperature, int top_k,
                            float top_p, uint64_t seed, int use_kv_cache,
                            int32_t *out);
int nnhip_generate_advanced_batch(nnhip_model *m, int B,
                                  const int32_t *prompts, int P, int max_new,
                                  float temperature, int top_k, float top_p,
                                  uint64_t seed, uint32_t seq0,
                                  int use_kv_cache, int32_t *out);

/* ---- fused device ops (dev buffers, stream-ordered) ------------------------ */
/* QuantizedDense ctor, INT8 (quantization.cpp:36-66): w [in][out] fp32 ->
 * codes [out][in] int8 (transposed for coalesced GEMV loads), scales [out]. */
int nnhip_quantize_w8(nnhip_ctx *ctx, const float *w, int in, int out,
                      int8_t *codes, float *scales);
/* The INT4 QuantizedDense ctor (quantization.cpp:38-86): scales = max|w| /
 * 7, codes clamp(round(w / scale), -7, 7), held one per byte in the same
 * [out][in] layout (every W8A32 entry point takes them); packing two to a
 * byte (packed_weights, low nibble = even [in][out] index) is a host
 * storage format the device does not use. */
int nnhip_quantize_w4(nnhip_ctx *ctx, const float *w, int in, int out,
                      int8_t *codes, float *scales);
/* QuantizedDense::forward (quantization.cpp:127-147): y [rows][N] =
 * x [rows][K] . (codes * scales)^T + bias.  path: 0 auto, 1 fp32 GEMV,
 * 2 int8-digit MFMA GEMM (K % 128 == 0, N % 64 == 0), 3 MFMA GEMM with the
 * digits formed in LDS from x, 4 the same GEMM fed with digit planes
 * (3 and 4: K in {128, 256, 512, 1024}, N % 32 == 0).  The MFMA paths (2-4)
 * agree bit for bit.  Stream-ordered: the digit planes and the codes in the
 * MFMA operand layout go to scratch the context keeps and reuses, which
 * grows (after draining the stream) only when a call needs more. */
int nnhip_linear_w8a32(nnhip_ctx *ctx, const float *x, int rows, int K,
                       const int8_t *codes, const float *scales,
                       const float *bias, int N, float *y, int path);
/* LayerNorm (layer.cpp:242-261) of h [rows][K] followed by
 * QuantizedDense::forward (quantization.cpp:127-147), the pair
 * TransformerDecoderLayer::forward runs at norm1 -> ffn and norm2 -> the next
 * layer (layer.cpp:1098-1113): y = LN(h) . W^T + b,
 * and LN(h) into ln_out when it is not NULL.  K in {128, 256, 512, 1024},
 * N % 32 == 0.  Rows below 16 run on the GEMV with the LayerNorm as its
 * prologue (the decode path of short batches), others on the LDS-resident
 * MFMA GEMM with the LayerNorm in its prologue.  Stream-ordered, with the
 * context's scratch as nnhip_linear_w8a32. */
int nnhip_layernorm_linear_w8a32(nnhip_ctx *ctx, const float *h, int rows,
                                 int K, const float *gamma, const float *beta,
                                 float *ln_out, const int8_t *codes,
                                 const float *scales, const float *bias, int N,
                                 float *y);
/* nnhip_linear_w8a32 without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, paths and results; its scratch (the codes in the MFMA operand
 * layout, digit planes, row exponents: N*K + 3*K*rows64 + 4*rows64 bytes,
 * rows64 = rows rounded up to 64) lives in one fixed 32 MiB device array per
 * GPU, held until the process ends; larger calls return NNHIP_EARG.  The
 * GEMV path (path 1, or path 0 below 16 rows) uses no scratch.  Stream-
 * ordered, no synchronisation.  The first context that calls it owns that
 * GPU's array until nnhip_destroy: calls from any other context on the same
 * GPU return NNHIP_EARG (two streams would race on the array).  Calls of
 * the owning context are ordered by its stream; each call overwrites the
 * array's contents. */
int nnhip_linear_w8a32_noalloc(nnhip_ctx *ctx, const float *x, int rows,
                               int K, const int8_t *codes,
                               const float *scales, const float *bias, int N,
                               float *y, int path);
/* Dense::forward (layer.cpp:162-171) with w [N][K] fp32 (transposed). */
int nnhip_linear_f32(nnhip_ctx *ctx, const float *x, int rows, int K,
                     const float *w, const float *bias, int N, float *y);
/* The MFMA path's exact integers: row exponents rexp [rows], digits
 * limbs [3][rows64][K] (rows64 = rows rounded up to 64) and the int64 dot
 * totals [rows][N] = sum_k (hi*65536 + mid*256 + lo) * code. */
int nnhip_linear_limb_totals(nnhip_ctx *ctx, const float *x, int rows, int K,
                             const int8_t *codes, int N, int64_t *totals,
                             int32_t *rexp, int8_t *limbs);
/* Tensor::rope (tensor.cpp:1126-1226) on q and k of qkv [B*S][3*H*D] rows
 * ([q | k | v], head-major within each) at positions pos[b] + s, then the KV
 * append of MultiHeadAttention::forward (layer.cpp:758-807) into kcache /
 * vcache [B][H][cap][D]; q_out [B*S][H*D]. */
int nnhip_rope_kv_append(nnhip_ctx *ctx, const float *qkv, int B, int S,
                         int H, int D, const int32_t *pos, float *q_out,
                         float *kcache, float *vcache, int cap);
/* nnhip_rope_kv_append with grouped-query heads (MultiHeadAttention's
 * num_kv_heads, layer.cpp:471-489): qkv rows [q: H heads | k: Hkv heads |
 * v: Hkv heads] of D, H a multiple of Hkv; kcache / vcache
 * [B][Hkv][cap][D]. */
int nnhip_rope_kv_append_gqa(nnhip_ctx *ctx, const float *qkv, int B, int S,
                             int H, int Hkv, int D, const int32_t *pos,
                             float *q_out, float *kcache, float *vcache,
                             int cap);
/* Fused causal attention of MultiHeadAttention::forward (layer.cpp:842-952)
 * for S queries per sequence: q [B*S][H*D], kcache / vcache [B][Hkv][cap][D]
 * holding pos0[b] + S valid entries; query s sees keys j <= pos0[b] + s.
 * out [B*S][H*D]. */
int nnhip_attention_kq(nnhip_ctx *ctx, const float *q, const float *kcache,
                       const float *vcache, int cap, const int32_t *pos0,
                       int B, int S, int H, int Hkv, int D, float *out);
/* nnhip_rope_kv_append into an int8 cache: RoPE on q and k, then each new
 * k and v row of one head quantised as quantize_kv does (layer.cpp:635-657:
 * scale = max|x| / 127, 1 when 0; code = clamp(round(x * (1 / scale)),
 * -127, 127)) into kcodes / vcodes [B][H][cap][D] and kscales / vscales
 * [B][H][cap].  D even and <= 64. */
int nnhip_rope_kv_append_q8(nnhip_ctx *ctx, const float *qkv, int B, int S,
                            int H, int D, const int32_t *pos, float *q_out,
                            int8_t *kcodes, float *kscales, int8_t *vcodes,
                            float *vscales, int cap);
/* nnhip_attention_kq over an int8 cache (layer.cpp:842-952, quantized
 * branches): element j of a cached row enters as (float)code * scale.
 * kcodes / vcodes [B][Hkv][cap][D], kscales / vscales [B][Hkv][cap]. */
int nnhip_attention_kq_q8(nnhip_ctx *ctx, const float *q, const int8_t *kcodes,
                          const float *kscales, const int8_t *vcodes,
                          const float *vscales, int cap, const int32_t *pos0,
                          int B, int S, int H, int Hkv, int D, float *out);
/* LayerNorm::forward (layer.cpp:242-261), eps 1e-5, over rows of d. */
int nnhip_layernorm(nnhip_ctx *ctx, const float *x, int rows, int d,
                    const float *gamma, const float *beta, float *y);
/* get_probs + sample_token (layer.cpp:1410-1498) per row: logits [B][V],
 * u [B]; tok [B]; probs [B][V] or NULL (not written when temperature <= 0).
 * top_k in (0, V) keeps the top_k largest probabilities, top_p in (0, 1)
 * the shortest prefix (descending, ties by lower index) whose sum reaches
 * top_p; both renormalise what is kept (layer.cpp:1447-1489).  Other values
 * leave the row unfiltered. */
int nnhip_sample_rows(nnhip_ctx *ctx, const float *logits, int B, int V,
                      float temperature, int top_k, float top_p,
                      const float *u, int32_t *tok, float *probs);
/* Accept loop + residual resample of generate_speculative (layer.cpp:
 * 1581-1630) for B sequences of k drafted positions, run by the kernels the
 * device loop itself uses: the draft rows' get_probs as the drafting steps
 * form them (layer.cpp:1554), then the verify rows' statistics and the
 * accept / residual kernel.  Target and draft logits [B][k][V], draft ids
 * [B][k], accept uniforms [B][k] (in place of the Philox slots k + j),
 * resample uniforms [B] (slot 2k).  n_accept [B]; next_tok [B] = resampled
 * id, or -1 when all k are accepted (no target row k for a bonus sample).
 * Allocates its scratch on the first call of a (B, k, V) and keeps it in
 * the context for the next such call; returns with the results written. */
int nnhip_spec_accept(nnhip_ctx *ctx, const float *tlogits,
                      const float *dlogits, const int32_t *dtok,
                      const float *u_accept, const float *u_resample, int B,
                      int k, int V, float temperature, int32_t *n_accept,
                      int32_t *next_tok);

/* ---- ExecutionBackend ops (dev buffers, stream-ordered) -------------------
 * The strided fp32 ops of the reference's backend interface
 * (include/backend/backend.hpp:35-220) with CpuBackend's semantics
 * (src/backend/cpu_backend.cpp), so that a HipBackend can run Tensor code
 * unchanged.  An operand is a view: a dev buffer, an element offset, a
 * shape and strides in elements (the reference passes DeviceBuffer, offset,
 * Shape, Strides).  Inputs are right-aligned against the output's shape and
 * their size-1 dimensions broadcast (get_input_offset, cpu_backend.cpp:
 * 69-88).  Errors carry the reference's messages where it has one
 * (cpu_backend.cpp:332-342). */
#define NNHIP_MAX_RANK 8
typedef struct {
  void *data;                      /* dev buffer                          */
  int64_t offset;                  /* elements                            */
  int32_t rank;                    /* 0 .. NNHIP_MAX_RANK                 */
  int64_t shape[NNHIP_MAX_RANK];
  int64_t strides[NNHIP_MAX_RANK]; /* elements                            */
} nnhip_view;
/* binary ops: out = a (op) b */
#define NNHIP_OP_ADD 0
#define NNHIP_OP_SUB 1
#define NNHIP_OP_MUL 2
#define NNHIP_OP_DIV 3
/* backward element-wise ops: grad_in = f(a, grad_out), a the forward input
 * (relu, log) or output (sigmoid, tanh, sqrt), as the *_backward virtuals
 * compute them (cpu_backend.cpp:473-481, 492-502, 513-521, 659-669,
 * 680-690) */
#define NNHIP_OP_RELU_BACKWARD 4
#define NNHIP_OP_SIGMOID_BACKWARD 5
#define NNHIP_OP_TANH_BACKWARD 6
#define NNHIP_OP_SQRT_BACKWARD 7
#define NNHIP_OP_LOG_BACKWARD 8
/* unary ops: out = f(in); log is log(x + 1e-8) as in cpu_backend.cpp:675 */
#define NNHIP_OP_RELU 16
#define NNHIP_OP_SIGMOID 17
#define NNHIP_OP_TANH 18
#define NNHIP_OP_SQRT 19
#define NNHIP_OP_LOG 20
/* ExecutionBackend::add / sub / mul / div (backend.hpp:35-61) and the
 * element-wise *_backward virtuals (:78-183): out = a (op) b. */
int nnhip_binary_f32(nnhip_ctx *ctx, int op, const nnhip_view *a,
                     const nnhip_view *b, const nnhip_view *out);
/* ExecutionBackend::relu / sigmoid / tanh / sqrt / log (backend.hpp:73-166). */
int nnhip_unary_f32(nnhip_ctx *ctx, int op, const nnhip_view *in,
                    const nnhip_view *out);
/* ExecutionBackend::matmul (backend.hpp:63-68, cpu_backend.cpp:326-387):
 * 2-D a [M][K] . b [K][N] -> out [M][N], any strides; each output adds its
 * products in ascending k. */
int nnhip_matmul_f32(nnhip_ctx *ctx, const nnhip_view *a, const nnhip_view *b,
                     const nnhip_view *out);
/* ExecutionBackend::sum (backend.hpp:70-74, cpu_backend.cpp:389-459): sums
 * over `axes`; out has the input's rank (summed dims of extent 1) or that
 * rank minus naxes.  Each output adds its inputs in ascending input index,
 * the reference's order. */
int nnhip_sum_f32(nnhip_ctx *ctx, const nnhip_view *in, const nnhip_view *out,
                  const int64_t *axes, int naxes);
/* ExecutionBackend::softmax (backend.hpp:117-121, cpu_backend.cpp:523-583):
 * exp(x - max) / sum along `axis`. */
int nnhip_softmax_f32(nnhip_ctx *ctx, const nnhip_view *in,
                      const nnhip_view *out, int axis);
/* ExecutionBackend::softmax_backward (backend.hpp:123-130, cpu_backend.cpp:
 * 586-638): dx = y * (dy - sum(dy * y)) along `axis`. */
int nnhip_softmax_backward_f32(nnhip_ctx *ctx, const nnhip_view *y,
                               const nnhip_view *dy, const nnhip_view *dx,
                               int axis);
/* ExecutionBackend::embedding (backend.hpp:199-206, cpu_backend.cpp:
 * 998-1033): weight [V][D], indices [N][T] holding fp32 ids, out [N][T][D];
 * an id outside [0, V) takes row 0. */
int nnhip_embedding_f32(nnhip_ctx *ctx, const nnhip_view *weight,
                        const nnhip_view *indices, const nnhip_view *out);
/* ExecutionBackend::slice_backward (backend.hpp:215-219, cpu_backend.cpp:
 * 1082-1120): grad_parent[..., index along axis, ...] += grad_slice. */
int nnhip_slice_backward_f32(nnhip_ctx *ctx, const nnhip_view *grad_slice,
                             const nnhip_view *grad_parent, int axis,
                             int64_t index);
/* ExecutionBackend::fill (backend.hpp:33, cpu_backend.cpp:49-67): count
 * fp32 values of dev set to value. */
int nnhip_fill_f32(nnhip_ctx *ctx, void *dev, size_t count, float value);

/* ---- microbenchmarks -------------------------------------------------------
 * Time one kernel on the context's stream with HIP events (one untimed
 * launch first), rotating over nbuf device-generated input sets; *ms is the
 * mean per launch.  No counterpart in the reference (it has no benchmarks);
 * they time the verify-step attention and acceptance-sampling steps and the
 * W8A32 Linear of the decode path in isolation. */
/* Verify attention over n_cached + S keys; quantized != 0 reads an int8
 * cache (codes and per-row scales). */
int nnhip_bench_attention(nnhip_ctx *ctx, int B, int S, int H, int D,
                          int n_cached, int iters, int nbuf, int quantized,
                          float *ms);
/* n_accept (host [B] or NULL): accepted counts on input set 0. */
int nnhip_bench_spec_accept(nnhip_ctx *ctx, int B, int k, int V,
                            float temperature, int iters, int nbuf, float *ms,
                            int32_t *n_accept);
/* path 1 = fp32 GEMV, 2 = int8-digit MFMA GEMM (digit split included),
 * 3 = LDS GEMM digitising fp32 rows, 4 = LDS GEMM over digit planes (their
 * digit split included), 5 = LDS GEMM with LayerNorm in its prologue,
 * 6 = LDS GEMM over digit planes made once, with the lm head's tile
 * softmax statistics (K of 512 or 1024); the GEMM alone over digit planes
 * made once: 7 = LDS GEMM, 8 = digit-plane GEMM, 9 = digit-plane GEMM with
 * one exponent per 64-wide K chunk (the output projection's; K <= 2048). */
int nnhip_bench_linear(nnhip_ctx *ctx, int rows, int K, int N, int path,
                       int iters, int nbuf, float *ms);
/* One TransformerDecoder::forward (layer.cpp:1159-1216) of m over B
 * sequences x S new tokens after n_cached cached positions (zeros), logits
 * of every row written -- the speculative loop's verify step at S = k + 1
 * -- replayed as a captured HIP graph; ms = milliseconds per forward.
 * quantized != 0: int8 KV cache. */
int nnhip_bench_forward(nnhip_model *m, int B, int S, int n_cached,
                        int quantized, int iters, float *ms);

#ifdef __cplusplus
}
#endif
#endif

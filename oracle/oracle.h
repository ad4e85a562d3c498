/*
 * oracle.h -- CPU restatement of the reference's speculative-decoding path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product (libnnhip.so).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product never links it.
 *
 * Every function restates the arithmetic of islhkafaa/neural-network's CPU
 * backend path in plain C, in the same fp32 operation order where the
 * reference fixes one (file:line citations at each definition in oracle.c).
 * Compiled with -ffp-contract=off so that no multiply-add is fused, as in
 * the reference's x86-64 build.
 *
 * Uniform source: the reference draws from std::mt19937 through libstdc++
 * distributions.  The oracle and the device path instead share one
 * counter-based Philox4x32-10 stream, addressed as u[seq][cycle][slot]:
 *   slots 0..k-1   draft sampling of step j
 *   slots k..2k-1  accept test of position j
 *   slot  2k       residual resample or bonus sample
 *   cycle 0, slot 2k: the first token after prefill.
 * generate_advanced's sampled mode uses u[seq][step][0].
 */
#ifndef NN_ORACLE_H
#define NN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct or_model or_model;
typedef struct or_cache or_cache;

typedef struct {
  int64_t cycles;       /* speculative cycles run after the first token */
  int64_t drafted;      /* sum of M over cycles */
  int64_t accepted;     /* accepted draft tokens */
  int64_t ties;         /* accept tests with |r - p/q| < 1e-6 */
  int64_t resampled;    /* cycles that ended in a residual resample */
  int64_t bonus;        /* cycles that ended in a bonus sample */
  double prefill_ms;    /* prompt forwards and first token (CLOCK_MONOTONIC) */
  double decode_ms;     /* the cycle loop */
} or_spec_stats;

/* Philox4x32-10 (Salmon et al., SC'11), the counter-based generator shared
 * with the device path. */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2],
                      uint32_t out[4]);
/* u[seq][cycle][slot] in [0,1): the top 24 bits of word 0, times 2^-24. */
float or_uniform(uint64_t seed, uint32_t seq, uint32_t cycle, uint32_t slot);

/* std::mt19937 (Matsumoto & Nishimura 1998, the parameters of C++
 * [rand.predef]) and the two draws generate_speculative and
 * generate_advanced take from it (layer.cpp:1249, 1394, 1493-1498,
 * 1596-1597) as libstdc++ forms them: uniform_real_distribution<float>(0, 1)
 * = generate_canonical<float, 24> (one output), and discrete_distribution's
 * generate_canonical<double, 53> (two outputs). */
typedef struct {
  uint32_t mt[624];
  int idx;
} or_mt;
void or_mt_seed(or_mt *g, uint32_t seed);
uint32_t or_mt_next(or_mt *g);
float or_mt_float(or_mt *g);
double or_mt_double(or_mt *g);
/* Uniform source of or_generate_speculative / or_generate_advanced:
 * 0 = Philox slots u[seq][cycle][slot] (the default), 1 = the reference's
 * sequential std::mt19937 stream seeded with (uint32)(seed + seq), draws in
 * the reference's order (first token, each draft sample, each accept test
 * up to the first rejection, the resample or bonus).  Greedy runs draw
 * nothing (every distribution they sample is one-hot). */
void or_set_rng(int mode);

/* Model: TransformerDecoder(vocab, d, heads, d_ff, layers, max_seq_len). */
or_model *or_model_create(int vocab, int d_model, int n_heads, int d_ff,
                          int n_layers, int max_seq_len);
void or_model_free(or_model *m);
int or_model_num_params(const or_model *m);
/* Shape of parameter idx in TransformerDecoder::parameters() order. */
int or_model_param_shape(const or_model *m, int idx, int64_t *rows,
                         int64_t *cols);
int or_model_set_param(or_model *m, int idx, const float *data);
/* Layer::save_weights / load_weights (layer.cpp:463-470) over parameters():
 * the NETW v1 file of serialization.cpp:8-109.  save: 0 or -1 (file).
 * load: 0; -1 open; -2 signature; -3 version; -4 tensor count; -5 rank;
 * -6 extent; -7 element count; -8 short read. */
int or_model_save_weights(const or_model *m, const char *path);
int or_model_load_weights(or_model *m, const char *path);
/* Quantise every Dense (q,k,v,o,gate,up,down,lm_head) to symmetric int8
 * per output channel; the embedding stays fp32. */
int or_model_quantize(or_model *m);
/* The same with INT4 codes (bits 4: scale = max|w| / 7, codes clamped to
 * +-7, quantization.cpp:38-86) or INT8 (bits 8); -1 for other widths. */
int or_model_quantize_bits(or_model *m, int bits);
/* Read back int8 codes ([in,out] reference layout) and scales of a Dense.
 * which: 0..6 = q,k,v,o,gate,up,down of layer `layer`; 7 = lm_head. */
int or_model_get_quantized(const or_model *m, int layer, int which,
                           int8_t *codes, float *scales);

or_cache *or_cache_create(const or_model *m);
/* KVCache(quantized): quantized != 0 keeps int8 codes and per-(head,
 * position) scales instead of fp32 rows. */
or_cache *or_cache_create_q(const or_model *m, int quantized);
void or_cache_free(or_cache *c);
/* Codes [H][len][D] and scales [H][len] of one layer of an int8 cache. */
int or_cache_read_q8(const or_cache *c, int layer, int8_t *kq, float *ks,
                     int8_t *vq, float *vs);
/* Checker hooks of an int8 cache (no counterpart in the reference):
 * the fp32 rows [H][len][D] that were quantised; codes / scales written
 * into positions [0, len) of one layer; the length set directly; and
 * freeze: while set, a forward leaves the codes already stored at its new
 * positions in place (so that a forward can be recomputed on codes taken
 * from elsewhere). */
int or_cache_read_raw(const or_cache *c, int layer, float *kraw, float *vraw);
int or_cache_write_q8(or_cache *c, int layer, int len, const int8_t *kq,
                      const float *ks, const int8_t *vq, const float *vs);
void or_cache_set_len(or_cache *c, int len);
void or_cache_freeze(or_cache *c, int frozen);
int or_cache_len(const or_cache *c);
void or_cache_truncate(or_cache *c, int len);

/* TransformerDecoder::forward for one sequence of S ids; logits [S][V].
 * cache may be NULL.  Returns 0, or -1 when S_past + S > max_seq_len with
 * no cache or an fp32 one; an int8 cache is not checked and grows
 * (layer.cpp:1171-1179 reads the length from caches[0].k, which an int8
 * cache leaves null). */
int or_forward(const or_model *m, or_cache *cache, const int32_t *ids, int S,
               float *logits);

/* Unit restatements used by kernel-level parity tests. */
void or_quantize_w8(const float *w, int64_t in, int64_t out, int8_t *codes,
                    float *scales);
/* QuantizedDense ctor for INT8 (bits 8) or INT4 (bits 4), codes [in][out]
 * one per byte. */
void or_quantize_w(const float *w, int64_t in, int64_t out, int bits,
                   int8_t *codes, float *scales);
/* INT4 codes <-> QuantizedDense::packed_weights (low nibble = even flat
 * index, sign-extended on unpacking). */
void or_pack_int4(const int8_t *codes, int64_t n, uint8_t *packed);
void or_unpack_int4(const uint8_t *packed, int64_t n, int8_t *codes);
void or_dense(const float *x, int64_t rows, int64_t in, int64_t out,
              const float *w, const int8_t *codes, const float *scales,
              const float *bias, float *y);
void or_rope(float *x, int64_t heads, int64_t S, int64_t D, int64_t s_past);
void or_layernorm(const float *x, int64_t rows, int64_t n, const float *gamma,
                  const float *beta, float eps, float *y);
/* Fused attention for one sequence: q [H][S][D] (already rotated),
 * k/v [H_kv][S_total][D] (cache after append), out [S][H][D]. */
void or_attention(const float *q, const float *k, const float *v, int64_t H,
                  int64_t H_kv, int64_t S, int64_t S_total, int64_t D,
                  int causal, float *out);
/* quantize_kv (layer.cpp:635-657): codes [rows][D], scales [rows]. */
void or_quantize_kv(const float *src, int64_t rows, int64_t D, int8_t *codes,
                    float *scales);
/* or_attention over an int8 cache: kq / vq [H_kv][S_total][D] codes,
 * ks / vs [H_kv][S_total] scales. */
void or_attention_q8(const float *q, const int8_t *kq, const float *ks,
                     const int8_t *vq, const float *vs, int64_t H,
                     int64_t H_kv, int64_t S, int64_t S_total, int64_t D,
                     int causal, float *out);

/* get_probs and sample_token of generate_speculative. */
void or_get_probs(const float *logits, int V, float temperature, int top_k,
                  float top_p, float *probs);
int or_sample(const float *probs, int V, double u);
int or_argmax(const float *x, int V);

/* Accept loop, residual resample and bonus of one cycle (see oracle.c). */
int or_accept_step(const float *p, const float *q, const int32_t *cand, int M,
                   int V, int greedy, int has_bonus, const float *u_accept,
                   float u_final, int *tok, int64_t *ties);
/* generate_speculative for one sequence; out receives P + max_new ids. */
int or_generate_speculative(const or_model *target, const or_model *draft,
                            const int32_t *prompt, int P, int max_new,
                            int lookahead, float temperature, int top_k,
                            float top_p, uint64_t seed, int quantized_cache,
                            uint32_t seq_index, int32_t *out,
                            or_spec_stats *stats);
/* Checker hook (not restated reference behaviour): when set, every cycle of
 * or_generate_speculative is recorded here, so that a test can compare the
 * draft logits of each drafting step with a no-cache forward of the token
 * sequence the reference's draft cache holds at that step
 * (layer.cpp:1541-1545, 1632-1653).  Arrays hold max_cycles cycles of
 * lookahead k and vocabulary V; cycles beyond max_cycles are not recorded. */
typedef struct {
  int max_cycles, k, V;
  int n;             /* cycles recorded */
  float *dlogits;    /* [max_cycles][k][V] draft logits of drafting step j */
  int32_t *cand;     /* [max_cycles][k] drafted candidates */
  int32_t *M;        /* [max_cycles] drafted this cycle */
  int32_t *acc;      /* [max_cycles] accepted drafts */
  int32_t *tok;      /* [max_cycles] resampled / bonus token, -1 if none */
  int32_t *dstart;   /* [max_cycles] draft cache length at cycle start */
  int32_t *tstart;   /* [max_cycles] target cache length at cycle start */
  double *margin;    /* [max_cycles] smallest distance of a random decision
                      * from its boundary: |r - p/q| of the accept tests,
                      * |u - cdf edge| of the draws */
  double first_margin;  /* the same for the first token's draw */
} or_spec_trace;
void or_set_spec_trace(or_spec_trace *trace);  /* NULL: recording off */
/* The smallest decision margin (as in or_spec_trace) of the random
 * decisions made since the last reset, e.g. by one or_accept_step; reset
 * != 0 starts a new record. */
double or_decision_margin(int reset);

/* Threads of the oracle's Dense products and attention heads (default 1).
 * Each output element keeps its single-thread summation order, so results
 * do not depend on the count. */
void or_set_threads(int n);

/* generate_advanced for one sequence; out receives P + max_new ids. */
int or_generate_advanced(const or_model *m, const int32_t *prompt, int P,
                         int max_new, float temperature, int top_k,
                         float top_p, uint64_t seed, uint32_t seq_index,
                         int use_kv_cache, int32_t *out);

#ifdef __cplusplus
}
#endif
#endif

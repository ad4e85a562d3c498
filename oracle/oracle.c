/*
 * oracle.c -- CPU restatement of islhkafaa/neural-network's speculative
 * decoding path (TEST INFRASTRUCTURE: the checker for libnnhip.so; the
 * product never links it).  Citations are file:line in the reference tree.
 *
 * Scope: TransformerDecoder forward with fp32 or W8A32 Dense layers, fp32
 * KV cache, RoPE, post-LN, SwiGLU, the fused attention arithmetic order,
 * get_probs / sample_token, the accept / residual / bonus logic and cache
 * rollback of generate_speculative, and generate_advanced.
 */
#define _POSIX_C_SOURCE 199309L
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <time.h>
#include <stdlib.h>
#include <string.h>

/* threads of the Dense products and attention heads (or_set_threads) */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n > 0 ? n : 1; }

/* ------------------------------------------------------------------ */
/* Philox4x32-10 (Random123 paper, Salmon et al. 2011).                */
/* ------------------------------------------------------------------ */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2],
                      uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float or_uniform(uint64_t seed, uint32_t seq, uint32_t cycle, uint32_t slot) {
  uint32_t ctr[4] = {slot, cycle, seq, 0u};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t o[4];
  or_philox4x32_10(ctr, key, o);
  return (float)(o[0] >> 8) * (1.0f / 16777216.0f);
}

/* std::mt19937: 624-word state, recurrence over words i, i + 1, i + 397,
 * matrix 0x9908b0df, tempering (11, 7 / 0x9d2c5680, 15 / 0xefc60000, 18);
 * seeding x_i = 1812433253 (x_{i-1} ^ (x_{i-1} >> 30)) + i. */
void or_mt_seed(or_mt *g, uint32_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < 624; ++i)
    g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
  g->idx = 624;
}

static void mt_twist(or_mt *g) {
  for (int i = 0; i < 624; ++i) {
    const uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
    g->mt[i] = g->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
  }
  g->idx = 0;
}

uint32_t or_mt_next(or_mt *g) {
  if (g->idx >= 624) mt_twist(g);
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* generate_canonical<float, 24>: one output, (float)x / 2^32, kept below 1 */
float or_mt_float(or_mt *g) {
  const float s = (float)or_mt_next(g);
  float r = s / 4294967296.0f;
  if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
  return r;
}

/* generate_canonical<double, 53>: two outputs x0 + x1 2^32 summed in double,
 * over 2^64, kept below 1 */
double or_mt_double(or_mt *g) {
  double s = (double)or_mt_next(g);
  s += (double)or_mt_next(g) * 4294967296.0;
  double r = s / 18446744073709551616.0;
  if (r >= 1.0) r = nextafter(1.0, 0.0);
  return r;
}

static int g_rng = 0;
void or_set_rng(int mode) { g_rng = mode; }

/* ------------------------------------------------------------------ */
/* Model                                                               */
/* ------------------------------------------------------------------ */
typedef struct {
  int64_t in, out;
  float *w;        /* [in][out] fp32, Dense::weight_ (layer.cpp:151-160) */
  float *b;        /* [out] */
  int8_t *codes;   /* [in][out] int8 after quantisation */
  float *scales;   /* [out] */
} or_dense_t;

typedef struct {
  or_dense_t q, k, v, o, gate, up, down;
  float *g1, *b1, *g2, *b2;
} or_layer_t;

struct or_model {
  int vocab, d, H, F, L, max_seq;
  float *emb;               /* [vocab][d] */
  or_layer_t *layers;
  or_dense_t lm;
};

struct or_cache {
  int L, H, D, cap, len;
  int quantized;            /* KVCache(quantized) (layer.hpp:223) */
  float *k, *v;             /* fp32 cache: [L][H][cap][D] */
  int8_t *kq, *vq;          /* int8 cache: codes [L][H][cap][D] */
  float *ks, *vs;           /*             scales [L][H][cap] */
  /* checker state of an int8 cache (no counterpart in the reference):
   * the rows as they were before quantisation, and `frozen`, under which an
   * append leaves the codes already stored at the new positions in place */
  float *kraw, *vraw;       /* [L][H][cap][D] */
  int frozen;
};

static void dense_init(or_dense_t *dn, int64_t in, int64_t out) {
  dn->in = in; dn->out = out;
  dn->w = (float *)calloc((size_t)(in * out), sizeof(float));
  dn->b = (float *)calloc((size_t)out, sizeof(float));
  dn->codes = NULL; dn->scales = NULL;
}
static void dense_free(or_dense_t *dn) {
  free(dn->w); free(dn->b); free(dn->codes); free(dn->scales);
}

or_model *or_model_create(int vocab, int d, int H, int F, int L, int max_seq) {
  if (vocab <= 0 || d <= 0 || H <= 0 || d % H != 0 || F <= 0 || L <= 0)
    return NULL;
  or_model *m = (or_model *)calloc(1, sizeof(or_model));
  m->vocab = vocab; m->d = d; m->H = H; m->F = F; m->L = L;
  m->max_seq = max_seq;
  m->emb = (float *)calloc((size_t)vocab * d, sizeof(float));
  m->layers = (or_layer_t *)calloc((size_t)L, sizeof(or_layer_t));
  for (int l = 0; l < L; ++l) {
    or_layer_t *ly = &m->layers[l];
    dense_init(&ly->q, d, d); dense_init(&ly->k, d, d);
    dense_init(&ly->v, d, d); dense_init(&ly->o, d, d);
    dense_init(&ly->gate, d, F); dense_init(&ly->up, d, F);
    dense_init(&ly->down, F, d);
    ly->g1 = (float *)malloc(sizeof(float) * d);
    ly->b1 = (float *)calloc((size_t)d, sizeof(float));
    ly->g2 = (float *)malloc(sizeof(float) * d);
    ly->b2 = (float *)calloc((size_t)d, sizeof(float));
    for (int i = 0; i < d; ++i) { ly->g1[i] = 1.0f; ly->g2[i] = 1.0f; }
  }
  dense_init(&m->lm, d, vocab);
  return m;
}

void or_model_free(or_model *m) {
  if (!m) return;
  for (int l = 0; l < m->L; ++l) {
    or_layer_t *ly = &m->layers[l];
    dense_free(&ly->q); dense_free(&ly->k); dense_free(&ly->v);
    dense_free(&ly->o); dense_free(&ly->gate); dense_free(&ly->up);
    dense_free(&ly->down);
    free(ly->g1); free(ly->b1); free(ly->g2); free(ly->b2);
  }
  free(m->layers); free(m->emb); dense_free(&m->lm); free(m);
}

/* TransformerDecoder::parameters() order (layer.cpp:1140-1154): token_emb;
 * per layer MHA q,k,v,o (w,b each, layer.cpp:491-502), SwiGLU gate,up,down
 * (layer.cpp:1712-1721), LN1 gamma,beta, LN2 gamma,beta (layer.cpp:
 * 1079-1090); lm_head w,b. */
int or_model_num_params(const or_model *m) { return 1 + 18 * m->L + 2; }

static float *param_ptr(const or_model *m, int idx, int64_t *rows,
                        int64_t *cols) {
  if (idx == 0) { *rows = m->vocab; *cols = m->d; return m->emb; }
  int last = 1 + 18 * m->L;
  if (idx == last) { *rows = m->d; *cols = m->vocab; return m->lm.w; }
  if (idx == last + 1) { *rows = 1; *cols = m->vocab; return m->lm.b; }
  if (idx < 0 || idx > last + 1) return NULL;
  int l = (idx - 1) / 18, j = (idx - 1) % 18;
  or_layer_t *ly = &m->layers[l];
  or_dense_t *dn[7] = {&ly->q, &ly->k, &ly->v, &ly->o, &ly->gate, &ly->up,
                       &ly->down};
  if (j < 14) {
    or_dense_t *x = dn[j / 2];
    if (j % 2 == 0) { *rows = x->in; *cols = x->out; return x->w; }
    *rows = 1; *cols = x->out; return x->b;
  }
  *rows = 1; *cols = m->d;
  float *ln[4] = {ly->g1, ly->b1, ly->g2, ly->b2};
  return ln[j - 14];
}

int or_model_param_shape(const or_model *m, int idx, int64_t *rows,
                         int64_t *cols) {
  return param_ptr(m, idx, rows, cols) ? 0 : -1;
}

int or_model_set_param(or_model *m, int idx, const float *data) {
  int64_t r, c;
  float *p = param_ptr(m, idx, &r, &c);
  if (!p) return -1;
  memcpy(p, data, sizeof(float) * (size_t)(r * c));
  return 0;
}

/* QuantizedDense ctor, INT8 branch (quantization.cpp:36-66): per output
 * column c, s_c = max_r |W[r,c]| / 127 (1 if 0); code = clamp(round(W/s),
 * -127, 127) with round-half-away-from-zero. */
void or_quantize_w(const float *w, int64_t in, int64_t out, int bits,
                   int8_t *codes, float *scales) {
  const float max_q = bits == 4 ? 7.0f : 127.0f;
  for (int64_t c = 0; c < out; ++c) {
    float mx = 0.0f;
    for (int64_t r = 0; r < in; ++r) {
      float a = fabsf(w[r * out + c]);
      if (a > mx) mx = a;
    }
    float s = mx / max_q;
    scales[c] = (s == 0.0f) ? 1.0f : s;
  }
  for (int64_t r = 0; r < in; ++r)
    for (int64_t c = 0; c < out; ++c) {
      float qf = roundf(w[r * out + c] / scales[c]);
      qf = fmaxf(-max_q, fminf(max_q, qf));
      codes[r * out + c] = (int8_t)qf;
    }
}

void or_quantize_w8(const float *w, int64_t in, int64_t out, int8_t *codes,
                    float *scales) {
  or_quantize_w(w, in, out, 8, codes, scales);
}

/* INT4 packing of QuantizedDense (quantization.cpp:68-86): two codes a
 * byte, the even flat index in the low nibble. */
void or_pack_int4(const int8_t *codes, int64_t n, uint8_t *packed) {
  for (int64_t i = 0; i < (n + 1) / 2; ++i) packed[i] = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint8_t v = (uint8_t)codes[i] & 0x0F;
    if (i % 2 == 0) packed[i / 2] = v;
    else packed[i / 2] |= (uint8_t)(v << 4);
  }
}

/* dequantize_weight's unpacking (quantization.cpp:106-122): a nibble with
 * bit 3 set is negative (sign-extended). */
void or_unpack_int4(const uint8_t *packed, int64_t n, int8_t *codes) {
  for (int64_t i = 0; i < n; ++i) {
    uint8_t b = i % 2 == 0 ? (packed[i / 2] & 0x0F) : ((packed[i / 2] >> 4) & 0x0F);
    codes[i] = (b & 0x08) ? (int8_t)(b | 0xF0) : (int8_t)b;
  }
}

/* The codes are kept one per byte: dequantize_weight gives the INT4 codes
 * the same values (code * scale) as INT8 codes, so the forward is shared. */
static void dense_quantize(or_dense_t *dn, int bits) {
  free(dn->codes); free(dn->scales);
  dn->codes = (int8_t *)malloc((size_t)(dn->in * dn->out));
  dn->scales = (float *)malloc(sizeof(float) * (size_t)dn->out);
  or_quantize_w(dn->w, dn->in, dn->out, bits, dn->codes, dn->scales);
}

int or_model_quantize_bits(or_model *m, int bits) {
  if (bits != 8 && bits != 4) return -1;
  for (int l = 0; l < m->L; ++l) {
    or_layer_t *ly = &m->layers[l];
    dense_quantize(&ly->q, bits); dense_quantize(&ly->k, bits);
    dense_quantize(&ly->v, bits); dense_quantize(&ly->o, bits);
    dense_quantize(&ly->gate, bits); dense_quantize(&ly->up, bits);
    dense_quantize(&ly->down, bits);
  }
  dense_quantize(&m->lm, bits);
  return 0;
}

int or_model_quantize(or_model *m) { return or_model_quantize_bits(m, 8); }

int or_model_get_quantized(const or_model *m, int layer, int which,
                           int8_t *codes, float *scales) {
  const or_dense_t *dn;
  if (which == 7) dn = &m->lm;
  else {
    if (layer < 0 || layer >= m->L || which < 0 || which > 6) return -1;
    const or_layer_t *ly = &m->layers[layer];
    const or_dense_t *all[7] = {&ly->q, &ly->k, &ly->v, &ly->o, &ly->gate,
                                &ly->up, &ly->down};
    dn = all[which];
  }
  if (!dn->codes) return -1;
  memcpy(codes, dn->codes, (size_t)(dn->in * dn->out));
  memcpy(scales, dn->scales, sizeof(float) * (size_t)dn->out);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Ops                                                                 */
/* ------------------------------------------------------------------ */

/* Dense::forward (layer.cpp:162-171) and QuantizedDense::forward
 * (quantization.cpp:127-147): y = x . W + b, W [in][out]; the quantised
 * weight is dequantised to fp32 q*s (quantization.cpp:97-105) before the
 * product.  Each output accumulates in fp32 in ascending k (the sgemm
 * order of cpu_backend.cpp:366 is not fixed by the reference; this is the
 * naive-loop order of cpu_backend.cpp:374-385). */
void or_dense(const float *x, int64_t rows, int64_t in, int64_t out,
              const float *w, const int8_t *codes, const float *scales,
              const float *bias, float *y) {
  /* column blocks are independent tasks; within a block the loop order is
   * the single-thread one, so every output keeps its summation order */
  enum { NB = 512 };
  const int64_t tasks = (out + NB - 1) / NB;
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && tasks > 1)
  for (int64_t t = 0; t < tasks; ++t) {
    const int64_t n0 = t * NB, n1 = out < n0 + NB ? out : n0 + NB;
    float wrow[NB];
    for (int64_t r = 0; r < rows; ++r)
      for (int64_t n = n0; n < n1; ++n) y[r * out + n] = 0.0f;
    for (int64_t k = 0; k < in; ++k) {
      const float *wr;
      if (codes) {
        const int8_t *cr = codes + k * out;
        for (int64_t n = n0; n < n1; ++n) wrow[n - n0] = (float)cr[n] * scales[n];
        wr = wrow - n0;
      } else {
        wr = w + k * out;
      }
      for (int64_t r = 0; r < rows; ++r) {
        float xk = x[r * in + k];
        float *yr = y + r * out;
        for (int64_t n = n0; n < n1; ++n) yr[n] += xk * wr[n];
      }
    }
    if (bias)
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t n = n0; n < n1; ++n) y[r * out + n] = y[r * out + n] + bias[n];
  }
}

static void dense_fwd(const or_dense_t *dn, const float *x, int64_t rows,
                      float *y) {
  or_dense(x, rows, dn->in, dn->out, dn->w, dn->codes, dn->scales, dn->b, y);
}

/* Tensor::rope (tensor.cpp:1141-1173), x [H][S][D] in place. */
void or_rope(float *x, int64_t H, int64_t S, int64_t D, int64_t s_past) {
  for (int64_t h = 0; h < H; ++h)
    for (int64_t s = 0; s < S; ++s) {
      float m = (float)(s_past + s);
      for (int64_t j = 0; j < D / 2; ++j) {
        float theta = powf(10000.0f, -2.0f * (float)j / (float)D);
        float omega = m * theta;
        float c = cosf(omega), sn = sinf(omega);
        float *p = x + (h * S + s) * D + 2 * j;
        float xe = p[0], xo = p[1];
        p[0] = xe * c - xo * sn;
        p[1] = xe * sn + xo * c;
      }
    }
}

/* LayerNorm::forward (layer.cpp:242-261) with the backend sum of
 * cpu_backend.cpp:389-459 (ascending index): mean = sum/N,
 * var = sum((x-mean)^2)/N, y = (x-mean)/sqrt(var+eps)*gamma + beta. */
void or_layernorm(const float *x, int64_t rows, int64_t n, const float *gamma,
                  const float *beta, float eps, float *y) {
  float N = (float)n;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * n;
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += xr[i];
    float mean = s / N;
    float sq = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      float df = xr[i] - mean;
      sq += df * df;
    }
    float var = sq / N;
    float sd = sqrtf(var + eps);
    for (int64_t i = 0; i < n; ++i) {
      float xh = (xr[i] - mean) / sd;
      y[r * n + i] = xh * gamma[i] + beta[i];
    }
  }
}

/* Fused attention of MultiHeadAttention::forward (layer.cpp:842-952):
 * score = dot/sqrt(D); masked positions (j > S_past + i) skip the max and
 * get probability 0; p = exp(s - max) * (1/sum); out[d] = sum_j p_j v_j[d]
 * in ascending j, skipping p == 0. */
void or_attention(const float *q, const float *k, const float *v, int64_t H,
                  int64_t H_kv, int64_t S, int64_t S_total, int64_t D,
                  int causal, float *out) {
  int64_t S_past = S_total - S;
  int64_t group = H / H_kv;
  float scale = sqrtf((float)D);
  /* heads are independent tasks (the reference's ThreadPool splits B*H,
   * layer.cpp:859-948) */
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && H > 1)
  for (int64_t h = 0; h < H; ++h) {
    float *row = (float *)malloc(sizeof(float) * (size_t)S_total);
    int64_t hk = h / group;
    for (int64_t i = 0; i < S; ++i) {
      float mx = -INFINITY;
      const float *qi = q + (h * S + i) * D;
      for (int64_t j = 0; j < S_total; ++j) {
        if (causal && j > S_past + i) { row[j] = -1e9f; continue; }
        const float *kj = k + (hk * S_total + j) * D;
        float dot = 0.0f;
        for (int64_t dd = 0; dd < D; ++dd) dot += qi[dd] * kj[dd];
        float sc = dot / scale;
        row[j] = sc;
        if (sc > mx) mx = sc;
      }
      float sum = 0.0f;
      for (int64_t j = 0; j < S_total; ++j) {
        if (causal && j > S_past + i) { row[j] = 0.0f; continue; }
        float e = expf(row[j] - mx);
        row[j] = e;
        sum += e;
      }
      if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int64_t j = 0; j < S_total; ++j) row[j] *= inv;
      }
      float *o = out + (i * H + h) * D;
      for (int64_t dd = 0; dd < D; ++dd) {
        float acc = 0.0f;
        for (int64_t j = 0; j < S_total; ++j) {
          if (row[j] == 0.0f) continue;
          acc += row[j] * v[(hk * S_total + j) * D + dd];
        }
        o[dd] = acc;
      }
    }
    free(row);
  }
}

/* quantize_kv of MultiHeadAttention::forward (layer.cpp:635-657) over rows
 * of D values: scale = max|x| / 127 (1 when 0), code = clamp(round(x *
 * (1 / scale)), -127, 127), round half away from zero. */
void or_quantize_kv(const float *src, int64_t rows, int64_t D, int8_t *codes,
                    float *scales) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *x = src + r * D;
    float mx = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
      float a = fabsf(x[d]);
      if (a > mx) mx = a;
    }
    float scale = mx / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[r] = scale;
    float inv = 1.0f / scale;
    for (int64_t d = 0; d < D; ++d) {
      float qv = roundf(x[d] * inv);
      qv = fmaxf(-127.0f, fminf(127.0f, qv));
      codes[r * D + d] = (int8_t)qv;
    }
  }
}

/* Fused attention over an int8 cache (layer.cpp:842-952, quantized
 * branches :878-890 and :925-938): every cached element enters as
 * (float)code * scale of its row, in the same products and order as the
 * fp32 path.  kq / vq [H_kv][S_total][D], ks / vs [H_kv][S_total]. */
void or_attention_q8(const float *q, const int8_t *kq, const float *ks,
                     const int8_t *vq, const float *vs, int64_t H,
                     int64_t H_kv, int64_t S, int64_t S_total, int64_t D,
                     int causal, float *out) {
  int64_t S_past = S_total - S;
  int64_t group = H / H_kv;
  float scale = sqrtf((float)D);
  /* heads are independent tasks (the reference's ThreadPool splits B*H,
   * layer.cpp:859-948) */
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && H > 1)
  for (int64_t h = 0; h < H; ++h) {
    float *row = (float *)malloc(sizeof(float) * (size_t)S_total);
    int64_t hk = h / group;
    for (int64_t i = 0; i < S; ++i) {
      float mx = -INFINITY;
      const float *qi = q + (h * S + i) * D;
      for (int64_t j = 0; j < S_total; ++j) {
        if (causal && j > S_past + i) { row[j] = -1e9f; continue; }
        const int8_t *kj = kq + (hk * S_total + j) * D;
        float ksc = ks[hk * S_total + j];
        float dot = 0.0f;
        for (int64_t dd = 0; dd < D; ++dd) dot += qi[dd] * ((float)kj[dd] * ksc);
        float sc = dot / scale;
        row[j] = sc;
        if (sc > mx) mx = sc;
      }
      float sum = 0.0f;
      for (int64_t j = 0; j < S_total; ++j) {
        if (causal && j > S_past + i) { row[j] = 0.0f; continue; }
        float e = expf(row[j] - mx);
        row[j] = e;
        sum += e;
      }
      if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int64_t j = 0; j < S_total; ++j) row[j] *= inv;
      }
      float *o = out + (i * H + h) * D;
      for (int64_t dd = 0; dd < D; ++dd) {
        float acc = 0.0f;
        for (int64_t j = 0; j < S_total; ++j) {
          if (row[j] == 0.0f) continue;
          acc += row[j] * ((float)vq[(hk * S_total + j) * D + dd] *
                           vs[hk * S_total + j]);
        }
        o[dd] = acc;
      }
    }
    free(row);
  }
}

/* ------------------------------------------------------------------ */
/* NETW weight files                                                   */
/* ------------------------------------------------------------------ */
/* The reference's rank of parameters()[idx]: LayerNorm gamma / beta are
 * Shape{embed_dim} (layer.cpp:204-209, 1063-1064); the embedding, Dense
 * weights and biases ([1][out], layer.cpp:153-157) are 2-D. */
static int param_rank(const or_model *m, int idx) {
  int last = 1 + 18 * m->L;
  return (idx >= 1 && idx < last && (idx - 1) % 18 >= 14) ? 1 : 2;
}

/* serialization::save_parameters (serialization.cpp:8-47): "NETW", uint16
 * version 1, uint32 count, per tensor uint32 rank, uint64 extents, uint64
 * element count, fp32 data.  Returns 0, or -1 when the file cannot be
 * written. */
int or_model_save_weights(const or_model *m, const char *path) {
  FILE *f = fopen(path, "wb");
  if (!f) return -1;
  uint16_t version = 1;
  uint32_t count = (uint32_t)or_model_num_params(m);
  fwrite("NETW", 1, 4, f);
  fwrite(&version, sizeof(version), 1, f);
  fwrite(&count, sizeof(count), 1, f);
  for (int i = 0; i < (int)count; ++i) {
    int64_t r = 0, c = 0;
    const float *p = param_ptr(m, i, &r, &c);
    uint32_t rank = (uint32_t)param_rank(m, i);
    uint64_t ext[2] = {(uint64_t)r, (uint64_t)c};
    uint64_t n = (uint64_t)(r * c);
    fwrite(&rank, sizeof(rank), 1, f);
    if (rank == 1) fwrite(&ext[1], sizeof(uint64_t), 1, f);
    else fwrite(ext, sizeof(uint64_t), 2, f);
    fwrite(&n, sizeof(n), 1, f);
    fwrite(p, sizeof(float), (size_t)n, f);
  }
  return fclose(f) == 0 ? 0 : -1;
}

/* serialization::load_parameters (serialization.cpp:49-109).  Returns 0;
 * -1 when the file cannot be opened; -2 bad signature; -3 version; -4
 * tensor count; -5 rank; -6 extent; -7 element count; -8 short read.
 * A quantised model's Dense layers are quantised again from the loaded
 * weights (what quantize_model after load_weights does). */
int or_model_load_weights(or_model *m, const char *path) {
  FILE *f = fopen(path, "rb");
  if (!f) return -1;
  int rc = 0;
  char magic[4];
  uint16_t version = 0;
  uint32_t count = 0;
  float *buf = NULL;
  if (fread(magic, 1, 4, f) != 4 || memcmp(magic, "NETW", 4) != 0) { rc = -2; goto out; }
  if (fread(&version, sizeof(version), 1, f) != 1) { rc = -8; goto out; }
  if (version != 1) { rc = -3; goto out; }
  if (fread(&count, sizeof(count), 1, f) != 1) { rc = -8; goto out; }
  if (count != (uint32_t)or_model_num_params(m)) { rc = -4; goto out; }
  for (int i = 0; i < (int)count; ++i) {
    int64_t r = 0, c = 0;
    float *p = param_ptr(m, i, &r, &c);
    uint32_t rank = 0;
    if (fread(&rank, sizeof(rank), 1, f) != 1) { rc = -8; goto out; }
    if (rank != (uint32_t)param_rank(m, i)) { rc = -5; goto out; }
    uint64_t want[2] = {(uint64_t)r, (uint64_t)c};
    for (uint32_t d = 0; d < rank; ++d) {
      uint64_t e = 0;
      if (fread(&e, sizeof(e), 1, f) != 1) { rc = -8; goto out; }
      if (e != want[2 - rank + d]) { rc = -6; goto out; }
    }
    uint64_t n = 0;
    if (fread(&n, sizeof(n), 1, f) != 1) { rc = -8; goto out; }
    if (n != (uint64_t)(r * c)) { rc = -7; goto out; }
    buf = (float *)realloc(buf, sizeof(float) * (size_t)n);
    if (fread(buf, sizeof(float), (size_t)n, f) != (size_t)n) { rc = -8; goto out; }
    memcpy(p, buf, sizeof(float) * (size_t)n);
  }
  if (m->lm.codes) or_model_quantize(m);
out:
  free(buf);
  fclose(f);
  return rc;
}

/* ------------------------------------------------------------------ */
/* Cache and forward                                                   */
/* ------------------------------------------------------------------ */
or_cache *or_cache_create_q(const or_model *m, int quantized) {
  or_cache *c = (or_cache *)calloc(1, sizeof(or_cache));
  c->L = m->L; c->H = m->H; c->D = m->d / m->H; c->cap = m->max_seq;
  c->quantized = quantized != 0;
  size_t n = (size_t)c->L * c->H * c->cap * c->D;
  if (c->quantized) {
    size_t ns = (size_t)c->L * c->H * c->cap;
    c->kq = (int8_t *)calloc(n, 1);
    c->vq = (int8_t *)calloc(n, 1);
    c->ks = (float *)calloc(ns, sizeof(float));
    c->vs = (float *)calloc(ns, sizeof(float));
    c->kraw = (float *)calloc(n, sizeof(float));
    c->vraw = (float *)calloc(n, sizeof(float));
  } else {
    c->k = (float *)calloc(n, sizeof(float));
    c->v = (float *)calloc(n, sizeof(float));
  }
  c->len = 0;
  return c;
}
or_cache *or_cache_create(const or_model *m) { return or_cache_create_q(m, 0); }

/* An int8 cache grows past max_seq_len, as the reference's does (its
 * quantised vectors have no capacity; see or_forward). */
static void *regrow(void *old, size_t esz, int L, int H, int cap, int ncap,
                    int len, int D) {
  char *nw = (char *)calloc((size_t)L * H * ncap * D, esz);
  for (int l = 0; l < L; ++l)
    for (int h = 0; h < H; ++h)
      memcpy(nw + (((size_t)l * H + h) * ncap) * D * esz,
             (char *)old + (((size_t)l * H + h) * cap) * D * esz,
             (size_t)len * D * esz);
  free(old);
  return nw;
}
static void cache_reserve(or_cache *c, int need) {
  if (need <= c->cap) return;
  int ncap = need > 2 * c->cap ? need : 2 * c->cap;
  c->kq = regrow(c->kq, 1, c->L, c->H, c->cap, ncap, c->len, c->D);
  c->vq = regrow(c->vq, 1, c->L, c->H, c->cap, ncap, c->len, c->D);
  c->ks = regrow(c->ks, sizeof(float), c->L, c->H, c->cap, ncap, c->len, 1);
  c->vs = regrow(c->vs, sizeof(float), c->L, c->H, c->cap, ncap, c->len, 1);
  c->kraw = regrow(c->kraw, sizeof(float), c->L, c->H, c->cap, ncap, c->len, c->D);
  c->vraw = regrow(c->vraw, sizeof(float), c->L, c->H, c->cap, ncap, c->len, c->D);
  c->cap = ncap;
}
void or_cache_free(or_cache *c) {
  if (!c) return;
  free(c->k); free(c->v); free(c->kq); free(c->vq); free(c->ks); free(c->vs);
  free(c->kraw); free(c->vraw);
  free(c);
}
int or_cache_read_raw(const or_cache *c, int layer, float *kraw, float *vraw) {
  if (!c->quantized || layer < 0 || layer >= c->L) return -1;
  for (int h = 0; h < c->H; ++h) {
    size_t src = (((size_t)layer * c->H + h) * c->cap) * c->D;
    size_t dst = (size_t)h * c->len * c->D;
    memcpy(kraw + dst, c->kraw + src, sizeof(float) * (size_t)c->len * c->D);
    memcpy(vraw + dst, c->vraw + src, sizeof(float) * (size_t)c->len * c->D);
  }
  return 0;
}
int or_cache_write_q8(or_cache *c, int layer, int len, const int8_t *kq,
                      const float *ks, const int8_t *vq, const float *vs) {
  if (!c->quantized || layer < 0 || layer >= c->L || len < 0 || len > c->cap)
    return -1;
  for (int h = 0; h < c->H; ++h) {
    size_t dst = ((size_t)layer * c->H + h) * c->cap;
    size_t src = (size_t)h * len;
    memcpy(c->kq + dst * c->D, kq + src * c->D, (size_t)len * c->D);
    memcpy(c->vq + dst * c->D, vq + src * c->D, (size_t)len * c->D);
    memcpy(c->ks + dst, ks + src, sizeof(float) * (size_t)len);
    memcpy(c->vs + dst, vs + src, sizeof(float) * (size_t)len);
  }
  return 0;
}
void or_cache_set_len(or_cache *c, int len) {
  if (len >= 0 && len <= c->cap) c->len = len;
}
void or_cache_freeze(or_cache *c, int frozen) { c->frozen = frozen != 0; }
int or_cache_read_q8(const or_cache *c, int layer, int8_t *kq, float *ks,
                     int8_t *vq, float *vs) {
  if (!c->quantized || layer < 0 || layer >= c->L) return -1;
  for (int h = 0; h < c->H; ++h) {
    size_t src = ((size_t)layer * c->H + h) * c->cap;
    size_t dst = (size_t)h * c->len;
    memcpy(kq + dst * c->D, c->kq + src * c->D, (size_t)c->len * c->D);
    memcpy(vq + dst * c->D, c->vq + src * c->D, (size_t)c->len * c->D);
    memcpy(ks + dst, c->ks + src, sizeof(float) * (size_t)c->len);
    memcpy(vs + dst, c->vs + src, sizeof(float) * (size_t)c->len);
  }
  return 0;
}
int or_cache_len(const or_cache *c) { return c->len; }
/* KVCache::truncate (layer.cpp:67-149): keep the first len positions. */
void or_cache_truncate(or_cache *c, int len) {
  if (len < c->len) c->len = len;
}

/* TransformerDecoder::forward (layer.cpp:1161-1193) for B = 1:
 * embedding gather with out-of-range ids -> row 0 (cpu_backend.cpp:
 * 1020-1025), decoder layers (layer.cpp:1097-1114), lm_head. */
int or_forward(const or_model *m, or_cache *cache, const int32_t *ids, int S,
               float *logits) {
  int d = m->d, H = m->H, D = d / H, F = m->F;
  int S_past = cache ? cache->len : 0;
  /* the reference reads S_past from caches[0].k (layer.cpp:1171-1179),
   * which an int8 cache leaves null: then nothing is checked */
  if (!(cache && cache->quantized) && S_past + S > m->max_seq) return -1;
  if (cache && cache->quantized) cache_reserve(cache, S_past + S);
  int S_total = S_past + S;
  size_t sd = (size_t)S * d;
  float *x = (float *)malloc(sizeof(float) * sd);
  float *q = (float *)malloc(sizeof(float) * sd);
  float *kk = (float *)malloc(sizeof(float) * sd);
  float *vv = (float *)malloc(sizeof(float) * sd);
  float *qh = (float *)malloc(sizeof(float) * sd);
  float *ctx = (float *)malloc(sizeof(float) * sd);
  float *t1 = (float *)malloc(sizeof(float) * sd);
  float *x1 = (float *)malloc(sizeof(float) * sd);
  float *g = (float *)malloc(sizeof(float) * (size_t)S * F);
  float *u = (float *)malloc(sizeof(float) * (size_t)S * F);
  float *kt = NULL, *vt = NULL;
  if (!cache) {
    kt = (float *)malloc(sizeof(float) * sd);
    vt = (float *)malloc(sizeof(float) * sd);
  }
  for (int s = 0; s < S; ++s) {
    int64_t id = ids[s];
    if (id < 0 || id >= m->vocab) id = 0;
    memcpy(x + (size_t)s * d, m->emb + (size_t)id * d, sizeof(float) * d);
  }
  for (int l = 0; l < m->L; ++l) {
    const or_layer_t *ly = &m->layers[l];
    /* MultiHeadAttention::forward (layer.cpp:593-994) */
    dense_fwd(&ly->q, x, S, q);
    dense_fwd(&ly->k, x, S, kk);
    dense_fwd(&ly->v, x, S, vv);
    /* [S][H][D] -> [H][S][D] (transpose(1,2), layer.cpp:619-621) */
    float *kh = cache ? (float *)malloc(sizeof(float) * sd) : kt;
    float *vh = cache ? (float *)malloc(sizeof(float) * sd) : vt;
    for (int h = 0; h < H; ++h)
      for (int s = 0; s < S; ++s)
        for (int e = 0; e < D; ++e) {
          size_t src = (size_t)s * d + h * D + e;
          size_t dst = ((size_t)h * S + s) * D + e;
          qh[dst] = q[src]; kh[dst] = kk[src]; vh[dst] = vv[src];
        }
    or_rope(qh, H, S, D, S_past);
    or_rope(kh, H, S, D, S_past);
    if (cache && cache->quantized) {
      /* int8 append (layer.cpp:683-757): the new rotated k and v rows are
       * quantised per (head, position), then attention reads the codes */
      size_t lay = (size_t)l * H * cache->cap;
      int8_t *cq = (int8_t *)malloc(sd);
      float *cs = (float *)malloc(sizeof(float) * (size_t)H * S);
      for (int pass = 0; pass < 2; ++pass) {
        const float *src = pass ? vh : kh;
        or_quantize_kv(src, (int64_t)H * S, D, cq, cs);
        int8_t *dq = pass ? cache->vq : cache->kq;
        float *ds = pass ? cache->vs : cache->ks;
        float *dr = pass ? cache->vraw : cache->kraw;
        for (int h = 0; h < H; ++h)
          for (int s = 0; s < S; ++s) {
            size_t dst = lay + (size_t)h * cache->cap + S_past + s;
            memcpy(dr + dst * D, src + ((size_t)h * S + s) * D, sizeof(float) * D);
            if (cache->frozen) continue;
            memcpy(dq + dst * D, cq + ((size_t)h * S + s) * D, (size_t)D);
            ds[dst] = cs[(size_t)h * S + s];
          }
      }
      free(cq); free(cs);
      int8_t *Kq = (int8_t *)malloc((size_t)H * S_total * D);
      int8_t *Vq = (int8_t *)malloc((size_t)H * S_total * D);
      float *Ks = (float *)malloc(sizeof(float) * (size_t)H * S_total);
      float *Vs = (float *)malloc(sizeof(float) * (size_t)H * S_total);
      for (int h = 0; h < H; ++h) {
        size_t src = lay + (size_t)h * cache->cap;
        memcpy(Kq + (size_t)h * S_total * D, cache->kq + src * D, (size_t)S_total * D);
        memcpy(Vq + (size_t)h * S_total * D, cache->vq + src * D, (size_t)S_total * D);
        memcpy(Ks + (size_t)h * S_total, cache->ks + src, sizeof(float) * (size_t)S_total);
        memcpy(Vs + (size_t)h * S_total, cache->vs + src, sizeof(float) * (size_t)S_total);
      }
      or_attention_q8(qh, Kq, Ks, Vq, Vs, H, H, S, S_total, D, 1, ctx);
      free(Kq); free(Vq); free(Ks); free(Vs); free(kh); free(vh);
    } else if (cache) {
      /* KV append (layer.cpp:758-807) */
      size_t lay = (size_t)l * H * cache->cap * D;
      for (int h = 0; h < H; ++h)
        for (int s = 0; s < S; ++s) {
          size_t dst = lay + ((size_t)h * cache->cap + S_past + s) * D;
          memcpy(cache->k + dst, kh + ((size_t)h * S + s) * D,
                 sizeof(float) * D);
          memcpy(cache->v + dst, vh + ((size_t)h * S + s) * D,
                 sizeof(float) * D);
        }
      /* gather the live cache rows of this layer as [H][S_total][D] */
      float *K = (float *)malloc(sizeof(float) * (size_t)H * S_total * D);
      float *V = (float *)malloc(sizeof(float) * (size_t)H * S_total * D);
      for (int h = 0; h < H; ++h) {
        memcpy(K + (size_t)h * S_total * D,
               cache->k + lay + (size_t)h * cache->cap * D,
               sizeof(float) * (size_t)S_total * D);
        memcpy(V + (size_t)h * S_total * D,
               cache->v + lay + (size_t)h * cache->cap * D,
               sizeof(float) * (size_t)S_total * D);
      }
      or_attention(qh, K, V, H, H, S, S_total, D, 1, ctx);
      free(K); free(V); free(kh); free(vh);
    } else {
      or_attention(qh, kh, vh, H, H, S, S, D, 1, ctx);
    }
    dense_fwd(&ly->o, ctx, S, t1);
    /* x1 = LN1(x + attn) (layer.cpp:1102; dropout is identity in eval) */
    for (size_t i = 0; i < sd; ++i) t1[i] = x[i] + t1[i];
    or_layernorm(t1, S, d, ly->g1, ly->b1, 1e-5f, x1);
    /* SwiGLU (layer.cpp:1704-1710): (g * sigmoid(g)) * u -> down;
     * sigmoid = 1/(1+exp(-x)) (cpu_backend.cpp:483-489) */
    dense_fwd(&ly->gate, x1, S, g);
    dense_fwd(&ly->up, x1, S, u);
    for (size_t i = 0; i < (size_t)S * F; ++i) {
      float sg = 1.0f / (1.0f + expf(-g[i]));
      float a = g[i] * sg;
      g[i] = a * u[i];
    }
    dense_fwd(&ly->down, g, S, t1);
    for (size_t i = 0; i < sd; ++i) t1[i] = x1[i] + t1[i];
    or_layernorm(t1, S, d, ly->g2, ly->b2, 1e-5f, x);
  }
  dense_fwd(&m->lm, x, S, logits);
  if (cache) cache->len = S_total;
  free(x); free(q); free(kk); free(vv); free(qh); free(ctx); free(t1);
  free(x1); free(g); free(u); free(kt); free(vt);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Sampling                                                            */
/* ------------------------------------------------------------------ */

/* First index of the maximum (strict >, layer.cpp:1413-1421;
 * std::max_element, layer.cpp:1591-1593). */
int or_argmax(const float *x, int V) {
  int a = 0;
  float mx = x[0];
  for (int v = 1; v < V; ++v)
    if (x[v] > mx) { mx = x[v]; a = v; }
  return a;
}

typedef struct { float p; int i; } or_pi;
static int cmp_desc(const void *a, const void *b) {
  const or_pi *x = (const or_pi *)a, *y = (const or_pi *)b;
  if (x->p > y->p) return -1;
  if (x->p < y->p) return 1;
  return (x->i < y->i) ? -1 : (x->i > y->i);
}

/* get_probs (layer.cpp:1410-1491).  T <= 0: one-hot at the first argmax.
 * Else logits/T, max-subtract, exp, float sum in index order, divide; then
 * sort descending, zero beyond top_k, zero after the cumulative sum first
 * reaches top_p, final_sum in sorted order, divide again.  Ties in the sort
 * are broken by index (std::sort leaves them unspecified; they change
 * nothing unless top_k/top_p cut between equal probabilities). */
void or_get_probs(const float *logits, int V, float T, int top_k, float top_p,
                  float *probs) {
  if (V <= 0) return;
  if (T <= 0.0f) {
    for (int v = 0; v < V; ++v) probs[v] = 0.0f;
    probs[or_argmax(logits, V)] = 1.0f;
    return;
  }
  float *sl = (float *)malloc(sizeof(float) * V);
  for (int v = 0; v < V; ++v) sl[v] = logits[v] / T;
  float mx = sl[0];
  for (int v = 1; v < V; ++v) if (sl[v] > mx) mx = sl[v];
  float sum = 0.0f;
  for (int v = 0; v < V; ++v) { probs[v] = expf(sl[v] - mx); sum += probs[v]; }
  for (int v = 0; v < V; ++v) probs[v] /= sum;
  or_pi *ip = (or_pi *)malloc(sizeof(or_pi) * V);
  for (int v = 0; v < V; ++v) { ip[v].p = probs[v]; ip[v].i = v; }
  qsort(ip, (size_t)V, sizeof(or_pi), cmp_desc);
  if (top_k > 0 && top_k < V)
    for (int i = top_k; i < V; ++i) ip[i].p = 0.0f;
  if (top_p > 0.0f && top_p < 1.0f) {
    float cs = 0.0f;
    int cut = 0;
    for (int i = 0; i < V; ++i) {
      if (cut) ip[i].p = 0.0f;
      else { cs += ip[i].p; if (cs >= top_p) cut = 1; }
    }
  }
  float fs = 0.0f;
  for (int v = 0; v < V; ++v) fs += ip[v].p;
  for (int v = 0; v < V; ++v) probs[v] = 0.0f;
  if (fs <= 0.0f) probs[ip[0].i] = 1.0f;
  else for (int v = 0; v < V; ++v) probs[ip[v].i] = ip[v].p / fs;
  free(ip); free(sl);
}

/* sample_token (layer.cpp:1493-1498) = std::discrete_distribution<size_t>
 * over the probabilities widened to double (libstdc++ random.tcc:
 * normalise by the double sum, partial_sum, last entry forced to 1.0,
 * lower_bound of the uniform): the first v with cdf[v] >= u. */
/* or_sample that also reports how far u lies from the drawn interval's
 * edges [cdf[v-1], cdf[v]] (checker use: a draw whose margin is below the
 * device's rounding may legitimately come out differently there). */
static int sample_margin(const float *probs, int V, double u, double *margin) {
  if (V < 2) { if (margin) *margin = 1.0; return 0; }
  double sum = 0.0;
  for (int v = 0; v < V; ++v) sum += (double)probs[v];
  double c = 0.0, prev = 0.0;
  for (int v = 0; v < V - 1; ++v) {
    c += (double)probs[v] / sum;
    if (c >= u) {
      if (margin) *margin = fmin(c - u, u - prev);
      return v;
    }
    prev = c;
  }
  if (margin) *margin = u - prev;
  return V - 1;
}

int or_sample(const float *probs, int V, double u) {
  return sample_margin(probs, V, u, NULL);
}

/* smallest decision margin of the current cycle (checker record) */
static double g_margin = 1.0;
double or_decision_margin(int reset) {
  double m = g_margin;
  if (reset) g_margin = 1.0;
  return m;
}

/* Draws of the speculative loop: greedy mode (T <= 0) samples only one-hot
 * vectors, where discrete_distribution returns the hot index; the oracle
 * takes it directly and consumes no uniform. */
static int draw(const float *probs, int V, int greedy, uint64_t seed,
                uint32_t seq, uint32_t cycle, uint32_t slot, or_mt *gen) {
  if (greedy) return or_argmax(probs, V);
  double m = 1.0;
  const double u = g_rng ? or_mt_double(gen) : (double)or_uniform(seed, seq, cycle, slot);
  int v = sample_margin(probs, V, u, &m);
  if (m < g_margin) g_margin = m;
  return v;
}

/* The accept loop and its ending (layer.cpp:1581-1630, 1643-1647) over
 * probability rows p [M (+1)][V] (target) and q [M][V] (draft) for the
 * candidates cand[M]: accept j while r_j * q_j[c_j] < p_j[c_j] (greedy: c_j
 * is the first argmax of p_j); at the first rejection r, *tok is drawn with
 * u_final from max(0, p_r - q_r) normalised by its float sum, or from p_r
 * when that sum is <= 0; after full acceptance *tok is drawn from p_M when
 * has_bonus, else -1.  Returns the number of accepted candidates. */
static int accept_step_d(const float *p, const float *q, const int32_t *cand, int M,
                         int V, int greedy, int has_bonus, const float *u_accept,
                         double u_final, int *tok, int64_t *ties);

int or_accept_step(const float *p, const float *q, const int32_t *cand, int M,
                   int V, int greedy, int has_bonus, const float *u_accept,
                   float u_final, int *tok, int64_t *ties) {
  return accept_step_d(p, q, cand, M, V, greedy, has_bonus, u_accept,
                       (double)u_final, tok, ties);
}

/* the number of candidates the accept loop accepts (its decisions only) */
static int accepted_count(const float *p, const float *q, const int32_t *cand,
                          int M, int V, int greedy, const float *u_accept) {
  for (int j = 0; j < M; ++j) {
    const int c = cand[j];
    const float *pj = p + (size_t)j * V, *qj = q + (size_t)j * V;
    const int acc = greedy ? c == or_argmax(pj, V) : u_accept[j] * qj[c] < pj[c];
    if (!acc) return j;
  }
  return M;
}

static int accept_step_d(const float *p, const float *q, const int32_t *cand, int M,
                         int V, int greedy, int has_bonus, const float *u_accept,
                         double u_final, int *tok, int64_t *ties) {
  *tok = -1;
  for (int j = 0; j < M; ++j) {
    int c = cand[j];
    const float *pj = p + (size_t)j * V, *qj = q + (size_t)j * V;
    int acc;
    if (greedy) {
      acc = c == or_argmax(pj, V);
    } else {
      float r = u_accept[j];
      acc = r * qj[c] < pj[c];
      double dist = fabs((double)r - (double)pj[c] / (double)qj[c]);
      if (ties && dist < 1e-6) (*ties)++;
      if (dist < g_margin) g_margin = dist;
    }
    if (acc) continue;
    if (greedy) { *tok = or_argmax(pj, V); return j; }
    float *rec = (float *)malloc(sizeof(float) * V);
    float sr = 0.0f;
    for (int v = 0; v < V; ++v) {
      rec[v] = fmaxf(0.0f, pj[v] - qj[v]);
      sr += rec[v];
    }
    double m = 1.0;
    if (sr <= 0.0f) *tok = sample_margin(pj, V, u_final, &m);
    else {
      for (int v = 0; v < V; ++v) rec[v] /= sr;
      *tok = sample_margin(rec, V, u_final, &m);
    }
    if (m < g_margin) g_margin = m;
    free(rec);
    return j;
  }
  if (has_bonus) {
    const float *pm = p + (size_t)M * V;
    if (greedy) *tok = or_argmax(pm, V);
    else {
      double m = 1.0;
      *tok = sample_margin(pm, V, u_final, &m);
      if (m < g_margin) g_margin = m;
    }
  }
  return M;
}

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

static or_spec_trace *g_trace = NULL;
void or_set_spec_trace(or_spec_trace *trace) { g_trace = trace; }

/* generate_speculative (layer.cpp:1382-1661) for one sequence. */
int or_generate_speculative(const or_model *t, const or_model *dm,
                            const int32_t *prompt, int P, int max_new, int k,
                            float T, int top_k, float top_p, uint64_t seed,
                            int quantized_cache, uint32_t seq, int32_t *out,
                            or_spec_stats *st) {
  int V = t->vocab;
  int greedy = T <= 0.0f;
  if (dm->vocab != V || P <= 0 || k <= 0 || k > 63) return -2;
  or_spec_stats local;
  memset(&local, 0, sizeof(local));
  /* KVCache(quantized_cache) for both models (layer.cpp:1396-1398) */
  or_cache *tc = or_cache_create_q(t, quantized_cache);
  or_cache *dc = or_cache_create_q(dm, quantized_cache);
  float *tl = (float *)malloc(sizeof(float) * (size_t)(P > k + 1 ? P : k + 1) * V);
  float *dl = (float *)malloc(sizeof(float) * (size_t)P * V);
  float *q = (float *)malloc(sizeof(float) * (size_t)k * V);
  float *p = (float *)malloc(sizeof(float) * (size_t)(k + 1) * V);
  float *rec = (float *)malloc(sizeof(float) * V);
  int32_t *cand = (int32_t *)malloc(sizeof(int32_t) * (k + 1));
  int rc = 0;
  int n = 0;
  double t0 = now_ms(), t1 = t0;
  for (int i = 0; i < P; ++i) out[n++] = prompt[i];
  /* prefill (layer.cpp:1400-1408) */
  if (or_forward(t, tc, prompt, P, tl) || or_forward(dm, dc, prompt, P, dl)) {
    rc = -1; goto done;
  }
  or_get_probs(tl + (size_t)(P - 1) * V, V, T, top_k, top_p, p);
  g_margin = 1.0;
  or_mt gen;
  or_mt_seed(&gen, (uint32_t)(seed + seq));
  out[n++] = draw(p, V, greedy, seed, seq, 0, 2 * k, &gen);
  if (g_trace) g_trace->first_margin = g_margin;
  int ngen = 1;
  uint32_t cycle = 0;
  t1 = now_ms();
  while (ngen < max_new) {
    int M = k < max_new - ngen ? k : max_new - ngen;
    ++cycle;
    int tstart = tc->len, dstart = dc->len;
    or_spec_trace *tr = g_trace;
    int tc_i = -1;
    g_margin = 1.0;
    if (tr && tr->n < tr->max_cycles && tr->k == k && tr->V == V) {
      tc_i = tr->n++;
      tr->dstart[tc_i] = dstart;
      tr->tstart[tc_i] = tstart;
      tr->M[tc_i] = M;
    }
    /* draft loop (layer.cpp:1541-1558) */
    for (int j = 0; j < M; ++j) {
      int32_t in = j == 0 ? out[n - 1] : cand[j - 1];
      if (or_forward(dm, dc, &in, 1, dl)) { rc = -1; goto done; }
      if (tc_i >= 0)
        memcpy(tr->dlogits + ((size_t)tc_i * k + j) * V, dl, sizeof(float) * V);
      or_get_probs(dl, V, T, top_k, top_p, q + (size_t)j * V);
      cand[j] = draw(q + (size_t)j * V, V, greedy, seed, seq, cycle, j, &gen);
      if (tc_i >= 0) tr->cand[(size_t)tc_i * k + j] = cand[j];
    }
    /* verify (layer.cpp:1560-1579) */
    int32_t tin[64];
    tin[0] = out[n - 1];
    for (int j = 0; j < M; ++j) tin[j + 1] = cand[j];
    if (or_forward(t, tc, tin, M + 1, tl)) { rc = -1; goto done; }
    for (int i = 0; i <= M; ++i)
      or_get_probs(tl + (size_t)i * V, V, T, top_k, top_p, p + (size_t)i * V);
    /* accept, resample or bonus (layer.cpp:1581-1630, 1643-1647) */
    float ua[64];
    double uf = 0.0;
    const int has_bonus = ngen + M < max_new;
    if (greedy) {
      for (int j = 0; j < M; ++j) ua[j] = 0.0f;
    } else if (g_rng) {
      /* the reference draws r_j only for the tests it makes (up to the
       * first rejection), then the resample or bonus: the tests' uniforms
       * from a copy of the stream, the stream then advanced past the ones
       * used */
      or_mt look = gen;
      for (int j = 0; j < M; ++j) ua[j] = or_mt_float(&look);
      const int a = accepted_count(p, q, cand, M, V, 0, ua);
      for (int j = 0; j < (a < M ? a + 1 : M); ++j) (void)or_mt_next(&gen);
      if (a < M || has_bonus) uf = or_mt_double(&gen);
    } else {
      for (int j = 0; j < M; ++j) ua[j] = or_uniform(seed, seq, cycle, k + j);
      uf = (double)or_uniform(seed, seq, cycle, 2 * k);
    }
    int tok = -1;
    int64_t ties = 0;
    int acc = accept_step_d(p, q, cand, M, V, greedy, has_bonus, ua, uf, &tok, &ties);
    for (int j = 0; j < acc; ++j) out[n++] = cand[j];
    if (tc_i >= 0) {
      tr->acc[tc_i] = acc; tr->tok[tc_i] = tok; tr->margin[tc_i] = g_margin;
    }
    ngen += acc;
    local.accepted += acc;
    local.ties += ties;
    local.cycles++;
    local.drafted += M;
    if (acc < M) {
      int rej = acc;
      out[n++] = tok; ngen++; local.resampled++;
      /* rollback (layer.cpp:1632-1637) and draft catch-up (:1639-1642) */
      or_cache_truncate(tc, tstart + rej + 1);
      or_cache_truncate(dc, dstart + rej + 1);
      if (or_forward(dm, dc, &tok, 1, dl)) { rc = -1; goto done; }
    } else if (tok >= 0) {
      /* bonus sample and draft catch-up (layer.cpp:1643-1655) */
      out[n++] = tok; ngen++; local.bonus++;
      int32_t last = cand[M - 1];
      if (or_forward(dm, dc, &last, 1, dl)) { rc = -1; goto done; }
    }
  }
done:
  local.prefill_ms = t1 - t0;
  local.decode_ms = now_ms() - t1;
  if (st) *st = local;
  or_cache_free(tc); or_cache_free(dc);
  free(tl); free(dl); free(q); free(p); free(rec); free(cand);
  return rc;
}

/* generate_advanced (layer.cpp:1240-1380) for one sequence.  Sampled mode
 * draws u[seq][step][0] (or, with or_set_rng(1), the next double of the
 * sequence's std::mt19937 stream); greedy takes the first argmax. */
int or_generate_advanced(const or_model *m, const int32_t *prompt, int P,
                         int max_new, float T, int top_k, float top_p,
                         uint64_t seed, uint32_t seq, int use_cache,
                         int32_t *out) {
  int V = m->vocab;
  int total = P + max_new;
  for (int i = 0; i < P; ++i) out[i] = prompt[i];
  int n = P;
  or_cache *c = use_cache ? or_cache_create(m) : NULL;
  float *lg = (float *)malloc(sizeof(float) * (size_t)total * V);
  float *pr = (float *)malloc(sizeof(float) * V);
  int rc = 0;
  or_mt gen;
  or_mt_seed(&gen, (uint32_t)(seed + seq));
  for (int step = 0; step < max_new; ++step) {
    int S;
    const int32_t *in;
    if (use_cache && step > 0) { S = 1; in = out + n - 1; }
    else {
      S = n;
      int start = 0;
      if (S > m->max_seq) { start = S - m->max_seq; S = m->max_seq; }
      in = out + start;
    }
    if (or_forward(m, c, in, S, lg)) { rc = -1; break; }
    const float *last = lg + (size_t)(S - 1) * V;
    int tok;
    if (T <= 0.0f) tok = or_argmax(last, V);
    else {
      or_get_probs(last, V, T, top_k, top_p, pr);
      tok = or_sample(pr, V, g_rng ? or_mt_double(&gen)
                                   : (double)or_uniform(seed, seq, (uint32_t)step, 0));
    }
    out[n++] = tok;
  }
  or_cache_free(c);
  free(lg); free(pr);
  return rc;
}

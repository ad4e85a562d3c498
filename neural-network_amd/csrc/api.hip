// extern "C" boundary of libnnhip.so (declared in include/nnhip.h).  Every
// entry point converts exceptions into a status code plus a thread-local
// message, the C form of the reference's std::runtime_error convention.
#include "api_common.hpp"

#include <cmath>
#include <cstring>

namespace {
thread_local std::string g_err;
}  // namespace

void nnhip::set_last_error(const std::string &msg) { g_err = msg; }

using nnhip::guard;

namespace {

#define REQ(cond, msg) NNHIP_REQUIRE((cond), nnhip::kErrArg, (msg))

void set_device(const nnhip_ctx *ctx) {
  NNHIP_CHECK(hipSetDevice(ctx->c.device));
}

// Allocate-and-copy helpers for the host-buffer entry points.
template <typename T>
nnhip::DevBuf<T> upload(hipStream_t st, const T *host, size_t n) {
  nnhip::DevBuf<T> d(n);
  NNHIP_CHECK(hipMemcpyAsync(d.p, host, n * sizeof(T), hipMemcpyHostToDevice, st));
  return d;
}

}  // namespace

extern "C" {

const char *nnhip_last_error(void) { return g_err.c_str(); }

int nnhip_init(int device, nnhip_ctx **out) {
  return guard([&] {
    REQ(out, "nnhip_init: out is NULL");
    int n = 0;
    NNHIP_CHECK(hipGetDeviceCount(&n));
    REQ(device >= 0 && device < n, "nnhip_init: no such device");
    NNHIP_CHECK(hipSetDevice(device));
    nnhip::noalloc_setup(device);
    std::unique_ptr<nnhip_ctx> c(new nnhip_ctx);
    c->c.device = device;
    NNHIP_CHECK(hipStreamCreateWithFlags(&c->c.stream, hipStreamNonBlocking));
    NNHIP_CHECK(hipEventCreate(&c->t0));
    NNHIP_CHECK(hipEventCreate(&c->t1));
    *out = c.release();
  });
}

int nnhip_destroy(nnhip_ctx *ctx) {
  return guard([&] {
    if (!ctx) return;
    set_device(ctx);
    (void)hipStreamSynchronize(ctx->c.stream);
    (void)hipEventDestroy(ctx->t0);
    (void)hipEventDestroy(ctx->t1);
    (void)hipStreamDestroy(ctx->c.stream);
    nnhip::noalloc_release(ctx);
    delete ctx;
  });
}

int nnhip_set_option(nnhip_ctx *ctx, const char *key, int value) {
  return guard([&] {
    REQ(ctx && key, "nnhip_set_option: NULL argument");
    if (std::strcmp(key, "graphs") == 0) ctx->c.use_graphs = value != 0;
    else if (std::strcmp(key, "rng") == 0) {
      REQ(value == 0 || value == 1, "rng must be 0 (Philox) or 1 (mt19937)");
      ctx->c.rng = value;
    }
    else if (std::strcmp(key, "gemm_wide") == 0) nnhip::g_gemm_wide = value;
    else if (std::strcmp(key, "gemv16") == 0) nnhip::g_gemv16 = value != 0;
    else if (std::strcmp(key, "accept_early") == 0) nnhip::g_accept_early = value != 0;
    else if (std::strcmp(key, "accept_split") == 0) nnhip::g_accept_split = value != 0;
    else if (std::strcmp(key, "lds_min_rows") == 0) {
      REQ(value >= 16, "lds_min_rows must be >= 16");
      nnhip::g_lds_min_rows = value;
    }
    else if (std::strcmp(key, "ln_split") == 0) nnhip::g_ln_split = value;
    else if (std::strcmp(key, "attn_short_q") == 0) {
      REQ(value == 1 || value == 2 || value == 4 || value == 8,
          "attn_short_q must be 1, 2, 4 or 8");
      nnhip::g_attn_short_q = value;
    }
    else if (std::strcmp(key, "attn_w4") == 0) {
      REQ(value >= 0 && value <= 2, "attn_w4 must be 0, 1 or 2");
      nnhip::g_attn_w4 = value;
    }
    else if (std::strcmp(key, "gemv_down_rows") == 0) {
      REQ(value >= 0, "gemv_down_rows must be >= 0");
      nnhip::g_gemv_down_rows = value;
    }
    else if (std::strcmp(key, "limb_k8") == 0) {
      REQ(value >= 128, "limb_k8 must be >= 128");
      nnhip::g_limb_k8 = value;
    }
    else if (std::strcmp(key, "o_limb_rows") == 0) {
      REQ(value >= 0, "o_limb_rows must be >= 0");
      nnhip::g_o_limb_rows = value;
    }
    else if (std::strcmp(key, "gemv_ln") == 0) {
      REQ(value >= 0, "gemv_ln must be >= 0");
      nnhip::g_gemv_ln = value;
    }
    else if (std::strcmp(key, "o_head_digits") == 0) nnhip::g_o_head_digits = value != 0;
    else if (std::strcmp(key, "persistent_draft") == 0) nnhip::g_persistent_draft = value != 0;
    else if (std::strcmp(key, "kv_stream") == 0) {
      REQ(value >= 0 && value <= 2, "kv_stream must be 0, 1 or 2");
      nnhip::g_kv_stream = value;
    }
    else if (std::strcmp(key, "attn_waves") == 0) {
      REQ(value >= 64 && value <= (1 << 20), "attn_waves must be in [64, 2^20]");
      nnhip::g_attn_waves = value;
    }
    else throw nnhip::Error(nnhip::kErrArg, std::string("unknown option ") + key);
  });
}

int nnhip_sync(nnhip_ctx *ctx) {
  return guard([&] {
    REQ(ctx, "nnhip_sync: NULL context");
    NNHIP_CHECK(hipStreamSynchronize(ctx->c.stream));
  });
}

int nnhip_malloc(nnhip_ctx *ctx, size_t bytes, void **out) {
  return guard([&] {
    REQ(ctx && out, "nnhip_malloc: NULL argument");
    set_device(ctx);
    *out = nullptr;
    if (bytes) NNHIP_CHECK(hipMalloc(out, bytes));
  });
}

int nnhip_free(nnhip_ctx *ctx, void *p) {
  return guard([&] {
    REQ(ctx, "nnhip_free: NULL context");
    if (p) {
      NNHIP_CHECK(hipStreamSynchronize(ctx->c.stream));
      NNHIP_CHECK(hipFree(p));
    }
  });
}

int nnhip_h2d(nnhip_ctx *ctx, void *dst, const void *src, size_t bytes) {
  return guard([&] {
    REQ(ctx && (bytes == 0 || (dst && src)), "nnhip_h2d: NULL argument");
    NNHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->c.stream));
    NNHIP_CHECK(hipStreamSynchronize(ctx->c.stream));
  });
}

int nnhip_d2h(nnhip_ctx *ctx, void *dst, const void *src, size_t bytes) {
  return guard([&] {
    REQ(ctx && (bytes == 0 || (dst && src)), "nnhip_d2h: NULL argument");
    NNHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->c.stream));
    NNHIP_CHECK(hipStreamSynchronize(ctx->c.stream));
  });
}

int nnhip_timer_begin(nnhip_ctx *ctx) {
  return guard([&] {
    REQ(ctx, "nnhip_timer_begin: NULL context");
    NNHIP_CHECK(hipEventRecord(ctx->t0, ctx->c.stream));
  });
}

int nnhip_timer_end(nnhip_ctx *ctx, float *ms) {
  return guard([&] {
    REQ(ctx && ms, "nnhip_timer_end: NULL argument");
    NNHIP_CHECK(hipEventRecord(ctx->t1, ctx->c.stream));
    NNHIP_CHECK(hipEventSynchronize(ctx->t1));
    NNHIP_CHECK(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
  });
}

// ---- decoder ---------------------------------------------------------------
int nnhip_decoder_create(nnhip_ctx *ctx, int vocab, int d_model, int n_heads,
                         int d_ff, int n_layers, int max_seq_len,
                         nnhip_model **out) {
  return guard([&] {
    REQ(ctx && out, "nnhip_decoder_create: NULL argument");
    set_device(ctx);
    std::unique_ptr<nnhip_model> m(new nnhip_model);
    m->m.reset(new nnhip::Model(&ctx->c, vocab, d_model, n_heads, d_ff,
                                n_layers, max_seq_len));
    *out = m.release();
  });
}

int nnhip_decoder_free(nnhip_model *m) {
  return guard([&] {
    if (!m) return;
    (void)hipStreamSynchronize(m->m->ctx->stream);
    delete m;
  });
}

int nnhip_decoder_num_params(const nnhip_model *m, int *n) {
  return guard([&] {
    REQ(m && n, "nnhip_decoder_num_params: NULL argument");
    *n = m->m->num_params();
  });
}

int nnhip_decoder_param_shape(const nnhip_model *m, int idx, int64_t *rows,
                              int64_t *cols) {
  return guard([&] {
    REQ(m && rows && cols, "nnhip_decoder_param_shape: NULL argument");
    m->m->param_shape(idx, rows, cols);
  });
}

int nnhip_decoder_set_param(nnhip_model *m, int idx, const float *host) {
  return guard([&] {
    REQ(m && host, "nnhip_decoder_set_param: NULL argument");
    m->m->set_param(idx, host);
  });
}

int nnhip_decoder_get_param(const nnhip_model *m, int idx, float *host) {
  return guard([&] {
    REQ(m && host, "nnhip_decoder_get_param: NULL argument");
    m->m->get_param(idx, host);
  });
}

int nnhip_decoder_init_normal(nnhip_model *m, uint64_t seed, float stdv) {
  return guard([&] {
    REQ(m, "nnhip_decoder_init_normal: NULL model");
    m->m->init_normal(seed, stdv);
  });
}

int nnhip_decoder_quantize(nnhip_model *m, int bits) {
  return guard([&] {
    REQ(m, "nnhip_decoder_quantize: NULL model");
    NNHIP_REQUIRE(bits == 8 || bits == 4, nnhip::kErrUnsupported,
                  "weight quantization: INT8 (8) or INT4 (4) only");
    m->m->quantize(bits);
  });
}

int nnhip_decoder_save_weights(const nnhip_model *m, const char *path) {
  return guard([&] {
    REQ(m && path, "nnhip_decoder_save_weights: NULL argument");
    nnhip::save_weights(*m->m, path);
  });
}

int nnhip_decoder_load_weights(nnhip_model *m, const char *path) {
  return guard([&] {
    REQ(m && path, "nnhip_decoder_load_weights: NULL argument");
    nnhip::load_weights(*m->m, path);
  });
}

int nnhip_decoder_get_quantized(const nnhip_model *m, int layer, int which,
                                int8_t *codes, float *scales) {
  return guard([&] {
    REQ(m && codes && scales, "nnhip_decoder_get_quantized: NULL argument");
    m->m->get_quantized(layer, which, codes, scales);
  });
}

int nnhip_decoder_forward(nnhip_model *mm, nnhip_kvcache *cache,
                          const int32_t *ids, int B, int S, float *logits) {
  return guard([&] {
    REQ(mm && ids && logits && B > 0 && S > 0, "nnhip_decoder_forward: bad argument");
    nnhip::Model &m = *mm->m;
    hipStream_t st = m.ctx->stream;
    nnhip::KVCache *kv = cache ? cache->c.get() : nullptr;
    if (kv) {
      REQ(kv->m == &m, "nnhip_decoder_forward: cache belongs to another model");
      REQ(kv->B == B, "nnhip_decoder_forward: cache batch differs from B");
      for (int b = 0; b < B; ++b)
        NNHIP_REQUIRE(kv->host_len[b] + S <= m.max_seq, nnhip::kErrCapacity,
                      "Sequence length S plus past cached length exceeds max_seq_len");
    } else {
      NNHIP_REQUIRE(S <= m.max_seq, nnhip::kErrCapacity,
                    "Sequence length S plus past cached length exceeds max_seq_len");
    }
    auto d_ids = upload(st, ids, (size_t)B * S);
    nnhip::DevBuf<float> d_log((size_t)B * S * m.V);
    int max_keys = S;
    if (kv) for (int b = 0; b < B; ++b) max_keys = std::max(max_keys, kv->host_len[b] + S);
    m.forward(kv, 0, d_ids.p, S, B, S, kv ? kv->len.p : nullptr, 0, nullptr,
              max_keys, d_log.p, false);
    NNHIP_CHECK(hipStreamSynchronize(st));
    m.check_pd();
    NNHIP_CHECK(hipMemcpyAsync(logits, d_log.p, d_log.bytes(), hipMemcpyDeviceToHost, st));
    if (kv) {
      for (int b = 0; b < B; ++b) kv->host_len[b] += S;
      NNHIP_CHECK(hipMemcpyAsync(kv->len.p, kv->host_len.data(), (size_t)B * 4,
                                 hipMemcpyHostToDevice, st));
    }
    NNHIP_CHECK(hipStreamSynchronize(st));
  });
}

// ---- KV cache --------------------------------------------------------------
int nnhip_kvcache_create(nnhip_model *m, int batch, int quantized,
                         nnhip_kvcache **out) {
  return guard([&] {
    REQ(m && out, "nnhip_kvcache_create: NULL argument");
    std::unique_ptr<nnhip_kvcache> c(new nnhip_kvcache);
    c->c.reset(new nnhip::KVCache(m->m.get(), batch, m->m->max_seq, quantized != 0));
    *out = c.release();
  });
}

int nnhip_kvcache_read_q8(const nnhip_kvcache *c, int layer, int b,
                          int8_t *kq, float *ks, int8_t *vq, float *vs) {
  return guard([&] {
    REQ(c && kq && ks && vq && vs, "nnhip_kvcache_read_q8: NULL argument");
    const nnhip::KVCache &kv = *c->c;
    REQ(kv.q8, "nnhip_kvcache_read_q8: the cache is not quantised");
    REQ(layer >= 0 && layer < kv.m->L && b >= 0 && b < kv.B,
        "nnhip_kvcache_read_q8: bad layer or sequence");
    hipStream_t st = kv.m->ctx->stream;
    NNHIP_CHECK(hipStreamSynchronize(st));
    const int H = kv.m->H, D = kv.m->D, n = kv.host_len[b];
    const nnhip::KvSrc src = kv.src(layer, b);
    for (int h = 0; h < H; ++h) {
      const int64_t row0 = (int64_t)h * kv.cap;
      NNHIP_CHECK(hipMemcpy(kq + (int64_t)h * n * D,
                            (const int8_t *)src.k + row0 * D, (size_t)n * D,
                            hipMemcpyDeviceToHost));
      NNHIP_CHECK(hipMemcpy(vq + (int64_t)h * n * D,
                            (const int8_t *)src.v + row0 * D, (size_t)n * D,
                            hipMemcpyDeviceToHost));
      NNHIP_CHECK(hipMemcpy(ks + (int64_t)h * n, src.ks + row0,
                            (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
      NNHIP_CHECK(hipMemcpy(vs + (int64_t)h * n, src.vs + row0,
                            (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
    }
  });
}

int nnhip_kvcache_read(const nnhip_kvcache *c, int layer, int b, float *k,
                       float *v) {
  return guard([&] {
    REQ(c && k && v, "nnhip_kvcache_read: NULL argument");
    const nnhip::KVCache &kv = *c->c;
    REQ(!kv.q8, "nnhip_kvcache_read: the cache is quantised");
    REQ(layer >= 0 && layer < kv.m->L && b >= 0 && b < kv.B,
        "nnhip_kvcache_read: bad layer or sequence");
    hipStream_t st = kv.m->ctx->stream;
    NNHIP_CHECK(hipStreamSynchronize(st));
    const int H = kv.m->H, D = kv.m->D, n = kv.host_len[b];
    const nnhip::KvSrc src = kv.src(layer, b);
    for (int h = 0; h < H; ++h) {
      const int64_t row0 = (int64_t)h * kv.cap;
      NNHIP_CHECK(hipMemcpy(k + (int64_t)h * n * D, (const float *)src.k + row0 * D,
                            (size_t)n * D * sizeof(float), hipMemcpyDeviceToHost));
      NNHIP_CHECK(hipMemcpy(v + (int64_t)h * n * D, (const float *)src.v + row0 * D,
                            (size_t)n * D * sizeof(float), hipMemcpyDeviceToHost));
    }
  });
}

int nnhip_kvcache_free(nnhip_kvcache *c) {
  return guard([&] {
    if (!c) return;
    (void)hipStreamSynchronize(c->c->m->ctx->stream);
    delete c;
  });
}

int nnhip_kvcache_length(const nnhip_kvcache *c, int b, int *len) {
  return guard([&] {
    REQ(c && len && b >= 0 && b < c->c->B, "nnhip_kvcache_length: bad argument");
    *len = c->c->host_len[b];
  });
}

int nnhip_kvcache_truncate(nnhip_kvcache *c, int b, int len) {
  return guard([&] {
    REQ(c && b >= 0 && b < c->c->B && len >= 0, "nnhip_kvcache_truncate: bad argument");
    if (len < c->c->host_len[b]) {
      c->c->host_len[b] = len;
      c->c->sync_len_to_device();
    }
  });
}

// ---- generation ------------------------------------------------------------
int nnhip_generate_speculative(nnhip_model *target, nnhip_model *draft,
                               const int32_t *prompt, int P, int max_new,
                               int lookahead, float temperature, int top_k,
                               float top_p, uint64_t seed,
                               int quantized_cache, int32_t *out,
                               nnhip_spec_stats *stats) {
  return guard([&] {
    REQ(target && draft && prompt && out, "nnhip_generate_speculative: NULL argument");
    nnhip::SpecStats st{};
    nnhip::generate_speculative_batch(*target->m, *draft->m, 1, prompt, P,
                                      max_new, lookahead, temperature, top_k,
                                      top_p, seed, 0, quantized_cache != 0,
                                      out, &st, nullptr);
    if (stats) std::memcpy(stats, &st, sizeof(st));
  });
}

int nnhip_generate_speculative_batch(nnhip_model *target, nnhip_model *draft,
                                     int B, const int32_t *prompts, int P,
                                     int max_new, int lookahead,
                                     float temperature, int top_k, float top_p,
                                     uint64_t seed, uint32_t seq0,
                                     int quantized_cache, int32_t *out,
                                     nnhip_spec_stats *stats,
                                     nnhip_spec_timing *timing) {
  return guard([&] {
    REQ(target && draft && prompts && out, "nnhip_generate_speculative_batch: NULL argument");
    static_assert(sizeof(nnhip::SpecStats) == sizeof(nnhip_spec_stats), "stats layout");
    static_assert(sizeof(nnhip::SpecTiming) == sizeof(nnhip_spec_timing), "timing layout");
    nnhip::generate_speculative_batch(
        *target->m, *draft->m, B, prompts, P, max_new, lookahead, temperature,
        top_k, top_p, seed, seq0, quantized_cache != 0, out,
        reinterpret_cast<nnhip::SpecStats *>(stats),
        reinterpret_cast<nnhip::SpecTiming *>(timing));
  });
}

int nnhip_generate_advanced(nnhip_model *m, const int32_t *prompt, int P,
                            int max_new, float temperature, int top_k,
                            float top_p, uint64_t seed, int use_kv_cache,
                            int32_t *out) {
  return guard([&] {
    REQ(m && prompt && out, "nnhip_generate_advanced: NULL argument");
    nnhip::generate_advanced_batch(*m->m, 1, prompt, P, max_new, temperature,
                                   top_k, top_p, seed, 0, use_kv_cache != 0,
                                   out);
  });
}

int nnhip_generate_advanced_batch(nnhip_model *m, int B,
                                  const int32_t *prompts, int P, int max_new,
                                  float temperature, int top_k, float top_p,
                                  uint64_t seed, uint32_t seq0,
                                  int use_kv_cache, int32_t *out) {
  return guard([&] {
    REQ(m && prompts && out, "nnhip_generate_advanced_batch: NULL argument");
    nnhip::generate_advanced_batch(*m->m, B, prompts, P, max_new, temperature,
                                   top_k, top_p, seed, seq0, use_kv_cache != 0,
                                   out);
  });
}

// ---- fused device ops --------------------------------------------------------
namespace {
int quantize_w(nnhip_ctx *ctx, const float *w, int in, int out, int8_t *codes,
               float *scales, int bits) {
  return guard([&] {
    REQ(ctx && w && codes && scales && in > 0 && out > 0,
        "nnhip_quantize_w: bad argument");
    hipStream_t st = ctx->c.stream;
    nnhip::DevBuf<float> t((size_t)in * out);
    nnhip::launch_transpose_into(st, w, in, out, t.p, 0, 1);
    nnhip::launch_quantize_w8(st, t.p, out, in, codes, scales, bits);
    NNHIP_CHECK(hipStreamSynchronize(st));
  });
}
}  // namespace

int nnhip_quantize_w8(nnhip_ctx *ctx, const float *w, int in, int out,
                      int8_t *codes, float *scales) {
  return quantize_w(ctx, w, in, out, codes, scales, 8);
}

int nnhip_quantize_w4(nnhip_ctx *ctx, const float *w, int in, int out,
                      int8_t *codes, float *scales) {
  return quantize_w(ctx, w, in, out, codes, scales, 4);
}

namespace {
struct LimbScratch {
  nnhip::DevBuf<int8_t> limbs;
  nnhip::DevBuf<int> rexp;
  int mpad = 0;
  void ensure(int rows, int K) {
    const int mp = (rows + 63) / 64 * 64;
    if ((size_t)3 * mp * K > limbs.n) limbs.alloc((size_t)3 * mp * K);
    if ((size_t)mp > rexp.n) rexp.alloc(mp);
    mpad = mp;
  }
};
// The context's scratch for `rows` rows of K digits and an N x K code copy
// in the operand layout; the stream drains first when a buffer must grow
// (earlier calls may still be reading it).  Returns the digit planes' mpad.
int ctx_scratch(nnhip_ctx *ctx, int rows, int K, int N) {
  const int mp = (rows + 63) / 64 * 64;
  const size_t nl = (size_t)3 * mp * K, nw = (size_t)N * K;
  if (nl > ctx->limbs.n || (size_t)mp > ctx->rexp.n || nw > ctx->sw.n) {
    NNHIP_CHECK(hipStreamSynchronize(ctx->c.stream));
    ctx->limbs.ensure(nl);
    ctx->rexp.ensure(mp);
    ctx->sw.ensure(nw);
  }
  return mp;
}
}  // namespace

int nnhip_linear_w8a32(nnhip_ctx *ctx, const float *x, int rows, int K,
                       const int8_t *codes, const float *scales,
                       const float *bias, int N, float *y, int path) {
  return guard([&] {
    REQ(ctx && x && codes && scales && bias && y && rows > 0 && K > 0 && N > 0,
        "nnhip_linear_w8a32: bad argument");
    hipStream_t st = ctx->c.stream;
    const bool mfma_ok = K % 128 == 0 && N % 64 == 0;
    bool mfma = path == 2 || (path == 0 && rows >= 16 && mfma_ok);
    NNHIP_REQUIRE(!(path == 2 && !mfma_ok), nnhip::kErrArg,
                  "MFMA path needs K % 128 == 0 and N % 64 == 0");
    NNHIP_REQUIRE(path >= 0 && path <= 4, nnhip::kErrArg, "unknown path");
    if (path == 3 || path == 4) {
      NNHIP_REQUIRE(nnhip::gemm_lds_supports(rows, K, N), nnhip::kErrArg,
                    "LDS GEMM needs K in {128, 256, 512, 1024} and N % 32 == 0");
      const int mpad = ctx_scratch(ctx, rows, K, N);
      nnhip::launch_swizzle_rows(st, codes, N, K, ctx->sw.p, false);
      if (path == 4)
        nnhip::launch_act_quant(st, x, K, rows, K, ctx->limbs.p, mpad, ctx->rexp.p);
      nnhip::launch_gemm_lds(st, path == 4 ? nnhip::kAFromDigits : nnhip::kAFromRows,
                             ctx->limbs.p, mpad, ctx->rexp.p, x, K, nullptr,
                             nullptr, nullptr, 0, rows, K, N, ctx->sw.p, scales,
                             bias, nullptr, 0, y, N, nnhip::kEpiBias);
    } else if (mfma) {
      const int mpad = ctx_scratch(ctx, rows, K, N);
      nnhip::launch_swizzle_rows(st, codes, N, K, ctx->sw.p, false);
      nnhip::launch_act_quant(st, x, K, rows, K, ctx->limbs.p, mpad, ctx->rexp.p);
      nnhip::launch_gemm_limb(st, ctx->limbs.p, mpad, ctx->rexp.p, rows, K, N,
                              ctx->sw.p, scales, bias, nullptr, 0, y, N,
                              nnhip::kEpiBias);
    } else {
      nnhip::launch_gemv(st, x, K, rows, K, N, codes, nullptr, scales, bias,
                         nullptr, 0, y, N, nnhip::kEpiBias);
    }
  });
}

int nnhip_layernorm_linear_w8a32(nnhip_ctx *ctx, const float *h, int rows,
                                 int K, const float *gamma, const float *beta,
                                 float *ln_out, const int8_t *codes,
                                 const float *scales, const float *bias, int N,
                                 float *y) {
  return guard([&] {
    REQ(ctx && h && gamma && beta && codes && scales && bias && y && rows > 0,
        "nnhip_layernorm_linear_w8a32: bad argument");
    NNHIP_REQUIRE(nnhip::gemm_lds_supports(rows, K, N), nnhip::kErrArg,
                  "fused LayerNorm GEMM needs K in {128, 256, 512, 1024} and N % 32 == 0");
    hipStream_t st = ctx->c.stream;
    if (rows < 16) {
      nnhip::GemvLn lf;
      lf.g = gamma; lf.b = beta; lf.out = ln_out; lf.ldo = K;
      nnhip::launch_gemv(st, h, K, rows, K, N, codes, nullptr, scales, bias,
                         nullptr, 0, y, N, nnhip::kEpiBias, nullptr, &lf);
      return;
    }
    ctx_scratch(ctx, 1, K, N);
    nnhip::launch_swizzle_rows(st, codes, N, K, ctx->sw.p, false);
    nnhip::launch_gemm_lds(st, nnhip::kAFromLayerNorm, nullptr, 0, nullptr, h,
                           K, gamma, beta, ln_out, K, rows, K, N, ctx->sw.p, scales,
                           bias, nullptr, 0, y, N, nnhip::kEpiBias);
  });
}

int nnhip_linear_f32(nnhip_ctx *ctx, const float *x, int rows, int K,
                     const float *w, const float *bias, int N, float *y) {
  return guard([&] {
    REQ(ctx && x && w && bias && y && rows > 0 && K > 0 && N > 0,
        "nnhip_linear_f32: bad argument");
    nnhip::launch_gemv(ctx->c.stream, x, K, rows, K, N, nullptr, w, nullptr,
                       bias, nullptr, 0, y, N, nnhip::kEpiBias);
  });
}

int nnhip_linear_limb_totals(nnhip_ctx *ctx, const float *x, int rows, int K,
                             const int8_t *codes, int N, int64_t *totals,
                             int32_t *rexp, int8_t *limbs) {
  return guard([&] {
    REQ(ctx && x && codes && totals && rows > 0, "nnhip_linear_limb_totals: bad argument");
    REQ(K % 128 == 0 && N % 64 == 0, "MFMA path needs K % 128 == 0 and N % 64 == 0");
    hipStream_t st = ctx->c.stream;
    LimbScratch ls;
    ls.ensure(rows, K);
    NNHIP_CHECK(hipMemsetAsync(ls.limbs.p, 0, ls.limbs.bytes(), st));
    nnhip::DevBuf<float> dummy(N);
    nnhip::DevBuf<int8_t> sw((size_t)N * K);
    nnhip::launch_swizzle_rows(st, codes, N, K, sw.p, false);
    nnhip::launch_act_quant(st, x, K, rows, K, ls.limbs.p, ls.mpad, ls.rexp.p);
    nnhip::launch_gemm_limb(st, ls.limbs.p, ls.mpad, ls.rexp.p, rows, K, N,
                            sw.p, dummy.p, dummy.p, nullptr, 0,
                            reinterpret_cast<float *>(totals), N,
                            nnhip::kEpiTotals);
    if (rexp) NNHIP_CHECK(hipMemcpyAsync(rexp, ls.rexp.p, (size_t)rows * 4, hipMemcpyDeviceToDevice, st));
    if (limbs)
      for (int l = 0; l < 3; ++l)
        nnhip::launch_swizzle_rows(st, ls.limbs.p + (size_t)l * ls.mpad * K,
                                   ls.mpad, K, limbs + (size_t)l * ls.mpad * K,
                                   true);
    NNHIP_CHECK(hipStreamSynchronize(st));
  });
}

// RoPE factors for positions [0, cap) by the reference's float formula
// (tensor.cpp:1141-1173): theta = pow(10000, -2j/D), omega = pos * theta.
static void rope_tables(int cap, int D, std::vector<float> &hc,
                        std::vector<float> &hs) {
  const int half = D / 2;
  hc.assign((size_t)cap * half, 0.f);
  hs.assign((size_t)cap * half, 0.f);
  for (int p = 0; p < cap; ++p)
    for (int j = 0; j < half; ++j) {
      const float theta = std::pow(10000.0f, -2.0f * (float)j / (float)D);
      const float omega = (float)p * theta;
      hc[(size_t)p * half + j] = std::cos(omega);
      hs[(size_t)p * half + j] = std::sin(omega);
    }
}

// The context's RoPE tables for head width D covering positions [0, cap):
// built once per width (and again only when a call needs more positions,
// after the stream has drained), so the append entry points neither compute
// tables nor synchronise per call.
static const nnhip_ctx::Rope &ctx_rope(nnhip_ctx *ctx, int cap, int D) {
  nnhip_ctx::Rope *slot = nullptr;
  for (auto &r : ctx->rope)
    if (r.D == D) { slot = &r; break; }
  if (!slot)
    for (auto &r : ctx->rope)
      if (r.D == 0) { slot = &r; break; }
  if (!slot) slot = &ctx->rope[0];
  if (slot->D == D && slot->n >= cap) return *slot;
  hipStream_t st = ctx->c.stream;
  NNHIP_CHECK(hipStreamSynchronize(st));   // earlier calls may read the old one
  const int n = std::max(cap, slot->D == D ? 2 * slot->n : 1024);
  std::vector<float> hc, hs;
  rope_tables(n, D, hc, hs);
  slot->c.alloc(hc.size());
  slot->s.alloc(hs.size());
  NNHIP_CHECK(hipMemcpyAsync(slot->c.p, hc.data(), hc.size() * 4,
                             hipMemcpyHostToDevice, st));
  NNHIP_CHECK(hipMemcpyAsync(slot->s.p, hs.data(), hs.size() * 4,
                             hipMemcpyHostToDevice, st));
  NNHIP_CHECK(hipStreamSynchronize(st));   // the host tables go out of scope
  slot->D = D;
  slot->n = n;
  return *slot;
}

int nnhip_rope_kv_append(nnhip_ctx *ctx, const float *qkv, int B, int S,
                         int H, int D, const int32_t *pos, float *q_out,
                         float *kcache, float *vcache, int cap) {
  return guard([&] {
    REQ(ctx && qkv && pos && q_out && kcache && vcache && B > 0 && S > 0 &&
            H > 0 && D > 0 && D % 2 == 0 && cap > 0,
        "nnhip_rope_kv_append: bad argument");
    hipStream_t st = ctx->c.stream;
    const nnhip_ctx::Rope &rt = ctx_rope(ctx, cap, D);
    nnhip::launch_rope_kv(st, qkv, B, S, H, D, pos, 0, nullptr, rt.c.p, rt.s.p,
                          q_out, kcache, vcache, cap, (int64_t)H * cap * D);
  });
}

int nnhip_rope_kv_append_gqa(nnhip_ctx *ctx, const float *qkv, int B, int S,
                             int H, int Hkv, int D, const int32_t *pos,
                             float *q_out, float *kcache, float *vcache,
                             int cap) {
  return guard([&] {
    REQ(ctx && qkv && pos && q_out && kcache && vcache && B > 0 && S > 0 &&
            H > 0 && Hkv > 0 && H % Hkv == 0 && D > 0 && D % 2 == 0 && cap > 0,
        "nnhip_rope_kv_append_gqa: bad argument");
    hipStream_t st = ctx->c.stream;
    const nnhip_ctx::Rope &rt = ctx_rope(ctx, cap, D);
    nnhip::launch_rope_kv(st, qkv, B, S, H, D, pos, 0, nullptr, rt.c.p, rt.s.p,
                          q_out, kcache, vcache, cap, (int64_t)Hkv * cap * D,
                          Hkv);
  });
}

int nnhip_attention_kq(nnhip_ctx *ctx, const float *q, const float *kcache,
                       const float *vcache, int cap, const int32_t *pos0,
                       int B, int S, int H, int Hkv, int D, float *out) {
  return guard([&] {
    REQ(ctx && q && kcache && vcache && pos0 && out && B > 0 && S > 0 &&
            H > 0 && Hkv > 0 && cap > 0,
        "nnhip_attention_kq: bad argument");
    hipStream_t st = ctx->c.stream;
    const int max_keys = cap;
    const int64_t pe = nnhip::attention_partial_elems(B, S, H, D, max_keys);
    if ((size_t)std::max<int64_t>(pe, 1) > ctx->part.n) {
      NNHIP_CHECK(hipStreamSynchronize(st));   // earlier calls may read it
      ctx->part.ensure((size_t)std::max<int64_t>(pe, 1));
    }
    nnhip::KvSrc kv;
    kv.k = kcache; kv.v = vcache; kv.seq_stride = (int64_t)Hkv * cap * D;
    nnhip::launch_attention(st, q, kv, B, S, H, Hkv, D, cap, pos0, 0, nullptr,
                            max_keys, ctx->part.p, pe, out);
  });
}

int nnhip_rope_kv_append_q8(nnhip_ctx *ctx, const float *qkv, int B, int S,
                            int H, int D, const int32_t *pos, float *q_out,
                            int8_t *kcodes, float *kscales, int8_t *vcodes,
                            float *vscales, int cap) {
  return guard([&] {
    REQ(ctx && qkv && pos && q_out && kcodes && kscales && vcodes && vscales &&
            B > 0 && S > 0 && H > 0 && D > 0 && D % 2 == 0 && D <= 64 && cap > 0,
        "nnhip_rope_kv_append_q8: bad argument");
    hipStream_t st = ctx->c.stream;
    const nnhip_ctx::Rope &rt = ctx_rope(ctx, cap, D);
    nnhip::launch_rope_kv_q8(st, qkv, B, S, H, D, pos, 0, nullptr, rt.c.p,
                             rt.s.p, q_out, kcodes, kscales, vcodes, vscales,
                             cap, (int64_t)H * cap * D, (int64_t)H * cap);
  });
}

int nnhip_attention_kq_q8(nnhip_ctx *ctx, const float *q, const int8_t *kcodes,
                          const float *kscales, const int8_t *vcodes,
                          const float *vscales, int cap, const int32_t *pos0,
                          int B, int S, int H, int Hkv, int D, float *out) {
  return guard([&] {
    REQ(ctx && q && kcodes && kscales && vcodes && vscales && pos0 && out &&
            B > 0 && S > 0 && H > 0 && Hkv > 0 && cap > 0,
        "nnhip_attention_kq_q8: bad argument");
    hipStream_t st = ctx->c.stream;
    const int max_keys = cap;
    const int64_t pe = nnhip::attention_partial_elems(B, S, H, D, max_keys);
    nnhip::DevBuf<float> part(pe > 0 ? pe : 1);
    nnhip::KvSrc kv;
    kv.q8 = true;
    kv.k = kcodes; kv.v = vcodes; kv.ks = kscales; kv.vs = vscales;
    kv.seq_stride = (int64_t)Hkv * cap * D;
    kv.sc_stride = (int64_t)Hkv * cap;
    nnhip::launch_attention(st, q, kv, B, S, H, Hkv, D, cap, pos0, 0, nullptr,
                            max_keys, part.p, pe, out);
    NNHIP_CHECK(hipStreamSynchronize(st));
  });
}

int nnhip_layernorm(nnhip_ctx *ctx, const float *x, int rows, int d,
                    const float *gamma, const float *beta, float *y) {
  return guard([&] {
    REQ(ctx && x && gamma && beta && y && rows > 0 && d > 0, "nnhip_layernorm: bad argument");
    nnhip::launch_layernorm(ctx->c.stream, x, rows, d, gamma, beta, y, nullptr,
                            0, nullptr);
  });
}

int nnhip_sample_rows(nnhip_ctx *ctx, const float *logits, int B, int V,
                      float temperature, int top_k, float top_p,
                      const float *u, int32_t *tok, float *probs) {
  return guard([&] {
    REQ(ctx && logits && u && tok && B > 0 && V > 0, "nnhip_sample_rows: bad argument");
    nnhip::launch_sample_rows(ctx->c.stream, logits, B, V, temperature, u, tok,
                              probs, top_k, top_p);
  });
}

int nnhip_spec_accept(nnhip_ctx *ctx, const float *tlogits,
                      const float *dlogits, const int32_t *dtok,
                      const float *u_accept, const float *u_resample, int B,
                      int k, int V, float temperature, int32_t *n_accept,
                      int32_t *next_tok) {
  return guard([&] {
    REQ(ctx && tlogits && dlogits && dtok && u_accept && u_resample &&
            n_accept && next_tok && B > 0 && k > 0 && V > 0,
        "nnhip_spec_accept: bad argument");
    hipStream_t st = ctx->c.stream;
    // the draft rows' get_probs as the loop's drafting steps leave them:
    // their logits and 128-column tile statistics, each probability formed
    // where the accept step reads it.  The state of the last call's sizes
    // is reused (the previous call has synchronized the stream).
    if (!ctx->accept || ctx->acc_B != B || ctx->acc_k != k || ctx->acc_V != V) {
      ctx->accept.reset();
      ctx->accept.reset(new nnhip::AcceptRows(B, k, V, temperature));
      ctx->acc_B = B; ctx->acc_k = k; ctx->acc_V = V;
    }
    nnhip::AcceptRows &ar = *ctx->accept;
    ar.s.T = temperature;
    ar.launch_logits(st, tlogits, dlogits, dtok, u_accept, u_resample,
                     n_accept, next_tok);
    NNHIP_CHECK(hipStreamSynchronize(st));
  });
}

}  // extern "C"

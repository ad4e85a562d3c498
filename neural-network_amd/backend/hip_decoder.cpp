// HipDecoder, HipKVCache, HipMultiHeadAttention and HipMhaCache
// (hip_nn.hpp) over libnnhip.so.  Nothing here uses the reference's compiled
// code, only its headers' types, so programs can run these objects without
// linking the reference's sources; the constructors from reference objects
// and the Tensor overloads are in hip_nn.cpp.
#include "hip_nn.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>

namespace nnhip_backend {

namespace {

std::vector<int32_t> to_ids(const std::vector<size_t> &v) {
  std::vector<int32_t> r(v.size());
  // ids the int32 ABI cannot hold behave as out-of-range ids (row 0 of the
  // embedding, cpu_backend.cpp:1022-1025)
  for (size_t i = 0; i < v.size(); ++i)
    r[i] = v[i] > 0x7fffffffu ? -1 : static_cast<int32_t>(v[i]);
  return r;
}

}  // namespace

HipDecoder::HipDecoder(HipBackend &backend, const DecoderConfig &cfg,
                       const std::vector<std::vector<float>> &params)
    : cfg_(cfg) {
  check(nnhip_decoder_create(backend.context(), (int)cfg.vocab_size,
                             (int)cfg.embed_dim, (int)cfg.num_heads,
                             (int)cfg.dim_feedforward, (int)cfg.num_layers,
                             (int)cfg.max_seq_len, &m_));
  try {
    int n = 0;
    check(nnhip_decoder_num_params(m_, &n));
    if ((size_t)n != params.size())
      throw std::runtime_error("HipDecoder: parameter count mismatch");
    for (size_t i = 0; i < params.size(); ++i) {
      int64_t rows = 0, cols = 0;
      check(nnhip_decoder_param_shape(m_, (int)i, &rows, &cols));
      if (params[i].size() != (size_t)(rows * cols))
        throw std::runtime_error("HipDecoder: parameter shape mismatch");
      check(nnhip_decoder_set_param(m_, (int)i, params[i].data()));
    }
  } catch (...) {
    (void)nnhip_decoder_free(m_);
    m_ = nullptr;
    throw;
  }
}

HipDecoder::~HipDecoder() { (void)nnhip_decoder_free(m_); }

void HipDecoder::quantize(const QuantizationConfig &config) {
  check(nnhip_decoder_quantize(
      m_, config.type == QuantizationType::INT4 ? 4 : 8));
}

std::vector<float> HipDecoder::forward(const std::vector<size_t> &ids,
                                       HipKVCache *cache) {
  const std::vector<int32_t> x = to_ids(ids);
  std::vector<float> logits(ids.size() * cfg_.vocab_size);
  check(nnhip_decoder_forward(m_, cache ? cache->handle() : nullptr, x.data(),
                              1, (int)x.size(), logits.data()));
  return logits;
}

std::vector<size_t> HipDecoder::generate_advanced(
    const std::vector<size_t> &prompt, size_t max_new_tokens, float temperature,
    size_t top_k, float top_p, unsigned int seed, bool use_kv_cache) {
  const std::vector<int32_t> p = to_ids(prompt);
  std::vector<int32_t> out(p.size() + max_new_tokens);
  check(nnhip_generate_advanced(m_, p.data(), (int)p.size(),
                                (int)max_new_tokens, temperature, (int)top_k,
                                top_p, seed, use_kv_cache ? 1 : 0,
                                out.data()));
  return std::vector<size_t>(out.begin(), out.end());
}

std::vector<size_t> HipDecoder::generate_speculative(
    HipDecoder *draft_model, const std::vector<size_t> &prompt,
    size_t max_new_tokens, size_t lookahead, float temperature, size_t top_k,
    float top_p, unsigned int seed, bool quantized_cache) {
  if (!draft_model) throw std::runtime_error("generate_speculative: no draft model");
  const std::vector<int32_t> p = to_ids(prompt);
  // the reference always appends the first token (layer.cpp:1508-1510)
  std::vector<int32_t> out(p.size() + std::max<size_t>(max_new_tokens, 1));
  nnhip_spec_stats st;
  check(nnhip_generate_speculative(m_, draft_model->m_, p.data(), (int)p.size(),
                                   (int)max_new_tokens, (int)lookahead,
                                   temperature, (int)top_k, top_p, seed,
                                   quantized_cache ? 1 : 0, out.data(), &st));
  return std::vector<size_t>(out.begin(), out.end());
}

HipKVCache::HipKVCache(HipDecoder &model, bool quantized) {
  check(nnhip_kvcache_create(model.handle(), 1, quantized ? 1 : 0, &c_));
}

HipKVCache::~HipKVCache() { (void)nnhip_kvcache_free(c_); }

void HipKVCache::truncate(size_t len) {
  check(nnhip_kvcache_truncate(c_, 0, (int)std::min<size_t>(len, 0x7fffffff)));
}

size_t HipKVCache::length() const {
  int n = 0;
  check(nnhip_kvcache_length(c_, 0, &n));
  return (size_t)n;
}

// ---- MultiHeadAttention ----------------------------------------------------

namespace {

std::unique_ptr<DeviceBuffer> upload_f32(HipBackend &be,
                                         const std::vector<float> &v) {
  std::unique_ptr<DeviceBuffer> d = be.allocate(v.size() * sizeof(float));
  be.copy_host_to_device(v.data(), *d, v.size() * sizeof(float));
  return d;
}

// w [in][out] -> rows [out][in] appended to dst
void append_transposed(std::vector<float> &dst, const std::vector<float> &w,
                       size_t in, size_t out) {
  const size_t base = dst.size();
  dst.resize(base + in * out);
  for (size_t k = 0; k < in; ++k)
    for (size_t n = 0; n < out; ++n) dst[base + n * in + k] = w[k * out + n];
}

float *fptr(DeviceBuffer &b) { return static_cast<float *>(b.data()); }
int8_t *cptr(DeviceBuffer &b) { return static_cast<int8_t *>(b.data()); }

}  // namespace

HipMultiHeadAttention::HipMultiHeadAttention(
    HipBackend &backend, const MhaConfig &cfg,
    const std::vector<std::vector<float>> &params)
    : be_(backend), cfg_(cfg) {
  // the reference constructor's checks (layer.cpp:477-482)
  if (cfg.num_heads == 0 || cfg.embed_dim % cfg.num_heads != 0)
    throw std::runtime_error("embed_dim must be divisible by num_heads");
  H_ = cfg.num_heads;
  Hkv_ = cfg.num_kv_heads == 0 ? H_ : cfg.num_kv_heads;
  if (H_ % Hkv_ != 0)
    throw std::runtime_error("num_heads must be divisible by num_kv_heads");
  D_ = cfg.embed_dim / H_;
  if (D_ % 2 != 0)
    throw std::runtime_error("HipMultiHeadAttention: RoPE needs an even head dim");
  if (!cfg.causal)
    throw std::runtime_error(
        "HipMultiHeadAttention: non-causal attention is not on the device path");
  const size_t E = cfg.embed_dim, Ekv = Hkv_ * D_;
  const size_t sizes[8] = {E * E, E, E * Ekv, Ekv, E * Ekv, Ekv, E * E, E};
  if (params.size() != 8)
    throw std::runtime_error("HipMultiHeadAttention: parameter count mismatch");
  for (int i = 0; i < 8; ++i)
    if (params[i].size() != sizes[i])
      throw std::runtime_error("HipMultiHeadAttention: parameter shape mismatch");
  master_ = params;
  std::vector<float> wqkv, bqkv;
  append_transposed(wqkv, params[0], E, E);
  append_transposed(wqkv, params[2], E, Ekv);
  append_transposed(wqkv, params[4], E, Ekv);
  for (int i : {1, 3, 5}) bqkv.insert(bqkv.end(), params[i].begin(), params[i].end());
  std::vector<float> wo;
  append_transposed(wo, params[6], E, E);
  wqkv_ = upload_f32(be_, wqkv);
  bqkv_ = upload_f32(be_, bqkv);
  wo_ = upload_f32(be_, wo);
  bo_ = upload_f32(be_, params[7]);
}

HipMultiHeadAttention::~HipMultiHeadAttention() = default;

void HipMultiHeadAttention::quantize(const QuantizationConfig &config) {
  const int bits = config.type == QuantizationType::INT4 ? 4 : 8;
  const size_t E = cfg_.embed_dim, Ekv = Hkv_ * D_, Nqkv = E + 2 * Ekv;
  cqkv_ = be_.allocate(Nqkv * E);
  sqkv_ = be_.allocate(Nqkv * sizeof(float));
  co_ = be_.allocate(E * E);
  so_ = be_.allocate(E * sizeof(float));
  // each projection from its fp32 [in][out] weights, into its rows of the
  // fused codes and scales
  auto quant = [&](const std::vector<float> &w, size_t out, int8_t *codes,
                   float *scales) {
    std::unique_ptr<DeviceBuffer> dw = upload_f32(be_, w);
    check(bits == 4 ? nnhip_quantize_w4(be_.context(), fptr(*dw), (int)E,
                                        (int)out, codes, scales)
                    : nnhip_quantize_w8(be_.context(), fptr(*dw), (int)E,
                                        (int)out, codes, scales));
    be_.synchronize();
  };
  quant(master_[0], E, cptr(*cqkv_), fptr(*sqkv_));
  quant(master_[2], Ekv, cptr(*cqkv_) + E * E, fptr(*sqkv_) + E);
  quant(master_[4], Ekv, cptr(*cqkv_) + (E + Ekv) * E, fptr(*sqkv_) + E + Ekv);
  quant(master_[6], E, cptr(*co_), fptr(*so_));
  quantized_ = true;
}

void HipMultiHeadAttention::forward_device(const float *x, size_t B, size_t S,
                                           float *y, HipMhaCache *cache) {
  if (B == 0 || S == 0) return;
  const size_t E = cfg_.embed_dim, Ekv = Hkv_ * D_, Nqkv = E + 2 * Ekv;
  const size_t rows = B * S;
  nnhip_ctx *ctx = be_.context();
  // the past: the cache's length for every sequence, or none
  std::unique_ptr<DeviceBuffer> tk, tv;
  float *kc = nullptr, *vc = nullptr;
  size_t cap = 0, past = 0;
  if (cache) {
    if (cache->B_ != B)
      throw std::runtime_error("HipMultiHeadAttention: cache batch differs from B");
    if (cache->len_ + S > cache->cap_)
      throw std::runtime_error(
          "HipMhaCache: cached length plus S exceeds its capacity");
    kc = fptr(*cache->k_);
    vc = fptr(*cache->v_);
    cap = cache->cap_;
    past = cache->len_;
  } else {
    tk = be_.allocate(B * Hkv_ * S * D_ * sizeof(float));
    tv = be_.allocate(B * Hkv_ * S * D_ * sizeof(float));
    kc = fptr(*tk);
    vc = fptr(*tv);
    cap = S;
  }
  // the layer's scratch, reused in stream order; grown after the stream has
  // drained (earlier calls may still read it)
  if (rows > s_rows_ || B > s_B_) {
    be_.synchronize();
    s_rows_ = std::max(rows, s_rows_);
    s_B_ = std::max(B, s_B_);
    s_qkv_ = be_.allocate(s_rows_ * Nqkv * sizeof(float));
    s_qrot_ = be_.allocate(s_rows_ * E * sizeof(float));
    s_ctx_ = be_.allocate(s_rows_ * E * sizeof(float));
    s_pos_ = be_.allocate(s_B_ * sizeof(int32_t));
  }
  DeviceBuffer *qkv = s_qkv_.get(), *qrot = s_qrot_.get(), *ctxo = s_ctx_.get();
  const std::vector<int32_t> hpos(B, (int32_t)past);
  check(nnhip_h2d(ctx, s_pos_->data(), hpos.data(), B * sizeof(int32_t)));
  const int32_t *dpos = static_cast<const int32_t *>(s_pos_->data());
  // q | k | v rows, RoPE at the cache length and the append, attention
  if (quantized_)
    check(nnhip_linear_w8a32(ctx, x, (int)rows, (int)E, cptr(*cqkv_),
                             fptr(*sqkv_), fptr(*bqkv_), (int)Nqkv,
                             fptr(*qkv), 0));
  else
    check(nnhip_linear_f32(ctx, x, (int)rows, (int)E, fptr(*wqkv_),
                           fptr(*bqkv_), (int)Nqkv, fptr(*qkv)));
  check(nnhip_rope_kv_append_gqa(ctx, fptr(*qkv), (int)B, (int)S, (int)H_,
                                 (int)Hkv_, (int)D_, dpos, fptr(*qrot), kc, vc,
                                 (int)cap));
  check(nnhip_attention_kq(ctx, fptr(*qrot), kc, vc, (int)cap, dpos, (int)B,
                           (int)S, (int)H_, (int)Hkv_, (int)D_, fptr(*ctxo)));
  if (quantized_)
    check(nnhip_linear_w8a32(ctx, fptr(*ctxo), (int)rows, (int)E, cptr(*co_),
                             fptr(*so_), fptr(*bo_), (int)E, y, 0));
  else
    check(nnhip_linear_f32(ctx, fptr(*ctxo), (int)rows, (int)E, fptr(*wo_),
                           fptr(*bo_), (int)E, y));
  if (!cache) be_.synchronize();  // the temporary K / V are freed on return
  if (cache) cache->len_ += S;
}

HipMhaCache::HipMhaCache(HipMultiHeadAttention &layer, size_t batch)
    : B_(batch), cap_(layer.cfg_.max_seq_len) {
  if (batch == 0 || cap_ == 0)
    throw std::runtime_error("HipMhaCache: empty batch or capacity");
  const size_t n = B_ * layer.Hkv_ * cap_ * layer.D_;
  k_ = layer.be_.allocate(n * sizeof(float));
  v_ = layer.be_.allocate(n * sizeof(float));
  layer.be_.fill(*k_, 0.0f);
  layer.be_.fill(*v_, 0.0f);
}

void HipMhaCache::truncate(size_t len) { len_ = std::min(len, len_); }

}  // namespace nnhip_backend

// HipDecoder and HipKVCache (hip_nn.hpp) over libnnhip.so.  Nothing here
// uses the reference's compiled code, only its headers' types, so programs
// can run these objects without linking the reference's sources; the
// constructor from a TransformerDecoder is in hip_nn.cpp.
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

}  // namespace nnhip_backend

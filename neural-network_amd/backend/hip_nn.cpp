// Drop-in decoder objects (hip_nn.hpp) over libnnhip.so.
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

HipDecoder::HipDecoder(HipBackend &backend, TransformerDecoder &d,
                       const DecoderConfig &cfg)
    : cfg_(cfg) {
  check(nnhip_decoder_create(backend.context(), (int)cfg.vocab_size,
                             (int)cfg.embed_dim, (int)cfg.num_heads,
                             (int)cfg.dim_feedforward, (int)cfg.num_layers,
                             (int)cfg.max_seq_len, &m_));
  auto params = d.parameters();
  int n = 0;
  check(nnhip_decoder_num_params(m_, &n));
  if ((size_t)n != params.size()) {
    nnhip_decoder_free(m_);
    throw std::runtime_error("HipDecoder: parameter count mismatch");
  }
  for (size_t i = 0; i < params.size(); ++i) {
    int64_t rows = 0, cols = 0;
    check(nnhip_decoder_param_shape(m_, (int)i, &rows, &cols));
    const std::vector<float> host = params[i]->to_host();
    if (host.size() != (size_t)(rows * cols))
      throw std::runtime_error("HipDecoder: parameter shape mismatch");
    check(nnhip_decoder_set_param(m_, (int)i, host.data()));
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

HipQuantizedDense::HipQuantizedDense(HipBackend &backend,
                                     const QuantizedDense &layer)
    : be_(backend) {
  if (layer.type() != QuantizationType::INT8)
    throw std::runtime_error("HipQuantizedDense: INT8 layers only");
  const Shape ws = layer.weight_shape();  // [in, out]
  in_ = ws.at(0);
  out_ = ws.at(1);
  // packed_weights hold int8 codes [in][out] (quantization.cpp:36-66); the
  // device reads them transposed, [out][in]
  const std::vector<uint8_t> &pw = layer.packed_weights();
  std::vector<int8_t> t(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n)
      t[n * in_ + k] = static_cast<int8_t>(pw[k * out_ + n]);
  codes_ = be_.allocate(t.size());
  check(nnhip_h2d(be_.context(), codes_->data(), t.data(), t.size()));
  const std::vector<float> sc = layer.scales()->to_host();
  scales_ = be_.allocate(sc.size() * sizeof(float));
  be_.copy_host_to_device(sc.data(), *scales_, sc.size() * sizeof(float));
  std::vector<float> b(out_, 0.0f);
  if (layer.bias()) b = layer.bias()->to_host();
  bias_ = be_.allocate(b.size() * sizeof(float));
  be_.copy_host_to_device(b.data(), *bias_, b.size() * sizeof(float));
}

std::shared_ptr<Tensor> HipQuantizedDense::forward(
    const std::shared_ptr<Tensor> &input) {
  const Shape &s = input->shape();
  if (input->backend() != &be_ || s.empty() || s.back() != in_ ||
      !is_contiguous(s, input->strides()))
    throw std::runtime_error(
        "HipQuantizedDense: input must be a contiguous HipBackend tensor "
        "whose last dimension is in_features");
  const size_t rows = count_elements(s) / in_;
  Shape out_shape = s;
  out_shape.back() = out_;
  std::shared_ptr<DeviceBuffer> y(be_.allocate(rows * out_ * sizeof(float)));
  const float *x =
      static_cast<const float *>(input->storage()->data()) + input->offset();
  check(nnhip_linear_w8a32(be_.context(), x, (int)rows, (int)in_,
                           static_cast<const int8_t *>(codes_->data()),
                           static_cast<const float *>(scales_->data()),
                           static_cast<const float *>(bias_->data()),
                           (int)out_, static_cast<float *>(y->data()), 0));
  return std::make_shared<Tensor>(out_shape, compute_strides(out_shape), 0, y,
                                  &be_, DataType::FP32);
}

}  // namespace nnhip_backend

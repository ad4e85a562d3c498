// The parts of the drop-in decoder objects (hip_nn.hpp) that use the
// reference's compiled code: HipDecoder's constructor from a
// TransformerDecoder and HipQuantizedDense over Tensor.
#include "hip_nn.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>

namespace nnhip_backend {

// The decoder's parameters() (layer.cpp:1140-1154) copied to the host in
// order, then the constructor from parameter arrays (hip_decoder.cpp).
static std::vector<std::vector<float>> host_params(TransformerDecoder &d) {
  std::vector<std::vector<float>> r;
  for (const auto &p : d.parameters()) r.push_back(p->to_host());
  return r;
}

HipDecoder::HipDecoder(HipBackend &backend, TransformerDecoder &d,
                       const DecoderConfig &cfg)
    : HipDecoder(backend, cfg, host_params(d)) {}

static std::vector<std::vector<float>> host_params(MultiHeadAttention &m) {
  std::vector<std::vector<float>> r;
  for (const auto &p : m.parameters()) r.push_back(p->to_host());
  return r;
}

HipMultiHeadAttention::HipMultiHeadAttention(HipBackend &backend,
                                             MultiHeadAttention &layer,
                                             const MhaConfig &cfg)
    : HipMultiHeadAttention(backend, cfg, host_params(layer)) {}

std::shared_ptr<Tensor> HipMultiHeadAttention::forward(
    const std::shared_ptr<Tensor> &input, HipMhaCache *cache) {
  const Shape &s = input->shape();
  // the reference's check (layer.cpp:596-599)
  if (s.size() != 3)
    throw std::runtime_error("MultiHeadAttention input must be of shape (B, S, E)");
  if (input->backend() != &be_ || s[2] != cfg_.embed_dim ||
      !is_contiguous(s, input->strides()))
    throw std::runtime_error(
        "HipMultiHeadAttention: input must be a contiguous HipBackend tensor "
        "whose last dimension is embed_dim");
  std::shared_ptr<DeviceBuffer> y(be_.allocate(count_elements(s) * sizeof(float)));
  const float *x =
      static_cast<const float *>(input->storage()->data()) + input->offset();
  forward_device(x, s[0], s[1], static_cast<float *>(y->data()), cache);
  return std::make_shared<Tensor>(s, compute_strides(s), 0, y, &be_,
                                  DataType::FP32);
}

void HipQuantizedDense::upload(const std::vector<int8_t> &codes_in_out,
                               const std::vector<float> &scales,
                               const std::vector<float> &bias) {
  host_codes_ = codes_in_out;
  host_scales_ = scales;
  host_bias_ = bias;
  // the device reads the codes transposed, [out][in], one per byte (INT4
  // codes in [-7, 7] go through the int8 kernels unchanged)
  std::vector<int8_t> t(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n) t[n * in_ + k] = codes_in_out[k * out_ + n];
  codes_ = be_.allocate(t.size());
  check(nnhip_h2d(be_.context(), codes_->data(), t.data(), t.size()));
  scales_ = be_.allocate(scales.size() * sizeof(float));
  be_.copy_host_to_device(scales.data(), *scales_, scales.size() * sizeof(float));
  bias_ = be_.allocate(bias.size() * sizeof(float));
  be_.copy_host_to_device(bias.data(), *bias_, bias.size() * sizeof(float));
}

HipQuantizedDense::HipQuantizedDense(HipBackend &backend,
                                     const QuantizedDense &layer)
    : be_(backend), type_(layer.type()) {
  const Shape ws = layer.weight_shape();  // [in, out]
  in_ = ws.at(0);
  out_ = ws.at(1);
  // packed_weights hold the codes of [in][out]: one int8 per byte (INT8,
  // quantization.cpp:36-66) or two 4-bit codes per byte, the even flat index
  // in the low nibble, sign-extended on reading (INT4, quantization.cpp:
  // 68-86, 106-122)
  packed_ = layer.packed_weights();
  const bool int4 = type_ == QuantizationType::INT4;
  std::vector<int8_t> codes(in_ * out_);
  for (size_t idx = 0; idx < codes.size(); ++idx) {
    if (!int4) {
      codes[idx] = static_cast<int8_t>(packed_[idx]);
    } else {
      const uint8_t nib = (idx % 2 == 0) ? (packed_[idx / 2] & 0x0F)
                                         : ((packed_[idx / 2] >> 4) & 0x0F);
      codes[idx] = (nib & 0x08) ? static_cast<int8_t>(nib | 0xF0)
                                : static_cast<int8_t>(nib);
    }
  }
  std::vector<float> b(out_, 0.0f);
  if (layer.bias()) b = layer.bias()->to_host();
  upload(codes, layer.scales()->to_host(), b);
}

HipQuantizedDense::HipQuantizedDense(HipBackend &backend,
                                     std::shared_ptr<Dense> float_dense,
                                     const QuantizationConfig &config)
    : be_(backend), type_(config.type) {
  const auto params = float_dense->parameters();  // weight [in, out], bias
  const Shape ws = params.at(0)->shape();
  in_ = ws.at(0);
  out_ = ws.at(1);
  const std::vector<float> w = params[0]->to_host();
  std::unique_ptr<DeviceBuffer> dw = be_.allocate(w.size() * sizeof(float));
  be_.copy_host_to_device(w.data(), *dw, w.size() * sizeof(float));
  std::unique_ptr<DeviceBuffer> dc = be_.allocate(in_ * out_);
  std::unique_ptr<DeviceBuffer> ds = be_.allocate(out_ * sizeof(float));
  const bool int4 = type_ == QuantizationType::INT4;
  check((int4 ? nnhip_quantize_w4 : nnhip_quantize_w8)(
      be_.context(), static_cast<const float *>(dw->data()), (int)in_, (int)out_,
      static_cast<int8_t *>(dc->data()), static_cast<float *>(ds->data())));
  std::vector<int8_t> t(in_ * out_);  // [out][in]
  std::vector<float> sc(out_);
  check(nnhip_d2h(be_.context(), t.data(), dc->data(), t.size()));
  check(nnhip_d2h(be_.context(), sc.data(), ds->data(), sc.size() * sizeof(float)));
  std::vector<int8_t> codes(in_ * out_);  // [in][out]
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n) codes[k * out_ + n] = t[n * in_ + k];
  // packed_weights in the reference's layout
  if (!int4) {
    packed_.assign(codes.begin(), codes.end());
  } else {
    packed_.assign((codes.size() + 1) / 2, 0);
    for (size_t idx = 0; idx < codes.size(); ++idx) {
      const uint8_t v = static_cast<uint8_t>(codes[idx]) & 0x0F;
      if (idx % 2 == 0) packed_[idx / 2] = v;
      else packed_[idx / 2] |= static_cast<uint8_t>(v << 4);
    }
  }
  std::vector<float> b(out_, 0.0f);
  if (params.size() > 1 && params[1]) b = params[1]->to_host();
  upload(codes, sc, b);
}

std::shared_ptr<Tensor> HipQuantizedDense::scales() const {
  return std::make_shared<Tensor>(Shape{out_}, host_scales_, &be_);
}

std::shared_ptr<Tensor> HipQuantizedDense::bias() const {
  return std::make_shared<Tensor>(Shape{1, out_}, host_bias_, &be_);
}

std::shared_ptr<Tensor> HipQuantizedDense::dequantize_weight() const {
  std::vector<float> w(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n)
      w[k * out_ + n] = static_cast<float>(host_codes_[k * out_ + n]) * host_scales_[n];
  return std::make_shared<Tensor>(Shape{in_, out_}, w, &be_);
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

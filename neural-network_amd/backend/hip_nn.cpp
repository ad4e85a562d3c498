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

HipQuantizedDense::HipQuantizedDense(HipBackend &backend,
                                     const QuantizedDense &layer)
    : be_(backend) {
  const Shape ws = layer.weight_shape();  // [in, out]
  in_ = ws.at(0);
  out_ = ws.at(1);
  // packed_weights hold the codes of [in][out]: one int8 per byte (INT8,
  // quantization.cpp:36-66) or two 4-bit codes per byte, the even flat index
  // in the low nibble, sign-extended on reading (INT4, quantization.cpp:
  // 68-86, 106-122); the device reads one code per byte, transposed
  // [out][in] (INT4 codes in [-7, 7] go through the int8 kernels unchanged)
  const bool int4 = layer.type() == QuantizationType::INT4;
  const std::vector<uint8_t> &pw = layer.packed_weights();
  auto code = [&](size_t idx) -> int8_t {
    if (!int4) return static_cast<int8_t>(pw[idx]);
    const uint8_t nib = (idx % 2 == 0) ? (pw[idx / 2] & 0x0F) : ((pw[idx / 2] >> 4) & 0x0F);
    return (nib & 0x08) ? static_cast<int8_t>(nib | 0xF0) : static_cast<int8_t>(nib);
  };
  std::vector<int8_t> t(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n)
      t[n * in_ + k] = code(k * out_ + n);
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

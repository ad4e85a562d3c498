// The parts of the drop-in decoder objects (hip_nn.hpp) that use the
// reference's compiled code: HipDecoder's constructor from a
// TransformerDecoder, HipMultiHeadAttention over Tensor and
// HipQuantizedDense, the Tensor face of HipQuantizedDenseCore.
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
                                     const QuantizedDense &layer) {
  const Shape ws = layer.weight_shape();  // [in, out]
  std::vector<float> b;
  if (layer.bias()) b = layer.bias()->to_host();
  core_ = std::make_unique<HipQuantizedDenseCore>(
      backend, layer.type(), ws.at(0), ws.at(1), layer.packed_weights(),
      layer.scales()->to_host(), b);
}

HipQuantizedDense::HipQuantizedDense(HipBackend &backend,
                                     std::shared_ptr<Dense> float_dense,
                                     const QuantizationConfig &config) {
  const auto params = float_dense->parameters();  // weight [in, out], bias
  const Shape ws = params.at(0)->shape();
  std::vector<float> b;
  if (params.size() > 1 && params[1]) b = params[1]->to_host();
  core_ = std::make_unique<HipQuantizedDenseCore>(
      backend, params[0]->to_host(), ws.at(0), ws.at(1), b, config.type);
}

std::shared_ptr<Tensor> HipQuantizedDense::scales() const {
  return std::make_shared<Tensor>(Shape{core_->out_features()}, core_->scales(),
                                  &core_->backend());
}

std::shared_ptr<Tensor> HipQuantizedDense::bias() const {
  return std::make_shared<Tensor>(Shape{1, core_->out_features()}, core_->bias(),
                                  &core_->backend());
}

std::shared_ptr<Tensor> HipQuantizedDense::dequantize_weight() const {
  return std::make_shared<Tensor>(weight_shape(), core_->dequantize_weight(),
                                  &core_->backend());
}

std::shared_ptr<Tensor> HipQuantizedDense::forward(
    const std::shared_ptr<Tensor> &input) {
  const Shape &s = input->shape();
  HipBackend &be = core_->backend();
  const size_t in = core_->in_features(), out = core_->out_features();
  if (input->backend() != &be || s.empty() || s.back() != in ||
      !is_contiguous(s, input->strides()))
    throw std::runtime_error(
        "HipQuantizedDense: input must be a contiguous HipBackend tensor "
        "whose last dimension is in_features");
  const size_t rows = count_elements(s) / in;
  Shape out_shape = s;
  out_shape.back() = out;
  std::shared_ptr<DeviceBuffer> y(be.allocate(rows * out * sizeof(float)));
  const float *x =
      static_cast<const float *>(input->storage()->data()) + input->offset();
  core_->forward_device(x, rows, static_cast<float *>(y->data()));
  return std::make_shared<Tensor>(out_shape, compute_strides(out_shape), 0, y,
                                  &be, DataType::FP32);
}

}  // namespace nnhip_backend

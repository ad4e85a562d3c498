// HipQuantizedDenseCore (hip_nn.hpp): QuantizedDense's codes, scales and
// forward on device pointers.  Uses only the reference's header types
// (QuantizationType), none of its compiled code.
#include "hip_nn.hpp"

#include <stdexcept>

namespace nnhip_backend {

namespace {

// one code of packed_weights (quantization.cpp:36-86, 100-122): INT8 one
// signed byte per weight; INT4 two per byte, the even flat index in the low
// nibble, sign-extended from 4 bits
int8_t unpack(const std::vector<uint8_t> &packed, size_t idx, bool int4) {
  if (!int4) return static_cast<int8_t>(packed[idx]);
  const uint8_t nib = (idx % 2 == 0) ? (packed[idx / 2] & 0x0F)
                                     : ((packed[idx / 2] >> 4) & 0x0F);
  return (nib & 0x08) ? static_cast<int8_t>(nib | 0xF0) : static_cast<int8_t>(nib);
}

std::vector<uint8_t> pack(const std::vector<int8_t> &codes, bool int4) {
  if (!int4) return std::vector<uint8_t>(codes.begin(), codes.end());
  std::vector<uint8_t> p((codes.size() + 1) / 2, 0);
  for (size_t idx = 0; idx < codes.size(); ++idx) {
    const uint8_t v = static_cast<uint8_t>(codes[idx]) & 0x0F;
    if (idx % 2 == 0) p[idx / 2] = v;
    else p[idx / 2] |= static_cast<uint8_t>(v << 4);
  }
  return p;
}

void check_sizes(size_t in, size_t out, size_t bias) {
  if (in == 0 || out == 0 || in > 0x7fffffff || out > 0x7fffffff)
    throw std::runtime_error("HipQuantizedDense: bad weight shape");
  if (bias != 0 && bias != out)
    throw std::runtime_error("HipQuantizedDense: bias size is not out_features");
}

}  // namespace

void HipQuantizedDenseCore::upload(const std::vector<int8_t> &codes_in_out,
                                   const std::vector<float> &scales,
                                   const std::vector<float> &bias) {
  host_codes_ = codes_in_out;
  host_scales_ = scales;
  host_bias_ = bias.empty() ? std::vector<float>(out_, 0.0f) : bias;
  // the device reads the codes transposed, [out][in], one per byte (INT4
  // codes in [-7, 7] go through the int8 kernels unchanged)
  std::vector<int8_t> t(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n) t[n * in_ + k] = codes_in_out[k * out_ + n];
  codes_ = be_.allocate(t.size());
  check(nnhip_h2d(be_.context(), codes_->data(), t.data(), t.size()));
  scales_ = be_.allocate(out_ * sizeof(float));
  be_.copy_host_to_device(host_scales_.data(), *scales_, out_ * sizeof(float));
  bias_ = be_.allocate(out_ * sizeof(float));
  be_.copy_host_to_device(host_bias_.data(), *bias_, out_ * sizeof(float));
}

HipQuantizedDenseCore::HipQuantizedDenseCore(HipBackend &backend,
                                             const std::vector<float> &weight,
                                             size_t in, size_t out,
                                             const std::vector<float> &bias,
                                             QuantizationType type)
    : be_(backend), type_(type), in_(in), out_(out) {
  check_sizes(in, out, bias.size());
  if (weight.size() != in * out)
    throw std::runtime_error("HipQuantizedDense: weight size is not in * out");
  std::unique_ptr<DeviceBuffer> dw = be_.allocate(weight.size() * sizeof(float));
  be_.copy_host_to_device(weight.data(), *dw, weight.size() * sizeof(float));
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
  packed_ = pack(codes, int4);
  upload(codes, sc, bias);
}

HipQuantizedDenseCore::HipQuantizedDenseCore(HipBackend &backend,
                                             QuantizationType type, size_t in,
                                             size_t out,
                                             const std::vector<uint8_t> &packed,
                                             const std::vector<float> &scales,
                                             const std::vector<float> &bias)
    : be_(backend), type_(type), in_(in), out_(out), packed_(packed) {
  check_sizes(in, out, bias.size());
  const bool int4 = type_ == QuantizationType::INT4;
  if (packed.size() != (int4 ? (in * out + 1) / 2 : in * out) ||
      scales.size() != out)
    throw std::runtime_error(
        "HipQuantizedDense: packed weights or scales do not match the shape");
  std::vector<int8_t> codes(in_ * out_);
  for (size_t idx = 0; idx < codes.size(); ++idx) codes[idx] = unpack(packed_, idx, int4);
  upload(codes, scales, bias);
}

void HipQuantizedDenseCore::forward_device(const float *x, size_t rows,
                                           float *y) const {
  if (rows == 0) return;
  check(nnhip_linear_w8a32(be_.context(), x, (int)rows, (int)in_,
                           static_cast<const int8_t *>(codes_->data()),
                           static_cast<const float *>(scales_->data()),
                           static_cast<const float *>(bias_->data()),
                           (int)out_, y, 0));
}

std::vector<float> HipQuantizedDenseCore::dequantize_weight() const {
  // static_cast<float>(Q) * s per element (quantization.cpp:96-122)
  std::vector<float> w(in_ * out_);
  for (size_t k = 0; k < in_; ++k)
    for (size_t n = 0; n < out_; ++n)
      w[k * out_ + n] = static_cast<float>(host_codes_[k * out_ + n]) * host_scales_[n];
  return w;
}

}  // namespace nnhip_backend

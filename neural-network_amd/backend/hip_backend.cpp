// HipBackend (hip_backend.hpp): each ExecutionBackend virtual packs its
// (buffer, offset, shape, strides) operands into nnhip_view and calls the
// matching libnnhip.so entry point.
#include "hip_backend.hpp"

#include <string>

namespace nnhip_backend {

void check(int status) {
  if (status != NNHIP_OK) throw std::runtime_error(nnhip_last_error());
}

namespace {

void require_fp32(const DeviceBuffer &b) {
  if (b.dtype() != DataType::FP32)
    throw std::runtime_error(
        "HipBackend: FP16 / BF16 buffers are not supported");
}

nnhip_view view(const DeviceBuffer &b, size_t offset, const Shape &shape,
                const Strides &strides) {
  require_fp32(b);
  if (shape.size() > NNHIP_MAX_RANK)
    throw std::runtime_error("HipBackend: more than 8 dimensions");
  if (strides.size() != shape.size())
    throw std::runtime_error("HipBackend: shape and strides differ in rank");
  // the last element the view reaches must lie inside the buffer; an empty
  // view reaches nothing
  size_t last = offset;
  bool empty = false;
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 0) empty = true;
    else last += (shape[i] - 1) * strides[i];
  }
  if (!empty && (last + 1) * sizeof(float) > b.size())
    throw std::runtime_error("HipBackend: view reaches past its buffer");
  nnhip_view v{};
  v.data = const_cast<void *>(b.data());
  v.offset = static_cast<int64_t>(offset);
  v.rank = static_cast<int32_t>(shape.size());
  for (size_t i = 0; i < shape.size(); ++i) {
    v.shape[i] = static_cast<int64_t>(shape[i]);
    v.strides[i] = static_cast<int64_t>(strides[i]);
  }
  return v;
}

[[noreturn]] void unsupported(const char *op) {
  throw std::runtime_error(std::string("HipBackend: ") + op +
                           " is not supported (not on the decode path)");
}

}  // namespace

HipBuffer::HipBuffer(nnhip_ctx *ctx, size_t bytes) : ctx_(ctx), bytes_(bytes) {
  check(nnhip_malloc(ctx_, bytes ? bytes : 1, &ptr_));
}

HipBuffer::~HipBuffer() { (void)nnhip_free(ctx_, ptr_); }

HipBackend::HipBackend(int device) {
  check(nnhip_init(device, &ctx_));
  // the decoder objects' sampled generation draws from std::mt19937 seeded
  // with the caller's seed, as TransformerDecoder's does (layer.cpp:1249,
  // 1394)
  try {
    check(nnhip_set_option(ctx_, "rng", 1));
  } catch (...) {
    (void)nnhip_destroy(ctx_);
    throw;
  }
}

HipBackend::~HipBackend() { (void)nnhip_destroy(ctx_); }

void HipBackend::synchronize() { check(nnhip_sync(ctx_)); }

std::unique_ptr<DeviceBuffer> HipBackend::allocate(size_t bytes) {
  return std::make_unique<HipBuffer>(ctx_, bytes);
}

void HipBackend::copy_host_to_device(const float *host_ptr,
                                     DeviceBuffer &device_buf,
                                     size_t size_bytes) {
  check(nnhip_h2d(ctx_, device_buf.data(), host_ptr, size_bytes));
}

void HipBackend::copy_to_device(const float *host_ptr, DeviceBuffer &device_buf,
                                size_t dest_offset_bytes, size_t size_bytes) {
  check(nnhip_h2d(ctx_, static_cast<char *>(device_buf.data()) + dest_offset_bytes,
                  host_ptr, size_bytes));
}

void HipBackend::copy_device_to_host(const DeviceBuffer &device_buf,
                                     float *host_ptr, size_t size_bytes) {
  check(nnhip_d2h(ctx_, host_ptr, device_buf.data(), size_bytes));
}

void HipBackend::fill(DeviceBuffer &buffer, float value) {
  require_fp32(buffer);
  check(nnhip_fill_f32(ctx_, buffer.data(), buffer.size() / sizeof(float), value));
}

void HipBackend::binary(int op, const DeviceBuffer &a, size_t a_offset,
                        const Shape &a_shape, const Strides &a_strides,
                        const DeviceBuffer &b, size_t b_offset,
                        const Shape &b_shape, const Strides &b_strides,
                        DeviceBuffer &out, size_t out_offset,
                        const Shape &out_shape, const Strides &out_strides) {
  const nnhip_view va = view(a, a_offset, a_shape, a_strides);
  const nnhip_view vb = view(b, b_offset, b_shape, b_strides);
  const nnhip_view vo = view(out, out_offset, out_shape, out_strides);
  check(nnhip_binary_f32(ctx_, op, &va, &vb, &vo));
}

void HipBackend::unary(int op, const DeviceBuffer &in, size_t in_offset,
                       const Shape &in_shape, const Strides &in_strides,
                       DeviceBuffer &out, size_t out_offset,
                       const Shape &out_shape, const Strides &out_strides) {
  const nnhip_view vi = view(in, in_offset, in_shape, in_strides);
  const nnhip_view vo = view(out, out_offset, out_shape, out_strides);
  check(nnhip_unary_f32(ctx_, op, &vi, &vo));
}

#define NNHIP_BINARY(name, op)                                                \
  void HipBackend::name(const DeviceBuffer &a, size_t a_offset,               \
                        const Shape &a_shape, const Strides &a_strides,       \
                        const DeviceBuffer &b, size_t b_offset,               \
                        const Shape &b_shape, const Strides &b_strides,       \
                        DeviceBuffer &out, size_t out_offset,                 \
                        const Shape &out_shape, const Strides &out_strides) { \
    binary(op, a, a_offset, a_shape, a_strides, b, b_offset, b_shape,         \
           b_strides, out, out_offset, out_shape, out_strides);               \
  }
NNHIP_BINARY(add, NNHIP_OP_ADD)
NNHIP_BINARY(sub, NNHIP_OP_SUB)
NNHIP_BINARY(mul, NNHIP_OP_MUL)
NNHIP_BINARY(div, NNHIP_OP_DIV)
NNHIP_BINARY(relu_backward, NNHIP_OP_RELU_BACKWARD)
NNHIP_BINARY(sigmoid_backward, NNHIP_OP_SIGMOID_BACKWARD)
NNHIP_BINARY(tanh_backward, NNHIP_OP_TANH_BACKWARD)
NNHIP_BINARY(sqrt_backward, NNHIP_OP_SQRT_BACKWARD)
NNHIP_BINARY(log_backward, NNHIP_OP_LOG_BACKWARD)
#undef NNHIP_BINARY

#define NNHIP_UNARY(name, op)                                                 \
  void HipBackend::name(const DeviceBuffer &in, size_t in_offset,             \
                        const Shape &in_shape, const Strides &in_strides,     \
                        DeviceBuffer &out, size_t out_offset,                 \
                        const Shape &out_shape, const Strides &out_strides) { \
    unary(op, in, in_offset, in_shape, in_strides, out, out_offset,           \
          out_shape, out_strides);                                            \
  }
NNHIP_UNARY(relu, NNHIP_OP_RELU)
NNHIP_UNARY(sigmoid, NNHIP_OP_SIGMOID)
NNHIP_UNARY(tanh, NNHIP_OP_TANH)
NNHIP_UNARY(sqrt, NNHIP_OP_SQRT)
NNHIP_UNARY(log, NNHIP_OP_LOG)
#undef NNHIP_UNARY

void HipBackend::matmul(const DeviceBuffer &a, size_t a_offset,
                        const Shape &a_shape, const Strides &a_strides,
                        const DeviceBuffer &b, size_t b_offset,
                        const Shape &b_shape, const Strides &b_strides,
                        DeviceBuffer &out, size_t out_offset,
                        const Shape &out_shape, const Strides &out_strides) {
  const nnhip_view va = view(a, a_offset, a_shape, a_strides);
  const nnhip_view vb = view(b, b_offset, b_shape, b_strides);
  const nnhip_view vo = view(out, out_offset, out_shape, out_strides);
  check(nnhip_matmul_f32(ctx_, &va, &vb, &vo));
}

void HipBackend::sum(const DeviceBuffer &input, size_t input_offset,
                     const Shape &input_shape, const Strides &input_strides,
                     DeviceBuffer &output, size_t output_offset,
                     const Shape &output_shape, const Strides &output_strides,
                     const std::vector<size_t> &axes) {
  const nnhip_view vi = view(input, input_offset, input_shape, input_strides);
  const nnhip_view vo = view(output, output_offset, output_shape, output_strides);
  std::vector<int64_t> ax(axes.begin(), axes.end());
  check(nnhip_sum_f32(ctx_, &vi, &vo, ax.data(), static_cast<int>(ax.size())));
}

void HipBackend::softmax(const DeviceBuffer &in, size_t in_offset,
                         const Shape &in_shape, const Strides &in_strides,
                         DeviceBuffer &out, size_t out_offset,
                         const Shape &out_shape, const Strides &out_strides,
                         size_t axis) {
  const nnhip_view vi = view(in, in_offset, in_shape, in_strides);
  const nnhip_view vo = view(out, out_offset, out_shape, out_strides);
  check(nnhip_softmax_f32(ctx_, &vi, &vo, static_cast<int>(axis)));
}

void HipBackend::softmax_backward(
    const DeviceBuffer &out, size_t out_offset, const Shape &out_shape,
    const Strides &out_strides, const DeviceBuffer &grad_out,
    size_t grad_out_offset, const Shape &grad_out_shape,
    const Strides &grad_out_strides, DeviceBuffer &grad_in,
    size_t grad_in_offset, const Shape &grad_in_shape,
    const Strides &grad_in_strides, size_t axis) {
  const nnhip_view vy = view(out, out_offset, out_shape, out_strides);
  const nnhip_view vg = view(grad_out, grad_out_offset, grad_out_shape, grad_out_strides);
  const nnhip_view vd = view(grad_in, grad_in_offset, grad_in_shape, grad_in_strides);
  check(nnhip_softmax_backward_f32(ctx_, &vy, &vg, &vd, static_cast<int>(axis)));
}

void HipBackend::embedding(const DeviceBuffer &weight, size_t weight_offset,
                           const Shape &weight_shape,
                           const Strides &weight_strides,
                           const DeviceBuffer &indices, size_t indices_offset,
                           const Shape &indices_shape,
                           const Strides &indices_strides, DeviceBuffer &out,
                           size_t out_offset, const Shape &out_shape,
                           const Strides &out_strides) {
  const nnhip_view vw = view(weight, weight_offset, weight_shape, weight_strides);
  const nnhip_view vi = view(indices, indices_offset, indices_shape, indices_strides);
  const nnhip_view vo = view(out, out_offset, out_shape, out_strides);
  check(nnhip_embedding_f32(ctx_, &vw, &vi, &vo));
}

void HipBackend::slice_backward(const DeviceBuffer &grad_slice,
                                size_t gs_offset, const Shape &gs_shape,
                                const Strides &gs_strides,
                                DeviceBuffer &grad_parent, size_t gp_offset,
                                const Shape &gp_shape,
                                const Strides &gp_strides, size_t axis,
                                size_t index) {
  const nnhip_view vs = view(grad_slice, gs_offset, gs_shape, gs_strides);
  const nnhip_view vp = view(grad_parent, gp_offset, gp_shape, gp_strides);
  check(nnhip_slice_backward_f32(ctx_, &vs, &vp, static_cast<int>(axis),
                                 static_cast<int64_t>(index)));
}

void HipBackend::conv2d(const DeviceBuffer &, size_t, const Shape &,
                        const Strides &, const DeviceBuffer &, size_t,
                        const Shape &, const Strides &, const DeviceBuffer &,
                        size_t, const Shape &, const Strides &, DeviceBuffer &,
                        size_t, const Shape &, const Strides &, size_t, size_t) {
  unsupported("conv2d");
}

void HipBackend::conv2d_backward(
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    DeviceBuffer &, size_t, const Shape &, const Strides &, DeviceBuffer &,
    size_t, const Shape &, const Strides &, DeviceBuffer &, size_t,
    const Shape &, const Strides &, size_t, size_t) {
  unsupported("conv2d_backward");
}

void HipBackend::maxpool2d(const DeviceBuffer &, size_t, const Shape &,
                           const Strides &, DeviceBuffer &, size_t,
                           const Shape &, const Strides &, size_t, size_t,
                           size_t) {
  unsupported("maxpool2d");
}

void HipBackend::maxpool2d_backward(
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    const DeviceBuffer &, size_t, const Shape &, const Strides &,
    DeviceBuffer &, size_t, const Shape &, const Strides &, size_t, size_t,
    size_t) {
  unsupported("maxpool2d_backward");
}

void HipBackend::embedding_backward(const DeviceBuffer &, size_t, const Shape &,
                                    const Strides &, const DeviceBuffer &,
                                    size_t, const Shape &, const Strides &,
                                    DeviceBuffer &, size_t, const Shape &,
                                    const Strides &) {
  unsupported("embedding_backward");
}

}  // namespace nnhip_backend

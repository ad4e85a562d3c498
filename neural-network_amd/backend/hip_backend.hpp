// HipBackend: the reference's ExecutionBackend plugin interface
// (include/backend/backend.hpp:20-221) served by libnnhip.so through its C
// ABI (include/nnhip.h), so that Tensor code (src/core/tensor.cpp) runs on
// an MI355X unchanged.  Compiled against the reference's headers
// (-I<reference>/include); it needs nothing else from the reference.
//
// Buffers are device memory (nnhip_malloc); ops are enqueued on the
// context's stream in call order, and copy_device_to_host returns with the
// data, so results are complete whenever the host reads them (the
// reference's ops are synchronous; its Tensor never dereferences
// DeviceBuffer::data() outside the backend).  Failures throw
// std::runtime_error with the library's message, the reference's
// convention.  FP32 buffers only: FP16 / BF16 storage belongs to the
// reference's AMP training path.  conv2d / maxpool2d (CNN layers) and
// embedding_backward throw: the decode path has neither.
#pragma once

#include "backend/backend.hpp"
#include "nnhip.h"

#include <memory>
#include <stdexcept>

namespace nnhip_backend {

// throws std::runtime_error(nnhip_last_error()) on a non-zero status
void check(int status);

class HipBuffer final : public DeviceBuffer {
 public:
  HipBuffer(nnhip_ctx *ctx, size_t bytes);
  ~HipBuffer() override;
  HipBuffer(const HipBuffer &) = delete;
  HipBuffer &operator=(const HipBuffer &) = delete;
  [[nodiscard]] size_t size() const noexcept override { return bytes_; }
  [[nodiscard]] void *data() noexcept override { return ptr_; }
  [[nodiscard]] const void *data() const noexcept override { return ptr_; }
  [[nodiscard]] DataType dtype() const noexcept override { return dtype_; }
  void set_dtype(DataType dt) noexcept override { dtype_ = dt; }

 private:
  nnhip_ctx *ctx_;
  void *ptr_ = nullptr;
  size_t bytes_;
  DataType dtype_ = DataType::FP32;
};

class HipBackend final : public ExecutionBackend {
 public:
  // one HIP stream on `device` (nnhip_init)
  explicit HipBackend(int device = 0);
  ~HipBackend() override;
  HipBackend(const HipBackend &) = delete;
  HipBackend &operator=(const HipBackend &) = delete;
  // the library context, for the fused entry points (nnhip_decoder_*,
  // nnhip_generate_speculative, ...)
  [[nodiscard]] nnhip_ctx *context() const noexcept { return ctx_; }
  // waits for every op enqueued so far
  void synchronize();

  [[nodiscard]] std::unique_ptr<DeviceBuffer> allocate(size_t bytes) override;
  void copy_host_to_device(const float *host_ptr, DeviceBuffer &device_buf,
                           size_t size_bytes) override;
  void copy_to_device(const float *host_ptr, DeviceBuffer &device_buf,
                      size_t dest_offset_bytes, size_t size_bytes) override;
  void copy_device_to_host(const DeviceBuffer &device_buf, float *host_ptr,
                           size_t size_bytes) override;
  void fill(DeviceBuffer &buffer, float value) override;

  void add(const DeviceBuffer &a, size_t a_offset, const Shape &a_shape,
           const Strides &a_strides, const DeviceBuffer &b, size_t b_offset,
           const Shape &b_shape, const Strides &b_strides, DeviceBuffer &out,
           size_t out_offset, const Shape &out_shape,
           const Strides &out_strides) override;
  void sub(const DeviceBuffer &a, size_t a_offset, const Shape &a_shape,
           const Strides &a_strides, const DeviceBuffer &b, size_t b_offset,
           const Shape &b_shape, const Strides &b_strides, DeviceBuffer &out,
           size_t out_offset, const Shape &out_shape,
           const Strides &out_strides) override;
  void mul(const DeviceBuffer &a, size_t a_offset, const Shape &a_shape,
           const Strides &a_strides, const DeviceBuffer &b, size_t b_offset,
           const Shape &b_shape, const Strides &b_strides, DeviceBuffer &out,
           size_t out_offset, const Shape &out_shape,
           const Strides &out_strides) override;
  void div(const DeviceBuffer &a, size_t a_offset, const Shape &a_shape,
           const Strides &a_strides, const DeviceBuffer &b, size_t b_offset,
           const Shape &b_shape, const Strides &b_strides, DeviceBuffer &out,
           size_t out_offset, const Shape &out_shape,
           const Strides &out_strides) override;
  void matmul(const DeviceBuffer &a, size_t a_offset, const Shape &a_shape,
              const Strides &a_strides, const DeviceBuffer &b, size_t b_offset,
              const Shape &b_shape, const Strides &b_strides, DeviceBuffer &out,
              size_t out_offset, const Shape &out_shape,
              const Strides &out_strides) override;
  void sum(const DeviceBuffer &input, size_t input_offset,
           const Shape &input_shape, const Strides &input_strides,
           DeviceBuffer &output, size_t output_offset,
           const Shape &output_shape, const Strides &output_strides,
           const std::vector<size_t> &axes) override;
  void relu(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
            const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
            const Shape &out_shape, const Strides &out_strides) override;
  void relu_backward(const DeviceBuffer &in, size_t in_offset,
                     const Shape &in_shape, const Strides &in_strides,
                     const DeviceBuffer &grad_out, size_t grad_out_offset,
                     const Shape &grad_out_shape,
                     const Strides &grad_out_strides, DeviceBuffer &grad_in,
                     size_t grad_in_offset, const Shape &grad_in_shape,
                     const Strides &grad_in_strides) override;
  void sigmoid(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
               const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
               const Shape &out_shape, const Strides &out_strides) override;
  void sigmoid_backward(const DeviceBuffer &out, size_t out_offset,
                        const Shape &out_shape, const Strides &out_strides,
                        const DeviceBuffer &grad_out, size_t grad_out_offset,
                        const Shape &grad_out_shape,
                        const Strides &grad_out_strides, DeviceBuffer &grad_in,
                        size_t grad_in_offset, const Shape &grad_in_shape,
                        const Strides &grad_in_strides) override;
  void tanh(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
            const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
            const Shape &out_shape, const Strides &out_strides) override;
  void tanh_backward(const DeviceBuffer &out, size_t out_offset,
                     const Shape &out_shape, const Strides &out_strides,
                     const DeviceBuffer &grad_out, size_t grad_out_offset,
                     const Shape &grad_out_shape,
                     const Strides &grad_out_strides, DeviceBuffer &grad_in,
                     size_t grad_in_offset, const Shape &grad_in_shape,
                     const Strides &grad_in_strides) override;
  void softmax(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
               const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
               const Shape &out_shape, const Strides &out_strides,
               size_t axis) override;
  void softmax_backward(const DeviceBuffer &out, size_t out_offset,
                        const Shape &out_shape, const Strides &out_strides,
                        const DeviceBuffer &grad_out, size_t grad_out_offset,
                        const Shape &grad_out_shape,
                        const Strides &grad_out_strides, DeviceBuffer &grad_in,
                        size_t grad_in_offset, const Shape &grad_in_shape,
                        const Strides &grad_in_strides, size_t axis) override;
  void sqrt(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
            const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
            const Shape &out_shape, const Strides &out_strides) override;
  void sqrt_backward(const DeviceBuffer &out, size_t out_offset,
                     const Shape &out_shape, const Strides &out_strides,
                     const DeviceBuffer &grad_out, size_t grad_out_offset,
                     const Shape &grad_out_shape,
                     const Strides &grad_out_strides, DeviceBuffer &grad_in,
                     size_t grad_in_offset, const Shape &grad_in_shape,
                     const Strides &grad_in_strides) override;
  void log(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
           const Strides &in_strides, DeviceBuffer &out, size_t out_offset,
           const Shape &out_shape, const Strides &out_strides) override;
  void log_backward(const DeviceBuffer &in, size_t in_offset,
                    const Shape &in_shape, const Strides &in_strides,
                    const DeviceBuffer &grad_out, size_t grad_out_offset,
                    const Shape &grad_out_shape,
                    const Strides &grad_out_strides, DeviceBuffer &grad_in,
                    size_t grad_in_offset, const Shape &grad_in_shape,
                    const Strides &grad_in_strides) override;
  void conv2d(const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
              const Strides &in_strides, const DeviceBuffer &weight,
              size_t weight_offset, const Shape &weight_shape,
              const Strides &weight_strides, const DeviceBuffer &bias,
              size_t bias_offset, const Shape &bias_shape,
              const Strides &bias_strides, DeviceBuffer &out,
              size_t out_offset, const Shape &out_shape,
              const Strides &out_strides, size_t padding,
              size_t stride) override;
  void conv2d_backward(
      const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
      const Strides &in_strides, const DeviceBuffer &weight,
      size_t weight_offset, const Shape &weight_shape,
      const Strides &weight_strides, const DeviceBuffer &grad_out,
      size_t grad_out_offset, const Shape &grad_out_shape,
      const Strides &grad_out_strides, DeviceBuffer &grad_in,
      size_t grad_in_offset, const Shape &grad_in_shape,
      const Strides &grad_in_strides, DeviceBuffer &grad_weight,
      size_t grad_weight_offset, const Shape &grad_weight_shape,
      const Strides &grad_weight_strides, DeviceBuffer &grad_bias,
      size_t grad_bias_offset, const Shape &grad_bias_shape,
      const Strides &grad_bias_strides, size_t padding,
      size_t stride) override;
  void maxpool2d(const DeviceBuffer &in, size_t in_offset,
                 const Shape &in_shape, const Strides &in_strides,
                 DeviceBuffer &out, size_t out_offset, const Shape &out_shape,
                 const Strides &out_strides, size_t pool_h, size_t pool_w,
                 size_t stride) override;
  void maxpool2d_backward(
      const DeviceBuffer &in, size_t in_offset, const Shape &in_shape,
      const Strides &in_strides, const DeviceBuffer &out, size_t out_offset,
      const Shape &out_shape, const Strides &out_strides,
      const DeviceBuffer &grad_out, size_t grad_out_offset,
      const Shape &grad_out_shape, const Strides &grad_out_strides,
      DeviceBuffer &grad_in, size_t grad_in_offset, const Shape &grad_in_shape,
      const Strides &grad_in_strides, size_t pool_h, size_t pool_w,
      size_t stride) override;
  void embedding(const DeviceBuffer &weight, size_t weight_offset,
                 const Shape &weight_shape, const Strides &weight_strides,
                 const DeviceBuffer &indices, size_t indices_offset,
                 const Shape &indices_shape, const Strides &indices_strides,
                 DeviceBuffer &out, size_t out_offset, const Shape &out_shape,
                 const Strides &out_strides) override;
  void embedding_backward(
      const DeviceBuffer &grad_out, size_t grad_out_offset,
      const Shape &grad_out_shape, const Strides &grad_out_strides,
      const DeviceBuffer &indices, size_t indices_offset,
      const Shape &indices_shape, const Strides &indices_strides,
      DeviceBuffer &grad_weight, size_t grad_weight_offset,
      const Shape &grad_weight_shape,
      const Strides &grad_weight_strides) override;
  void slice_backward(const DeviceBuffer &grad_slice, size_t gs_offset,
                      const Shape &gs_shape, const Strides &gs_strides,
                      DeviceBuffer &grad_parent, size_t gp_offset,
                      const Shape &gp_shape, const Strides &gp_strides,
                      size_t axis, size_t index) override;

 private:
  void binary(int op, const DeviceBuffer &a, size_t a_offset,
              const Shape &a_shape, const Strides &a_strides,
              const DeviceBuffer &b, size_t b_offset, const Shape &b_shape,
              const Strides &b_strides, DeviceBuffer &out, size_t out_offset,
              const Shape &out_shape, const Strides &out_strides);
  void unary(int op, const DeviceBuffer &in, size_t in_offset,
             const Shape &in_shape, const Strides &in_strides,
             DeviceBuffer &out, size_t out_offset, const Shape &out_shape,
             const Strides &out_strides);
  nnhip_ctx *ctx_ = nullptr;
};

}  // namespace nnhip_backend

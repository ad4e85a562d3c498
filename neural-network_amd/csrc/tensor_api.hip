// C ABI of the ExecutionBackend ops (include/nnhip.h, "ExecutionBackend
// ops"): argument checks and the conversion of nnhip_view into the kernels'
// TensorView; the kernels are in tensor_ops.hip.
#include "api_common.hpp"

using nnhip::guard;

namespace {

void set_device(nnhip_ctx *ctx) { NNHIP_CHECK(hipSetDevice(ctx->c.device)); }

nnhip::TensorView view_of(const nnhip_view *v, const char *what) {
  NNHIP_REQUIRE(v, nnhip::kErrArg, std::string(what) + ": view is NULL");
  NNHIP_REQUIRE(v->rank >= 0 && v->rank <= NNHIP_MAX_RANK, nnhip::kErrArg,
                std::string(what) + ": rank out of range");
  NNHIP_REQUIRE(v->offset >= 0, nnhip::kErrArg,
                std::string(what) + ": negative offset");
  nnhip::TensorView t;
  t.data = v->data;
  t.offset = v->offset;
  t.rank = v->rank;
  for (int i = 0; i < v->rank; ++i) {
    t.shape[i] = v->shape[i];
    t.strides[i] = v->strides[i];
  }
  return t;
}

}  // namespace

extern "C" {

int nnhip_binary_f32(nnhip_ctx *ctx, int op, const nnhip_view *a,
                     const nnhip_view *b, const nnhip_view *out) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_binary_f32: ctx is NULL");
    NNHIP_REQUIRE(op >= NNHIP_OP_ADD && op <= NNHIP_OP_LOG_BACKWARD,
                  nnhip::kErrArg, "nnhip_binary_f32: unknown op");
    set_device(ctx);
    nnhip::launch_binary(ctx->c.stream, op, view_of(a, "binary"),
                         view_of(b, "binary"), view_of(out, "binary"));
  });
}

int nnhip_unary_f32(nnhip_ctx *ctx, int op, const nnhip_view *in,
                    const nnhip_view *out) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_unary_f32: ctx is NULL");
    NNHIP_REQUIRE(op >= NNHIP_OP_RELU && op <= NNHIP_OP_LOG, nnhip::kErrArg,
                  "nnhip_unary_f32: unknown op");
    set_device(ctx);
    nnhip::launch_unary(ctx->c.stream, op, view_of(in, "unary"),
                        view_of(out, "unary"));
  });
}

int nnhip_matmul_f32(nnhip_ctx *ctx, const nnhip_view *a, const nnhip_view *b,
                     const nnhip_view *out) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_matmul_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_matmul(ctx->c.stream, view_of(a, "matmul"),
                         view_of(b, "matmul"), view_of(out, "matmul"));
  });
}

int nnhip_sum_f32(nnhip_ctx *ctx, const nnhip_view *in, const nnhip_view *out,
                  const int64_t *axes, int naxes) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_sum_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_sum(ctx->c.stream, view_of(in, "sum"), view_of(out, "sum"),
                      axes, naxes);
  });
}

int nnhip_softmax_f32(nnhip_ctx *ctx, const nnhip_view *in,
                      const nnhip_view *out, int axis) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_softmax_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_softmax(ctx->c.stream, view_of(in, "softmax"),
                          view_of(out, "softmax"), axis);
  });
}

int nnhip_softmax_backward_f32(nnhip_ctx *ctx, const nnhip_view *y,
                               const nnhip_view *dy, const nnhip_view *dx,
                               int axis) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_softmax_backward_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_softmax_backward(ctx->c.stream, view_of(y, "softmax_backward"),
                                   view_of(dy, "softmax_backward"),
                                   view_of(dx, "softmax_backward"), axis);
  });
}

int nnhip_embedding_f32(nnhip_ctx *ctx, const nnhip_view *weight,
                        const nnhip_view *indices, const nnhip_view *out) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_embedding_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_embedding(ctx->c.stream, view_of(weight, "embedding"),
                            view_of(indices, "embedding"),
                            view_of(out, "embedding"));
  });
}

int nnhip_slice_backward_f32(nnhip_ctx *ctx, const nnhip_view *grad_slice,
                             const nnhip_view *grad_parent, int axis,
                             int64_t index) {
  return guard([&] {
    NNHIP_REQUIRE(ctx, nnhip::kErrArg, "nnhip_slice_backward_f32: ctx is NULL");
    set_device(ctx);
    nnhip::launch_slice_backward(ctx->c.stream,
                                 view_of(grad_slice, "slice_backward"),
                                 view_of(grad_parent, "slice_backward"), axis,
                                 index);
  });
}

int nnhip_fill_f32(nnhip_ctx *ctx, void *dev, size_t count, float value) {
  return guard([&] {
    NNHIP_REQUIRE(ctx && (dev || count == 0), nnhip::kErrArg,
                  "nnhip_fill_f32: bad argument");
    set_device(ctx);
    if (count)
      nnhip::launch_fill(ctx->c.stream, static_cast<float *>(dev),
                         (int64_t)count, value);
  });
}

}  // extern "C"

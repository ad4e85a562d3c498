// Strided tensor ops of the reference's ExecutionBackend on gfx950: the
// element-wise binary and unary ops, matmul, sum over axes, softmax along
// an axis and the embedding gather (include/backend/backend.hpp:35-206),
// with the CpuBackend's semantics (src/backend/cpu_backend.cpp):
//
// * operands are (buffer, element offset, shape, strides); an input's shape
//   is right-aligned against the output's and its size-1 dimensions
//   broadcast (get_input_offset, cpu_backend.cpp:69-88);
// * matmul is 2-D, out[r][c] = sum_k a[r][k] * b[k][c] accumulated in
//   ascending k with separately rounded products and sums (the naive loop of
//   cpu_backend.cpp:374-385; the sgemm it uses for row-major operands fixes
//   no order);
// * sum adds the inputs of each output in ascending input index, as the
//   serial loop of cpu_backend.cpp:389-459 does, so results are bit-equal;
// * softmax is exp(x - max) / sum along the axis (cpu_backend.cpp:523-583);
// * embedding reads fp32 ids, out-of-range ids take row 0
//   (cpu_backend.cpp:998-1033).
//
// These ops are HBM-bound streams (matmul aside, which is not on the decode
// path): a thread per output element, coalesced along the innermost
// dimension, float4 on contiguous same-shape operands.
#include "nnhip_internal.hpp"

#include <hip/hip_runtime.h>

// Every product and sum below is rounded on its own, as in the reference's
// scalar loops (no multiply-add is fused).
#pragma clang fp contract(off)

namespace nnhip {

namespace {

constexpr int kBlock = 256;

struct Dims {
  int rank;
  int64_t shape[kMaxRank];
  int64_t stride[kMaxRank];
};

__device__ __forceinline__ float apply_binary(int op, float a, float b) {
  switch (op) {
    case kOpAdd: return a + b;
    case kOpSub: return a - b;
    case kOpMul: return a * b;
    case kOpDiv: return a / b;
    // backward ops: a is the forward input or output, b the upstream gradient
    // (cpu_backend.cpp:473-481, 492-502, 513-521, 659-669, 680-690)
    case kOpReluBack: return a > 0.0f ? b : 0.0f;
    case kOpSigmoidBack: return (b * a) * (1.0f - a);
    case kOpTanhBack: return b * (1.0f - a * a);
    case kOpSqrtBack: return b * (0.5f / (a + 1e-8f));
    default: return b / (a + 1e-8f);  // kOpLogBack
  }
}

__device__ __forceinline__ float apply_unary(int op, float x) {
  switch (op) {
    case kOpRelu: return fmaxf(x, 0.0f);
    case kOpSigmoid: return 1.0f / (1.0f + expf(-x));
    case kOpTanh: return tanhf(x);
    case kOpSqrt: return sqrtf(x);
    default: return logf(x + 1e-8f);  // kOpLog
  }
}

// offset of the operand element that output element `flat` reads: the
// operand's dims are right-aligned against the output's, size-1 dims
// broadcast
__device__ __forceinline__ int64_t operand_offset(int64_t flat, const Dims &out,
                                                  const Dims &in) {
  int64_t off = 0;
  const int lead = out.rank - in.rank;
  for (int d = out.rank - 1; d >= 0; --d) {
    const int64_t c = flat % out.shape[d];
    flat /= out.shape[d];
    const int id = d - lead;
    if (id >= 0 && in.shape[id] > 1) off += c * in.stride[id];
  }
  return off;
}

__global__ __launch_bounds__(kBlock) void binary_kernel(
    int op, const float *__restrict__ a, Dims da, const float *__restrict__ b,
    Dims db, float *__restrict__ o, Dims dout, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    const float x = a[operand_offset(i, dout, da)];
    const float y = b[operand_offset(i, dout, db)];
    o[operand_offset(i, dout, dout)] = apply_binary(op, x, y);
  }
}

// contiguous operands of one shape: four elements a thread
__global__ __launch_bounds__(kBlock) void binary_flat_kernel(
    int op, const float *__restrict__ a, const float *__restrict__ b,
    float *__restrict__ o, int64_t n) {
  const int64_t n4 = n / 4;
  for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kBlock) {
    const float4 x = reinterpret_cast<const float4 *>(a)[i];
    const float4 y = reinterpret_cast<const float4 *>(b)[i];
    reinterpret_cast<float4 *>(o)[i] =
        make_float4(apply_binary(op, x.x, y.x), apply_binary(op, x.y, y.y),
                    apply_binary(op, x.z, y.z), apply_binary(op, x.w, y.w));
  }
  for (int64_t i = n4 * 4 + blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    o[i] = apply_binary(op, a[i], b[i]);
}

__global__ __launch_bounds__(kBlock) void unary_kernel(
    int op, const float *__restrict__ a, Dims da, float *__restrict__ o,
    Dims dout, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    o[operand_offset(i, dout, dout)] = apply_unary(op, a[operand_offset(i, dout, da)]);
}

// 2-D matmul on 64 x 64 output tiles: a 16 x 16 thread block, each thread
// 4 x 4 outputs; K staged through LDS 16 at a time.  Every output adds its
// products in ascending k, each product and sum rounded on its own.
constexpr int kMT = 64, kKT = 16;
__global__ __launch_bounds__(kBlock) void matmul_kernel(
    const float *__restrict__ a, int64_t sa0, int64_t sa1,
    const float *__restrict__ b, int64_t sb0, int64_t sb1,
    float *__restrict__ o, int64_t so0, int64_t so1, int M, int N, int K) {
  __shared__ float As[kKT][kMT + 1];
  __shared__ float Bs[kKT][kMT + 1];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int r0 = blockIdx.y * kMT, c0 = blockIdx.x * kMT;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kKT) {
    for (int e = threadIdx.x; e < kKT * kMT; e += kBlock) {
      const int kk = e / kMT, mm = e % kMT;
      const int r = r0 + mm, c = c0 + mm, k = k0 + kk;
      As[kk][mm] = (r < M && k < K) ? a[r * sa0 + k * sa1] : 0.0f;
      Bs[kk][mm] = (c < N && k < K) ? b[k * sb0 + c * sb1] : 0.0f;
    }
    __syncthreads();
    const int kn = min(kKT, K - k0);
    for (int kk = 0; kk < kn; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = acc[i][j] + av[i] * bv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + ty * 4 + i, c = c0 + tx * 4 + j;
      if (r < M && c < N) o[r * so0 + c * so1] = acc[i][j];
    }
}

// One thread per output element: its inputs are the input elements whose
// kept coordinates equal the output's; they are visited with the summed
// coordinates in row-major order, i.e. in ascending input index.
__global__ __launch_bounds__(kBlock) void sum_kernel(
    const float *__restrict__ in, Dims din, float *__restrict__ o, Dims dout,
    uint32_t axes_mask, int keepdims, int64_t n_out, int64_t n_red) {
  for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n_out;
       i += (int64_t)gridDim.x * kBlock) {
    // coordinates of the kept input dims, from the output index
    int64_t base = 0, t = i;
    for (int d = din.rank - 1, od = dout.rank - 1; d >= 0; --d) {
      const bool summed = (axes_mask >> d) & 1u;
      if (summed) {
        if (keepdims) {
          t /= dout.shape[od];
          --od;
        }
        continue;
      }
      const int64_t c = t % dout.shape[od];
      t /= dout.shape[od];
      --od;
      base += c * din.stride[d];
    }
    float acc = 0.0f;
    for (int64_t r = 0; r < n_red; ++r) {
      int64_t off = base, u = r;
      for (int d = din.rank - 1; d >= 0; --d) {
        if (!((axes_mask >> d) & 1u)) continue;
        off += (u % din.shape[d]) * din.stride[d];
        u /= din.shape[d];
      }
      acc = acc + in[off];
    }
    o[operand_offset(i, dout, dout)] = acc;
  }
}

// One workgroup per slice along `axis`: max, sum of exp(x - max), then
// exp(x - max) / sum.
__global__ __launch_bounds__(kBlock) void softmax_kernel(
    const float *__restrict__ in, Dims din, float *__restrict__ o, Dims dout,
    int axis, int64_t n_slices) {
  __shared__ float red[kBlock / 64];
  const int64_t L = din.shape[axis];
  for (int64_t sl = blockIdx.x; sl < n_slices; sl += gridDim.x) {
    // coordinates of the slice (all dims but axis), row-major
    int64_t ib = 0, ob = 0, t = sl;
    for (int d = din.rank - 1; d >= 0; --d) {
      if (d == axis) continue;
      const int64_t c = t % din.shape[d];
      t /= din.shape[d];
      if (din.shape[d] > 1) ib += c * din.stride[d];
      if (dout.shape[d] > 1) ob += c * dout.stride[d];
    }
    const int64_t si = din.shape[axis] > 1 ? din.stride[axis] : 0;
    const int64_t so = dout.shape[axis] > 1 ? dout.stride[axis] : 0;
    float mx = -INFINITY;
    for (int64_t j = threadIdx.x; j < L; j += kBlock) mx = fmaxf(mx, in[ib + j * si]);
    mx = wave_max_all(mx);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s = 0.0f;
    for (int64_t j = threadIdx.x; j < L; j += kBlock) s += expf(in[ib + j * si] - mx);
    s = wave_sum_all(s);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    for (int64_t j = threadIdx.x; j < L; j += kBlock)
      o[ob + j * so] = expf(in[ib + j * si] - mx) / s;
  }
}

// softmax_backward (cpu_backend.cpp:586-638): per slice along `axis`,
// s = sum_j dy_j * y_j, dx_j = y_j * (dy_j - s).
__global__ __launch_bounds__(kBlock) void softmax_backward_kernel(
    const float *__restrict__ y, Dims dy_, const float *__restrict__ g, Dims dg,
    float *__restrict__ o, Dims dout, int axis, int64_t n_slices) {
  __shared__ float red[kBlock / 64];
  const int64_t L = dout.shape[axis];
  for (int64_t sl = blockIdx.x; sl < n_slices; sl += gridDim.x) {
    // the slice's flat index with coordinate 0 along the axis
    int64_t t = sl, f0 = 0, mul = 1;
    for (int d = dout.rank - 1; d >= 0; --d) {
      if (d == axis) { mul *= dout.shape[d]; continue; }
      f0 += (t % dout.shape[d]) * mul;
      t /= dout.shape[d];
      mul *= dout.shape[d];
    }
    int64_t ax = 1;
    for (int d = dout.rank - 1; d > axis; --d) ax *= dout.shape[d];
    float s = 0.0f;
    for (int64_t j = threadIdx.x; j < L; j += kBlock) {
      const int64_t f = f0 + j * ax;
      s += g[operand_offset(f, dout, dg)] * y[operand_offset(f, dout, dy_)];
    }
    s = wave_sum_all(s);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    for (int64_t j = threadIdx.x; j < L; j += kBlock) {
      const int64_t f = f0 + j * ax;
      const float yv = y[operand_offset(f, dout, dy_)];
      o[operand_offset(f, dout, dout)] =
          yv * (g[operand_offset(f, dout, dg)] - s);
    }
  }
}

// slice_backward (cpu_backend.cpp:1082-1120): the parent gradient at index
// `index` along `axis` gains the slice's gradient.
__global__ __launch_bounds__(kBlock) void slice_backward_kernel(
    const float *__restrict__ gs, Dims dgs, float *__restrict__ gp, Dims dgp,
    int axis, int64_t index, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    int64_t t = i, off = 0;
    for (int d = dgp.rank - 1, sd = dgs.rank - 1; d >= 0; --d) {
      int64_t c;
      if (d == axis) {
        c = index;
      } else {
        c = t % dgs.shape[sd];
        t /= dgs.shape[sd];
        --sd;
      }
      off += c * dgp.stride[d];
    }
    gp[off] += gs[operand_offset(i, dgs, dgs)];
  }
}

// out[n][t][:] = weight[id][:] with id = (size_t)indices[n][t], 0 when out
// of range; one wave per (n, t) row.
__global__ __launch_bounds__(kBlock) void embedding_kernel(
    const float *__restrict__ w, int64_t V, int64_t D, int64_t sw0, int64_t sw1,
    const float *__restrict__ ids, int64_t T, int64_t si0, int64_t si1,
    float *__restrict__ o, int64_t so0, int64_t so1, int64_t so2, int64_t rows) {
  const int64_t row = blockIdx.x * (int64_t)(kBlock / 64) + threadIdx.x / 64;
  if (row >= rows) return;
  const int64_t n = row / T, t = row % T;
  const float f = ids[n * si0 + t * si1];
  // (size_t) of a negative or NaN id is out of range in the reference
  const int64_t id = (f >= 0.0f && f < (float)V) ? (int64_t)f : 0;
  const int64_t v = id < V ? id : 0;
  for (int64_t d = threadIdx.x & 63; d < D; d += 64)
    o[n * so0 + t * so1 + d * so2] = w[v * sw0 + d * sw1];
}

Dims to_dims(const TensorView &v) {
  Dims d;
  d.rank = v.rank;
  for (int i = 0; i < kMaxRank; ++i) {
    d.shape[i] = i < v.rank ? v.shape[i] : 1;
    d.stride[i] = i < v.rank ? v.strides[i] : 0;
  }
  return d;
}

int64_t numel(const TensorView &v) {
  int64_t n = 1;
  for (int i = 0; i < v.rank; ++i) n *= v.shape[i];
  return n;
}

bool contiguous(const TensorView &v) {
  int64_t e = 1;
  for (int i = v.rank - 1; i >= 0; --i) {
    if (v.shape[i] != 1 && v.strides[i] != e) return false;
    e *= v.shape[i];
  }
  return true;
}

bool same_shape(const TensorView &a, const TensorView &b) {
  if (a.rank != b.rank) return false;
  for (int i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i]) return false;
  return true;
}

// `in` broadcasts to `out` under CpuBackend's rule (right-aligned dims, each
// equal to the output's or 1); anything else would index past `in`
bool broadcasts_to(const TensorView &in, const TensorView &out) {
  if (in.rank > out.rank) return false;
  const int lead = out.rank - in.rank;
  for (int i = 0; i < in.rank; ++i)
    if (in.shape[i] != 1 && in.shape[i] != out.shape[lead + i]) return false;
  return true;
}

void check_view(const TensorView &v, const char *what) {
  NNHIP_REQUIRE(v.data && v.rank >= 0 && v.rank <= kMaxRank, kErrArg,
                std::string(what) + ": bad tensor view");
  for (int i = 0; i < v.rank; ++i)
    NNHIP_REQUIRE(v.shape[i] >= 0 && v.strides[i] >= 0, kErrArg,
                  std::string(what) + ": negative extent or stride");
}

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kBlock - 1) / kBlock;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, 65536));
}

const float *at(const TensorView &v) { return static_cast<const float *>(v.data) + v.offset; }
float *at_mut(const TensorView &v) { return static_cast<float *>(v.data) + v.offset; }

}  // namespace

void launch_binary(hipStream_t st, int op, const TensorView &a,
                   const TensorView &b, const TensorView &out) {
  check_view(a, "binary"); check_view(b, "binary"); check_view(out, "binary");
  NNHIP_REQUIRE(op >= kOpAdd && op <= kOpLogBack, kErrArg, "binary: unknown op");
  NNHIP_REQUIRE(broadcasts_to(a, out) && broadcasts_to(b, out), kErrArg,
                "binary: operand shape does not broadcast to the output's");
  const int64_t n = numel(out);
  if (n == 0) return;
  if (same_shape(a, out) && same_shape(b, out) && contiguous(a) &&
      contiguous(b) && contiguous(out) && ((a.offset | b.offset | out.offset) & 3) == 0) {
    hipLaunchKernelGGL(binary_flat_kernel, dim3(grid_for((n + 3) / 4)), dim3(kBlock),
                       0, st, op, at(a), at(b), at_mut(out), n);
  } else {
    hipLaunchKernelGGL(binary_kernel, dim3(grid_for(n)), dim3(kBlock), 0, st, op,
                       at(a), to_dims(a), at(b), to_dims(b), at_mut(out),
                       to_dims(out), n);
  }
  NNHIP_CHECK(hipGetLastError());
}

void launch_unary(hipStream_t st, int op, const TensorView &in,
                  const TensorView &out) {
  check_view(in, "unary"); check_view(out, "unary");
  NNHIP_REQUIRE(op >= kOpRelu && op <= kOpLog, kErrArg, "unary: unknown op");
  NNHIP_REQUIRE(broadcasts_to(in, out), kErrArg,
                "unary: input shape does not broadcast to the output's");
  const int64_t n = numel(out);
  if (n == 0) return;
  hipLaunchKernelGGL(unary_kernel, dim3(grid_for(n)), dim3(kBlock), 0, st, op,
                     at(in), to_dims(in), at_mut(out), to_dims(out), n);
  NNHIP_CHECK(hipGetLastError());
}

void launch_matmul(hipStream_t st, const TensorView &a, const TensorView &b,
                   const TensorView &out) {
  check_view(a, "matmul"); check_view(b, "matmul"); check_view(out, "matmul");
  // messages of cpu_backend.cpp:332-342
  NNHIP_REQUIRE(a.rank == 2 && b.rank == 2 && out.rank == 2, kErrArg,
                "Matmul only supports 2D matrices.");
  const int64_t M = a.shape[0], K = a.shape[1], N = b.shape[1];
  NNHIP_REQUIRE(b.shape[0] == K && out.shape[0] == M && out.shape[1] == N,
                kErrArg, "Incompatible shapes for matmul.");
  NNHIP_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), kErrArg,
                "matmul: extent too large");
  if (M == 0 || N == 0) return;
  const dim3 grid((unsigned)((N + kMT - 1) / kMT), (unsigned)((M + kMT - 1) / kMT));
  hipLaunchKernelGGL(matmul_kernel, grid, dim3(kBlock), 0, st, at(a), a.strides[0],
                     a.strides[1], at(b), b.strides[0], b.strides[1], at_mut(out),
                     out.strides[0], out.strides[1], (int)M, (int)N, (int)K);
  NNHIP_CHECK(hipGetLastError());
}

void launch_sum(hipStream_t st, const TensorView &in, const TensorView &out,
                const int64_t *axes, int naxes) {
  check_view(in, "sum"); check_view(out, "sum");
  NNHIP_REQUIRE(naxes >= 0 && (naxes == 0 || axes), kErrArg, "sum: bad axes");
  uint32_t mask = 0;
  for (int i = 0; i < naxes; ++i) {
    NNHIP_REQUIRE(axes[i] >= 0 && axes[i] < in.rank, kErrArg, "sum: axis out of range");
    mask |= 1u << axes[i];
  }
  int nsum = 0;
  int64_t n_red = 1;
  for (int d = 0; d < in.rank; ++d)
    if ((mask >> d) & 1u) { ++nsum; n_red *= in.shape[d]; }
  // the reference keeps the summed dims when the output has the input's
  // rank (cpu_backend.cpp:413-426), else drops them (:427-437)
  const bool keep = out.rank == in.rank;
  NNHIP_REQUIRE(keep || out.rank == in.rank - nsum, kErrArg,
                "sum: output rank does not match the axes");
  for (int d = 0, od = 0; d < in.rank; ++d) {
    const bool summed = (mask >> d) & 1u;
    if (summed && !keep) continue;
    NNHIP_REQUIRE(out.shape[od] == (summed ? 1 : in.shape[d]), kErrArg,
                  "sum: output shape does not match the axes");
    ++od;
  }
  const int64_t n_out = numel(out);
  if (n_out == 0) return;
  hipLaunchKernelGGL(sum_kernel, dim3(grid_for(n_out)), dim3(kBlock), 0, st,
                     at(in), to_dims(in), at_mut(out), to_dims(out), mask,
                     keep ? 1 : 0, n_out, n_red);
  NNHIP_CHECK(hipGetLastError());
}

void launch_softmax(hipStream_t st, const TensorView &in, const TensorView &out,
                    int axis) {
  check_view(in, "softmax"); check_view(out, "softmax");
  NNHIP_REQUIRE(axis >= 0 && axis < in.rank && same_shape(in, out), kErrArg,
                "softmax: bad axis or shapes");
  const int64_t n = numel(in);
  if (n == 0) return;
  const int64_t slices = n / in.shape[axis];
  hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)std::min<int64_t>(slices, 65536)),
                     dim3(kBlock), 0, st, at(in), to_dims(in), at_mut(out),
                     to_dims(out), axis, slices);
  NNHIP_CHECK(hipGetLastError());
}

void launch_softmax_backward(hipStream_t st, const TensorView &y,
                             const TensorView &dy, const TensorView &dx,
                             int axis) {
  check_view(y, "softmax_backward"); check_view(dy, "softmax_backward");
  check_view(dx, "softmax_backward");
  // grad_out broadcasts against the output's shape, as in
  // CpuBackend::softmax_backward (get_input_offset over out_shape)
  NNHIP_REQUIRE(axis >= 0 && axis < y.rank && same_shape(y, dx) && broadcasts_to(dy, y),
                kErrArg, "softmax_backward: bad axis or shapes");
  const int64_t n = numel(y);
  if (n == 0) return;
  const int64_t slices = n / y.shape[axis];
  hipLaunchKernelGGL(softmax_backward_kernel,
                     dim3((unsigned)std::min<int64_t>(slices, 65536)), dim3(kBlock), 0,
                     st, at(y), to_dims(y), at(dy), to_dims(dy), at_mut(dx),
                     to_dims(dx), axis, slices);
  NNHIP_CHECK(hipGetLastError());
}

void launch_slice_backward(hipStream_t st, const TensorView &gs,
                           const TensorView &gp, int axis, int64_t index) {
  check_view(gs, "slice_backward"); check_view(gp, "slice_backward");
  NNHIP_REQUIRE(axis >= 0 && axis < gp.rank && gs.rank == gp.rank - 1 &&
                    index >= 0 && index < gp.shape[axis],
                kErrArg, "slice_backward: bad axis, index or ranks");
  for (int d = 0, sd = 0; d < gp.rank; ++d) {
    if (d == axis) continue;
    NNHIP_REQUIRE(gs.shape[sd] == gp.shape[d], kErrArg,
                  "slice_backward: slice shape does not match the parent");
    ++sd;
  }
  const int64_t n = numel(gs);
  if (n == 0) return;
  hipLaunchKernelGGL(slice_backward_kernel, dim3(grid_for(n)), dim3(kBlock), 0, st,
                     at(gs), to_dims(gs), at_mut(gp), to_dims(gp), axis, index, n);
  NNHIP_CHECK(hipGetLastError());
}

void launch_embedding(hipStream_t st, const TensorView &w, const TensorView &ids,
                      const TensorView &out) {
  check_view(w, "embedding"); check_view(ids, "embedding"); check_view(out, "embedding");
  NNHIP_REQUIRE(w.rank == 2 && ids.rank == 2 && out.rank == 3 &&
                    out.shape[0] == ids.shape[0] && out.shape[1] == ids.shape[1] &&
                    out.shape[2] == w.shape[1],
                kErrArg, "embedding: weight [V][D], indices [N][T], out [N][T][D]");
  const int64_t rows = ids.shape[0] * ids.shape[1];
  if (rows == 0 || w.shape[1] == 0) return;
  const int64_t per = kBlock / 64;
  hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)((rows + per - 1) / per)),
                     dim3(kBlock), 0, st, at(w), w.shape[0], w.shape[1],
                     w.strides[0], w.strides[1], at(ids), ids.shape[1],
                     ids.strides[0], ids.strides[1], at_mut(out), out.strides[0],
                     out.strides[1], out.strides[2], rows);
  NNHIP_CHECK(hipGetLastError());
}

}  // namespace nnhip

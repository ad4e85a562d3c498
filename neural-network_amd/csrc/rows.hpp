// Row-wise LayerNorm and activation-digit arithmetic of the LayerNorm and
// act_quant kernels: one wave per row, the row held in "quads".
#pragma once

#include "nnhip_internal.hpp"

namespace nnhip {

// A row held by a wave in "quads": lane l has the 4 consecutive entries
// 256 i + 4 l .. + 3 for i < NQ (a quad is valid while 256 i + 4 l < d), so
// every wave-wide load or store of a quad index i is one contiguous 1 KB.
__device__ __forceinline__ bool quad_ok(int i, int lane, int d) {
  return 256 * i + 4 * lane < d;
}
// start of quad i of a lane (the last quad of the row for invalid ones, so
// that loads stay unconditional)
__device__ __forceinline__ int quad_at(int i, int lane, int d) {
  return min(256 * i + 4 * lane, d - 4);
}

// LayerNorm of one row (layer.cpp:242-261) held by a wave in quads with
// their gamma / beta: mean = sum / N, var = sum((x - mean)^2) / N,
// (x - mean) / sqrt(var + 1e-5) * gamma + beta; the sums are DPP wave
// reductions.  y gets the normalised row; with limbs its digits for the next
// MFMA GEMM (row exponent from the row's max, as aq_row_finish).
template <int NQ>
__device__ __forceinline__ void ln_row_finish(
    float (&v)[NQ][4], const float (&gv)[NQ][4], const float (&bv)[NQ][4],
    int d, int row, float *__restrict__ y, int8_t *__restrict__ limbs,
    int mpad, int *__restrict__ rexp, int lane) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NQ; ++i)
    if (quad_ok(i, lane, d)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) s += v[i][j];
    }
  s = wave_sum_all(s);
  const float N = (float)d;
  const float mean = s / N;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NQ; ++i)
    if (quad_ok(i, lane, d)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) { const float df = v[i][j] - mean; sq += df * df; }
    }
  sq = wave_sum_all(sq);
  const float sd = sqrtf(sq / N + 1e-5f);
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    if (!quad_ok(i, lane, d)) break;
    float *w = v[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (w[j] - mean) / sd * gv[i][j] + bv[i][j];
    *reinterpret_cast<float4 *>(y + (int64_t)row * d + 256 * i + 4 * lane) =
        make_float4(w[0], w[1], w[2], w[3]);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(w[0]), fabsf(w[1])),
                         fmaxf(fabsf(w[2]), fabsf(w[3]))));
  }
  if (!limbs) return;
  mx = wave_max_all(mx);
  const int e = digit_exponent(mx);
  if (lane == 0) rexp[row] = e;
  const int64_t plane = (int64_t)mpad * d;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    if (!quad_ok(i, lane, d)) break;
    const int3 t = digits4(v[i], e);
    // the quad's 4 bytes are adjacent in the operand layout
    const int64_t off = mfma_operand_offset(row, 256 * i + 4 * lane, d);
    *reinterpret_cast<int *>(limbs + off) = t.x;
    *reinterpret_cast<int *>(limbs + plane + off) = t.y;
    *reinterpret_cast<int *>(limbs + 2 * plane + off) = t.z;
  }
}

// max |x| over the valid quads of a row slice of span entries held by a wave
// (this lane's part)
template <int NQ>
__device__ __forceinline__ float quads_absmax(const float (&v)[NQ][4], int span,
                                              int lane) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < NQ; ++i)
    if (quad_ok(i, lane, span)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(v[i][j]));
    }
  return mx;
}

// Digits of the quads of row m's entries [s0, s0 + span) (of K) held by a
// wave, with the row exponent e = 22 - exponent(max|x|) over the whole row:
// X = rint(x * 2^e) split into balanced base-256 digits (hi, mid, lo) in the
// MFMA operand layout.
template <int NQ>
__device__ __forceinline__ void aq_store_digits(const float (&v)[NQ][4], int s0,
                                                int span, int K, int m, int e,
                                                int8_t *__restrict__ limbs,
                                                int mpad, int lane) {
  const int64_t plane = (int64_t)mpad * K;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    if (!quad_ok(i, lane, span)) break;
    const int3 t = digits4(v[i], e);
    const int64_t off = mfma_operand_offset(m, s0 + 256 * i + 4 * lane, K);
    *reinterpret_cast<int *>(limbs + off) = t.x;
    *reinterpret_cast<int *>(limbs + plane + off) = t.y;
    *reinterpret_cast<int *>(limbs + 2 * plane + off) = t.z;
  }
}

// Digits of one row for the MFMA GEMM (same rule as act_quant_kernel): the
// row (d floats, d % 128 == 0) is in LDS, mx is the thread's max |value|;
// NT threads reduce it through sred, then the row exponent goes to rexp and
// the three digit planes to limbs (MFMA operand layout, planes mpad x d).
template <int NT>
__device__ inline void store_row_digits(const float *srow, int d, float mx,
                                 int64_t row, int8_t *__restrict__ limbs,
                                 int mpad, int *__restrict__ rexp,
                                 float *sred) {
  typedef int v4i __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) mx = fmaxf(mx, sred[w]);
  const int e = digit_exponent(mx);
  if (threadIdx.x == 0) rexp[row] = e;
  const int64_t plane = (int64_t)mpad * d;
  for (int p = threadIdx.x; p < d / 16; p += NT) {
    const int k = p * 16;
    v4i hi, mid, lo;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int3 t = digits4(srow + k + 4 * q, e);
      hi[q] = t.x; mid[q] = t.y; lo[q] = t.z;
    }
    const int64_t off = mfma_operand_offset((int)row, k, d);
    *reinterpret_cast<v4i *>(limbs + off) = hi;
    *reinterpret_cast<v4i *>(limbs + plane + off) = mid;
    *reinterpret_cast<v4i *>(limbs + 2 * plane + off) = lo;
  }
}

// quads of a row with ordinary loads
template <int NQ>
__device__ __forceinline__ void load_quads(const float *__restrict__ xr, int d,
                                           int lane, float (&v)[NQ][4]) {
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const float4 f = *reinterpret_cast<const float4 *>(xr + quad_at(i, lane, d));
    v[i][0] = f.x; v[i][1] = f.y; v[i][2] = f.z; v[i][3] = f.w;
  }
}

}  // namespace nnhip

// W8A32 / fp32 Linear layers for gfx950.
//
// Replaces QuantizedDense::forward (quantization.cpp:127-147, dequantise the
// whole weight then cblas_sgemm) and Dense::forward (layer.cpp:162-171).
// Weights live on the device transposed to [N][K] (output channel major, K
// contiguous) so that both kernels stream them with coalesced loads:
//
//  * gemv_kernel  -- rows <= 4 per pass (batch-1 draft / verify): fp32 VALU
//    dot products, int8 codes dequantised in registers, per-channel scale
//    and bias applied once per output in the epilogue.
//  * gemm_limb_kernel -- rows >= 16 (batched verify, prefill): the fp32
//    activations are split exactly into three int8 digits with a per-row
//    power-of-two scale; each digit is multiplied with the int8 codes on the
//    MFMA (v_mfma_i32_32x32x32_i8) with exact int32 accumulation, and the
//    three int32 sums are recombined exactly in int64 before one rounding to
//    fp32.  Result: an fp32 product whose only error is the 2^-23 (relative
//    to the row maximum) digit truncation of x and one final rounding.
#include "nnhip_internal.hpp"
#include "rows.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace nnhip {

namespace {

constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));


// ---------------------------------------------------------------------------
// GEMV: y[r][n] = epi( sum_k x[r][k] * w[n][k] ), r < R (<= 8).
// A workgroup of 4 waves covers NC columns for each of CG = 4/nks column
// sets; wave (c, s) reduces K-slice s of column set c.  Each lane owns
// 4-element groups of K at stride 256 and keeps its slice of x for all R rows
// in registers; the int8 weights of all NC columns are requested together
// with x.  The NC x R partial sums of a lane are then reduced over the wave
// by a butterfly reduce-scatter (each exchange step halves the values a lane
// carries), which leaves one (column, row) total per lane.
// ---------------------------------------------------------------------------
constexpr int kGemvNC = 8;  // columns per column set

// Butterfly reduce-scatter of NP (a power of two <= 64) values per lane over
// the 64 lanes of a wave: afterwards v[0] of lane l is the wave's total of
// slot gemv_slot<NP>(l).  Step O (32, 16, ..., 1) halves the CNT values a
// lane carries while CNT > 1 (the lane with bit O set keeps the upper half),
// then adds the partner's single value; every index is a constant, so v
// stays in registers.
template <int NP, int CNT, int O>
__device__ __forceinline__ void rs_step(float (&v)[NP], int lane) {
  if constexpr (O >= 1) {
    if constexpr (CNT > 1) {
      constexpr int H = CNT / 2;
      const bool up = (lane & O) != 0;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const float send = up ? v[i] : v[i + H];
        const float keep = up ? v[i + H] : v[i];
        v[i] = keep + __shfl_xor(send, O, 64);
      }
      rs_step<NP, H, O / 2>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], O, 64);
      rs_step<NP, 1, O / 2>(v, lane);
    }
  }
}
template <int NP>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[NP]) {
  rs_step<NP, NP, 32>(v, (int)threadIdx.x & 63);
}
template <int NP>
__device__ __forceinline__ int gemv_slot(int lane) {
  int slot = 0, cnt = NP;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
    if (cnt > 1) { cnt /= 2; if (lane & o) slot += cnt; }
  return slot;
}

// lf.g set: the rows x are first normalised, LayerNorm (layer.cpp:242-261)
// with the arithmetic of layernorm_rows_kernel (row sums in quads, DPP wave
// reductions), so the normalised entries are the ones that kernel writes;
// workgroup 0 also writes them to lf.out when set.
template <int R, bool Q8>
__global__ __launch_bounds__(256) void gemv_kernel(
    const float *__restrict__ x, int64_t ldx, int K, int N,
    const int8_t *__restrict__ wq, const float *__restrict__ wf,
    const float *__restrict__ scale, const float *__restrict__ bias,
    const float *__restrict__ resid, int64_t ldr, float *__restrict__ y,
    int64_t ldy, int epi, int nks, int64_t row0, RopeArgs ra, GemvLn lf) {
  // row group blockIdx.y: rows [R * blockIdx.y, R * blockIdx.y + R) of the
  // launch
  {
    const int64_t g = (int64_t)blockIdx.y * R;
    x += g * ldx;
    if (resid) resid += g * ldr;
    if (y) y += g * ldy;
    if (lf.out) lf.out += g * lf.ldo;
    row0 += g;
  }
  constexpr int kMaxIt = 4;  // slice <= 1024 elements
  constexpr int P = kGemvNC * R;
  constexpr int NP = P <= 8 ? 8 : P <= 16 ? 16 : P <= 32 ? 32 : 64;
  __shared__ float red[4][kGemvNC][R];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cset = w / nks, slice = w % nks;
  const int cg = 4 / nks;
  const int slen = (((K + nks - 1) / nks) + 3) & ~3;
  const int k0 = slice * slen;
  const int iters = (slen + 255) / 256;
  const int64_t ncol0 = (int64_t)blockIdx.x * cg * kGemvNC + cset * kGemvNC;

  // The epilogue's operands, requested first so that they arrive with the
  // main loads: thread t < cg * 8 * R owns item (row e_r, column e_n) --
  // an output, or the even column of a SwiGLU / RoPE pair.
  const bool pair = epi == kEpiSwiGLU || epi == kEpiRope;
  const int e_r = (int)threadIdx.x % R, e_cc = ((int)threadIdx.x / R) % kGemvNC;
  const int e_cs = (int)threadIdx.x / (R * kGemvNC);
  const int64_t e_n = (int64_t)blockIdx.x * cg * kGemvNC + e_cs * kGemvNC + e_cc;
  const bool e_ok = (int)threadIdx.x < cg * kGemvNC * R && e_n < N &&
                    (!pair || (e_n & 1) == 0);
  float e_sc0 = 1.f, e_sc1 = 1.f, e_bi0 = 0.f, e_bi1 = 0.f, e_rs = 0.f;
  int e_pos = -1;
  float2 e_cos = make_float2(0.f, 0.f);
  if (e_ok) {
    if (Q8) e_sc0 = scale[e_n];
    e_bi0 = bias[e_n];
    if (pair) {
      if (Q8) e_sc1 = scale[e_n + 1];
      e_bi1 = bias[e_n + 1];
    }
    if (epi == kEpiResid) e_rs = resid[e_r * ldr + e_n];
    if (epi == kEpiRope) {
      e_pos = rope_row_pos(ra, row0 + e_r);
      if (e_pos >= 0 && e_n / (ra.H * ra.D) != 2) e_cos = rope_cos_sin(ra, e_pos, (int)e_n);
    }
  }

  float xr[R][kMaxIt][4];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      int k = k0 + it * 256 + lane * 4;
      bool ok = it < iters && k < k0 + slen && k < K;
      float4 v = ok ? *reinterpret_cast<const float4 *>(x + r * ldx + k)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
      xr[r][it][0] = v.x; xr[r][it][1] = v.y;
      xr[r][it][2] = v.z; xr[r][it][3] = v.w;
    }
  // int8 weights of all the wave's columns (zero past N or the slice)
  int wpk[Q8 ? kGemvNC : 1][kMaxIt];
  if constexpr (Q8) {
#pragma unroll
    for (int c = 0; c < kGemvNC; ++c)
#pragma unroll
      for (int it = 0; it < kMaxIt; ++it) {
        const int k = k0 + it * 256 + lane * 4;
        const int64_t n = ncol0 + c;
        const bool ok = it < iters && k < k0 + slen && k < K && n < N;
        wpk[c][it] = ok ? *reinterpret_cast<const int *>(wq + n * K + k) : 0;
      }
  }

  if (lf.g) {
#pragma clang fp contract(off)
    // each row's mean and deviation over all K, then the wave's slice
    // normalised in place
    float mean[R], sd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float q[4][4];
      load_quads<4>(x + r * ldx, K, lane, q);
      float sm = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (quad_ok(i, lane, K)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) sm += q[i][j];
        }
      sm = wave_sum_all(sm);
      const float Nf = (float)K;
      mean[r] = sm / Nf;
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (quad_ok(i, lane, K)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) { const float df = q[i][j] - mean[r]; sq += df * df; }
        }
      sq = wave_sum_all(sq);
      sd[r] = sqrtf(sq / Nf + 1e-5f);
    }
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
      const int k = k0 + it * 256 + lane * 4;
      if (!(it < iters && k < k0 + slen && k < K)) continue;
      const float4 gg = *reinterpret_cast<const float4 *>(lf.g + k);
      const float4 bb = *reinterpret_cast<const float4 *>(lf.b + k);
      const float ga[4] = {gg.x, gg.y, gg.z, gg.w}, ba[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xr[r][it][e] = (xr[r][it][e] - mean[r]) / sd[r] * ga[e] + ba[e];
        if (lf.out && blockIdx.x == 0 && cset == 0)
          *reinterpret_cast<float4 *>(lf.out + r * lf.ldo + k) =
              make_float4(xr[r][it][0], xr[r][it][1], xr[r][it][2], xr[r][it][3]);
      }
    }
  }
  float acc[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) acc[i] = 0.f;
#pragma unroll
  for (int it = 0; it < kMaxIt; ++it) {
    int k = k0 + it * 256 + lane * 4;
    if (!(it < iters && k < k0 + slen && k < K)) continue;
#pragma unroll
    for (int c = 0; c < kGemvNC; ++c) {
      float wv[4];
      if constexpr (Q8) {
        const int pk = wpk[c][it];
        wv[0] = (float)(int8_t)(pk & 0xff);
        wv[1] = (float)(int8_t)((pk >> 8) & 0xff);
        wv[2] = (float)(int8_t)((pk >> 16) & 0xff);
        wv[3] = (float)(int8_t)((pk >> 24) & 0xff);
      } else {
        const int64_t n = ncol0 + c;
        if (n >= N) continue;
        float4 f = *reinterpret_cast<const float4 *>(wf + n * K + k);
        wv[0] = f.x; wv[1] = f.y; wv[2] = f.z; wv[3] = f.w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[c * R + r] += xr[r][it][e] * wv[e];
    }
  }
  wave_reduce_scatter<NP>(acc);
  {
    const int slot = gemv_slot<NP>(lane);
    // lanes sharing a slot (NP < 64) hold the same total: the first writes
    if (slot < P && (lane & (64 / NP - 1)) == 0)
      red[w][slot / R][slot % R] = acc[0];
  }
  __syncthreads();
  // combine the nks slices and apply the epilogue (one item per thread:
  // cg * 8 * R <= 256)
  if (e_ok) {
    const int r = e_r, cc = e_cc, cs = e_cs;
    const int64_t n = e_n;
    float a = 0.f;
    for (int s = 0; s < nks; ++s) a += red[cs * nks + s][cc][r];
    float v = Q8 ? a * e_sc0 : a;
    v = v + e_bi0;
    if (pair) {
      float a1 = 0.f;
      for (int s = 0; s < nks; ++s) a1 += red[cs * nks + s][cc + 1][r];
      float u = (Q8 ? a1 * e_sc1 : a1) + e_bi1;
      if (epi == kEpiSwiGLU) y[r * ldy + n / 2] = swiglu_pair(v, u);
      else if (e_pos >= 0) rope_store_pair_at(ra, row0 + r, e_pos, (int)n, v, u, e_cos.x, e_cos.y);
    } else if (epi == kEpiResid) {
      y[r * ldy + n] = e_rs + v;
    } else {
      y[r * ldy + n] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// int8 GEMV with 128-bit code loads: y[r][n] = epi( sum_k x[r][k] * w[n][k] ),
// r < R (<= 8), K = 16 G with G (chunks of 16 codes per column) a power of
// two from 16 to 256.  A workgroup (256 threads) covers NB = CPI * NIT
// columns, CPI = 256 / G of them at a time: thread t owns chunk t % G of
// column t / G of each of its NIT column groups, so it loads 16 codes of a
// column with one 16-byte load, and its 16 entries of each row once, kept in
// registers for all its columns.  Every code load is issued with the row
// loads; the columns' scales and biases are staged in LDS first.  The R x NIT
// partial sums of a thread are reduced over the G threads of its column
// (within a wave: butterfly reduce-scatter over lane offsets G/2 .. 1, or
// 32 .. 1 when G > 64, then the G / 64 waves of a column through LDS), then
// the epilogue of gemv_kernel runs one (row, column) item per thread.
// ---------------------------------------------------------------------------
template <int G>
struct Gemv16Shape {
  static constexpr int CPI = 256 / G;                 // columns per pass
  static constexpr int NIT = G <= 32 ? (G == 16 ? 1 : 2) : 4;
  static constexpr int NB = CPI * NIT;                // columns per workgroup
  static constexpr int WPC = G > 64 ? G / 64 : 1;     // waves per column
  static constexpr int OMAX = G > 64 ? 32 : G / 2;    // first butterfly offset
};

template <int NP, int OMAX>
__device__ __forceinline__ int gemv16_slot(int lane) {
  int slot = 0, cnt = NP;
#pragma unroll
  for (int o = OMAX; o >= 1; o >>= 1)
    if (cnt > 1) { cnt /= 2; if (lane & o) slot += cnt; }
  return slot;
}

template <int R, int G>
__global__ __launch_bounds__(256) void gemv16_kernel(
    const float *__restrict__ x, int64_t ldx, int K, int N,
    const int8_t *__restrict__ wq, const float *__restrict__ scale,
    const float *__restrict__ bias, const float *__restrict__ resid,
    int64_t ldr, float *__restrict__ y, int64_t ldy, int epi, int64_t row0,
    RopeArgs ra, GemvLn lf) {
  using SH = Gemv16Shape<G>;
  constexpr int CPI = SH::CPI, NIT = SH::NIT, NB = SH::NB, WPC = SH::WPC;
  constexpr int P = NIT * R;
  constexpr int NP = P <= 1 ? 1 : P <= 2 ? 2 : P <= 4 ? 4 : P <= 8 ? 8
                   : P <= 16 ? 16 : P <= 32 ? 32 : 64;
  static_assert(P <= 64, "gemv16: too many partial sums per thread");
  {
    const int64_t g = (int64_t)blockIdx.y * R;
    x += g * ldx;
    if (resid) resid += g * ldr;
    if (y) y += g * ldy;
    if (lf.out) lf.out += g * lf.ldo;
    row0 += g;
  }
  __shared__ float s_scale[NB], s_bias[NB];
  __shared__ float red[WPC][NB][R];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int chunk = t % G, cpos = t / G;
  const int64_t col0 = (int64_t)blockIdx.x * NB;
  if (t < NB) {
    const int64_t n = col0 + t;
    s_scale[t] = n < N ? scale[n] : 0.f;
    s_bias[t] = n < N ? bias[n] : 0.f;
  }
  // epilogue operands of the thread's item (row e_r, column e_c), requested
  // first: the residual, the RoPE position and angle
  const bool pair = epi == kEpiSwiGLU || epi == kEpiRope;
  const int e_r = t % R, e_c = t / R;
  const int64_t e_n = col0 + e_c;
  const bool e_ok = t < NB * R && e_n < N && (!pair || (e_n & 1) == 0);
  float e_rs = 0.f;
  int e_pos = -1;
  float2 e_cos = make_float2(0.f, 0.f);
  if (e_ok) {
    if (epi == kEpiResid) e_rs = resid[e_r * ldr + e_n];
    if (epi == kEpiRope) {
      e_pos = rope_row_pos(ra, row0 + e_r);
      if (e_pos >= 0 && e_n / (ra.H * ra.D) != 2) e_cos = rope_cos_sin(ra, e_pos, (int)e_n);
    }
  }
  // the thread's 16 entries of every row and its NIT 16-byte code chunks
  const int k = chunk * 16;
  float xr[R][16];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = *reinterpret_cast<const float4 *>(x + r * ldx + k + 4 * q);
      xr[r][4 * q] = v.x; xr[r][4 * q + 1] = v.y;
      xr[r][4 * q + 2] = v.z; xr[r][4 * q + 3] = v.w;
    }
  v4i wc[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int64_t n = col0 + it * CPI + cpos;
    wc[it] = n < N ? *reinterpret_cast<const v4i *>(wq + n * K + k) : v4i{0, 0, 0, 0};
  }
  if (lf.g) {
#pragma clang fp contract(off)
    // each row's mean and deviation over all K with layernorm_rows_kernel's
    // arithmetic (every wave forms them from the whole row), then the
    // thread's entries normalised
    float mean[R], sd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float q4[4][4];
      load_quads<4>(x + r * ldx, K, lane, q4);
      float sm = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (quad_ok(i, lane, K)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) sm += q4[i][j];
        }
      sm = wave_sum_all(sm);
      const float Nf = (float)K;
      mean[r] = sm / Nf;
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (quad_ok(i, lane, K)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) { const float df = q4[i][j] - mean[r]; sq += df * df; }
        }
      sq = wave_sum_all(sq);
      sd[r] = sqrtf(sq / Nf + 1e-5f);
    }
    float ga[16], ba[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 gg = *reinterpret_cast<const float4 *>(lf.g + k + 4 * q);
      const float4 bb = *reinterpret_cast<const float4 *>(lf.b + k + 4 * q);
      ga[4 * q] = gg.x; ga[4 * q + 1] = gg.y; ga[4 * q + 2] = gg.z; ga[4 * q + 3] = gg.w;
      ba[4 * q] = bb.x; ba[4 * q + 1] = bb.y; ba[4 * q + 2] = bb.z; ba[4 * q + 3] = bb.w;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int e = 0; e < 16; ++e) xr[r][e] = (xr[r][e] - mean[r]) / sd[r] * ga[e] + ba[e];
      if (lf.out && blockIdx.x == 0 && cpos == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<float4 *>(lf.out + r * lf.ldo + k + 4 * q) =
              make_float4(xr[r][4 * q], xr[r][4 * q + 1], xr[r][4 * q + 2], xr[r][4 * q + 3]);
      }
    }
  }
  float acc[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) acc[i] = 0.f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      const int pk = wc[it][wd];
      float wv[4];
      wv[0] = (float)(int8_t)(pk & 0xff);
      wv[1] = (float)(int8_t)((pk >> 8) & 0xff);
      wv[2] = (float)(int8_t)((pk >> 16) & 0xff);
      wv[3] = (float)(int8_t)((pk >> 24) & 0xff);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[it * R + r] += xr[r][4 * wd + e] * wv[e];
    }
  }
  rs_step<NP, NP, SH::OMAX>(acc, lane);
  {
    const int slot = gemv16_slot<NP, SH::OMAX>(lane);
    // lanes of a column holding the same slot (NP < the butterfly's span)
    // hold the same total: the first writes
    constexpr int span = 2 * SH::OMAX;
    const int first = (span / NP > 1) ? ((lane & (span / NP - 1)) == 0) : 1;
    if (slot < P && first)
      red[WPC > 1 ? w % WPC : 0][(slot / R) * CPI + cpos][slot % R] = acc[0];
  }
  __syncthreads();
  if (e_ok) {
    const int r = e_r, c = e_c;
    const int64_t n = e_n;
    float a = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < WPC; ++s2) a += red[s2][c][r];
    float v = a * s_scale[c] + s_bias[c];
    if (pair) {
      float a1 = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < WPC; ++s2) a1 += red[s2][c + 1][r];
      const float u = a1 * s_scale[c + 1] + s_bias[c + 1];
      if (epi == kEpiSwiGLU) y[r * ldy + n / 2] = swiglu_pair(v, u);
      else if (e_pos >= 0) rope_store_pair_at(ra, row0 + r, e_pos, (int)n, v, u, e_cos.x, e_cos.y);
    } else if (epi == kEpiResid) {
      y[r * ldy + n] = e_rs + v;
    } else {
      y[r * ldy + n] = v;
    }
  }
}

// Digits of activation rows for the MFMA GEMM: X = rint(x * 2^e) with
// e = 22 - exponent(max|x|) per row, split into balanced base-256 digits
// (hi, mid, lo), written in the MFMA operand layout.  WPR waves per row, each
// holding a slice of K / WPR entries in quads (rows.hpp: lane l has entries
// 256 i + 4 l .. + 3 of the slice, i < NQ) in registers, so the row is read
// once and every load is a contiguous 1 KB per wave; the slices' maxima are
// combined through LDS (max is exact, so the exponent does not depend on WPR).
template <int NQ, int WPR>
__global__ __launch_bounds__(256) void act_quant_kernel(
    const float *__restrict__ x, int64_t ldx, int K, int rows,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
  __shared__ float s_mx[4];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = blockIdx.x * (4 / WPR) + wv / WPR;
  const int span = K / WPR, s0 = (wv % WPR) * span;
  float v[NQ][4];
  load_quads<NQ>(x + (int64_t)min(m, rows - 1) * ldx + s0, span, lane, v);
  float mx = wave_max_all(quads_absmax<NQ>(v, span, lane));
  if constexpr (WPR > 1) {
    if (lane == 0) s_mx[wv] = mx;
    __syncthreads();
    const int w0 = wv - wv % WPR;
#pragma unroll
    for (int j = 0; j < WPR; ++j) mx = fmaxf(mx, s_mx[w0 + j]);
  }
  if (m >= rows) return;
  const int e = digit_exponent(mx);
  if (lane == 0 && s0 == 0) rexp[m] = e;
  aq_store_digits<NQ>(v, s0, span, K, m, e, limbs, mpad, lane);
}

// ---------------------------------------------------------------------------
// int8 MFMA GEMM over the activation digits.  Workgroup tile 32 rows x 64
// columns; the four waves split K (chunks of 128, wave w takes chunks w,
// w+4, ...) with the next chunk's loads issued before the current chunk's
// MFMAs, and the three int32 accumulators per 32x32 sub-tile (one per digit)
// are summed across waves with LDS integer atomics (exact, order-free).
// Both operands are stored in the MFMA operand layout (mfma_operand_offset):
// within each 128-wide K chunk, lane (r, h) supplies bytes
// [s*32 + h*16, s*32 + h*16 + 16) of its row for MFMA step s, identically for
// the digit operand and the weight operand, so each MFMA contracts matching
// k indices whatever order the hardware assigns to a lane's 16 bytes, and
// every operand load of a wave is one contiguous 1 KB block.
// Tiles are dealt to the 8 XCDs in contiguous runs (row tiles of one column
// tile adjacent), so a weight tile is fetched from HBM into one XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kGemmMT = 32;

// NSUB 32-column sub-tiles per workgroup (tile 32 x 32*NSUB); NW waves
// split K (chunks w, w + NW, ...).
// HX: the digits carry one exponent per 64-wide K chunk (rexp is then
// [M][K/64], the merged attention's per-head exponents): a 128-wide chunk's
// MFMA steps 0-1 and 2-3 are two such chunks (mfma_operand_offset), each
// chunk's exact integer total is scaled by its own 2^-e in double, and the
// waves' sums are added in wave order through LDS (deterministic); one
// rounding to float, then the bias / residual epilogue.
template <int NSUB, int NW = 4, bool HX = false>
__global__ __launch_bounds__(64 * NW, NSUB == 1 && NW == 4 ? 2 : 1) void gemm_limb_kernel(
    const int8_t *__restrict__ limbs, int mpad, const int *__restrict__ rexp,
    int M, int K, int N, const int8_t *__restrict__ wq,
    const float *__restrict__ scale, const float *__restrict__ bias,
    const float *__restrict__ resid, int64_t ldr, float *__restrict__ y,
    int64_t ldy, int epi, int ntm, int ntn, RopeArgs ra) {
  constexpr int NT = 32 * NSUB;
  constexpr int kThr = 64 * NW;
  static_assert(!HX || NSUB == 1, "chunk exponents with 32-column tiles");
  __shared__ int red[kLimbs][kGemmMT][NT];
  __shared__ double dred[HX ? NW : 1][kGemmMT][HX ? NT : 1];
  __shared__ int s_hx[HX ? kGemmMT * kMaxHxChunks : 1];
  const int T = ntm * ntn;
  const int per = (T + 7) / 8;
  const int wi = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (wi >= T) return;
  const int tn = wi / ntm, tm = wi % ntm;
  const int m0 = tm * kGemmMT, n0 = tn * NT;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  for (int i = threadIdx.x; i < kLimbs * kGemmMT * NT; i += kThr)
    (&red[0][0][0])[i] = 0;
  // the epilogue's operands (thread -> (row, column pair) items), requested
  // now so that they arrive with the MFMA operands
  // (the thread count is a multiple of NT/2, so a thread's items share one
  // column pair)
  constexpr int IT = kGemmMT * NT / 2 / kThr;
  static_assert(IT >= 1 && IT * kThr == kGemmMT * NT / 2, "one item set per thread");
  static_assert(kThr % (NT / 2) == 0, "items must share their columns");
  const int e_n = n0 + 2 * ((int)threadIdx.x % (NT / 2));
  const bool e_cols = epi != kEpiTotals;
  const float e_sc0 = e_cols ? scale[e_n] : 0.f, e_sc1 = e_cols ? scale[e_n + 1] : 0.f;
  const float e_bi0 = e_cols ? bias[e_n] : 0.f, e_bi1 = e_cols ? bias[e_n + 1] : 0.f;
  int e_ex[IT];
  float e_rs[IT][2];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int m = m0 + ((int)threadIdx.x + it * kThr) / (NT / 2);
    const bool ok = m < M && e_cols;
    e_ex[it] = ok && !HX ? rexp[m] : 0;
    e_rs[it][0] = ok && epi == kEpiResid ? resid[(int64_t)m * ldr + e_n] : 0.f;
    e_rs[it][1] = ok && epi == kEpiResid ? resid[(int64_t)m * ldr + e_n + 1] : 0.f;
  }
  const int nhx = K / 64;
  if constexpr (HX) {
    // the tile's chunk exponents (rows past M: 0)
    for (int i = threadIdx.x; i < kGemmMT * nhx; i += kThr) {
      const int rr = i / nhx, cc = i % nhx;
      s_hx[i] = m0 + rr < M ? rexp[(int64_t)(m0 + rr) * nhx + cc] : 0;
    }
  }
  __syncthreads();

  v16i acc[NSUB][kLimbs];
#pragma unroll
  for (int t = 0; t < NSUB; ++t)
#pragma unroll
    for (int l = 0; l < kLimbs; ++l) acc[t][l] = v16i{};
  const int nch = K / 128;
  const int cb = 0, ce = nch;
  // tile bases in the operand layout: 32 rows x 128 k = 4 KB per chunk
  const int8_t *pb = wq + (int64_t)(n0 >> 5) * nch * 4096 + lane * 16;
  const int8_t *pa = limbs + (int64_t)(m0 >> 5) * nch * 4096 + lane * 16;
  const int64_t plane = (int64_t)mpad * K;
  struct Frag { v4i b[NSUB][4], a[kLimbs][4]; };
  auto load = [&](int c, Frag &f) {
    const int kb = c * 4096;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < NSUB; ++t)
        f.b[t][s] = *reinterpret_cast<const v4i *>(pb + (int64_t)t * nch * 4096 + kb + s * 1024);
#pragma unroll
      for (int l = 0; l < kLimbs; ++l)
        f.a[l][s] = *reinterpret_cast<const v4i *>(pa + l * plane + kb + s * 1024);
    }
  };
  auto mma = [&](const Frag &f) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < NSUB; ++t)
#pragma unroll
        for (int l = 0; l < kLimbs; ++l)
          acc[t][l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[l][s], f.b[t][s], acc[t][l], 0, 0, 0);
  };
  if constexpr (HX) {
    // lane holds column (lane & 31) of rows (j >> 2) * 8 + h * 4 + (j & 3)
    double dsum[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) dsum[j] = 0.0;
    for (int c = cb + w; c < ce; c += NW) {
      Frag f;
      load(c, f);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        v16i a3[kLimbs];
#pragma unroll
        for (int l = 0; l < kLimbs; ++l) a3[l] = v16i{};
#pragma unroll
        for (int s = 2 * half; s < 2 * half + 2; ++s)
#pragma unroll
          for (int l = 0; l < kLimbs; ++l)
            a3[l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[l][s], f.b[0][s], a3[l], 0, 0, 0);
        const int hc = 2 * c + half;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int row = (j >> 2) * 8 + h * 4 + (j & 3);
          // the chunk's exact total (|digit sums| < 2^21), then its scale
          const double tot = fma((double)a3[0][j], 65536.0,
                                 fma((double)a3[1][j], 256.0, (double)a3[2][j]));
          dsum[j] += ldexp(tot, -s_hx[row * nhx + hc]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      dred[w][(j >> 2) * 8 + h * 4 + (j & 3)][r] = dsum[j];
    __syncthreads();
  }
  // ping-pong over the wave's chunks w, w+NW, w+2NW, ...: the loads of the
  // next chunk are in flight while the current chunk's MFMAs run
  Frag fa, fb;
  int c = HX ? ce : cb + w;
  if (c < ce) load(c, fa);
  while (c < ce) {
    if (c + NW < ce) load(c + NW, fb);
    mma(fa);
    c += NW;
    if (c >= ce) break;
    if (c + NW < ce) load(c + NW, fa);
    mma(fb);
    c += NW;
  }
  if (!HX && cb + w < ce) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t)
#pragma unroll
      for (int l = 0; l < kLimbs; ++l)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int row = (j >> 2) * 8 + h * 4 + (j & 3);
          atomicAdd(&red[l][row][t * 32 + r], acc[t][l][j]);
        }
  }
  if constexpr (!HX) __syncthreads();
  // epilogue: thread -> (row, column pair)
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int idx = threadIdx.x + it * kThr;
    const int row = idx / (NT / 2), cp = idx % (NT / 2);
    const int m = m0 + row;
    if (m >= M) continue;
    const int c0 = 2 * cp;
    const int n = n0 + c0;
    float v[2];
    if constexpr (HX) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        double dt = 0.0;
#pragma unroll
        for (int u = 0; u < NW; ++u) dt += dred[u][row][c0 + e];
        v[e] = fmaf((float)dt, e == 0 ? e_sc0 : e_sc1, e == 0 ? e_bi0 : e_bi1);
      }
    } else {
      long long tot[2];
#pragma unroll
      for (int e = 0; e < 2; ++e)
        tot[e] = (long long)red[0][row][c0 + e] * 65536LL +
                 (long long)red[1][row][c0 + e] * 256LL +
                 (long long)red[2][row][c0 + e];
      if (epi == kEpiTotals) {
        long long *yt = reinterpret_cast<long long *>(y) + (int64_t)m * ldy + n;
        yt[0] = tot[0]; yt[1] = tot[1];
        continue;
      }
      v[0] = dequant_epilogue(tot[0], e_ex[it], e_sc0, e_bi0);
      v[1] = dequant_epilogue(tot[1], e_ex[it], e_sc1, e_bi1);
    }
    if (epi == kEpiSwiGLU) {
      y[(int64_t)m * ldy + n / 2] = swiglu_pair(v[0], v[1]);
    } else if (epi == kEpiRope) {
      if (ra.kq) rope_store_pair_q8(ra, m, n, v[0], v[1]);
      else rope_store_pair(ra, m, n, v[0], v[1]);
    } else {
      if (epi == kEpiResid) { v[0] = e_rs[it][0] + v[0]; v[1] = e_rs[it][1] + v[1]; }
      y[(int64_t)m * ldy + n] = v[0];
      y[(int64_t)m * ldy + n + 1] = v[1];
    }
  }
}

// ---------------------------------------------------------------------------
// int8 MFMA GEMM with the activation digits resident in LDS (K <= 1024).
// One workgroup of 16 waves owns a 32*CT-column block and walks `rpt`
// consecutive 32-row tiles with its weight slice held in registers, so the
// weights are read once per workgroup however many rows there are: wave
// (column tile ct, K slice ks) multiplies its 32 columns over K/KS of the K
// range (KS = min(4, K/128), CT = 16/KS); the slices' int64 totals are
// summed in LDS with 64-bit integer atomics (exact, order-free) and the
// epilogue runs over the summed tile.
// Loads are issued in the order they are needed -- the per-column vectors
// and the residual, the first row tile's activations, then the weight slice
// -- so the prologue works on the activations while the weights stream in,
// and the first tile's MFMAs on a chunk wait only for that chunk.  The next
// row tile's digits are copied into LDS as soon as every wave is done with
// the current tile's, so they arrive during its epilogue.
// The 32 x K digit tile (3 planes, MFMA operand layout) is built by the
// prologue:
//   kAFromDigits     copied from digit planes written by another kernel,
//   kAFromRows       digitised from fp32 rows (x, ldx),
//   kAFromLayerNorm  LayerNorm (layer.cpp:242-261) of fp32 rows, written
//                    to ln_out by the first column block, then digitised.
// Only kAFromDigits walks more than one row tile (rpt > 1).
// ---------------------------------------------------------------------------
constexpr int kLdsThreads = 1024;

template <int MODE, int KPT, bool Q8KV = false>
__global__ __launch_bounds__(kLdsThreads) void gemm_lds_kernel(
    const int8_t *__restrict__ limbs, int mpad, const int *__restrict__ rexp,
    const float *__restrict__ x, int64_t ldx, const float *__restrict__ lng,
    const float *__restrict__ lnb, float *__restrict__ ln_out, int64_t ldo,
    int M, int N, const int8_t *__restrict__ wq,
    const float *__restrict__ scale, const float *__restrict__ bias,
    const float *__restrict__ resid, int64_t ldr, float *__restrict__ y,
    int64_t ldy, int epi, int ntm, int ntn, int rpt, RopeArgs ra,
    TileStatsArgs tsa) {
  constexpr int K = KPT * 32;
  constexpr int nch = K / 128;
  constexpr int KS = nch < 4 ? nch : 4;       // K slices
  constexpr int CT = 16 / KS;                 // 32-column tiles per workgroup
  constexpr int CPW = nch / KS;               // 128-wide chunks per wave
  constexpr int NC = 32 * CT;                 // columns per workgroup
  constexpr int kPlane = kGemmMT * K;         // bytes per digit plane
  constexpr int kRedLd = 33;                  // padded row of the sum tile
  constexpr int kABytes = kLimbs * kPlane;
  constexpr bool kLN = MODE == kAFromLayerNorm;
  constexpr bool kDig = MODE == kAFromDigits;
  __shared__ __attribute__((aligned(16))) int8_t sa[kABytes];
  __shared__ long long red[CT][kGemmMT][kRedLd];
  __shared__ float s_sc[NC], s_bi[NC];
  __shared__ __attribute__((aligned(16))) float s_g[kLN ? K : 4], s_b[kLN ? K : 4];
  __shared__ int s_e[2][kGemmMT];
  const int rt = kDig ? rpt : 1;              // row tiles per workgroup
  const int ngr = (ntm + rt - 1) / rt;        // row-tile groups
  const int T = ngr * ntn;
  const int per = (T + 7) / 8;
  const int wi = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (wi >= T) return;
  const int tn = wi / ngr, tg = wi % ngr;
  const int tmb = tg * rt, tme = min(ntm, tmb + rt);
  const int n0 = tn * NC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ct = w % CT, ks = w / CT;
  const int nw = n0 + 32 * ct;                // this wave's column tile

  // ---- small operands: per-column and LayerNorm vectors, residual ----
  float vsc = 0.f, vbi = 0.f;
  if (tid < NC && n0 + tid < N && epi != kEpiTotals) {
    vsc = scale[n0 + tid];
    vbi = bias[n0 + tid];
  }
  float vg = 0.f, vb = 0.f;
  if (kLN && tid < K) { vg = lng[tid]; vb = lnb[tid]; }
  // epilogue items: thread -> (row, column pair)
  constexpr int ITEMS = kGemmMT * NC / 2 / kLdsThreads;
  float e_rs[ITEMS][2];
  auto load_resid = [&](int tm) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = tid + it * kLdsThreads;
      const int row = idx / (NC / 2), c0 = 2 * (idx % (NC / 2));
      const int m = tm * kGemmMT + row, n = n0 + c0;
      const bool ok = epi == kEpiResid && m < M && n < N;
      e_rs[it][0] = ok ? resid[(int64_t)m * ldr + n] : 0.f;
      e_rs[it][1] = ok ? resid[(int64_t)m * ldr + n + 1] : 0.f;
    }
  };
  load_resid(tmb);

  // ---- the first row tile's activations ----
  // digits: 16-byte pieces of the 32 x K tile, consecutive pieces on
  // consecutive lanes (a wave's 64 pieces are one 1 KB run of a plane);
  // rows: thread (row rr, part pp) takes entries 4pp + 128i, i < K/128
  constexpr int kPieces = kABytes / 16;
  constexpr int kPer = kDig ? (kPieces + kLdsThreads - 1) / kLdsThreads : 1;
  constexpr int PP = kDig ? 1 : K / 128;
  const int64_t plane = (int64_t)mpad * K;
  auto row_exps = [&](int tm) {
    return tid < kGemmMT && tm * kGemmMT + tid < M ? rexp[tm * kGemmMT + tid] : 0;
  };
  float4 v[PP];
  int a_e = 0;
  const int rr = tid >> 5, pp = tid & 31;
  const bool live = tmb * kGemmMT + rr < M;
  if constexpr (kDig) {
    // straight into LDS (global_load_lds puts lane i's 16 bytes at the
    // wave's LDS address + 16 i); waited for before the prologue's barrier
    a_e = row_exps(tmb);
    const int8_t *src = limbs + (int64_t)tmb * nch * 4096;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i0 = w * kWave + j * kLdsThreads;
      if (kPieces % kLdsThreads == 0 || i0 < kPieces) {
        const int l = i0 / (kPlane / 16), o = (i0 % (kPlane / 16)) * 16;
        __builtin_amdgcn_global_load_lds(
            (__attribute__((address_space(1))) void *)(src + l * plane + o + lane * 16),
            (__attribute__((address_space(3))) void *)(sa + l * kPlane + o), 16, 0, 0);
      }
    }
  } else {
    const int m = tmb * kGemmMT + rr;
#pragma unroll
    for (int i = 0; i < PP; ++i)
      v[i] = live ? *reinterpret_cast<const float4 *>(x + (int64_t)m * ldx + 4 * pp + 128 * i)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // ---- the weight slice ----
  v4i bf[CPW][4];
  {
    const int nt = min(nw, N - 32);           // past N: the last tile, unused
    const int8_t *pb = wq + (int64_t)(nt >> 5) * nch * 4096 + lane * 16;
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        bf[c][s] = *reinterpret_cast<const v4i *>(pb + (ks * CPW + c) * 4096 + s * 1024);
  }

  if constexpr (KS > 1)
    for (int i = tid; i < CT * kGemmMT * kRedLd; i += kLdsThreads)
      (&red[0][0][0])[i] = 0;
  if (tid < NC) { s_sc[tid] = vsc; s_bi[tid] = vbi; }

  // ---- prologue: the first 32 x K digit tile in LDS ----
  if constexpr (kDig) {
    if (tid < kGemmMT) s_e[0][tid] = a_e;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // digits in LDS
  } else {
#pragma clang fp contract(off)
    const int m = tmb * kGemmMT + rr;
    if (kLN && tid < K) { s_g[tid] = vg; s_b[tid] = vb; }
    // sums / maxima over the 32 lanes of a row (aligned half-waves)
    auto row_sum = [](float a) {
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) a += __shfl_xor(a, o, kWave);
      return a;
    };
    auto row_max = [](float a) {
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, kWave));
      return a;
    };
    if constexpr (kLN) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < PP; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
      const float Nf = (float)K;
      const float mean = row_sum(s) / Nf;
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < PP; ++i) {
        const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean,
                    d = v[i].w - mean;
        sq += (a * a + b * b) + (c * c + d * d);
      }
      const float sd = sqrtf(row_sum(sq) / Nf + 1e-5f);
      __syncthreads();                        // s_g, s_b written
      const bool wr = ln_out && tn == 0 && live;
#pragma unroll
      for (int i = 0; i < PP; ++i) {
        const int k = 4 * pp + 128 * i;
        const float4 gg = *reinterpret_cast<const float4 *>(s_g + k);
        const float4 bb = *reinterpret_cast<const float4 *>(s_b + k);
        v[i].x = (v[i].x - mean) / sd * gg.x + bb.x;
        v[i].y = (v[i].y - mean) / sd * gg.y + bb.y;
        v[i].z = (v[i].z - mean) / sd * gg.z + bb.z;
        v[i].w = (v[i].w - mean) / sd * gg.w + bb.w;
        if (wr) *reinterpret_cast<float4 *>(ln_out + (int64_t)m * ldo + k) = v[i];
      }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < PP; ++i)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)),
                           fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    mx = row_max(mx);
    const int e = digit_exponent(mx);
    if (pp == 0) s_e[0][rr] = live ? e : 0;
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const int k = 4 * pp + 128 * i;
      const float f[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      int3 d = digits4(f, e);
      if (!live) d = make_int3(0, 0, 0);
      const int o = (int)mfma_operand_offset(rr, k, K);
      *reinterpret_cast<int *>(sa + o) = d.x;
      *reinterpret_cast<int *>(sa + kPlane + o) = d.y;
      *reinterpret_cast<int *>(sa + 2 * kPlane + o) = d.z;
    }
  }
  __syncthreads();

  // one row tile: MFMAs over the wave's K slice, the slices summed into the
  // tile of totals, then the epilogue; when another tile follows, its digits
  // go straight into the tile buffer meanwhile (global_load_lds puts lane
  // i's 16 bytes at the wave's LDS address + 16 i)
  auto row_tile = [&](int tm) {
    const int buf = (tm - tmb) & 1;
    const bool more = tm + 1 < tme;
    if (nw < N) {
      v16i acc[kLimbs];
#pragma unroll
      for (int l = 0; l < kLimbs; ++l) acc[l] = v16i{};
      const int8_t *pa = sa + lane * 16;
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int off = (ks * CPW + c) * 4096 + s * 1024;
#pragma unroll
          for (int l = 0; l < kLimbs; ++l) {
            const v4i a = *reinterpret_cast<const v4i *>(pa + l * kPlane + off);
            acc[l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bf[c][s], acc[l], 0, 0, 0);
          }
        }
      // lane holds column (lane & 31) of rows (j >> 2) * 8 + (lane >> 5) * 4 +
      // (j & 3), j < 16
      long long *rp = &red[ct][(lane >> 5) * 4][lane & 31];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const long long tot = (long long)acc[0][j] * 65536LL +
                              (long long)acc[1][j] * 256LL + (long long)acc[2][j];
        long long *q = rp + ((j >> 2) * 8 + (j & 3)) * kRedLd;
        if constexpr (KS == 1) *q = tot;
        else atomicAdd(reinterpret_cast<unsigned long long *>(q), (unsigned long long)tot);
      }
    }
    __syncthreads();

    // ---- epilogue over the summed tile: its LDS operands are read first
    // (the totals cleared behind them when another tile follows), then the
    // next tile's digit copy is started, then the outputs are formed ----
    const int m0 = tm * kGemmMT;
    long long et[ITEMS][2];
    float esc[ITEMS][2], ebi[ITEMS][2];
    int eex[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = tid + it * kLdsThreads;
      const int row = idx / (NC / 2), c0 = 2 * (idx % (NC / 2));
      long long *rq = &red[c0 >> 5][row][c0 & 31];
      et[it][0] = rq[0]; et[it][1] = rq[1];
      if (KS > 1 && more) { rq[0] = 0; rq[1] = 0; }
      eex[it] = s_e[buf][row];
      esc[it][0] = s_sc[c0]; esc[it][1] = s_sc[c0 + 1];
      ebi[it][0] = s_bi[c0]; ebi[it][1] = s_bi[c0 + 1];
    }
    if (kDig && more) {
      a_e = row_exps(tm + 1);
      const int8_t *src = limbs + (int64_t)(tm + 1) * nch * 4096;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i0 = w * kWave + j * kLdsThreads;
        if (kPieces % kLdsThreads == 0 || i0 < kPieces) {
          const int l = i0 / (kPlane / 16), o = (i0 % (kPlane / 16)) * 16;
          __builtin_amdgcn_global_load_lds(
              (__attribute__((address_space(1))) void *)(src + l * plane + o + lane * 16),
              (__attribute__((address_space(3))) void *)(sa + l * kPlane + o), 16, 0, 0);
        }
      }
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = tid + it * kLdsThreads;
      const int row = idx / (NC / 2), c0 = 2 * (idx % (NC / 2));
      const int m = m0 + row, n = n0 + c0;
      if (m >= M || n >= N) continue;
      if (epi == kEpiTotals) {
        long long *yt = reinterpret_cast<long long *>(y) + (int64_t)m * ldy + n;
        yt[0] = et[it][0]; yt[1] = et[it][1];
        continue;
      }
      float v0 = dequant_epilogue(et[it][0], eex[it], esc[it][0], ebi[it][0]);
      float v1 = dequant_epilogue(et[it][1], eex[it], esc[it][1], ebi[it][1]);
      if (epi == kEpiSwiGLU) {
        y[(int64_t)m * ldy + n / 2] = swiglu_pair(v0, v1);
      } else if (epi == kEpiRope) {
        if constexpr (Q8KV) rope_store_pair_q8(ra, m, n, v0, v1);
        else rope_store_pair(ra, m, n, v0, v1);
      } else {
        if (epi == kEpiResid) { v0 = e_rs[it][0] + v0; v1 = e_rs[it][1] + v1; }
        y[(int64_t)m * ldy + n] = v0;
        y[(int64_t)m * ldy + n + 1] = v1;
      }
    }
    // softmax statistics of this column block (NC == 128: item `it` of a
    // wave is one row's whole block, two columns a lane)
    if (NC == 2 * kWave && tsa.out && epi == kEpiBias) {
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        const int idx = tid + it * kLdsThreads;
        const int row = idx / (NC / 2), c0 = 2 * (idx % (NC / 2));
        const int m = m0 + row, n = n0 + c0;
        if (m >= M) continue;                  // whole wave
        const float l0 = dequant_epilogue(et[it][0], eex[it], esc[it][0], ebi[it][0]);
        const float l1 = dequant_epilogue(et[it][1], eex[it], esc[it][1], ebi[it][1]);
        if (tsa.T > 0.f) {
          float s0 = n < N ? (tsa.T == 1.f ? l0 : l0 / tsa.T) : -INFINITY;
          float s1 = n + 1 < N ? (tsa.T == 1.f ? l1 : l1 / tsa.T) : -INFINITY;
          const float mx = wave_max_all(fmaxf(s0, s1));
          const float e = wave_sum_all((n < N ? expf(s0 - mx) : 0.f) +
                                       (n + 1 < N ? expf(s1 - mx) : 0.f));
          if (lane == 0) tsa.out[(int64_t)m * tsa.ld + tn] = make_float2(mx, e);
        } else {
          const float a0 = n < N ? l0 : -INFINITY, a1 = n + 1 < N ? l1 : -INFINITY;
          const float mx = wave_max_all(fmaxf(a0, a1));
          const int ix = wave_min_all(a0 == mx ? n : (a1 == mx ? n + 1 : 0x7fffffff));
          if (lane == 0) tsa.out[(int64_t)m * tsa.ld + tn] = make_float2(mx, __int_as_float(ix));
        }
      }
    }
    if (kDig && more) {
      if (tid < kGemmMT) s_e[buf ^ 1][tid] = a_e;
      load_resid(tm + 1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // digits in LDS
      __syncthreads();
    }
  };
  // the first tile apart from the loop, so that its MFMAs wait for the
  // weight chunks one at a time
  row_tile(tmb);
  for (int tm = tmb + 1; tm < tme; ++tm) row_tile(tm);
}

__global__ __launch_bounds__(256) void quantize_w8_kernel(
    const float *__restrict__ w, int K, float max_q, int8_t *__restrict__ q,
    float *__restrict__ scales) {
  __shared__ float smax[4];
  const int64_t n = blockIdx.x;
  const float *wr = w + n * K;
  float mx = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) mx = fmaxf(mx, fabsf(wr[k]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
  float s = mx / max_q;
  if (s == 0.0f) s = 1.0f;
  if (threadIdx.x == 0) scales[n] = s;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    float qf = roundf(wr[k] / s);
    qf = fmaxf(-max_q, fminf(max_q, qf));
    q[n * K + k] = (int8_t)qf;
  }
}

// Row-major int8 [R][K] <-> MFMA operand layout, one 16-byte piece per
// thread (piece p is the p-th 16 bytes of the operand layout).
__global__ __launch_bounds__(256) void swizzle_rows_kernel(
    const int8_t *__restrict__ src, int R, int K, int8_t *__restrict__ dst,
    int inverse) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= (int64_t)R * K / 16) return;
  const int nch = K / 128;
  const int lane = (int)(p & 63);
  int64_t q = p >> 6;
  const int s = (int)(q & 3);
  q >>= 2;
  const int c = (int)(q % nch);
  const int64_t t = q / nch;
  const int64_t row = t * 32 + (lane & 31);
  const int col = c * 128 + s * 32 + (lane >> 5) * 16;
  if (inverse)
    *reinterpret_cast<v4i *>(dst + row * K + col) =
        *reinterpret_cast<const v4i *>(src + p * 16);
  else
    *reinterpret_cast<v4i *>(dst + p * 16) =
        *reinterpret_cast<const v4i *>(src + row * K + col);
}

// dst[(row_base + n*row_stride)][k] = src[k][n]  (32x32 tiles through LDS)
__global__ __launch_bounds__(256) void transpose_into_kernel(
    const float *__restrict__ src, int K, int N, float *__restrict__ dst,
    int64_t row_base, int64_t row_stride) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    int k = k0 + i, n = n0 + tx;
    tile[i][tx] = (k < K && n < N) ? src[(int64_t)k * N + n] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    int n = n0 + i, k = k0 + tx;
    if (k < K && n < N) dst[(row_base + n * row_stride) * K + k] = tile[tx][i];
  }
}

__global__ __launch_bounds__(256) void transpose_out_kernel(
    const float *__restrict__ src, int K, int N, int64_t row_base,
    int64_t row_stride, float *__restrict__ dst) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    int n = n0 + i, k = k0 + tx;
    tile[i][tx] = (k < K && n < N) ? src[(row_base + n * row_stride) * K + k] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    int k = k0 + i, n = n0 + tx;
    if (k < K && n < N) dst[(int64_t)k * N + n] = tile[tx][i];
  }
}

__device__ __forceinline__ void philox10(uint32_t c[4], uint32_t k0,
                                         uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
    uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
}

// Seeded N(0, std) for element (k, n) of parameter `param` (logical
// [K][N] index k*N + n): Philox4x32-10 + Box-Muller.
__global__ __launch_bounds__(256) void init_normal_kernel(
    float *__restrict__ dst, int K, int N, int64_t row_base,
    int64_t row_stride, uint64_t seed, uint32_t param, float stdv,
    int transposed) {
  int64_t total = (int64_t)K * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    uint32_t c[4] = {(uint32_t)i, (uint32_t)(i >> 32), param, 0x4E4E5744u};
    philox10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    float u1 = ((float)(c[0] >> 8) + 1.0f) * (1.0f / 16777216.0f);
    float u2 = (float)(c[1] >> 8) * (1.0f / 16777216.0f);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795864f * u2);
    int64_t k = i / N, n = i % N;
    int64_t off = transposed ? (row_base + n * row_stride) * K + k : i;
    dst[off] = z * stdv;
  }
}

__global__ void fill_kernel(float *p, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

template <int R, int G>
void gemv16_launch(hipStream_t st, const float *x, int64_t ldx, int K, int N,
                   const int8_t *wq, const float *scale, const float *bias,
                   const float *resid, int64_t ldr, float *y, int64_t ldy,
                   int epi, int64_t row0, const RopeArgs &ra, const GemvLn &lf,
                   int groups) {
  constexpr int NB = Gemv16Shape<G>::NB;
  dim3 grid((N + NB - 1) / NB, groups);
  hipLaunchKernelGGL((gemv16_kernel<R, G>), grid, dim3(256), 0, st, x, ldx, K, N,
                     wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf);
}

template <int R>
void gemv_dispatch(hipStream_t st, const float *x, int64_t ldx, int K, int N,
                   const int8_t *wq, const float *wf, const float *scale,
                   const float *bias, const float *resid, int64_t ldr,
                   float *y, int64_t ldy, int epi, int64_t row0,
                   const RopeArgs &ra, const GemvLn &lf, int groups = 1) {
  // int8 codes, K = 16 G with G a power of two in [16, 256], aligned rows:
  // the 128-bit-load GEMV
  if (wq && g_gemv16 && ldx % 4 == 0 &&
      reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(wq) % 16 == 0) {
    switch (K) {
      case 256: gemv16_launch<R, 16>(st, x, ldx, K, N, wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf, groups); return;
      case 512: gemv16_launch<R, 32>(st, x, ldx, K, N, wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf, groups); return;
      case 1024: gemv16_launch<R, 64>(st, x, ldx, K, N, wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf, groups); return;
      case 2048: gemv16_launch<R, 128>(st, x, ldx, K, N, wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf, groups); return;
      case 4096: gemv16_launch<R, 256>(st, x, ldx, K, N, wq, scale, bias, resid, ldr, y, ldy, epi, row0, ra, lf, groups); return;
      default: break;
    }
  }
  int nks = K >= 1024 ? 4 : (K >= 512 ? 2 : 1);
  int cols = (4 / nks) * kGemvNC;
  dim3 grid((N + cols - 1) / cols, groups);
  if (wq)
    hipLaunchKernelGGL((gemv_kernel<R, true>), grid, dim3(256), 0, st, x, ldx,
                       K, N, wq, wf, scale, bias, resid, ldr, y, ldy, epi,
                       nks, row0, ra, lf);
  else
    hipLaunchKernelGGL((gemv_kernel<R, false>), grid, dim3(256), 0, st, x,
                       ldx, K, N, wq, wf, scale, bias, resid, ldr, y, ldy,
                       epi, nks, row0, ra, lf);
}

}  // namespace

// 1: allow 32x64 GEMM tiles for large grids; 0: always 32x32 (default,
// measured faster on every decode shape).
int g_gemm_wide = 1;
// 1: int8 GEMVs with K of 256-4096 use 128-bit code loads (gemv16_kernel)
int g_gemv16 = 1;

void launch_gemv(hipStream_t st, const float *x, int64_t ldx, int rows, int K,
                 int N, const int8_t *wq, const float *wf, const float *scale,
                 const float *bias, const float *resid, int64_t ldr, float *y,
                 int64_t ldy, int epi, const RopeArgs *ra, const GemvLn *ln) {
  NNHIP_REQUIRE(K % 4 == 0 && K <= 4096, kErrArg, "gemv: K must be a multiple of 4 and <= 4096");
  const GemvLn lz = ln ? *ln : GemvLn{};
  NNHIP_REQUIRE(!lz.g || (lz.b && K <= 1024 && ldx % 4 == 0 &&
                          (!lz.out || lz.ldo % 4 == 0)),
                kErrArg, "gemv: a folded LayerNorm needs K <= 1024 and aligned rows");
  NNHIP_REQUIRE(epi != kEpiSwiGLU || N % 2 == 0, kErrArg, "gemv: SwiGLU needs even N");
  NNHIP_REQUIRE(epi != kEpiRope || ra, kErrArg, "gemv: RoPE epilogue needs its arguments");
  NNHIP_REQUIRE(!(ra && ra->kq), kErrArg,
                "gemv: no int8 KV append in this epilogue (use rope_kv_q8)");
  const RopeArgs rz = ra ? *ra : RopeArgs{};
  // 32 or more rows (the draft's down projection): groups of 4 rows, twice
  // the workgroups of 8-row groups with half the work each (measured faster)
  if (rows >= 32 && rows % 4 == 0) {
    gemv_dispatch<4>(st, x, ldx, K, N, wq, wf, scale, bias, resid, ldr, y,
                     ldy, epi, 0, rz, lz, rows / 4);
    NNHIP_CHECK(hipGetLastError());
    return;
  }
  // 8 rows per workgroup, so that a verify step's k+1 rows (k <= 7) read
  // the weights once: the whole groups of 8 rows in one launch (one row
  // group per grid row), the remainder in a second
  const int full = rows / 8;
  if (full > 0)
    gemv_dispatch<8>(st, x, ldx, K, N, wq, wf, scale, bias, resid, ldr, y,
                     ldy, epi, 0, rz, lz, full);
  for (int r0 = full * 8; r0 < rows; r0 += 8) {
    int rr = rows - r0 < 8 ? rows - r0 : 8;
    const float *xp = x + r0 * ldx;
    const float *rp = resid ? resid + r0 * ldr : nullptr;
    float *yp = y ? y + r0 * ldy : nullptr;
    GemvLn lp = lz;
    if (lp.out) lp.out += r0 * lp.ldo;
#define NNHIP_GEMV(R) \
    gemv_dispatch<R>(st, xp, ldx, K, N, wq, wf, scale, bias, rp, ldr, yp, ldy, epi, r0, rz, lp)
    switch (rr) {
      case 1: NNHIP_GEMV(1); break;
      case 2: NNHIP_GEMV(2); break;
      case 3: NNHIP_GEMV(3); break;
      case 4: NNHIP_GEMV(4); break;
      case 5: NNHIP_GEMV(5); break;
      case 6: NNHIP_GEMV(6); break;
      case 7: NNHIP_GEMV(7); break;
      default: NNHIP_GEMV(8); break;
    }
#undef NNHIP_GEMV
  }
  NNHIP_CHECK(hipGetLastError());
}

void launch_act_quant(hipStream_t st, const float *x, int64_t ldx, int rows,
                      int K, int8_t *limbs, int mpad, int *rexp) {
  if (rows <= 0) return;
  NNHIP_REQUIRE(K % 128 == 0 && ldx % 4 == 0 && rows <= mpad, kErrArg,
                "act_quant: K % 128 and ldx % 4 must be 0");
  NNHIP_REQUIRE(K <= 4096, kErrArg, "act_quant: K must be <= 4096");
  // one wave per 1024 entries of a row (at most 4 per row)
  if (K <= 1024)
    hipLaunchKernelGGL((act_quant_kernel<4, 1>), dim3((rows + 3) / 4), dim3(256),
                       0, st, x, ldx, K, rows, limbs, mpad, rexp);
  else if (K <= 2048)
    hipLaunchKernelGGL((act_quant_kernel<4, 2>), dim3((rows + 1) / 2), dim3(256),
                       0, st, x, ldx, K, rows, limbs, mpad, rexp);
  else
    hipLaunchKernelGGL((act_quant_kernel<4, 4>), dim3(rows), dim3(256), 0, st,
                       x, ldx, K, rows, limbs, mpad, rexp);
  NNHIP_CHECK(hipGetLastError());
}

int g_limb_k8 = 512;

// The int8 KV append in gemm_limb_kernel's epilogue needs each head's pairs
// within one tile row's 16 (32x32 tiles) column pairs.
bool gemm_limb_q8_ok(int D) { return rope_q8_head_dim_ok(D) && D <= 32; }

void launch_gemm_limb(hipStream_t st, const int8_t *limbs, int mpad,
                      const int *rexp, int rows, int K, int N,
                      const int8_t *wq, const float *scale, const float *bias,
                      const float *resid, int64_t ldr, float *y, int64_t ldy,
                      int epi, const RopeArgs *ra) {
  NNHIP_REQUIRE(K % 128 == 0 && N % 64 == 0, kErrArg,
                "gemm_limb: K % 128 and N % 64 must be 0");
  NNHIP_REQUIRE(epi != kEpiRope || ra, kErrArg,
                "gemm_limb: RoPE epilogue needs its arguments");
  const RopeArgs rz = ra ? *ra : RopeArgs{};
  NNHIP_REQUIRE(mpad % 64 == 0 && rows <= mpad, kErrArg, "gemm_limb: bad mpad");
  const bool q8 = epi == kEpiRope && rz.kq;
  NNHIP_REQUIRE(!q8 || gemm_limb_q8_ok(rz.D), kErrArg,
                "gemm_limb: int8 KV append needs a power-of-two head dim <= 32");
  // 32x64 tiles when they alone give enough workgroups to fill the chip,
  // otherwise 32x32 tiles (twice the workgroups, two resident per CU)
  const int ntm = (rows + kGemmMT - 1) / kGemmMT;
  const bool wide = ntm * (N / 64) >= 512 && g_gemm_wide != 0;
  if (wide) {
    const int ntn = N / 64, per = (ntm * ntn + 7) / 8;
    hipLaunchKernelGGL(gemm_limb_kernel<2>, dim3(8 * per), dim3(256), 0, st,
                       limbs, mpad, rexp, rows, K, N, wq, scale, bias, resid,
                       ldr, y, ldy, epi, ntm, ntn, rz);
  } else if (K >= g_limb_k8) {
    // K >= 512: 8 waves split it, half the chunks each (at K = 512 four of
    // them have no chunk and add zeros; the epilogue is still spread over 512
    // threads, measured faster than 4 waves)
    const int ntn = N / 32, per = (ntm * ntn + 7) / 8;
    hipLaunchKernelGGL((gemm_limb_kernel<1, 8>), dim3(8 * per), dim3(512), 0, st,
                       limbs, mpad, rexp, rows, K, N, wq, scale, bias, resid,
                       ldr, y, ldy, epi, ntm, ntn, rz);
  } else {
    const int ntn = N / 32, per = (ntm * ntn + 7) / 8;
    hipLaunchKernelGGL(gemm_limb_kernel<1>, dim3(8 * per), dim3(256), 0, st,
                       limbs, mpad, rexp, rows, K, N, wq, scale, bias, resid,
                       ldr, y, ldy, epi, ntm, ntn, rz);
  }
  NNHIP_CHECK(hipGetLastError());
}

void launch_gemm_limb_hx(hipStream_t st, const int8_t *limbs, int mpad,
                         const int *hexp, int rows, int K, int N,
                         const int8_t *wq, const float *scale, const float *bias,
                         const float *resid, int64_t ldr, float *y, int64_t ldy,
                         int epi) {
  NNHIP_REQUIRE(K % 128 == 0 && K / 64 <= kMaxHxChunks && N % 64 == 0 && rows > 0,
                kErrArg, "gemm_limb_hx: K % 128 == 0, K <= 2048, N % 64 == 0");
  NNHIP_REQUIRE(limbs && hexp && mpad % 64 == 0 && rows <= mpad, kErrArg,
                "gemm_limb_hx: digit planes missing or bad mpad");
  NNHIP_REQUIRE(epi == kEpiBias || epi == kEpiResid, kErrArg,
                "gemm_limb_hx: bias or residual epilogue only");
  const int ntm = (rows + kGemmMT - 1) / kGemmMT;
  const int ntn = N / 32, per = (ntm * ntn + 7) / 8;
  if (K >= g_limb_k8)
    hipLaunchKernelGGL((gemm_limb_kernel<1, 8, true>), dim3(8 * per), dim3(512), 0, st,
                       limbs, mpad, hexp, rows, K, N, wq, scale, bias, resid,
                       ldr, y, ldy, epi, ntm, ntn, RopeArgs{});
  else
    hipLaunchKernelGGL((gemm_limb_kernel<1, 4, true>), dim3(8 * per), dim3(256), 0, st,
                       limbs, mpad, hexp, rows, K, N, wq, scale, bias, resid,
                       ldr, y, ldy, epi, ntm, ntn, RopeArgs{});
  NNHIP_CHECK(hipGetLastError());
}

int gemm_lds_tile_width(int K) {
  // 16 waves of 32 columns over K/KS each: 128-column blocks when KS = 4
  return K == 512 || K == 1024 ? 2 * kWave : 0;
}

void launch_gemm_lds(hipStream_t st, int mode, const int8_t *limbs, int mpad,
                     const int *rexp, const float *x, int64_t ldx,
                     const float *lng, const float *lnb, float *ln_out,
                     int64_t ldo, int rows, int K, int N, const int8_t *wq,
                     const float *scale, const float *bias,
                     const float *resid, int64_t ldr, float *y, int64_t ldy,
                     int epi, const RopeArgs *ra, const TileStatsArgs *ts) {
  NNHIP_REQUIRE(gemm_lds_supports(rows, K, N), kErrArg,
                "gemm_lds: needs K in {128, 256, 512, 1024}, N % 32 == 0");
  NNHIP_REQUIRE(epi != kEpiRope || ra, kErrArg,
                "gemm_lds: RoPE epilogue needs its arguments");
  if (mode == kAFromDigits)
    NNHIP_REQUIRE(limbs && rexp && rows <= mpad && mpad % 32 == 0, kErrArg,
                  "gemm_lds: digit planes missing");
  else
    NNHIP_REQUIRE(x && ldx >= K && ldx % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(x) & 15) == 0,
                  kErrArg, "gemm_lds: rows must be 16-byte aligned, ldx >= K");
  if (mode == kAFromLayerNorm)
    NNHIP_REQUIRE(lng && lnb && (!ln_out || (ldo >= K && ldo % 4 == 0)),
                  kErrArg, "gemm_lds: LayerNorm parameters missing");
  const RopeArgs rz = ra ? *ra : RopeArgs{};
  const bool q8 = epi == kEpiRope && rz.kq;
  NNHIP_REQUIRE(!q8 || rope_q8_head_dim_ok(rz.D), kErrArg,
                "gemm_lds: int8 KV append needs a power-of-two head dim <= 64");
  const int ntm = (rows + kGemmMT - 1) / kGemmMT;
  NNHIP_REQUIRE(!ts || !ts->out || (gemm_lds_tile_width(K) > 0 && epi == kEpiBias),
                kErrArg, "gemm_lds: tile statistics need K of 512 or 1024 and a bias epilogue");
  const TileStatsArgs tz = ts ? *ts : TileStatsArgs{};
  const int ntn = (int)(gemm_lds_workgroups(rows, K, N) / ntm);
  // digit planes: a workgroup walks as many row tiles as it takes for all
  // workgroups to be resident at once (one per CU), so that the weights are
  // read once and no second wave of workgroups waits behind the first
  int rpt = 1;
  if (mode == kAFromDigits && ntm * ntn > kGemmSlots)
    rpt = ntn >= kGemmSlots ? ntm : (ntm + kGemmSlots / ntn - 1) / (kGemmSlots / ntn);
  const int per = ((ntm + rpt - 1) / rpt * ntn + 7) / 8;
  dim3 grid(8 * per);
#define NNHIP_GL(MD, KP)                                                      \
  if (q8)                                                                     \
    hipLaunchKernelGGL((gemm_lds_kernel<MD, KP, true>), grid,                 \
                       dim3(kLdsThreads), 0, st, limbs, mpad, rexp, x, ldx,   \
                       lng, lnb, ln_out, ldo, rows, N, wq, scale, bias, resid, \
                       ldr, y, ldy, epi, ntm, ntn, rpt, rz, tz);              \
  else                                                                        \
    hipLaunchKernelGGL((gemm_lds_kernel<MD, KP, false>), grid,                \
                       dim3(kLdsThreads), 0, st, limbs, mpad, rexp, x, ldx,   \
                       lng, lnb, ln_out, ldo, rows, N, wq, scale, bias, resid, \
                       ldr, y, ldy, epi, ntm, ntn, rpt, rz, tz)
#define NNHIP_GL_K(MD)                                                        \
  switch (K) {                                                                \
    case 128: { NNHIP_GL(MD, 4); } break;                                     \
    case 256: { NNHIP_GL(MD, 8); } break;                                     \
    case 512: { NNHIP_GL(MD, 16); } break;                                    \
    default: { NNHIP_GL(MD, 32); } break;                                     \
  }
  if (mode == kAFromDigits) { NNHIP_GL_K(kAFromDigits) }
  else if (mode == kAFromRows) { NNHIP_GL_K(kAFromRows) }
  else { NNHIP_GL_K(kAFromLayerNorm) }
#undef NNHIP_GL_K
#undef NNHIP_GL
  NNHIP_CHECK(hipGetLastError());
}

void launch_quantize_w8(hipStream_t st, const float *w_nk, int N, int K,
                        int8_t *q_nk, float *scales, int bits) {
  NNHIP_REQUIRE(bits == 8 || bits == 4, kErrUnsupported,
                "weight quantization: INT8 or INT4 only");
  hipLaunchKernelGGL(quantize_w8_kernel, dim3(N), dim3(256), 0, st, w_nk, K,
                     bits == 8 ? 127.0f : 7.0f, q_nk, scales);
  NNHIP_CHECK(hipGetLastError());
}

void launch_swizzle_rows(hipStream_t st, const int8_t *src, int R, int K,
                         int8_t *dst, bool inverse) {
  NNHIP_REQUIRE(R % 32 == 0 && K % 128 == 0, kErrArg,
                "swizzle: R % 32 and K % 128 must be 0");
  const int64_t pieces = (int64_t)R * K / 16;
  hipLaunchKernelGGL(swizzle_rows_kernel, dim3((unsigned)((pieces + 255) / 256)),
                     dim3(256), 0, st, src, R, K, dst, inverse ? 1 : 0);
  NNHIP_CHECK(hipGetLastError());
}

void launch_transpose_into(hipStream_t st, const float *src_kn, int K, int N,
                           float *dst, int64_t row_base, int64_t row_stride) {
  dim3 grid((N + 31) / 32, (K + 31) / 32);
  hipLaunchKernelGGL(transpose_into_kernel, grid, dim3(256), 0, st, src_kn, K,
                     N, dst, row_base, row_stride);
  NNHIP_CHECK(hipGetLastError());
}

void launch_transpose_out(hipStream_t st, const float *src, int K, int N,
                          int64_t row_base, int64_t row_stride, float *dst_kn) {
  dim3 grid((N + 31) / 32, (K + 31) / 32);
  hipLaunchKernelGGL(transpose_out_kernel, grid, dim3(256), 0, st, src, K, N,
                     row_base, row_stride, dst_kn);
  NNHIP_CHECK(hipGetLastError());
}

void launch_init_normal(hipStream_t st, float *dst, int K, int N,
                        int64_t row_base, int64_t row_stride, uint64_t seed,
                        uint32_t param, float stdv, int transposed) {
  int64_t total = (int64_t)K * N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(init_normal_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     st, dst, K, N, row_base, row_stride, seed, param, stdv,
                     transposed);
  NNHIP_CHECK(hipGetLastError());
}

void launch_fill(hipStream_t st, float *p, int64_t n, float v) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p,
                     n, v);
  NNHIP_CHECK(hipGetLastError());
}

}  // namespace nnhip

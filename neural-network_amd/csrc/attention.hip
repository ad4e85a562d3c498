// Token embedding, RoPE + KV-cache append, k-query causal attention over the
// device-resident KV cache, and LayerNorm for gfx950.
//
// Replaces the host loops of MultiHeadAttention::forward (layer.cpp:593-994):
// RoPE (tensor.cpp:1126-1226), the O(S) KV concat (layer.cpp:758-807), the
// fused ThreadPool attention (layer.cpp:842-952), plus Embedding
// (cpu_backend.cpp:998-1033) and LayerNorm (layer.cpp:242-261).
//
// KV cache layout: per layer [B][H_kv][cap][D] fp32, so one (sequence, head)
// is a contiguous [cap][D] slab; appending is a write at the sequence's own
// length and truncation (KVCache::truncate, layer.cpp:67-149) is a length
// update.  Each sequence carries its own length, so a batch is ragged.
#include "nnhip_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace nnhip {

namespace {

constexpr int kWave = 64;
constexpr int kKeysPerSplit = 128;
constexpr int kMaxQ = 8;       // queries per workgroup
constexpr int kMaxD = 64;      // head dim handled by the attention kernel

// Embedding gather (cpu_backend.cpp:1020-1025): ids outside [0, vocab) read
// row 0.  Row t = b*S + s takes ids[b*stride_b + s].
__global__ __launch_bounds__(256) void embed_kernel(
    const float *__restrict__ emb, int vocab, int d,
    const int32_t *__restrict__ ids, int S, int stride_b,
    float *__restrict__ x) {
  const int t = blockIdx.x;
  const int b = t / S, s = t % S;
  int id = ids[(int64_t)b * stride_b + s];
  if (id < 0 || id >= vocab) id = 0;
  const float *src = emb + (int64_t)id * d;
  float *dst = x + (int64_t)t * d;
  for (int i = threadIdx.x; i < d; i += blockDim.x) dst[i] = src[i];
}

// verify input of one cycle: [generated.back(), c_0 .. c_{k-1}] per sequence
// (layer.cpp:1560-1566).
__global__ void build_verify_ids_kernel(const int32_t *__restrict__ cur,
                                        const int32_t *__restrict__ cand, int B,
                                        int k, int32_t *__restrict__ ids) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * (k + 1)) return;
  int b = i / (k + 1), s = i % (k + 1);
  ids[i] = s == 0 ? cur[b] : cand[b * k + s - 1];
}

// RoPE on q and k at position base[b] + off + s (tensor.cpp:1141-1173, with
// the cos/sin table computed on the host by the same float formula), then
// append rotated k and v to the cache.  qkv row t = b*S + s holds
// [q(H*D) | k(H*D) | v(H*D)].
__global__ __launch_bounds__(256) void rope_kv_kernel(
    const float *__restrict__ qkv, int S, int H, int D,
    const int32_t *__restrict__ base, int off,
    const int32_t *__restrict__ active, const float *__restrict__ cosb,
    const float *__restrict__ sinb, float *__restrict__ qrot,
    float *__restrict__ kc, float *__restrict__ vc, int cap,
    int64_t seq_stride) {
#pragma clang fp contract(off)
  const int t = blockIdx.x;
  const int b = t / S, s = t % S;
  if (active && !active[b]) return;
  const int pos = base[b] + off + s;
  if (pos < 0 || pos >= cap) return;
  const int E = H * D, half = D / 2;
  const float *row = qkv + (int64_t)t * 3 * E;
  for (int i = threadIdx.x; i < H * half; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float c = cosb[(int64_t)pos * half + j];
    const float sn = sinb[(int64_t)pos * half + j];
    const int e = h * D + 2 * j;
    float xe = row[e], xo = row[e + 1];
    qrot[(int64_t)t * E + e] = xe * c - xo * sn;
    qrot[(int64_t)t * E + e + 1] = xe * sn + xo * c;
    xe = row[E + e]; xo = row[E + e + 1];
    float *kd = kc + b * seq_stride + ((int64_t)h * cap + pos) * D + 2 * j;
    kd[0] = xe * c - xo * sn;
    kd[1] = xe * sn + xo * c;
    float *vd = vc + b * seq_stride + ((int64_t)h * cap + pos) * D + 2 * j;
    vd[0] = row[2 * E + e];
    vd[1] = row[2 * E + e + 1];
  }
}

// ---------------------------------------------------------------------------
// Split-K attention.  Grid (split of 128 keys, head, b * n_qblocks).  Each of
// the 32 lane groups (8 lanes, 8 dims per lane) loads 4 consecutive keys at
// once, scores them for every query of the block, and keeps (max, sum, acc)
// per query; groups merge by shuffles, waves through LDS, and the split's
// partial state is written for attn_combine_kernel.  Arithmetic: score =
// dot / sqrt(D), keys j > q_pos masked, p = exp(score - max), out =
// (sum p v) * (1 / sum p), as layer.cpp:859-948.
// ---------------------------------------------------------------------------
constexpr int kKeysPerGroup = 4;

// Sum over the 8 lanes of an aligned lane group with DPP: swap neighbours,
// swap pairs, then mirror the two quads (row_half_mirror).
__device__ __forceinline__ float group8_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
           0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
           0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
           0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}

template <int SQ>
__global__ __launch_bounds__(256) void attn_kernel(
    const float *__restrict__ q, const float *__restrict__ kc,
    const float *__restrict__ vc, int S, int H, int Hkv, int D, int cap,
    int64_t seq_stride, const int32_t *__restrict__ base, int off,
    const int32_t *__restrict__ active, int nsplit, int nqb, int kps,
    float *__restrict__ part) {
  constexpr int kGroups = 32;
  __shared__ float s_m[kGroups][SQ], s_l[kGroups][SQ], s_f[kGroups][SQ];
  __shared__ float s_acc[kGroups][SQ][kMaxD];
  __shared__ float s_M[SQ];
  const int sp = blockIdx.x, h = blockIdx.y;
  const int b = blockIdx.z / nqb, qb = blockIdx.z % nqb;
  if (active && !active[b]) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = w * 8 + (lane >> 3), sub = lane & 7;
  const int q0 = qb * kMaxQ;
  const int nq = min(SQ, S - q0);
  const int E = H * D;
  const int hk = h / (H / Hkv);
  const int pos0 = base[b] + off + q0;         // position of query q0
  const int kend_all = min(pos0 + nq, cap);    // keys [0, kend_all) visible
  const int ks = sp * kps;
  const int kend = min(ks + kps, kend_all);
  const float scale = sqrtf((float)D);
  const int dl = D / 8;                        // dims per lane (<= 8)
  const float *kb = kc + b * seq_stride + (int64_t)hk * cap * D;
  const float *vb = vc + b * seq_stride + (int64_t)hk * cap * D;

  // the block's queries, read by every lane group through LDS broadcasts
  __shared__ float s_q[SQ][kMaxD];
  for (int t = threadIdx.x; t < SQ * kMaxD; t += blockDim.x) {
    const int i = t / kMaxD, dd = t % kMaxD;
    s_q[i][dd] = (i < nq && dd < D) ? q[((int64_t)b * S + q0 + i) * E + h * D + dd] : 0.f;
  }
  __syncthreads();
  float m[SQ], l[SQ], acc[SQ][8];
#pragma unroll
  for (int i = 0; i < SQ; ++i) {
    m[i] = -INFINITY; l[i] = 0.f;
#pragma unroll
    for (int x = 0; x < 8; ++x) acc[i][x] = 0.f;
  }

  struct Blk { float k[kKeysPerGroup][8], v[kKeysPerGroup][8]; };
  auto load = [&](int j0, Blk &bk) {
#pragma unroll
    for (int e = 0; e < kKeysPerGroup; ++e) {
      const int j = j0 + e;
      const bool ok = j < kend;
      if (dl == 8) {
        float4 k0 = make_float4(0.f, 0.f, 0.f, 0.f), k1 = k0, v0 = k0, v1 = k0;
        if (ok) {
          const float4 *kp = reinterpret_cast<const float4 *>(kb + (int64_t)j * D + sub * 8);
          const float4 *vp = reinterpret_cast<const float4 *>(vb + (int64_t)j * D + sub * 8);
          k0 = kp[0]; k1 = kp[1]; v0 = vp[0]; v1 = vp[1];
        }
        bk.k[e][0] = k0.x; bk.k[e][1] = k0.y; bk.k[e][2] = k0.z; bk.k[e][3] = k0.w;
        bk.k[e][4] = k1.x; bk.k[e][5] = k1.y; bk.k[e][6] = k1.z; bk.k[e][7] = k1.w;
        bk.v[e][0] = v0.x; bk.v[e][1] = v0.y; bk.v[e][2] = v0.z; bk.v[e][3] = v0.w;
        bk.v[e][4] = v1.x; bk.v[e][5] = v1.y; bk.v[e][6] = v1.z; bk.v[e][7] = v1.w;
      } else {
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          bk.k[e][x] = (ok && x < dl) ? kb[(int64_t)j * D + sub * dl + x] : 0.f;
          bk.v[e][x] = (ok && x < dl) ? vb[(int64_t)j * D + sub * dl + x] : 0.f;
        }
      }
    }
  };
  // online softmax over one block of 4 keys starting at j0
  auto consume = [&](int j0, const Blk &bk) {
#pragma unroll
    for (int i = 0; i < SQ; ++i) {
      float qv[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) qv[x] = x < dl ? s_q[i][sub * dl + x] : 0.f;
      float sc[kKeysPerGroup];
      float mb = -INFINITY;
#pragma unroll
      for (int e = 0; e < kKeysPerGroup; ++e) {
        float dot = 0.f;
#pragma unroll
        for (int x = 0; x < 8; ++x) dot += qv[x] * bk.k[e][x];
        dot = group8_sum(dot);
        const int j = j0 + e;
        const bool valid = i < nq && j < kend && j <= pos0 + i;   // causal
        sc[e] = valid ? dot / scale : -INFINITY;
        mb = fmaxf(mb, sc[e]);
      }
      if (mb == -INFINITY) continue;
      const float mn = fmaxf(m[i], mb);
      const float a = (m[i] == -INFINITY) ? 0.f : expf(m[i] - mn);
      l[i] *= a;
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[i][x] *= a;
      m[i] = mn;
#pragma unroll
      for (int e = 0; e < kKeysPerGroup; ++e) {
        const float p = expf(sc[e] - mn);        // 0 for masked keys
        l[i] += p;
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[i][x] += p * bk.v[e][x];
      }
    }
  };
  // group g takes blocks g, g+32, ... of the split; the next block's loads
  // are in flight while the current one is scored
  constexpr int kStride = kGroups * kKeysPerGroup;
  Blk ba, bb;
  int j0 = ks + g * kKeysPerGroup;
  if (j0 < kend) load(j0, ba);
  while (j0 < kend) {
    if (j0 + kStride < kend) load(j0 + kStride, bb);
    consume(j0, ba);
    j0 += kStride;
    if (j0 >= kend) break;
    if (j0 + kStride < kend) load(j0 + kStride, ba);
    consume(j0, bb);
    j0 += kStride;
  }
#pragma unroll
  for (int i = 0; i < SQ; ++i) {
    if (sub == 0) { s_m[g][i] = m[i]; s_l[g][i] = l[i]; }
#pragma unroll
    for (int x = 0; x < 8; ++x)
      if (x < dl) s_acc[g][i][sub * dl + x] = acc[i][x];
  }
  __syncthreads();
  // merge the 32 groups: per query the common max, per (group, query) the
  // rescale factor, then per (query, dim) the weighted sums
  if (threadIdx.x < nq) {
    float mn = -INFINITY;
    for (int gg = 0; gg < kGroups; ++gg) mn = fmaxf(mn, s_m[gg][threadIdx.x]);
    s_M[threadIdx.x] = mn;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < kGroups * nq; t += blockDim.x) {
    const int gg = t / nq, i = t % nq;
    const float mg = s_m[gg][i];
    s_f[gg][i] = (mg == -INFINITY) ? 0.f : expf(mg - s_M[i]);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nq * D; t += blockDim.x) {
    const int i = t / D, dd = t % D;
    float ls = 0.f, as = 0.f;
    for (int gg = 0; gg < kGroups; ++gg) {
      const float f = s_f[gg][i];
      ls += s_l[gg][i] * f;
      as += s_acc[gg][i][dd] * f;
    }
    const int64_t row = (int64_t)b * S + q0 + i;
    const int64_t pi = (row * H + h) * nsplit + sp;
    float *pp = part + pi * (D + 2);
    if (dd == 0) { pp[0] = s_M[i]; pp[1] = ls; }
    pp[2 + dd] = as;
  }
}

// Merges the splits of every head of one row (b, s), writes the context row
// [H*D] and, when requested, its int8 digits for the output projection
// (same rule as act_quant_kernel).
__global__ __launch_bounds__(256) void attn_combine_kernel(
    const float *__restrict__ part, int S, int H, int D, int nsplit,
    const int32_t *__restrict__ active, float *__restrict__ out,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
  __shared__ float srow[4096];
  __shared__ float sred[4];
  const int64_t row = blockIdx.x;
  if (active && !active[row / S]) return;
  const int E = H * D;
  float mx = 0.f;
  for (int t = threadIdx.x; t < E; t += blockDim.x) {
    const int h = t / D, dd = t % D;
    const float *pp = part + (row * H + h) * nsplit * (D + 2);
    float mn = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) mn = fmaxf(mn, pp[sp * (D + 2)]);
    float ls = 0.f, as = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float ms = pp[sp * (D + 2)];
      const float f = (ms == -INFINITY) ? 0.f : expf(ms - mn);
      ls += pp[sp * (D + 2) + 1] * f;
      as += pp[sp * (D + 2) + 2 + dd] * f;
    }
    const float inv = ls > 0.f ? 1.0f / ls : 0.f;
    const float v = as * inv;
    out[row * E + t] = v;
    if (limbs) { srow[t] = v; mx = fmaxf(mx, fabsf(v)); }
  }
  if (!limbs) return;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
  const int e = digit_exponent(mx);
  if (threadIdx.x == 0) rexp[row] = e;
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int64_t plane = (int64_t)mpad * E;
  for (int p = threadIdx.x; p < E / 16; p += blockDim.x) {
    const int k = p * 16;
    v4i hi, mid, lo;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int3 t = digits4(srow + k + 4 * qq, e);
      hi[qq] = t.x; mid[qq] = t.y; lo[qq] = t.z;
    }
    const int64_t o2 = mfma_operand_offset((int)row, k, E);
    *reinterpret_cast<v4i *>(limbs + o2) = hi;
    *reinterpret_cast<v4i *>(limbs + plane + o2) = mid;
    *reinterpret_cast<v4i *>(limbs + 2 * plane + o2) = lo;
  }
}

// LayerNorm (layer.cpp:242-261): mean = sum/N, var = sum((x-mean)^2)/N,
// y = (x - mean) / sqrt(var + 1e-5) * gamma + beta.  Optionally also writes
// the int8 digits of y for the next MFMA GEMM (same rule as act_quant).
__global__ __launch_bounds__(256) void layernorm_kernel(
    const float *__restrict__ hin, int d, const float *__restrict__ g,
    const float *__restrict__ bt, float *__restrict__ y,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
#pragma clang fp contract(off)
  __shared__ float sred[4];
  constexpr int kPer = 16;                 // d <= 4096
  const int64_t row = blockIdx.x;
  const float *xr = hin + row * d;
  float v[kPer];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    int c = threadIdx.x + i * 256;
    v[i] = c < d ? xr[c] : 0.f;
    s += v[i];
  }
  auto block_sum = [&](float a) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o, kWave);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = a;
    __syncthreads();
    return (sred[0] + sred[1]) + (sred[2] + sred[3]);
  };
  const float N = (float)d;
  const float mean = block_sum(s) / N;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    int c = threadIdx.x + i * 256;
    if (c < d) { float df = v[i] - mean; sq += df * df; }
  }
  const float var = block_sum(sq) / N;
  const float sd = sqrtf(var + 1e-5f);
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    int c = threadIdx.x + i * 256;
    if (c < d) {
      float xh = (v[i] - mean) / sd;
      v[i] = xh * g[c] + bt[c];
      y[row * d + c] = v[i];
      mx = fmaxf(mx, fabsf(v[i]));
    }
  }
  if (!limbs) return;
  // digits of y for the next MFMA GEMM, in the MFMA operand layout
  __shared__ float srow[4096];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    int c = threadIdx.x + i * 256;
    if (c < d) srow[c] = v[i];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
  const int e = digit_exponent(mx);
  if (threadIdx.x == 0) rexp[row] = e;
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int64_t plane = (int64_t)mpad * d;
  for (int p = threadIdx.x; p < d / 16; p += 256) {
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

__global__ void add_scalar_kernel(int32_t *p, int n, int v) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] += v;
}

}  // namespace

void launch_add_scalar(hipStream_t st, int32_t *p, int n, int v) {
  hipLaunchKernelGGL(add_scalar_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     st, p, n, v);
  NNHIP_CHECK(hipGetLastError());
}

void launch_embed(hipStream_t st, const float *emb, int vocab, int d,
                  const int32_t *ids, int rows, float *x) {
  // ids contiguous, one per row
  hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(256), 0, st, emb, vocab, d,
                     ids, 1, 1, x);
  NNHIP_CHECK(hipGetLastError());
}

void launch_embed_strided(hipStream_t st, const float *emb, int vocab, int d,
                          const int32_t *ids, int B, int S, int stride_b,
                          float *x) {
  hipLaunchKernelGGL(embed_kernel, dim3(B * S), dim3(256), 0, st, emb, vocab,
                     d, ids, S, stride_b, x);
  NNHIP_CHECK(hipGetLastError());
}

void launch_build_verify_ids(hipStream_t st, const int32_t *cur,
                             const int32_t *cand, int B, int k, int32_t *ids) {
  int n = B * (k + 1);
  hipLaunchKernelGGL(build_verify_ids_kernel, dim3((n + 255) / 256), dim3(256),
                     0, st, cur, cand, B, k, ids);
  NNHIP_CHECK(hipGetLastError());
}

void launch_rope_kv(hipStream_t st, const float *qkv, int B, int S, int H,
                    int D, const int32_t *base, int off, const int32_t *active,
                    const float *cosb, const float *sinb, float *qrot,
                    float *kc, float *vc, int cap, int64_t seq_stride) {
  hipLaunchKernelGGL(rope_kv_kernel, dim3(B * S), dim3(256), 0, st, qkv, S, H,
                     D, base, off, active, cosb, sinb, qrot, kc, vc, cap,
                     seq_stride);
  NNHIP_CHECK(hipGetLastError());
}

// Splits of the key range: enough (sequence, head, query block, split)
// workgroups to fill the GPU about 3 times over, each split a multiple of
// 128 keys.
static int attention_splits(int B, int S, int H, int max_keys, int *kps) {
  const int nqb = (S + kMaxQ - 1) / kMaxQ;
  const int units = std::max(1, B * H * nqb);
  const int max_split = std::max(1, (std::max(max_keys, 1) + kKeysPerSplit - 1) / kKeysPerSplit);
  int ns = std::min(max_split, std::max(1, (768 + units - 1) / units));
  int k = (std::max(max_keys, 1) + ns - 1) / ns;
  k = (k + kKeysPerSplit - 1) / kKeysPerSplit * kKeysPerSplit;
  ns = (std::max(max_keys, 1) + k - 1) / k;
  if (kps) *kps = k;
  return ns;
}

int64_t attention_partial_elems(int B, int S, int H, int D, int max_keys) {
  const int nsplit = attention_splits(B, S, H, max_keys, nullptr);
  return (int64_t)B * S * H * nsplit * (D + 2);
}

void launch_attention(hipStream_t st, const float *q, const float *kc,
                      const float *vc, int B, int S, int H, int Hkv, int D,
                      int cap, int64_t seq_stride, const int32_t *base,
                      int off, const int32_t *active, int max_keys,
                      float *part, int64_t part_elems, float *out,
                      int8_t *limbs, int mpad, int *rexp) {
  NNHIP_REQUIRE(D % 8 == 0 && D <= kMaxD, kErrArg,
                "attention: head dim must be a multiple of 8 and <= 64");
  NNHIP_REQUIRE(Hkv > 0 && H % Hkv == 0, kErrArg, "attention: bad kv heads");
  NNHIP_REQUIRE(H * D <= 4096, kErrArg, "attention: H*D must be <= 4096");
  NNHIP_REQUIRE(!limbs || ((H * D) % 128 == 0 && B * S <= mpad), kErrArg,
                "attention: digit output needs H*D % 128 == 0");
  if (max_keys < 1) max_keys = 1;
  int kps = 0;
  const int nsplit = attention_splits(B, S, H, max_keys, &kps);
  NNHIP_REQUIRE(part_elems >= attention_partial_elems(B, S, H, D, max_keys),
                kErrArg, "attention: partial buffer too small");
  const int nqb = (S + kMaxQ - 1) / kMaxQ;
  const int sq = S < kMaxQ ? S : kMaxQ;
  dim3 grid(nsplit, H, B * nqb);
#define NNHIP_ATTN(SQV)                                                      \
  hipLaunchKernelGGL((attn_kernel<SQV>), grid, dim3(256), 0, st, q, kc, vc, S, \
                     H, Hkv, D, cap, seq_stride, base, off, active, nsplit,    \
                     nqb, kps, part)
  switch (sq) {
    case 1: NNHIP_ATTN(1); break;
    case 2: NNHIP_ATTN(2); break;
    case 3: NNHIP_ATTN(3); break;
    case 4: NNHIP_ATTN(4); break;
    case 5: NNHIP_ATTN(5); break;
    case 6: NNHIP_ATTN(6); break;
    case 7: NNHIP_ATTN(7); break;
    default: NNHIP_ATTN(8); break;
  }
#undef NNHIP_ATTN
  NNHIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(attn_combine_kernel, dim3(B * S), dim3(256), 0, st, part,
                     S, H, D, nsplit, active, out, limbs, mpad, rexp);
  NNHIP_CHECK(hipGetLastError());
}

void launch_layernorm(hipStream_t st, const float *h, int rows, int d,
                      const float *g, const float *b, float *y,
                      int8_t *limbs, int mpad, int *rexp) {
  NNHIP_REQUIRE(d <= 4096, kErrArg, "layernorm: d must be <= 4096");
  NNHIP_REQUIRE(!limbs || (d % 128 == 0 && rows <= mpad), kErrArg,
                "layernorm: digit output needs d % 128 == 0");
  hipLaunchKernelGGL(layernorm_kernel, dim3(rows), dim3(256), 0, st, h, d, g,
                     b, y, limbs, mpad, rexp);
  NNHIP_CHECK(hipGetLastError());
}

}  // namespace nnhip

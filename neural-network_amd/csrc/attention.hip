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
#include "rows.hpp"

#include <hip/hip_runtime.h>

#include <type_traits>

#include <algorithm>
#include <cmath>

namespace nnhip {

namespace {

constexpr int kWave = 64;
constexpr int kMaxQ = 8;       // queries per workgroup
// attn_short_q: launches of fewer (sequence, head) pairs than this take
// their queries in blocks of g_attn_short_q
constexpr int kAttnShortUnits = 64;
constexpr int kMaxD = 64;      // head dim handled by the attention kernel

// Embedding gather (cpu_backend.cpp:1020-1025): ids outside [0, vocab) read
// row 0.  Row t = b*S + s takes ids[b*stride_b + s], or with lead set
// lead[b] for s = 0 and ids[b*stride_b + s - 1] after it (the verify rows
// [generated.back(), c_0 .. c_{k-1}] of layer.cpp:1560-1566 read from the
// last tokens and the candidates).  With limbs, the row's digits for the
// first q/k/v GEMM are written too.
__global__ __launch_bounds__(256) void embed_kernel(
    const float *__restrict__ emb, int vocab, int d,
    const int32_t *__restrict__ ids, int S, int stride_b,
    const int32_t *__restrict__ lead, float *__restrict__ x,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
  __shared__ float srow[4096];
  __shared__ float sred[4];
  const int t = blockIdx.x;
  const int b = t / S, s = t % S;
  int id = !lead ? ids[(int64_t)b * stride_b + s]
                 : (s == 0 ? lead[b] : ids[(int64_t)b * stride_b + s - 1]);
  if (id < 0 || id >= vocab) id = 0;
  const float *src = emb + (int64_t)id * d;
  float *dst = x + (int64_t)t * d;
  float mx = 0.f;
  if (d <= 4096 && ((d & 3) | (((uintptr_t)emb | (uintptr_t)x) & 15)) == 0) {
    // float4 pieces, at most 4 per thread (d <= 4096), all requested before
    // any is stored
    const int np = d >> 2;
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = reinterpret_cast<const float4 *>(src)[min((int)threadIdx.x + 256 * j, np - 1)];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = threadIdx.x + 256 * j;
      if (p >= np) break;
      reinterpret_cast<float4 *>(dst)[p] = v[j];
      if (limbs) {
        reinterpret_cast<float4 *>(srow)[p] = v[j];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)),
                             fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
      }
    }
  } else {
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
      const float v = src[i];
      dst[i] = v;
      if (limbs) { srow[i] = v; mx = fmaxf(mx, fabsf(v)); }
    }
  }
  if (limbs) store_row_digits<256>(srow, d, mx, t, limbs, mpad, rexp, sred);
}

// RoPE on q and k at position base[b] + off + s (tensor.cpp:1141-1173, with
// the cos/sin table computed on the host by the same float formula), then
// append rotated k and v to the cache.  qkv row t = b*S + s holds
// [q(H*D) | k(H*D) | v(H*D)].
__global__ __launch_bounds__(256) void rope_kv_kernel(
    const float *__restrict__ qkv, int S, int H, int Hkv, int D,
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
  // row t: [q: H heads | k: Hkv heads | v: Hkv heads] of D
  const int E = H * D, Ekv = Hkv * D, half = D / 2;
  const float *row = qkv + (int64_t)t * (E + 2 * Ekv);
  for (int i = threadIdx.x; i < H * half; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float c = cosb[(int64_t)pos * half + j];
    const float sn = sinb[(int64_t)pos * half + j];
    const int e = h * D + 2 * j;
    const float xe = row[e], xo = row[e + 1];
    qrot[(int64_t)t * E + e] = xe * c - xo * sn;
    qrot[(int64_t)t * E + e + 1] = xe * sn + xo * c;
  }
  for (int i = threadIdx.x; i < Hkv * half; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float c = cosb[(int64_t)pos * half + j];
    const float sn = sinb[(int64_t)pos * half + j];
    const int e = h * D + 2 * j;
    const float xe = row[E + e], xo = row[E + e + 1];
    float *kd = kc + b * seq_stride + ((int64_t)h * cap + pos) * D + 2 * j;
    kd[0] = xe * c - xo * sn;
    kd[1] = xe * sn + xo * c;
    float *vd = vc + b * seq_stride + ((int64_t)h * cap + pos) * D + 2 * j;
    vd[0] = row[E + Ekv + e];
    vd[1] = row[E + Ekv + e + 1];
  }
}

// RoPE on q and k as rope_kv_kernel, then the append into an int8 cache:
// quantize_kv of layer.cpp:635-657 on each new k row (after RoPE) and v row
// of one head: scale = max|x| / 127 (1 when 0), code = clamp(round(x *
// (1 / scale)), +-127), round half away from zero.  One wave per (row,
// head): lane j < D/2 rotates pair j of q and k, lane 32 + j holds pair j
// of v; each half-wave reduces its row's max.
__global__ __launch_bounds__(256) void rope_kv_q8_kernel(
    const float *__restrict__ qkv, int R, int S, int H, int D,
    const int32_t *__restrict__ base, int off,
    const int32_t *__restrict__ active, const float *__restrict__ cosb,
    const float *__restrict__ sinb, float *__restrict__ qrot,
    int8_t *__restrict__ kq, float *__restrict__ ks, int8_t *__restrict__ vq,
    float *__restrict__ vs, int cap, int64_t seq_stride, int64_t sc_stride) {
#pragma clang fp contract(off)
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= R * H) return;
  const int t = wid / H, h = wid % H;
  const int b = t / S, s = t % S;
  if (active && !active[b]) return;
  const int pos = base[b] + off + s;
  if (pos < 0 || pos >= cap) return;
  const int lane = threadIdx.x & 63, half = D / 2, E = H * D;
  const bool vlane = lane >= 32;
  const int j = lane & 31;
  const bool own = j < half;
  const int jj = own ? j : half - 1;
  const float *row = qkv + (int64_t)t * 3 * E + h * D + 2 * jj;
  float xe, xo;
  if (!vlane) {
    const float c = cosb[(int64_t)pos * half + jj];
    const float sn = sinb[(int64_t)pos * half + jj];
    const float qe = row[0], qo = row[1];
    if (own) {
      float *qd = qrot + (int64_t)t * E + h * D + 2 * jj;
      qd[0] = qe * c - qo * sn;
      qd[1] = qe * sn + qo * c;
    }
    const float ke = row[E], ko = row[E + 1];
    xe = ke * c - ko * sn;
    xo = ke * sn + ko * c;
  } else {
    xe = row[2 * E];
    xo = row[2 * E + 1];
  }
  float mx = own ? fmaxf(fabsf(xe), fabsf(xo)) : 0.f;
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  float scale = mx / 127.0f;
  if (scale == 0.0f) scale = 1.0f;
  const float inv = 1.0f / scale;
  const float ce = fmaxf(-127.0f, fminf(127.0f, roundf(xe * inv)));
  const float co = fmaxf(-127.0f, fminf(127.0f, roundf(xo * inv)));
  const int64_t rix = b * sc_stride + (int64_t)h * cap + pos;
  int8_t *dst = (vlane ? vq : kq) + b * seq_stride + ((int64_t)h * cap + pos) * D + 2 * jj;
  if (own) {
    dst[0] = (int8_t)ce;
    dst[1] = (int8_t)co;
  }
  if (j == 0) (vlane ? vs : ks)[rix] = scale;
}

// ---------------------------------------------------------------------------
// Split-K attention: a wave per (key split, head, sequence, query block).
// Either each wave is its own workgroup and writes its split's partial state
// for attn_combine_kernel (W = 1), or the W waves of one workgroup are the
// splits of one (head, sequence, query block) and merge in LDS, writing the
// context rows (W > 1, short contexts).
// Arithmetic as layer.cpp:859-948: score = q.k / sqrt(D), keys j > q_pos
// masked, softmax, out = (sum p v) / (sum p).  The exponentials are taken in
// base 2: the dot product is scaled by log2(e)/sqrt(D) and p = 2^(s - max),
// which is the same function.
//
// A split is walked in chunks of 32 keys; a chunk's K and V rows are all
// requested before any arithmetic.
//  * Scores: lane group g (8 lanes, D/8 dims per lane) owns keys c0+g+8t,
//    t < 4.  Each lane forms partial dot products for all SQP (power of two
//    >= queries) queries and a reduce-scatter over the 8 lanes (DPP
//    row_half_mirror, quad xor 2, quad xor 1) leaves lane `sub` with the full
//    score of query g8(sub) & (SQP-1): log2(SQP) exchange-adds instead of
//    3 * SQP.  For that, position p of a lane's query registers holds query
//    p ^ (g8(sub) & (SQP-1)) with g8(s) = s ^ 3 * bit2(s).
//  * Softmax: per-query running max across chunks (online rescale), chunk
//    probabilities written to LDS as [key][query].
//    With int8 rows, 5-8 queries of 64 dims and merged splits (the verify
//    step over an int8 cache), the scores are one int8 MFMA product per
//    chunk instead: the queries in three digit planes against the K codes
//    as stored (see MS in attn_kernel).
//  * PV: lane (r, dq) owns dims 4dq..4dq+3 of keys c0 + r + kpi*t, with
//    kpi = 256 / D key rows per wave instruction; the SQP probabilities of a
//    key are one broadcast LDS read.
// The split's (max, sum, acc) per query goes to `part` for the combine, or to
// LDS for the in-workgroup merge.
// ---------------------------------------------------------------------------
constexpr int kChunk = 32;
constexpr double kL2StreamBytes = 32.0 * 1024 * 1024;   // 8 XCDs x 4 MB of L2
constexpr int kMergedWaves = 8;    // key splits of a merged workgroup
constexpr int kMergedWaves4 = 4;   // ... for 4+ queries (option attn_w4)
constexpr int kMergedChunks = 4;   // at most this many chunks per split

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
             0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Orders a wave's LDS accesses across its lanes (a wave's LDS operations
// complete in program order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// max / sum over the 8 lanes l, l^8, ..., l^56 (same `sub`, all groups)
__device__ __forceinline__ float groups_max(float v) {
  v = fmaxf(v, dppf<0x128>(v));                // row_ror:8
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float groups_sum(float v) {
  v += dppf<0x128>(v);
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

// KV-cache rows of a launch whose rows (counted up to its key bound) exceed
// the L2s are streamed: non-temporal loads, so that they do not evict the
// weights and activations held in L2 between launches.  At 32 sequences
// both models' launches stream (the draft's too, although each draft step
// re-reads its cache: loading those rows normally, so that the memory-side
// cache could keep them between steps, measured 2.4% slower).  Launches
// within the L2s (short contexts, batch 1) load normally.
typedef float nnhip_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float *p) {
  const nnhip_f4 v = __builtin_nontemporal_load(reinterpret_cast<const nnhip_f4 *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
template <int DL>
__device__ __forceinline__ void load_lane_dims_stream(const float *p, int sub,
                                                      float (&x)[8]) {
  if constexpr (DL == 8) {
    const float4 a = ld_stream4(p + 4 * sub);
    const float4 c = ld_stream4(p + 32 + 4 * sub);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
  } else if constexpr (DL == 4) {
    const float4 a = ld_stream4(p + 4 * sub);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
#pragma unroll
    for (int i = 4; i < 8; ++i) x[i] = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = i < DL ? __builtin_nontemporal_load(p + DL * sub + i) : 0.f;
  }
}

// Dims of a lane in the score phase (DL = D/8 of them): for DL = 8 the two
// float4 runs 4*sub.. and 32+4*sub.. (a wave instruction then reads whole
// 128-byte halves of 8 key rows), for DL = 4 the run 4*sub.., otherwise
// DL*sub + x.  `p` is the row start; every load is unconditional.
template <int DL>
__device__ __forceinline__ void load_lane_dims(const float *p, int sub,
                                               float (&x)[8]) {
  if constexpr (DL == 8) {
    const float4 a = *reinterpret_cast<const float4 *>(p + 4 * sub);
    const float4 c = *reinterpret_cast<const float4 *>(p + 32 + 4 * sub);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
  } else if constexpr (DL == 4) {
    const float4 a = *reinterpret_cast<const float4 *>(p + 4 * sub);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
#pragma unroll
    for (int i = 4; i < 8; ++i) x[i] = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = i < DL ? p[DL * sub + i] : 0.f;
  }
}

// The same dims of an int8 row as int8 codes packed four to a word (byte i
// of the lane's run in bits 8(i&3) of word i>>2).
template <int DL>
__device__ __forceinline__ void load_lane_codes(const int8_t *p, int sub,
                                                uint32_t (&w)[2]) {
  if constexpr (DL == 8) {
    w[0] = *reinterpret_cast<const uint32_t *>(p + 4 * sub);
    w[1] = *reinterpret_cast<const uint32_t *>(p + 32 + 4 * sub);
  } else if constexpr (DL == 4) {
    w[0] = *reinterpret_cast<const uint32_t *>(p + 4 * sub);
    w[1] = 0u;
  } else {
    w[0] = 0u; w[1] = 0u;
#pragma unroll
    for (int i = 0; i < DL; ++i)
      w[i >> 2] |= (uint32_t)(uint8_t)p[DL * sub + i] << (8 * (i & 3));
  }
}

__device__ __forceinline__ float code_at(uint32_t w, int i) {
  return (float)(int8_t)(w >> (8 * i));
}

// A chunk's K rows in flight: fp32 dims, or codes and the rows' scales.
template <bool Q8> struct KChunk { float kr[4][8]; };
template <> struct KChunk<true> { uint32_t kc[4][2]; float ks[4]; };
// ... for the int8 MFMA scores: lane (c, hh) holds key c's codes for dims
// [32 s + 16 hh, +16), s = 0, 1 (the B operand of two 32-dim steps), and
// that key's scale
typedef int attn_v4i __attribute__((ext_vector_type(4)));
typedef int attn_v16i __attribute__((ext_vector_type(16)));
struct KChunkMfma { attn_v4i kb[2]; float ks; };

template <int SQP, int DL, int W, bool Q8>
__global__ __launch_bounds__(kWave * W, W == 4 ? 2 : 1) void attn_kernel(
    const float *__restrict__ q, KvSrc kv, int S, int H, int Hkv, int cap,
    const int32_t *__restrict__ base, int off,
    const int32_t *__restrict__ active, int nsplit, int nqb, int kps,
    float qscale, float *__restrict__ part, float *__restrict__ out, int nt,
    int8_t *__restrict__ hlimbs, int mpad, int *__restrict__ hexp) {
  constexpr int D = DL * 8;
  constexpr int NQ4 = D / 4, KPI = kWave / NQ4;   // PV: key rows per wave op
  constexpr int TPV = (kChunk + KPI - 1) / KPI;   // PV keys per lane
  // per wave: chunk probabilities [kChunk][SQP], later the PV partials
  // [KPI][SQP][D]; with W > 1 also the wave's (max, sum) per query
  constexpr int kBuf = (KPI * SQP * D > kChunk * SQP ? KPI * SQP * D
                                                      : kChunk * SQP) / 4;
  __shared__ float4 s_buf4[W][kBuf];
  __shared__ float s_alpha[W][SQP];
  __shared__ float s_ml[W][SQP][2];
  const int wv = threadIdx.x >> 6;
  float *s_buf = reinterpret_cast<float *>(s_buf4[wv]);
  // W == 1: one key split per workgroup (blockIdx.x); W > 1: the splits are
  // the workgroup's waves and are merged here
  const int sp = W == 1 ? (int)blockIdx.x : wv, h = blockIdx.y;
  const int b = blockIdx.z / nqb, qb = blockIdx.z % nqb;
  if (active && !active[b]) return;
  const int lane = threadIdx.x & 63, g = lane >> 3, sub = lane & 7;
  const int g8 = sub ^ (((sub >> 2) & 1) * 3);
  const int myq = g8 & (SQP - 1);
  const bool uniq = g8 < SQP;                 // one lane per (group, query)
  // query blocks of SQP (kMaxQ whenever a launch has more than one block,
  // except short launches: blocks of g_attn_short_q)
  const int q0 = qb * SQP;
  const int nq = min(SQP, S - q0);
  const int E = H * D;
  const int hk = h / (H / Hkv);
  const int pos0 = base[b] + off + q0;
  const int kend_all = min(pos0 + nq, cap);
  // W > 1: the workgroup's visible keys are shared out over its W waves in
  // whole chunks (kps from the host only bounds the capacity)
  const int kspan = W == 1 ? kps
      : (((kend_all + kChunk - 1) / kChunk + W - 1) / W) * kChunk;
  const int ks = sp * kspan;
  const int kend = min(ks + kspan, kend_all);
  using KT = typename std::conditional<Q8, int8_t, float>::type;
  const KT *kb = static_cast<const KT *>(kv.k) + b * kv.seq_stride + (int64_t)hk * cap * D;
  const KT *vb = static_cast<const KT *>(kv.v) + b * kv.seq_stride + (int64_t)hk * cap * D;
  // int8 rows: the scales of this (sequence, kv head)
  const float *ksb = Q8 ? kv.ks + b * kv.sc_stride + (int64_t)hk * cap : nullptr;
  const float *vsb = Q8 ? kv.vs + b * kv.sc_stride + (int64_t)hk * cap : nullptr;
  const int r = min(lane / NQ4, KPI - 1), dq = lane % NQ4;
  const bool pv_lane = lane < KPI * NQ4;

  // int8 rows, up to 8 queries of 64 dims, merged key splits: the scores on
  // the int8 MFMA (v_mfma_i32_32x32x32_i8).  A operand: the queries as three
  // digit planes (act_quant's rule: one exponent e per query row, X =
  // rint(q 2^e) in balanced base-256 digits; rows 8-31 zero); B operand: a
  // chunk's 32 K rows' codes as stored.  Each score is the exact integer
  // total sum_x X_x code_x, scaled by 2^-e and the K row's scale.  The
  // softmax and the PV products are those of the other path.
  constexpr bool MS = Q8 && SQP == 8 && DL == 8 && W > 1;
  const int kc_ = lane & 31, hh = lane >> 5;   // MS: key / query row, half
  float qv[MS ? 1 : SQP][8];
  attn_v4i qa[MS ? kLimbs : 1][2];
  int eq4[4];                                  // MS: exponents of queries 4 hh + j
  if constexpr (MS) {
    float f[2][16];
    float mx = 0.f;
    const bool qok = kc_ < nq;
    const float *qrow = q + ((int64_t)b * S + q0 + min(kc_, nq - 1)) * E + h * D;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 v4 = *reinterpret_cast<const float4 *>(qrow + 32 * s2 + 16 * hh + 4 * i);
        f[s2][4 * i] = qok ? v4.x : 0.f; f[s2][4 * i + 1] = qok ? v4.y : 0.f;
        f[s2][4 * i + 2] = qok ? v4.z : 0.f; f[s2][4 * i + 3] = qok ? v4.w : 0.f;
#pragma unroll
        for (int x = 0; x < 4; ++x) mx = fmaxf(mx, fabsf(f[s2][4 * i + x]));
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const int e = digit_exponent(mx);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int3 t = digits4(&f[s2][4 * i], e);
        qa[0][s2][i] = t.x; qa[1][s2][i] = t.y; qa[2][s2][i] = t.z;
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) eq4[j] = __shfl(e, 4 * hh + j, kWave);
  } else {
#pragma unroll
    for (int p = 0; p < SQP; ++p) {
      const int qi = p ^ myq;
      load_lane_dims<DL>(q + ((int64_t)b * S + q0 + min(qi, nq - 1)) * E + h * D,
                         sub, qv[p]);
    }
  }
  float acc[SQP][4];
#pragma unroll
  for (int i = 0; i < SQP; ++i)
#pragma unroll
    for (int x = 0; x < 4; ++x) acc[i][x] = 0.f;
  float m_run = -INFINITY, l_loc = 0.f;
  // MS: running max and partial sum of queries 4 hh + j (this lane's keys)
  float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, l4[4] = {0.f, 0.f, 0.f, 0.f};

  // A chunk's K and V rows are all requested before any arithmetic; rows
  // past the split end re-read the last valid row and are masked.  The
  // next chunk's K rows are requested before the current chunk is worked on
  // (two register buffers, used in turn); its V rows, needed only after the
  // scores, at the start of its own turn.  An int8 row enters as
  // (float)code * scale per element, the product layer.cpp:886-887 and
  // :932-934 form (the V rows always; the K rows except on the MFMA score
  // path, whose exact integer totals are scaled once per key).
  using Chunk = std::conditional_t<MS, KChunkMfma, KChunk<Q8>>;
  auto load_chunk = [&](int c0, Chunk &ck) {
    if constexpr (MS) {
      // lane (c, hh): key c0 + c's codes for dims 16 hh .. and 32 + 16 hh ..
      const int j = min(c0 + kc_, kend - 1);
      const int8_t *kr8 = reinterpret_cast<const int8_t *>(kb) + (int64_t)j * D + 16 * hh;
      ck.kb[0] = *reinterpret_cast<const attn_v4i *>(kr8);
      ck.kb[1] = *reinterpret_cast<const attn_v4i *>(kr8 + 32);
      ck.ks = ksb[j];
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = min(c0 + g + 8 * t, kend - 1);
        if constexpr (Q8) {
          load_lane_codes<DL>(kb + (int64_t)j * D, sub, ck.kc[t]);
          ck.ks[t] = ksb[j];
        } else {
          if (nt) load_lane_dims_stream<DL>(kb + (int64_t)j * D, sub, ck.kr[t]);
          else load_lane_dims<DL>(kb + (int64_t)j * D, sub, ck.kr[t]);
        }
      }
    }
  };
  auto work_chunk = [&](int c0, const Chunk &ck) {
    float4 vv[TPV];
    float kr[4][8];
    if constexpr (Q8) {
      uint32_t vw[TPV];
      float vsc[TPV];
#pragma unroll
      for (int t = 0; t < TPV; ++t) {
        const int row = min(c0 + r + KPI * t, kend - 1);
        vw[t] = *reinterpret_cast<const uint32_t *>(vb + (int64_t)row * D + dq * 4);
        vsc[t] = vsb[row];
      }
      if constexpr (!MS) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int x = 0; x < 8; ++x) kr[t][x] = code_at(ck.kc[t][x >> 2], x & 3) * ck.ks[t];
      }
#pragma unroll
      for (int t = 0; t < TPV; ++t)
        vv[t] = make_float4(code_at(vw[t], 0) * vsc[t], code_at(vw[t], 1) * vsc[t],
                            code_at(vw[t], 2) * vsc[t], code_at(vw[t], 3) * vsc[t]);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int x = 0; x < 8; ++x) kr[t][x] = ck.kr[t][x];
#pragma unroll
      for (int t = 0; t < TPV; ++t) {
        const float *pv = vb + (int64_t)min(c0 + r + KPI * t, kend - 1) * D + dq * 4;
        vv[t] = nt ? ld_stream4(pv) : *reinterpret_cast<const float4 *>(pv);
      }
    }
    if constexpr (MS) {
      // the chunk's scores: rows 4 hh + j (j < 4) of key c0 + c in lane
      // (c, hh)'s accumulator entries j; the chunk maximum of each query
      // over the 32 lanes of its half, then the online softmax as below
      attn_v16i sacc[kLimbs];
#pragma unroll
      for (int l = 0; l < kLimbs; ++l) sacc[l] = attn_v16i{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int l = 0; l < kLimbs; ++l)
          sacc[l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa[l][s2], ck.kb[s2], sacc[l], 0, 0, 0);
      const int key = c0 + kc_;
      float p4[4], al4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int qq = 4 * hh + j;
        const double tot = fma((double)sacc[0][j], 65536.0,
                               fma((double)sacc[1][j], 256.0, (double)sacc[2][j]));
        const bool valid = qq < nq && key < kend && key <= pos0 + qq;
        const float scj = valid ? ((float)ldexp(tot, -eq4[j]) * ck.ks) * qscale : -INFINITY;
        float cmj = scj;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) cmj = fmaxf(cmj, __shfl_xor(cmj, o, kWave));
        const float mn = fmaxf(m4[j], cmj);
        const float ms = (mn == -INFINITY) ? 0.f : mn;
        al4[j] = __builtin_amdgcn_exp2f(m4[j] - ms);   // 0 at start
        m4[j] = mn;
        p4[j] = __builtin_amdgcn_exp2f(scj - ms);      // 0 if masked
        l4[j] = l4[j] * al4[j] + p4[j];
      }
      *reinterpret_cast<float4 *>(s_buf + kc_ * SQP + 4 * hh) =
          make_float4(p4[0], p4[1], p4[2], p4[3]);
      if (kc_ == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s_alpha[wv][4 * hh + j] = al4[j];
      }
    } else {
    // scores of this lane's query for keys c0 + g + 8t
    float sc[4], cm = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float pr[SQP];
#pragma unroll
      for (int p = 0; p < SQP; ++p) {
        float s = 0.f;
#pragma unroll
        for (int x = 0; x < 8; ++x)
          if (x < DL) s += qv[p][x] * kr[t][x];
        pr[p] = s;
      }
      // bit 2 of g8 (partner sub ^ 7)
      if constexpr (SQP == 8) {
#pragma unroll
        for (int p = 0; p < 4; ++p) pr[p] += dppf<0x141>(pr[p + 4]);
      } else {
#pragma unroll
        for (int p = 0; p < SQP; ++p) pr[p] += dppf<0x141>(pr[p]);
      }
      // bit 1 (partner sub ^ 2)
      if constexpr (SQP >= 4) {
#pragma unroll
        for (int p = 0; p < 2; ++p) pr[p] += dppf<0x4E>(pr[p + 2]);
      } else {
#pragma unroll
        for (int p = 0; p < SQP; ++p) pr[p] += dppf<0x4E>(pr[p]);
      }
      // bit 0 (partner sub ^ 1)
      if constexpr (SQP >= 2) pr[0] += dppf<0xB1>(pr[1]);
      else pr[0] += dppf<0xB1>(pr[0]);
      const int j = c0 + g + 8 * t;
      const bool valid = myq < nq && j < kend && j <= pos0 + myq;
      sc[t] = valid ? pr[0] * qscale : -INFINITY;
      cm = fmaxf(cm, sc[t]);
    }
    cm = groups_max(cm);
    const float mn = fmaxf(m_run, cm);
    const float ms = (mn == -INFINITY) ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m_run - ms);   // 0 at start
    m_run = mn;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float p = __builtin_amdgcn_exp2f(sc[t] - ms);    // 0 if masked
      ps += p;
      if (uniq) s_buf[(g + 8 * t) * SQP + myq] = p;
    }
    l_loc = l_loc * alpha + ps;
    if (uniq && g == 0) s_alpha[wv][myq] = alpha;
    }
    wave_lds_sync();
    float al[SQP];
#pragma unroll
    for (int i = 0; i < SQP; ++i) al[i] = s_alpha[wv][i];
#pragma unroll
    for (int i = 0; i < SQP; ++i)
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[i][x] *= al[i];
#pragma unroll
    for (int t = 0; t < TPV; ++t) {
      // rows past the chunk (KPI not dividing it) read a masked row's zeros
      const int jj = min(r + KPI * t, kChunk - 1);
      const float m = (r + KPI * t < kChunk) ? 1.f : 0.f;
      float pk[SQP];
      const float *pp = s_buf + jj * SQP;
      if constexpr (SQP >= 4) {
#pragma unroll
        for (int i = 0; i < SQP; i += 4) {
          const float4 w = *reinterpret_cast<const float4 *>(pp + i);
          pk[i] = w.x * m; pk[i + 1] = w.y * m; pk[i + 2] = w.z * m;
          pk[i + 3] = w.w * m;
        }
      } else {
#pragma unroll
        for (int i = 0; i < SQP; ++i) pk[i] = pp[i] * m;
      }
#pragma unroll
      for (int i = 0; i < SQP; ++i) {
        acc[i][0] += pk[i] * vv[t].x; acc[i][1] += pk[i] * vv[t].y;
        acc[i][2] += pk[i] * vv[t].z; acc[i][3] += pk[i] * vv[t].w;
      }
    }
    wave_lds_sync();
  };
  Chunk ca, cb;
  if (ks < kend) load_chunk(ks, ca);
  for (int c0 = ks; c0 < kend; c0 += 2 * kChunk) {
    if (c0 + kChunk < kend) load_chunk(c0 + kChunk, cb);
    work_chunk(c0, ca);
    if (c0 + kChunk >= kend) break;
    if (c0 + 2 * kChunk < kend) load_chunk(c0 + 2 * kChunk, ca);
    work_chunk(c0 + kChunk, cb);
  }
  const float l = groups_sum(l_loc);
  float lq4[4];                               // MS: each query's sum over its keys
  if constexpr (MS) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = l4[j];
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) v += __shfl_xor(v, o, kWave);
      lq4[j] = v;
    }
  }
  if (pv_lane) {
#pragma unroll
    for (int i = 0; i < SQP; ++i)
      *reinterpret_cast<float4 *>(s_buf + (r * SQP + i) * D + dq * 4) =
          make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
  }
  wave_lds_sync();
  const int64_t row0 = (int64_t)b * S + q0;
  if constexpr (W > 1) {
    // the wave's reduced acc into the front of its buffer, (max, sum) per
    // query beside it, then the W splits merged as attn_combine_kernel does
    for (int t = lane; t < nq * D; t += kWave) {
      const int i = t / D, dd = t % D;
      float s = 0.f;
#pragma unroll
      for (int rr = 0; rr < KPI; ++rr) s += s_buf[(rr * SQP + i) * D + dd];
      s_buf[i * D + dd] = s;
    }
    if constexpr (MS) {
      if (kc_ == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s_ml[wv][4 * hh + j][0] = m4[j];
          s_ml[wv][4 * hh + j][1] = lq4[j];
        }
      }
    } else if (uniq && g == 0) {
      s_ml[wv][myq][0] = m_run;
      s_ml[wv][myq][1] = l;
    }
    __syncthreads();
    const int E = H * D;
    for (int t = threadIdx.x; t < nq * D; t += kWave * W) {
      const int i = t / D, dd = t % D;
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < W; ++u) mx = fmaxf(mx, s_ml[u][i][0]);
      float ls = 0.f, as = 0.f;
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const float mu = s_ml[u][i][0];
        const float f = mu == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mu - mx);
        ls += s_ml[u][i][1] * f;
        as += reinterpret_cast<const float *>(s_buf4[u])[i * D + dd] * f;
      }
      const float inv = ls > 0.f ? 1.0f / ls : 0.f;
      const float v = as * inv;
      out[(row0 + i) * E + h * D + dd] = v;
      if (D == kWave && hlimbs) {
        // the output projection's digits of this head's 64 entries of the
        // row (one per lane of this wave): the exponent of the row's head
        // chunk, then X = rint(v 2^e) in balanced base-256 digits (the
        // act_quant_kernel rule applied per head), at k = h D + dd
        const float mx = wave_max_all(fabsf(v));
        const int e = digit_exponent(mx);
        const int X = (int)rintf(ldexpf(v, e));
        const int lo = (int)(int8_t)(X & 0xff);
        const int t1 = (X - lo) >> 8;
        const int md = (int)(int8_t)(t1 & 0xff);
        const int hi = (t1 - md) >> 8;
        const int64_t o = mfma_operand_offset((int)(row0 + i), h * D + dd, E);
        const int64_t plane = (int64_t)mpad * E;
        hlimbs[o] = (int8_t)hi;
        hlimbs[plane + o] = (int8_t)md;
        hlimbs[2 * plane + o] = (int8_t)lo;
        if (dd == 0) hexp[(row0 + i) * H + h] = e;
      }
    }
    return;
  }
  if (uniq && g == 0 && myq < nq) {
    float *pp = part + (((row0 + myq) * H + h) * nsplit + sp) * (D + 2);
    pp[0] = m_run;
    pp[1] = l;
  }
  for (int t = lane; t < nq * D; t += kWave) {
    const int i = t / D, dd = t % D;
    float s = 0.f;
#pragma unroll
    for (int rr = 0; rr < KPI; ++rr) s += s_buf[(rr * SQP + i) * D + dd];
    part[(((row0 + i) * H + h) * nsplit + sp) * (D + 2) + 2 + dd] = s;
  }
}

// Merges the splits of every head of one row (b, s), writes the context row
// [H*D] and, when requested, its int8 digits for the output projection
// (same rule as act_quant_kernel).  The per-split weights
// 2^(m_s - M) / L are formed once per head in LDS, then every output element
// is a weighted sum over the splits.
constexpr int kCombineThreads = 1024;
constexpr int kMaxHeadSplits = 2048;         // H * nsplit bound

__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(
    const float *__restrict__ part, int S, int H, int D, int nsplit,
    const int32_t *__restrict__ active, float *__restrict__ out,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
  __shared__ float srow[4096];
  __shared__ float s_m[kMaxHeadSplits], s_l[kMaxHeadSplits];
  __shared__ float sred[kCombineThreads / kWave];
  const int64_t row = blockIdx.x;
  if (active && !active[row / S]) return;
  const int E = H * D, HS = H * nsplit;
  const float *prow = part + row * HS * (D + 2);
  for (int t = threadIdx.x; t < HS; t += blockDim.x) {
    s_m[t] = prow[(int64_t)t * (D + 2)];
    s_l[t] = prow[(int64_t)t * (D + 2) + 1];
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += blockDim.x) {
    float mn = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) mn = fmaxf(mn, s_m[h * nsplit + sp]);
    float ls = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float ms = s_m[h * nsplit + sp];
      const float f = (ms == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms - mn);
      s_m[h * nsplit + sp] = f;
      ls += s_l[h * nsplit + sp] * f;
    }
    const float inv = ls > 0.f ? 1.0f / ls : 0.f;
    for (int sp = 0; sp < nsplit; ++sp) s_m[h * nsplit + sp] *= inv;
  }
  __syncthreads();
  float mx = 0.f;
  for (int t = threadIdx.x; t < E; t += blockDim.x) {
    const int h = t / D, dd = t % D;
    const float *pp = prow + (int64_t)h * nsplit * (D + 2) + 2 + dd;
    const float *w = s_m + h * nsplit;
    float v = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) v += w[sp] * pp[(int64_t)sp * (D + 2)];
    out[row * E + t] = v;
    if (limbs) { srow[t] = v; mx = fmaxf(mx, fabsf(v)); }
  }
  if (!limbs) return;
  store_row_digits<kCombineThreads>(srow, E, mx, row, limbs, mpad, rexp, sred);
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
  store_row_digits<256>(srow, d, mx, row, limbs, mpad, rexp, sred);
}

// LayerNorm as layernorm_kernel, one wave per row for d % 16 == 0: the row
// is held in quads (rows.hpp: lane l has entries 256 i + 4 l .. + 3, i < NQ)
// with its gamma and beta, all requested at once; the row sums and the max
// are DPP wave reductions, and the digits of y (for the next MFMA GEMM) are
// written from the same registers.
template <int NQ>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(
    const float *__restrict__ hin, int d, int rows, const float *__restrict__ g,
    const float *__restrict__ bt, float *__restrict__ y,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  // the row, gamma and beta in quads (rows.hpp), all requested at once
  float v[NQ][4], gv[NQ][4], bv[NQ][4];
  load_quads<NQ>(g, d, lane, gv);
  load_quads<NQ>(bt, d, lane, bv);
  load_quads<NQ>(hin + (int64_t)row * d, d, lane, v);
  ln_row_finish<NQ>(v, gv, bv, d, row, y, limbs, mpad, rexp, lane);
}

// LayerNorm as layernorm_rows_kernel with a row spread over WPR waves
// (256 entries each, one quad a lane): the sums and the max of the row are
// combined through LDS in wave order.
template <int WPR>
__global__ __launch_bounds__(256) void layernorm_split_kernel(
    const float *__restrict__ hin, int d, int rows, const float *__restrict__ g,
    const float *__restrict__ bt, float *__restrict__ y,
    int8_t *__restrict__ limbs, int mpad, int *__restrict__ rexp) {
#pragma clang fp contract(off)
  __shared__ float s_sum[4], s_sq[4], s_mx[4];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * (4 / WPR) + wv / WPR;
  const int s0 = (wv % WPR) * 256, w0 = wv - wv % WPR;
  const bool live = row < rows;
  const int64_t rr = live ? row : rows - 1;
  const int k = s0 + 4 * lane;
  const float4 hv = *reinterpret_cast<const float4 *>(hin + rr * d + k);
  const float4 gq = *reinterpret_cast<const float4 *>(g + k);
  const float4 bq = *reinterpret_cast<const float4 *>(bt + k);
  float v[4] = {hv.x, hv.y, hv.z, hv.w};
  const float gv[4] = {gq.x, gq.y, gq.z, gq.w}, bv[4] = {bq.x, bq.y, bq.z, bq.w};
  float sm = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) sm += v[j];
  sm = wave_sum_all(sm);
  if (lane == 0) s_sum[wv] = sm;
  __syncthreads();
  sm = 0.f;
#pragma unroll
  for (int j = 0; j < WPR; ++j) sm += s_sum[w0 + j];
  const float N = (float)d;
  const float mean = sm / N;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) { const float df = v[j] - mean; sq += df * df; }
  sq = wave_sum_all(sq);
  if (lane == 0) s_sq[wv] = sq;
  __syncthreads();
  sq = 0.f;
#pragma unroll
  for (int j = 0; j < WPR; ++j) sq += s_sq[w0 + j];
  const float sd = sqrtf(sq / N + 1e-5f);
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = (v[j] - mean) / sd * gv[j] + bv[j];
    mx = fmaxf(mx, fabsf(v[j]));
  }
  if (live)
    *reinterpret_cast<float4 *>(y + rr * d + k) = make_float4(v[0], v[1], v[2], v[3]);
  if (!limbs) return;
  mx = wave_max_all(mx);
  if (lane == 0) s_mx[wv] = mx;
  __syncthreads();
  mx = 0.f;
#pragma unroll
  for (int j = 0; j < WPR; ++j) mx = fmaxf(mx, s_mx[w0 + j]);
  if (!live) return;
  const int e = digit_exponent(mx);
  if (lane == 0 && s0 == 0) rexp[row] = e;
  const int64_t plane = (int64_t)mpad * d;
  const int3 t = digits4(v, e);
  const int64_t off = mfma_operand_offset(row, k, d);
  *reinterpret_cast<int *>(limbs + off) = t.x;
  *reinterpret_cast<int *>(limbs + plane + off) = t.y;
  *reinterpret_cast<int *>(limbs + 2 * plane + off) = t.z;
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
                     ids, 1, 1, nullptr, x, nullptr, 0, nullptr);
  NNHIP_CHECK(hipGetLastError());
}

void launch_embed_strided(hipStream_t st, const float *emb, int vocab, int d,
                          const int32_t *ids, int B, int S, int stride_b,
                          float *x, int8_t *limbs, int mpad, int *rexp,
                          const int32_t *lead) {
  NNHIP_REQUIRE(d <= 4096 && (!limbs || (d % 128 == 0 && B * S <= mpad)),
                kErrArg, "embed: digit output needs d % 128 == 0, d <= 4096");
  hipLaunchKernelGGL(embed_kernel, dim3(B * S), dim3(256), 0, st, emb, vocab,
                     d, ids, S, stride_b, lead, x, limbs, mpad, rexp);
  NNHIP_CHECK(hipGetLastError());
}

void launch_rope_kv(hipStream_t st, const float *qkv, int B, int S, int H,
                    int D, const int32_t *base, int off, const int32_t *active,
                    const float *cosb, const float *sinb, float *qrot,
                    float *kc, float *vc, int cap, int64_t seq_stride,
                    int Hkv) {
  if (Hkv <= 0) Hkv = H;
  NNHIP_REQUIRE(H % Hkv == 0 && D % 2 == 0, kErrArg,
                "rope_kv: H must be a multiple of Hkv, D even");
  hipLaunchKernelGGL(rope_kv_kernel, dim3(B * S), dim3(256), 0, st, qkv, S, H,
                     Hkv, D, base, off, active, cosb, sinb, qrot, kc, vc, cap,
                     seq_stride);
  NNHIP_CHECK(hipGetLastError());
}

void launch_rope_kv_q8(hipStream_t st, const float *qkv, int B, int S, int H,
                       int D, const int32_t *base, int off,
                       const int32_t *active, const float *cosb,
                       const float *sinb, float *qrot, int8_t *kq, float *ks,
                       int8_t *vq, float *vs, int cap, int64_t seq_stride,
                       int64_t sc_stride) {
  NNHIP_REQUIRE(D % 2 == 0 && D <= 64, kErrArg,
                "rope_kv_q8: head dim must be even and <= 64");
  const int R = B * S;
  hipLaunchKernelGGL(rope_kv_q8_kernel, dim3((R * H + 3) / 4), dim3(256), 0,
                     st, qkv, R, S, H, D, base, off, active, cosb, sinb, qrot,
                     kq, ks, vq, vs, cap, seq_stride, sc_stride);
  NNHIP_CHECK(hipGetLastError());
}

int g_attn_waves = 4096;
int g_kv_stream = 1;
int g_attn_w4 = 1;
int g_attn_short_q = 1;
int g_ln_split = 1;

// Splits of the key range: about g_attn_waves waves over the whole launch
// (4 per SIMD by default), each split a whole number of 32-key chunks.
static int attention_splits(int B, int S, int H, int max_keys, int *kps) {
  const int nqb = (S + kMaxQ - 1) / kMaxQ;
  const int units = std::max(1, B * H * nqb);
  const int keys = std::max(max_keys, 1);
  const int max_split = (keys + kChunk - 1) / kChunk;
  int ns = std::min(max_split, std::max(1, (g_attn_waves + units - 1) / units));
  ns = std::max(1, std::min(ns, kMaxHeadSplits / std::max(H, 1)));
  int k = (keys + ns - 1) / ns;
  k = (k + kChunk - 1) / kChunk * kChunk;
  ns = (keys + k - 1) / k;
  if (kps) *kps = k;
  return ns;
}

int64_t attention_partial_elems(int B, int S, int H, int D, int max_keys) {
  const int nsplit = attention_splits(B, S, H, max_keys, nullptr);
  return (int64_t)B * S * H * nsplit * (D + 2);
}

bool attention_merged(int D, int max_keys) {
  return (D == 32 || D == 64) &&
         max_keys <= kMergedWaves * kMergedChunks * kChunk;
}

bool launch_attention(hipStream_t st, const float *q, const KvSrc &kv, int B,
                      int S, int H, int Hkv, int D, int cap,
                      const int32_t *base, int off, const int32_t *active,
                      int max_keys, float *part, int64_t part_elems,
                      float *out, int8_t *limbs, int mpad, int *rexp,
                      int *hexp) {
  NNHIP_REQUIRE(D % 8 == 0 && D <= kMaxD, kErrArg,
                "attention: head dim must be a multiple of 8 and <= 64");
  NNHIP_REQUIRE(!kv.q8 || (kv.ks && kv.vs), kErrArg,
                "attention: int8 rows need their scales");
  NNHIP_REQUIRE(Hkv > 0 && H % Hkv == 0, kErrArg, "attention: bad kv heads");
  NNHIP_REQUIRE(H * D <= 4096, kErrArg, "attention: H*D must be <= 4096");
  NNHIP_REQUIRE(!limbs || ((H * D) % 128 == 0 && B * S <= mpad), kErrArg,
                "attention: digit output needs H*D % 128 == 0");
  if (max_keys < 1) max_keys = 1;
  const int nqb_all = (S + kMaxQ - 1) / kMaxQ;
  const int sq_all = S < kMaxQ ? S : kMaxQ;
  const float qscale = (float)(1.4426950408889634 / std::sqrt((double)D));
  // stream the fp32 rows when the launch reads more than the L2s hold
  const double kv_bytes = 2.0 * B * Hkv * (double)std::min(max_keys, cap) * D *
                          (kv.q8 ? 1.0 : 4.0);
  const int nt = !kv.q8 && (g_kv_stream == 2 ||
                            (g_kv_stream == 1 && kv_bytes > kL2StreamBytes));
  if (attention_merged(D, max_keys)) {
    // one workgroup per (head, sequence, query block); its waves are the key
    // splits, merged in LDS, and the context rows are written directly, with
    // hexp also their digits per head (exponent per row and head).  A launch
    // of few (sequence, head) pairs (one sequence's verify or catch-up step)
    // takes its queries in blocks of g_attn_short_q (default 1): more
    // workgroups, each with fewer queries' products, the K / V rows read
    // once per block (from L2 after the first)
    const int qblk = g_attn_short_q;
    const bool short_q = qblk < kMaxQ && S > qblk && S <= kMaxQ &&
                         B * H < kAttnShortUnits;
    const int nqb = short_q ? (S + qblk - 1) / qblk : nqb_all;
    const int sq = short_q ? qblk : sq_all;
    NNHIP_REQUIRE(!hexp || (limbs && D == kWave && (H * D) % 128 == 0 && B * S <= mpad),
                  kErrArg, "attention: head digits need D == 64, H*D % 128 == 0");
    int8_t *hl = hexp ? limbs : nullptr;
    int kps = (max_keys + kMergedWaves - 1) / kMergedWaves;
    kps = (kps + kChunk - 1) / kChunk * kChunk;
    dim3 grid(1, H, B * nqb);
#define NNHIP_ATTN(SQP, DL, W)                                                \
  if (kv.q8)                                                                  \
    hipLaunchKernelGGL((attn_kernel<SQP, DL, W, true>), grid, dim3(kWave * W),  \
                       0, st, q, kv, S, H, Hkv, cap, base, off, active, W, nqb, \
                       kps, qscale, nullptr, out, nt, hl, mpad, hexp);         \
  else                                                                        \
    hipLaunchKernelGGL((attn_kernel<SQP, DL, W, false>), grid, dim3(kWave * W), \
                       0, st, q, kv, S, H, Hkv, cap, base, off, active, W, nqb, \
                       kps, qscale, nullptr, out, nt, hl, mpad, hexp)
#define NNHIP_ATTN_D(SQP, W)                                                  \
  if (D == 32) { NNHIP_ATTN(SQP, 4, W); } else { NNHIP_ATTN(SQP, 8, W); }
    // many-query rows hold many registers (one workgroup of 8 waves per CU):
    // with 4 waves two workgroups share a CU and a launch runs in one round;
    // a launch of few workgroups (one sequence) keeps 8 waves each, which
    // shortens every wave's walk (batch-1 verify: 183.1 -> 181.7 ms)
    const bool w4 = g_attn_w4 && max_keys <= kMergedWaves4 * kMergedChunks * kChunk &&
                    (g_attn_w4 == 2 || B * H * nqb >= 128);
    if (sq == 1) { NNHIP_ATTN_D(1, kMergedWaves) }
    else if (sq == 2) { NNHIP_ATTN_D(2, kMergedWaves) }
    else if (sq <= 4) { if (w4) { NNHIP_ATTN_D(4, kMergedWaves4) } else { NNHIP_ATTN_D(4, kMergedWaves) } }
    else { if (w4) { NNHIP_ATTN_D(8, kMergedWaves4) } else { NNHIP_ATTN_D(8, kMergedWaves) } }
#undef NNHIP_ATTN_D
#undef NNHIP_ATTN
    NNHIP_CHECK(hipGetLastError());
    return false;
  }
  const int nqb = nqb_all, sq = sq_all;
  int kps = 0;
  const int nsplit = attention_splits(B, S, H, max_keys, &kps);
  NNHIP_REQUIRE(part_elems >= attention_partial_elems(B, S, H, D, max_keys),
                kErrArg, "attention: partial buffer too small");
  dim3 grid(nsplit, H, B * nqb);
#define NNHIP_ATTN(SQP, DL)                                                   \
  if (kv.q8)                                                                  \
    hipLaunchKernelGGL((attn_kernel<SQP, DL, 1, true>), grid, dim3(kWave), 0,  \
                       st, q, kv, S, H, Hkv, cap, base, off, active, nsplit,  \
                       nqb, kps, qscale, part, nullptr, nt, nullptr, 0,       \
                       nullptr);                                              \
  else                                                                        \
    hipLaunchKernelGGL((attn_kernel<SQP, DL, 1, false>), grid, dim3(kWave), 0, \
                       st, q, kv, S, H, Hkv, cap, base, off, active, nsplit,  \
                       nqb, kps, qscale, part, nullptr, nt, nullptr, 0, nullptr)
#define NNHIP_ATTN_D(SQP)                                                     \
  switch (D / 8) {                                                            \
    case 1: { NNHIP_ATTN(SQP, 1); } break;                                    \
    case 2: { NNHIP_ATTN(SQP, 2); } break;                                    \
    case 3: { NNHIP_ATTN(SQP, 3); } break;                                    \
    case 4: { NNHIP_ATTN(SQP, 4); } break;                                    \
    case 5: { NNHIP_ATTN(SQP, 5); } break;                                    \
    case 6: { NNHIP_ATTN(SQP, 6); } break;                                    \
    case 7: { NNHIP_ATTN(SQP, 7); } break;                                    \
    default: { NNHIP_ATTN(SQP, 8); } break;                                   \
  }
  if (sq == 1) NNHIP_ATTN_D(1)
  else if (sq == 2) NNHIP_ATTN_D(2)
  else if (sq <= 4) NNHIP_ATTN_D(4)
  else NNHIP_ATTN_D(8)
#undef NNHIP_ATTN_D
#undef NNHIP_ATTN
  NNHIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(attn_combine_kernel, dim3(B * S), dim3(kCombineThreads), 0,
                     st, part, S, H, D, nsplit, active, out, limbs, mpad, rexp);
  NNHIP_CHECK(hipGetLastError());
  return limbs != nullptr;
}

void launch_layernorm(hipStream_t st, const float *h, int rows, int d,
                      const float *g, const float *b, float *y,
                      int8_t *limbs, int mpad, int *rexp) {
  NNHIP_REQUIRE(d <= 4096, kErrArg, "layernorm: d must be <= 4096");
  NNHIP_REQUIRE(!limbs || (d % 128 == 0 && rows <= mpad), kErrArg,
                "layernorm: digit output needs d % 128 == 0");
  if (g_ln_split && (d == 512 || d == 1024) &&
      ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(y) |
        reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(b)) & 15) == 0) {
    // 256 entries a wave: 2 or 4 waves a row
    if (d == 512)
      hipLaunchKernelGGL((layernorm_split_kernel<2>), dim3((rows + 1) / 2), dim3(256), 0,
                         st, h, d, rows, g, b, y, limbs, mpad, rexp);
    else
      hipLaunchKernelGGL((layernorm_split_kernel<4>), dim3(rows), dim3(256), 0, st, h,
                         d, rows, g, b, y, limbs, mpad, rexp);
  } else if (d % 16 == 0 && d <= 4096) {
    const dim3 grid((rows + 3) / 4);
#define NNHIP_LN(P)                                                           \
  hipLaunchKernelGGL((layernorm_rows_kernel<P>), grid, dim3(256), 0, st, h, d, \
                     rows, g, b, y, limbs, mpad, rexp)
    if (d <= 1024) { NNHIP_LN(4); }
    else if (d <= 2048) { NNHIP_LN(8); }
    else { NNHIP_LN(16); }
#undef NNHIP_LN
  } else {
    hipLaunchKernelGGL(layernorm_kernel, dim3(rows), dim3(256), 0, st, h, d, g,
                       b, y, limbs, mpad, rexp);
  }
  NNHIP_CHECK(hipGetLastError());
}

}  // namespace nnhip

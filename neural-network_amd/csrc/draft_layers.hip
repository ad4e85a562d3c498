// The decoder layers of one forward of a short batch (the draft model's
// drafting steps, layer.cpp:1541-1558, and any other forward of a few rows)
// as ONE persistent kernel: every CU runs one workgroup, and the layer's
// five dependent steps are separated by waits on per-tile flags instead of
// kernel launches.  Off by default (option persistent_draft): on the
// 4-layer d 512 draft at batch 32 it takes 151 us per forward (per layer
// about 7.5 us q/k/v, 12 attention, 2.6 O, 10 gate/up, 5.5 down, timed
// per step with wall_clock64), more than the per-kernel path, and two
// faster variants of it (V rows requested before the softmax, MFMA tile
// products) made GPU memory faults whose cause was not found.  Per layer (TransformerDecoderLayer::forward, layer.cpp:
// 1097-1114, post-LN):
//   A  q | k | v = x . Wqkv + b, with x = LN2 of the previous layer's output
//      (the layer input itself for layer 0); RoPE on q and k
//      (tensor.cpp:1141-1173) and the KV append (layer.cpp:758-807)
//   B  attention per (sequence, head) over the cache (layer.cpp:842-952)
//   C  t1 = x + (ctx . Wo + bo)
//   D  x1 = LN1(t1); ff = SwiGLU(x1 . Wgu + bgu) (layer.cpp:1704-1710)
//   E  t2 = x1 + (ff . Wdown + bdown)
// The kernel ends with t2 of the last layer; the lm head applies its LN2.
//
// Every step reads whole rows of its input (a tile of rows x columns of a
// Dense, K in full), so each LayerNorm is applied where its rows are read
// and needs no launch of its own.  Products are fp32 on the vector ALUs:
// int8 codes times fp32 activations, summed in a fixed order per output
// (lanes split K, one butterfly reduce-scatter per wave), then scale and
// bias, as QuantizedDense::forward's dequantised product
// (quantization.cpp:127-147).
//
// Cross-workgroup data: each step writes its outputs to fresh addresses of
// a per-forward ring (never read before in the launch) with stores that
// write through to memory (agent scope), every 128-byte line by one
// workgroup only.  Synchronisation is by data flow: every tile of every step
// publishes a flag word once its outputs are stored, and a tile waits only
// for the flags of the tiles whose outputs it reads (6 to 64 of them), so
// workgroups run ahead into later steps as soon as their inputs exist.  A
// flag holds the launch's generation (each workgroup counts its launches in
// its own word; all of them agree).  Every wait is bounded: after kPdSpin
// polls the waiting workgroup sets the error word, every workgroup leaves at
// its next wait, and the host reports the failure.  A tile issues the loads
// of its weight codes (and the attention step those of the keys cached
// before the launch) before it waits, so they overlap the wait.
#include "nnhip_internal.hpp"

#include <algorithm>

// RoPE and the softmax round each product and sum on their own, as the
// reference's scalar code does; the dot products use fmaf explicitly.
#pragma clang fp contract(off)

namespace nnhip {

namespace {

constexpr int kPdThreads = 256;
constexpr int kPdWaves = kPdThreads / 64;
constexpr int kPdSpin = 1 << 21;        // polls before a wait gives up
constexpr int kPdMaxKeys = 1024;        // keys of one (sequence, head)
constexpr int kPdHead = 64;             // head width the attention step takes
constexpr int kPdSmem = 8192 + 512 + 64;  // floats of LDS
enum PdStep { kStepQkv = 0, kStepAttn = 1, kStepO = 2, kStepGu = 3, kStepDown = 4 };

__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_dev(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PdRing {
  float *xl, *q, *ctx, *t1, *x1, *ff, *t2;
};

__device__ inline PdRing ring_of(const PdArgs &a, int l) {
  const int64_t rd = (int64_t)a.R * a.d;
  float *base = a.ring + (int64_t)l * pd_ring_layer_floats(a.R, a.d, a.F);
  PdRing r;
  r.xl = base;
  r.q = base + rd;
  r.ctx = base + 2 * rd;
  r.t1 = base + 3 * rd;
  r.x1 = base + 4 * rd;
  r.ff = base + 5 * rd;
  r.t2 = base + 5 * rd + (int64_t)a.R * a.F;
  return r;
}

// flag word of tile `t` of step `st` in layer l
__device__ __forceinline__ int flag_ix(int l, int st, int t) {
  return (l * 5 + st) * kPdFlagSlot + t;
}

// Tile t of step (l, st) is stored: every thread's stores have completed,
// then one thread publishes the generation in the tile's flag word.
__device__ inline void publish(const PdArgs &a, int ix, unsigned want) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(a.tflags + ix, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until the flag words dep(i), i < n <= 64 (dep(i) < 0: none), hold
// `want`: one lane of the first wave per word.  Returns false when this wait
// timed out or another workgroup's did (the caller leaves the kernel).
template <class Dep>
__device__ inline bool wait_deps(const PdArgs &a, int n, Dep dep, unsigned want) {
  __shared__ int s_ok;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int ix = lane < n ? dep(lane) : -1;
    int ok = 1;
    for (int it = 0;; ++it) {
      const int done = ix < 0 || (int)(ld_dev(a.tflags + ix) - want) >= 0;
      if (__all(done)) break;
      if ((it & 63) == 63) {
        const int e = __shfl(lane == 0 ? (int)ld_dev((const unsigned *)a.err) : 0, 0);
        if (e) { ok = 0; break; }
      }
      if (it >= kPdSpin) {
        if (lane == 0) atomicExch(a.err, 1);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) s_ok = ok;
  }
  __syncthreads();
  return s_ok != 0;
}

// RT rows [r0, r0 + RT) of src (rows of K floats, ld K) into LDS xs, zeros
// for rows past R
template <int RT>
__device__ inline void load_rows(const float *__restrict__ src, int r0, int R,
                                 int K, float *xs) {
  const int n4 = RT * K / 4;
  for (int i = threadIdx.x; i < n4; i += kPdThreads) {
    const int r = (4 * i) / K;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r0 + r < R)
      v = reinterpret_cast<const float4 *>(src + (int64_t)(r0 + r) * K)[i - r * (K / 4)];
    reinterpret_cast<float4 *>(xs)[i] = v;
  }
}

// rows [r0, r0 + RT) of xs (LDS) to dst (rows of K floats), rows < R
template <int RT>
__device__ inline void store_rows(const float *xs, int r0, int R, int K, float *dst) {
  for (int i = threadIdx.x; i < RT * K; i += kPdThreads)
    if (r0 + i / K < R) st_dev(dst + (int64_t)r0 * K + i, xs[i]);
}

// LayerNorm::forward (layer.cpp:242-261) of the RT rows in xs, in place:
// mean = sum / N, var = sum((x - mean)^2) / N, (x - mean) / sqrt(var + eps)
// * gamma + beta; one wave per row, lane l holding [l*KL, l*KL + KL).
// gamma and beta of the lane's K slice, requested before a wait
template <int KL>
struct LnParams {
  float g[KL], b[KL];
};
template <int KL>
__device__ inline void load_ln(const float *__restrict__ g, const float *__restrict__ b,
                               LnParams<KL> &p) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KL; i += 4) {
    const float4 vg = *reinterpret_cast<const float4 *>(g + lane * KL + i);
    const float4 vb = *reinterpret_cast<const float4 *>(b + lane * KL + i);
    p.g[i] = vg.x; p.g[i + 1] = vg.y; p.g[i + 2] = vg.z; p.g[i + 3] = vg.w;
    p.b[i] = vb.x; p.b[i + 1] = vb.y; p.b[i + 2] = vb.z; p.b[i + 3] = vb.w;
  }
}

template <int RT, int KL>
__device__ inline void ln_rows(float *xs, const LnParams<KL> &p) {
  constexpr int K = 64 * KL;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int r = wave; r < RT; r += kPdWaves) {
    float *x = xs + r * K + lane * KL;
    float v[KL];
#pragma unroll
    for (int i = 0; i < KL; ++i) v[i] = x[i];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < KL; ++i) s += v[i];
    const float N = (float)K;
    const float mean = wave_sum_all(s) / N;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const float df = v[i] - mean;
      sq += df * df;
    }
    const float var = wave_sum_all(sq) / N;
    const float sd = sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const float xh = (v[i] - mean) / sd;
      x[i] = xh * p.g[i] + p.b[i];
    }
  }
}

// The codes one lane of wave w feeds to a tile: columns c0 + w*CW + c,
// k in [l*KL, l*KL + KL), as 32-bit words
template <int CW, int KL>
struct TileCodes {
  uint32_t w[CW][KL / 4];
};
template <int CW, int KL>
__device__ inline void load_tile_codes(const int8_t *__restrict__ wq, int c0,
                                       TileCodes<CW, KL> &tc) {
  constexpr int K = 64 * KL;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int8_t *p0 = wq + (int64_t)(c0 + wave * CW) * K + lane * KL;
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int8_t *p = p0 + (int64_t)c * K;
    if constexpr (KL % 16 == 0) {
#pragma unroll
      for (int i = 0; i < KL / 16; ++i) {
        const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
        tc.w[c][4 * i] = v.x; tc.w[c][4 * i + 1] = v.y;
        tc.w[c][4 * i + 2] = v.z; tc.w[c][4 * i + 3] = v.w;
      }
    } else if constexpr (KL == 8) {
      const uint2 v = *reinterpret_cast<const uint2 *>(p);
      tc.w[c][0] = v.x; tc.w[c][1] = v.y;
    } else {
      tc.w[c][0] = *reinterpret_cast<const uint32_t *>(p);
    }
  }
}

__device__ __forceinline__ float code_at(uint32_t w, int j) {
  return (float)(int)(int8_t)(w >> (8 * j));
}

// Butterfly reduce-scatter of M values per lane over the lanes of a wave,
// offsets O, O/2, .., 1: at offset O a lane keeps the half of its values its
// bit O selects and adds the partner's copy of that half; once one value is
// left the remaining offsets add it up.  Afterwards lane l holds the total
// of value l / (64 / M).
template <int M, int O, int P>
__device__ __forceinline__ void reduce_scatter(float (&acc)[P], int lane) {
  if constexpr (O >= 1) {
    if constexpr (M > 1) {
      const bool up = (lane & O) != 0;
#pragma unroll
      for (int i = 0; i < M / 2; ++i) {
        const float keep = up ? acc[i + M / 2] : acc[i];
        const float send = up ? acc[i] : acc[i + M / 2];
        acc[i] = keep + __shfl_xor(send, O, 64);
      }
      reduce_scatter<M / 2, O / 2, P>(acc, lane);
    } else {
      acc[0] += __shfl_xor(acc[0], O, 64);
      reduce_scatter<1, O / 2, P>(acc, lane);
    }
  }
}

// Dot products of one tile: rows [0, RT) of xs (LDS, rows of K = 64*KL)
// against the wave's CW columns (codes in registers).  Lane l sums its K
// slice in ascending k (fmaf), then a butterfly reduce-scatter over the 64
// lanes adds the slices; os[r * NC + w*CW + c] receives the total.  RT*CW
// is a power of two <= 64.
template <int RT, int CW, int KL>
__device__ inline void tile_dot(const float *xs, const TileCodes<CW, KL> &tc,
                                float *os, int NC) {
  constexpr int K = 64 * KL;
  constexpr int P = RT * CW;
  static_assert(P <= 64 && (P & (P - 1)) == 0, "tile partials");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float x[RT][KL];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int i = 0; i < KL; i += 4) {
      const float4 v = *reinterpret_cast<const float4 *>(xs + r * K + lane * KL + i);
      x[r][i] = v.x; x[r][i + 1] = v.y; x[r][i + 2] = v.z; x[r][i + 3] = v.w;
    }
  float acc[P];
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    float wf[KL];
#pragma unroll
    for (int i = 0; i < KL; ++i) wf[i] = code_at(tc.w[c][i >> 2], i & 3);
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < KL; ++i) s = fmaf(x[r][i], wf[i], s);
      acc[r * CW + c] = s;
    }
  }
  reduce_scatter<P, 32, P>(acc, lane);
  // lane l holds partial p = l / (64 / P)
  constexpr int G = 64 / P;
  if (lane % G == 0) {
    const int p = lane / G;
    const int r = p / CW, c = p % CW;
    os[r * NC + wave * CW + c] = acc[0];
  }
}

// Tile grids of the steps: tile t = cg * ngr + gi covers rows [gi * RT, ..)
// and columns [cg * NC, ..).
constexpr int RT_A = 8, NC_A = 32;     // q | k | v
constexpr int RT_CE = 2, NC_CE = 32;   // output and down projections
constexpr int RT_D = 4, NC_D = 128;    // gate | up (interleaved): 64 outputs
__host__ __device__ __forceinline__ int ngroups(int R, int RT) { return (R + RT - 1) / RT; }

// ---------------------------------------------------------------------------
// Step A: q | k | v of RT_A rows x 32 columns per tile.  Waits for the rows
// of the previous layer's down projection (64 tiles: 4 row groups x the
// column groups).
// ---------------------------------------------------------------------------
template <int KLD>
__device__ bool step_qkv(const PdArgs &a, int l, float *sm, unsigned want) {
  constexpr int K = 64 * KLD, CW = NC_A / kPdWaves;
  const PdLayer &ly = a.ly[l];
  const PdRing rg = ring_of(a, l);
  const int ngr = ngroups(a.R, RT_A), ncg = 3 * K / NC_A;
  const int ngrE = ngroups(a.R, RT_CE), ncgE = K / NC_CE;
  float *xs = sm, *os = sm + 8192;
  const float *src = l == 0 ? a.x0 : ring_of(a, l - 1).t2;
  for (int t = blockIdx.x; t < ngr * ncg; t += gridDim.x) {
    const int gi = t % ngr, cg = t / ngr;
    const int r0 = gi * RT_A, c0 = cg * NC_A;
    TileCodes<CW, KLD> tc;
    load_tile_codes<CW, KLD>(ly.wqkv, c0, tc);
    LnParams<KLD> lp;
    if (l > 0) load_ln<KLD>(a.ly[l - 1].g2, a.ly[l - 1].b2, lp);
    // the epilogue's operands of this thread's pair (n, n + 1) of row r
    const int tid = threadIdx.x;
    const int er = tid / (NC_A / 2), en = c0 + 2 * (tid % (NC_A / 2));
    const int64_t emrow = r0 + er;
    const bool epi = tid < RT_A * NC_A / 2 && emrow < a.R;
    float esc0 = 0.f, esc1 = 0.f, ebi0 = 0.f, ebi1 = 0.f, ecos = 0.f, esin = 0.f;
    int epos = -1;
    if (epi) {
      esc0 = ly.sqkv[en]; esc1 = ly.sqkv[en + 1];
      ebi0 = ly.bqkv[en]; ebi1 = ly.bqkv[en + 1];
      const int b = (int)(emrow / a.S), s = (int)(emrow % a.S);
      const bool act = !a.active || a.active[b] != 0;
      const int pos = a.base[b] + a.off + s;
      if (act && pos >= 0 && pos < a.cap) {
        epos = pos;
        if (en / K != 2) {
          const int j = ((en % K) % a.D) >> 1, half = a.D >> 1;
          ecos = a.cosb[(int64_t)pos * half + j];
          esin = a.sinb[(int64_t)pos * half + j];
        }
      }
    }
    if (l > 0 && !wait_deps(a, 64, [&](int i) {
          const int ge = 4 * gi + (i & 3), ce = i >> 2;
          return ge < ngrE && ce < ncgE ? flag_ix(l - 1, kStepDown, ce * ngrE + ge) : -1;
        }, want))
      return false;
    load_rows<RT_A>(src, r0, a.R, K, xs);
    __syncthreads();
    if (l > 0) {
      ln_rows<RT_A, KLD>(xs, lp);
      __syncthreads();
      // the layer input, the output projection's residual
      if (cg == 0) store_rows<RT_A>(xs, r0, a.R, K, rg.xl);
    }
    tile_dot<RT_A, CW, KLD>(xs, tc, os, NC_A);
    __syncthreads();
    // pairs (n, n+1): bias, RoPE of q and k, the append of k and v
    if (epi && epos >= 0) {
      const int n = en, pos = epos;
      const int64_t mrow = emrow;
      const float v0 = os[er * NC_A + n - c0] * esc0 + ebi0;
      const float v1 = os[er * NC_A + n - c0 + 1] * esc1 + ebi1;
      const int b = (int)(mrow / a.S);
      const int part = n / K, nn = n % K;
      const int h = nn / a.D, j = (nn % a.D) >> 1;
      if (part == 2) {
        float *vd = ly.vc + b * a.seq_stride + ((int64_t)h * a.cap + pos) * a.D + 2 * j;
        st_dev(vd, v0);
        st_dev(vd + 1, v1);
      } else {
        const float q0 = v0 * ecos - v1 * esin;
        const float q1 = v0 * esin + v1 * ecos;
        float *dst = part == 0
            ? rg.q + mrow * K + nn
            : ly.kc + b * a.seq_stride + ((int64_t)h * a.cap + pos) * a.D + 2 * j;
        st_dev(dst, q0);
        st_dev(dst + 1, q1);
      }
    }
    publish(a, flag_ix(l, kStepQkv, t), want);
  }
  return true;
}

// ---------------------------------------------------------------------------
// Step B: attention of one (sequence, head) per tile.  Waits for the six
// q | k | v tiles of its rows and head; the keys cached before the launch
// are requested first.
// ---------------------------------------------------------------------------
__device__ float block_max4(float v, float *red) {
  v = wave_max_all(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ float block_sum4(float v, float *red) {
  v = wave_sum_all(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ inline void load_key(const float *kr, float4 (&k)[kPdHead / 4]) {
#pragma unroll
  for (int i = 0; i < kPdHead / 4; ++i) k[i] = reinterpret_cast<const float4 *>(kr)[i];
}

__device__ inline float qk_dot(const float *q, const float4 (&k)[kPdHead / 4]) {
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < kPdHead / 4; ++i) {
    dot += q[4 * i] * k[i].x;
    dot += q[4 * i + 1] * k[i].y;
    dot += q[4 * i + 2] * k[i].z;
    dot += q[4 * i + 3] * k[i].w;
  }
  return dot;
}

__device__ bool step_attention(const PdArgs &a, int l, float *sm, unsigned want) {
  const PdLayer &ly = a.ly[l];
  const PdRing rg = ring_of(a, l);
  const int D = kPdHead, S = a.S, d = a.d;
  float *sc = sm;                       // [S][kPdMaxKeys] scores, then p
  float *qs = sm + 2 * kPdMaxKeys;      // [S][D]
  float *pv = qs + 2 * D;               // [waves][S][D]
  float *red = pv + kPdWaves * 2 * D;   // [4]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
  const int ngrA = ngroups(a.R, RT_A), ncq = d / NC_A;
  const float scale = sqrtf((float)D);
  for (int t = blockIdx.x; t < a.B * a.H; t += gridDim.x) {
    const int b = t / a.H, h = t % a.H;
    const bool act = !a.active || a.active[b] != 0;
    const int p0 = act ? a.base[b] + a.off : 0;   // position of query 0
    const int nk = act ? min(p0 + S, a.cap) : 0;  // keys of the last query
    const int nold = min(max(p0, 0), nk);         // keys cached before
    const float *kb = ly.kc + b * a.seq_stride + (int64_t)h * a.cap * D;
    const float *vb = ly.vc + b * a.seq_stride + (int64_t)h * a.cap * D;
    float4 k0[kPdHead / 4], k1[kPdHead / 4];
    if (tid < nold) load_key(kb + (int64_t)tid * D, k0);
    if (tid + kPdThreads < nold) load_key(kb + (int64_t)(tid + kPdThreads) * D, k1);
    const int ga = (b * S) / RT_A;
    if (!wait_deps(a, 6, [&](int i) {
          const int cg = (i >> 1) * ncq + 2 * h + (i & 1);
          return flag_ix(l, kStepQkv, cg * ngrA + ga);
        }, want))
      return false;
    if (!act) {   // rows of a finished sequence: zeros
      for (int i = tid; i < S * D; i += kPdThreads)
        st_dev(rg.ctx + (int64_t)(b * S + i / D) * d + h * D + i % D, 0.f);
      publish(a, flag_ix(l, kStepAttn, t), want);
      continue;
    }
    for (int i = tid; i < S * D; i += kPdThreads)
      qs[i] = rg.q[(int64_t)(b * S + i / D) * d + h * D + i % D];
    // the keys appended in this launch, now stored
    if (tid >= nold && tid < nk) load_key(kb + (int64_t)tid * D, k0);
    if (tid + kPdThreads >= nold && tid + kPdThreads < nk)
      load_key(kb + (int64_t)(tid + kPdThreads) * D, k1);
    __syncthreads();
    for (int s = 0; s < S; ++s) {
      if (tid < nk)
        sc[s * kPdMaxKeys + tid] = tid > p0 + s ? -INFINITY : qk_dot(qs + s * D, k0) / scale;
      if (tid + kPdThreads < nk)
        sc[s * kPdMaxKeys + tid + kPdThreads] =
            tid + kPdThreads > p0 + s ? -INFINITY : qk_dot(qs + s * D, k1) / scale;
    }
    for (int j = tid + 2 * kPdThreads; j < nk; j += kPdThreads) {
      float4 kx[kPdHead / 4];
      load_key(kb + (int64_t)j * D, kx);
      for (int s = 0; s < S; ++s)
        sc[s * kPdMaxKeys + j] = j > p0 + s ? -INFINITY : qk_dot(qs + s * D, kx) / scale;
    }
    __syncthreads();
    for (int s = 0; s < S; ++s) {
      float mx = -INFINITY;
      for (int j = tid; j < nk; j += kPdThreads) mx = fmaxf(mx, sc[s * kPdMaxKeys + j]);
      mx = block_max4(mx, red);
      float sum = 0.f;
      for (int j = tid; j < nk; j += kPdThreads) {
        const float x = sc[s * kPdMaxKeys + j];
        const float e = x == -INFINITY ? 0.f : expf(x - mx);
        sc[s * kPdMaxKeys + j] = e;
        sum += e;
      }
      sum = block_sum4(sum, red);
      const float inv = 1.0f / sum;
      for (int j = tid; j < nk; j += kPdThreads)
        sc[s * kPdMaxKeys + j] = sc[s * kPdMaxKeys + j] * inv;
    }
    __syncthreads();
    // p . V: lane (jo = l / 16, dims 4*(l % 16) .. +3) of wave w takes keys
    // j = 16 i + 4 w + jo, eight rows requested at a time
    const int e4 = 4 * (lane & 15), jo = lane >> 4;
    float4 acc[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
    for (int j0 = 4 * wave + jo; j0 < nk; j0 += 16 * 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + 16 * u;
        v[u] = j < nk ? *reinterpret_cast<const float4 *>(vb + (int64_t)j * D + e4)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + 16 * u;
        if (j >= nk) continue;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s >= S) continue;
          const float p = sc[s * kPdMaxKeys + j];
          if (p == 0.f) continue;
          acc[s].x += p * v[u].x; acc[s].y += p * v[u].y;
          acc[s].z += p * v[u].z; acc[s].w += p * v[u].w;
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s >= S) continue;
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        acc[s].x += __shfl_xor(acc[s].x, o, 64);
        acc[s].y += __shfl_xor(acc[s].y, o, 64);
        acc[s].z += __shfl_xor(acc[s].z, o, 64);
        acc[s].w += __shfl_xor(acc[s].w, o, 64);
      }
      if (jo == 0)
        *reinterpret_cast<float4 *>(pv + (wave * 2 + s) * D + e4) = acc[s];
    }
    __syncthreads();
    for (int i = tid; i < S * D; i += kPdThreads) {
      const int s = i / D, e = i % D;
      const float o = (pv[(0 * 2 + s) * D + e] + pv[(1 * 2 + s) * D + e]) +
                      (pv[(2 * 2 + s) * D + e] + pv[(3 * 2 + s) * D + e]);
      st_dev(rg.ctx + (int64_t)(b * S + s) * d + h * D + e, o);
    }
    publish(a, flag_ix(l, kStepAttn, t), want);
  }
  return true;
}

// ---------------------------------------------------------------------------
// Steps C and E: y = resid + (x . W + b) on RT_CE rows x 32 columns per tile.
// C (the output projection) waits for the attention tiles of its rows'
// sequences (and the q | k | v tile that stored the layer input); E (the
// down projection) for the gate | up tiles of its rows.
// ---------------------------------------------------------------------------
template <int KL, bool DOWN>
__device__ bool step_resid(const PdArgs &a, int l, float *sm, unsigned want) {
  constexpr int K = 64 * KL, CW = NC_CE / kPdWaves;
  const PdLayer &ly = a.ly[l];
  const PdRing rg = ring_of(a, l);
  const float *x = DOWN ? rg.ff : rg.ctx;
  const int8_t *w = DOWN ? ly.wdn : ly.wo;
  const float *sc = DOWN ? ly.sdn : ly.so, *bi = DOWN ? ly.bdn : ly.bo;
  const float *resid = DOWN ? rg.x1 : (l == 0 ? a.x0 : rg.xl);
  float *y = DOWN ? (l + 1 == a.L ? a.out : rg.t2) : rg.t1;
  const int N = a.d;
  const int ngr = ngroups(a.R, RT_CE), ncg = N / NC_CE;
  const int ngrD = ngroups(a.R, RT_D), ncgD = 2 * a.F / NC_D;
  float *xs = sm, *os = sm + 8192;
  for (int t = blockIdx.x; t < ngr * ncg; t += gridDim.x) {
    const int gi = t % ngr, cg = t / ngr;
    const int r0 = gi * RT_CE, c0 = cg * NC_CE;
    TileCodes<CW, KL> tc;
    load_tile_codes<CW, KL>(w, c0, tc);
    const int tid = threadIdx.x;
    const int er = tid / NC_CE, en = c0 + tid % NC_CE;
    const int64_t emrow = r0 + er;
    const bool epi = tid < RT_CE * NC_CE && emrow < a.R;
    const float esc = epi ? sc[en] : 0.f, ebi = epi ? bi[en] : 0.f;
    bool ok;
    if constexpr (DOWN) {
      const int gd = r0 / RT_D;
      ok = wait_deps(a, ncgD, [&](int i) {
        return flag_ix(l, kStepGu, i * ngrD + gd);
      }, want);
    } else {
      const int b0 = r0 / a.S, b1 = min(r0 + RT_CE - 1, a.R - 1) / a.S;
      const int H = a.H;
      ok = wait_deps(a, 2 * H + 1, [&](int i) {
        if (i < H) return flag_ix(l, kStepAttn, b0 * H + i);
        if (i < 2 * H) return b1 != b0 ? flag_ix(l, kStepAttn, b1 * H + i - H) : -1;
        return l > 0 ? flag_ix(l, kStepQkv, r0 / RT_A) : -1;   // cg 0 of its group
      }, want);
    }
    if (!ok) return false;
    const float eres = epi ? resid[emrow * N + en] : 0.f;
    load_rows<RT_CE>(x, r0, a.R, K, xs);
    __syncthreads();
    tile_dot<RT_CE, CW, KL>(xs, tc, os, NC_CE);
    __syncthreads();
    if (epi) st_dev(y + emrow * N + en, eres + (os[tid] * esc + ebi));
    publish(a, flag_ix(l, DOWN ? kStepDown : kStepO, t), want);
  }
  return true;
}

// ---------------------------------------------------------------------------
// Step D: x1 = LN1(t1); ff = SwiGLU(x1 . Wgu + bgu) on RT_D rows x NC_D
// interleaved columns (NC_D / 2 outputs) per tile, as two halves of 64
// columns over the same normalised rows.  Waits for the output projection's
// tiles of its rows.
// ---------------------------------------------------------------------------
template <int KLD>
__device__ bool step_gate_up(const PdArgs &a, int l, float *sm, unsigned want) {
  constexpr int K = 64 * KLD, NH = NC_D / 2, CW = NH / kPdWaves;
  const PdLayer &ly = a.ly[l];
  const PdRing rg = ring_of(a, l);
  const int ngr = ngroups(a.R, RT_D), ncg = 2 * a.F / NC_D;
  const int ngrC = ngroups(a.R, RT_CE), ncgC = K / NC_CE;
  float *xs = sm, *os = sm + 8192;
  for (int t = blockIdx.x; t < ngr * ncg; t += gridDim.x) {
    const int gi = t % ngr, cg = t / ngr;
    const int r0 = gi * RT_D, c0 = cg * NC_D;
    TileCodes<CW, KLD> tc0, tc1;
    load_tile_codes<CW, KLD>(ly.wgu, c0, tc0);
    load_tile_codes<CW, KLD>(ly.wgu, c0 + NH, tc1);
    LnParams<KLD> lp;
    load_ln<KLD>(ly.g1, ly.b1, lp);
    // this thread's output: row er, pair jj (columns c0 + 2 jj, + 1)
    const int tid = threadIdx.x;
    const int er = tid / (NC_D / 2), jj = tid % (NC_D / 2), en = c0 + 2 * jj;
    const int64_t emrow = r0 + er;
    const bool epi = tid < RT_D * NC_D / 2 && emrow < a.R;
    const float sg = epi ? ly.sgu[en] : 0.f, su = epi ? ly.sgu[en + 1] : 0.f;
    const float bg = epi ? ly.bgu[en] : 0.f, bu = epi ? ly.bgu[en + 1] : 0.f;
    if (!wait_deps(a, 2 * ncgC, [&](int i) {
          const int gc = 2 * gi + (i & 1), cc = i >> 1;
          return gc < ngrC ? flag_ix(l, kStepO, cc * ngrC + gc) : -1;
        }, want))
      return false;
    load_rows<RT_D>(rg.t1, r0, a.R, K, xs);
    __syncthreads();
    ln_rows<RT_D, KLD>(xs, lp);
    __syncthreads();
    if (cg == 0) store_rows<RT_D>(xs, r0, a.R, K, rg.x1);   // the down projection's residual
    tile_dot<RT_D, CW, KLD>(xs, tc0, os, NC_D);
    tile_dot<RT_D, CW, KLD>(xs, tc1, os + NH, NC_D);
    __syncthreads();
    if (epi) {
      const float g = os[er * NC_D + 2 * jj] * sg + bg;
      const float u = os[er * NC_D + 2 * jj + 1] * su + bu;
      st_dev(rg.ff + emrow * a.F + en / 2, swiglu_pair(g, u));
    }
    publish(a, flag_ix(l, kStepGu, t), want);
  }
  return true;
}

template <int KLD, int KLF>
__global__ __launch_bounds__(kPdThreads, 1) void draft_layers_kernel(PdArgs a) {
  __shared__ __align__(16) float sm[kPdSmem];
  if (ld_dev((const unsigned *)a.err)) return;
  // this launch's generation: every workgroup has counted the same launches
  const unsigned want = ld_dev(a.flags + blockIdx.x) + 1;
  for (int l = 0; l < a.L; ++l) {
    if (!step_qkv<KLD>(a, l, sm, want)) return;
    if (!step_attention(a, l, sm, want)) return;
    if (!step_resid<KLD, false>(a, l, sm, want)) return;
    if (!step_gate_up<KLD>(a, l, sm, want)) return;
    if (!step_resid<KLF, true>(a, l, sm, want)) return;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(a.flags + blockIdx.x, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool draft_layers_supported(int d, int H, int F, int L, int R, int cap) {
  const int kld = d / 64, klf = F / 64;
  const bool shapes = (kld == 8 && klf == 32) || (kld == 4 && klf == 16);
  if (!(shapes && d % 64 == 0 && F % 64 == 0 && d / H == kPdHead && L >= 1 &&
        L <= kPdMaxLayers && R >= 1 && R <= 64 && cap <= kPdMaxKeys))
    return false;
  // every step's tiles fit a flag slot; every wait names <= 64 tiles
  const int tiles[5] = {ngroups(R, RT_A) * 3 * d / NC_A, R * H,
                        ngroups(R, RT_CE) * d / NC_CE,
                        ngroups(R, RT_D) * 2 * F / NC_D,
                        ngroups(R, RT_CE) * d / NC_CE};
  for (int t : tiles)
    if (t > kPdFlagSlot) return false;
  return 2 * F / NC_D <= 64 && 2 * (d / NC_CE) <= 64 && 2 * H + 1 <= 64;
}

void launch_draft_layers(hipStream_t st, const PdArgs &a, int nwg) {
  NNHIP_REQUIRE(draft_layers_supported(a.d, a.H, a.F, a.L, a.R, a.cap) &&
                    a.S >= 1 && a.S <= 2 && a.B * a.S == a.R && a.D == kPdHead &&
                    nwg >= 1 && a.flags && a.err && a.ring,
                kErrArg, "draft layers: unsupported shape or missing state");
  const int kld = a.d / 64;
  if (kld == 8)
    hipLaunchKernelGGL((draft_layers_kernel<8, 32>), dim3(nwg), dim3(kPdThreads),
                       0, st, a);
  else
    hipLaunchKernelGGL((draft_layers_kernel<4, 16>), dim3(nwg), dim3(kPdThreads),
                       0, st, a);
  NNHIP_CHECK(hipGetLastError());
}

}  // namespace nnhip

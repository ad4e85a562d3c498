// Softmax, sampling and the speculative accept / reject step for gfx950.
//
// Replaces the host side of generate_speculative (layer.cpp:1410-1655):
// get_probs (:1410-1491), sample_token (:1493-1498), the accept loop
// (:1581-1609), the residual resample (:1611-1630), the bonus sample
// (:1643-1647) and the cache rollback (:1632-1637).  One workgroup of 1024
// threads owns one sequence; a vocabulary row of probabilities is held in
// LDS (up to 32768 entries, 132 KB), so every pass after the first read of
// the logits is on-chip.  No host round trip happens per token.
//
// Uniforms: Philox4x32-10 keyed by the seed, counter {slot, cycle, seq, 0},
// u = (word0 >> 8) * 2^-24 (the oracle's default stream), or with
// SpecState::mt set the reference's own std::mt19937 per sequence, drawn in
// the reference's order (mt_seed_kernel, mt_commit).
#include "nnhip_internal.hpp"
#include "rows.hpp"

#include <hip/hip_runtime.h>

#include <type_traits>

// Every product and sum below is rounded on its own, as the reference's
// scalar loops round them (p - q of the residual, the probabilities, the
// tile sums): no fused multiply-add, so the decisions follow the reference's
// arithmetic (the exponentials' own implementation is unaffected).
#pragma clang fp contract(off)

namespace nnhip {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxV = 32768;
// Probability rows live in LDS at a padded address (one spare word every 32)
// so that both the strided passes (v = tid + 1024 i) and the per-thread
// contiguous chunks of the inverse CDF are free of bank conflicts.
constexpr int kRowWords = kMaxV + kMaxV / 32;

__device__ __forceinline__ int la(int v) { return v + (v >> 5); }

__device__ __forceinline__ float uniform(uint64_t seed, uint32_t seq,
                                         uint32_t cycle, uint32_t slot) {
  uint32_t c0 = slot, c1 = cycle, c2 = seq, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
  return (float)(c0 >> 8) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------------------
// std::mt19937 (SpecState::mt), the generator generate_advanced and
// generate_speculative draw from (layer.cpp:1249, 1394).  The engine is the
// standard's: 624-word state, seeding x_i = 1812433253 (x_{i-1} ^
// (x_{i-1} >> 30)) + i, twist, tempering.  Its outputs are produced 624 at a
// time by a whole workgroup into a per-sequence ring; the draws are
// libstdc++'s generate_canonical: a float from one output ((float)g / 2^32),
// a double from two ((g1 + g2 2^32) / 2^64), each the largest value below 1
// when rounding reaches 1.
// ---------------------------------------------------------------------------
constexpr int kMtM = 397;
constexpr int kMtD = kMtN - kMtM;   // 227

__device__ __forceinline__ uint32_t mt_mix(uint32_t cur, uint32_t nxt) {
  const uint32_t y = (cur & 0x80000000u) | (nxt & 0x7fffffffu);
  return (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
}

__device__ __forceinline__ uint32_t mt_temper(uint32_t y) {
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  return y ^ (y >> 18);
}

// One twist of a sequence's state mt (global) and its 624 tempered outputs
// written to ring slots wp .. wp + 623 (mod kMtRing), by a workgroup of at
// least kMtN threads; every thread calls it.  New word i is old[i + 397] ^
// mix(old[i], old[i + 1]) for i < 227 and new[i - 227] ^ mix(old[i],
// old[i + 1]) after (new[0] in place of old[624]), so three phases separated
// by barriers give the sequential recurrence's words.
__device__ void mt_twist(uint32_t *mt, uint32_t *ring, uint32_t wp) {
  const int i = threadIdx.x;
  const bool on = i < kMtN;
  const uint32_t cur = on ? mt[i] : 0u;
  const uint32_t nxt = (on && i + 1 < kMtN) ? mt[i + 1] : 0u;
  const uint32_t far = i < kMtD ? mt[i + kMtM] : 0u;
  __syncthreads();   // every old word read
  uint32_t v = 0u;
  if (i < kMtD) {
    v = far ^ mt_mix(cur, nxt);
    mt[i] = v;
  }
  __syncthreads();
  if (i >= kMtD && i < 2 * kMtD) {
    v = mt[i - kMtD] ^ mt_mix(cur, nxt);
    mt[i] = v;
  }
  __syncthreads();
  if (i >= 2 * kMtD && on) {
    v = mt[i - kMtD] ^ mt_mix(cur, i + 1 < kMtN ? nxt : mt[0]);
    mt[i] = v;
  }
  if (on) ring[(wp + (uint32_t)i) & (kMtRing - 1)] = mt_temper(v);
  __syncthreads();   // the ring's new outputs visible to the workgroup
}

__device__ __forceinline__ uint32_t mt_out(const SpecState &s, int b, uint32_t p) {
  return s.mt_ring[(int64_t)b * kMtRing + (p & (kMtRing - 1))];
}
__device__ __forceinline__ double mt_double_at(const SpecState &s, int b, uint32_t p) {
  double x = (double)mt_out(s, b, p);
  x += (double)mt_out(s, b, p + 1) * 4294967296.0;
  const double r = x * 0x1p-64;
  return r >= 1.0 ? 0x1.fffffffffffffp-1 : r;
}
__device__ __forceinline__ float mt_float_at(const SpecState &s, int b, uint32_t p) {
  const float r = (float)mt_out(s, b, p) * 0x1p-32f;
  return r >= 1.0f ? 0x1.fffffep-1f : r;
}

// The uniform of sequence b's sampled draw: with the mt19937 stream the
// double `off` outputs past the read counter, else the Philox uniform of
// (cycle, slot).  test_u: the same for an accept test's float.
__device__ __forceinline__ double draw_u(const SpecState &s, int b, uint32_t off,
                                         uint32_t cyc, uint32_t slot) {
  if (s.mt_ring) return mt_double_at(s, b, s.mt_rw[2 * b] + off);
  return (double)uniform(s.seed, s.seq0 + b, cyc, slot);
}
__device__ __forceinline__ float test_u(const SpecState &s, int b, uint32_t off,
                                        uint32_t cyc, uint32_t slot) {
  if (s.mt_ring) return mt_float_at(s, b, s.mt_rw[2 * b] + off);
  return uniform(s.seed, s.seq0 + b, cyc, slot);
}

// After a launch's draws for sequence b (block-uniform call, every thread):
// the read counter advanced by `used` outputs, and when fewer than kMtLow
// remain unread the next 624 appended.  Each thread has read the counters
// before the barrier; the ring slots rewritten lie outside the unread ones.
__device__ void mt_commit(const SpecState &s, int b, uint32_t used) {
  uint32_t *rw = s.mt_rw + 2 * b;
  const uint32_t rp = rw[0] + used, wp = rw[1];
  __syncthreads();
  const bool fill = wp - rp < (uint32_t)kMtLow;
  if (fill)
    mt_twist(s.mt + (int64_t)b * kMtN, s.mt_ring + (int64_t)b * kMtRing, wp);
  if (threadIdx.x == 0) {
    rw[0] = rp;
    if (fill) rw[1] = wp + kMtN;
  }
}

// Seeds sequence b's engine with (uint32_t)(seed + seq0 + b) -- the
// reference's seed is an unsigned int, and the engine keeps the value mod
// 2^32 -- and fills the ring with its first 624 outputs.
__global__ __launch_bounds__(1024) void mt_seed_kernel(SpecState s) {
  const int b = blockIdx.x;
  uint32_t *mt = s.mt + (int64_t)b * kMtN;
  if (threadIdx.x == 0) {
    uint32_t x = (uint32_t)(s.seed + s.seq0 + (uint64_t)b);
    mt[0] = x;
    for (int i = 1; i < kMtN; ++i) {
      x = 1812433253u * (x ^ (x >> 30)) + (uint32_t)i;
      mt[i] = x;
    }
  }
  __syncthreads();
  mt_twist(mt, s.mt_ring + (int64_t)b * kMtRing, 0u);
  if (threadIdx.x == 0) {
    s.mt_rw[2 * b] = 0u;
    s.mt_rw[2 * b + 1] = kMtN;
  }
}

// Row statistics of get_probs (T > 0), see row_pass; tau / tix: the top-k /
// top-p rule (block_filter), which keeps entry v iff bits(p1_v) > tau or
// (bits(p1_v) == tau and v <= tix) -- everything by default.
struct RowStats {
  float mx, rsum, rfs;
  uint32_t tau;
  int tix;
};
__device__ __forceinline__ RowStats mk_stats(float mx, float rsum, float rfs) {
  return RowStats{mx, rsum, rfs, 0u, 0x7fffffff};
}

__device__ __forceinline__ bool kept(float p1, int v, const RowStats &st) {
  const uint32_t u = __float_as_uint(p1);
  return u > st.tau || (u == st.tau && v <= st.tix);
}

// workgroup reduction slots; `rows` holds per-row statistics formed by
// single waves (accept step, up to one row per wave)
constexpr int kDigits = 16;   // digit values of one level of block_filter
struct Shared {
  float f[kWaves];
  double d[kWaves];
  int i[kWaves];
  RowStats rows[kWaves];
  int argm[kWaves];
  double xd;
  int hn[kWaves][kDigits];
  double hs[kWaves][kDigits];
  float prow[kRowWords];
};
// the same without the probability row, for kernels that need no full row
struct SmallShared {
  float f[kWaves];
  double d[kWaves];
  int i[kWaves];
  double xd;
};

template <class SH>
__device__ __forceinline__ float block_max(float v, SH &sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh.f[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, sh.f[w]);
  return r;
}

template <class SH>
__device__ __forceinline__ float block_sum(float v, SH &sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r += sh.f[w];
  return r;
}

// exclusive prefix sum over threads in index order; *total = the block sum
template <class SH>
__device__ __forceinline__ double block_excl_scan_d(double v, SH &sh,
                                                    double *total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    double t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  __syncthreads();
  if (lane == 63) sh.d[w] = incl;
  __syncthreads();
  double pre = 0.0, tot = 0.0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const double x = sh.d[i];
    pre += i < w ? x : 0.0;
    tot += x;
  }
  *total = tot;
  return pre + incl - v;
}

template <class SH>
__device__ __forceinline__ int block_min_i(int v, SH &sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.i[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = sh.i[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = min(r, sh.i[w]);
  return r;
}

// The thread's row entries v = tid + kThreads * i, i < kPer, all requested
// before the first is used (indices past V re-read entry V-1 and are
// replaced by `fill`).
constexpr int kPer = kMaxV / kThreads;   // row entries per thread

__device__ __forceinline__ void load_row(const float *__restrict__ row, int V,
                                         float fill, float (&x)[kPer]) {
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    x[i] = row[min((int)threadIdx.x + i * kThreads, V - 1)];
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if ((int)threadIdx.x + i * kThreads >= V) x[i] = fill;
}

// First index of the maximum (layer.cpp:1413-1421, std::max_element).
template <class SH>
__device__ __forceinline__ int block_argmax(const float *__restrict__ row,
                                            int V, SH &sh) {
  float x[kPer];
  load_row(row, V, -INFINITY, x);
  float bv = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) bv = fmaxf(bv, x[i]);
  const float mx = block_max(bv, sh);
  // lowest index holding the maximum (entries ascend with i)
  int cand = 0x7fffffff;
#pragma unroll
  for (int i = kPer - 1; i >= 0; --i) {
    const int v = (int)threadIdx.x + i * kThreads;
    if (v < V && x[i] == mx) cand = v;
  }
  const int r = block_min_i(cand, sh);
  return r == 0x7fffffff ? 0 : r;
}

// get_probs (layer.cpp:1426-1489) for T > 0 without top-k / top-p:
// s = l / T, e = exp(s - max), p1 = e / sum, p = p1 / sum(p1).  The two
// normalisations multiply by the correctly rounded reciprocals 1/sum and
// 1/sum(p1), so p may differ from the divided value in the last place.
// RowStats holds what recomputes p at one index (prob_at).
__device__ __forceinline__ float scaled(float l, float T) {
  return T == 1.0f ? l : l / T;
}

// p at index v of a row with logit l, from the row's statistics
__device__ __forceinline__ float prob_of(float l, int v, float T,
                                         const RowStats &st) {
  const float p1 = expf(scaled(l, T) - st.mx) * st.rsum;
  return kept(p1, v, st) ? p1 * st.rfs : 0.f;
}

// ---------------------------------------------------------------------------
// top-k / top-p of get_probs (layer.cpp:1447-1489).  The reference sorts p1
// (the probabilities after the first normalisation) descending, zeroes the
// ranks from top_k on, then zeroes every rank after the one at which the
// running sum first reaches top_p, and renormalises by what is left: the
// kept set is the first R = min(top_k, r + 1) ranks, r the top-p crossing.
// Ties in the order go to the lower index (std::sort leaves them
// unspecified; the oracle does the same).  No sort here: a most-significant-
// digit search over the bit patterns of p1 (non-negative floats order as
// their bits), 4 bits a level; per level, counts and double sums of the
// candidates per digit value are reduced over the workgroup and the digit
// where the running count from the top reaches top_k or the running sum
// reaches top_p is taken.  After 8 levels the boundary value tau is exact;
// of the entries equal to tau, those in index order up to what the rule
// allows are kept (tix: the last kept index; all of them when no cut falls
// inside the group).  The running sum is double here and a float sum in
// sorted order in the reference, so the crossing rank can differ where that
// float sum lies within its rounding error of top_p (a tie).
// x: p1 of entries v = tid + kThreads i (entries v >= V ignored).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void block_filter(const float (&x)[kPer], int V,
                                          int top_k, float top_p, Shared &sh,
                                          RowStats &st) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p > 0.f && top_p < 1.f;
  const int kcap = use_k ? top_k : V;
  uint32_t prefix = 0u;
  int above_n = 0, gcnt = 0;
  double above_s = 0.0;
  bool p_cut = false;
  for (int level = 0; level < 8; ++level) {
    const int shift = 28 - 4 * level;
    // a thread's counts and (float) sums per digit, eight digits at a time,
    // then summed over the wave (double) into the wave's LDS slots
    __syncthreads();
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      int cnt[kDigits / 2];
      float smf[kDigits / 2];
#pragma unroll
      for (int d = 0; d < kDigits / 2; ++d) { cnt[d] = 0; smf[d] = 0.f; }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int v = tid + i * kThreads;
        const uint32_t u = __float_as_uint(x[i]);
        const bool cand = v < V && (level == 0 || (u >> (shift + 4)) == prefix);
        const int dg = cand ? (int)((u >> shift) & 15u) - half * (kDigits / 2) : -1;
#pragma unroll
        for (int d = 0; d < kDigits / 2; ++d) {
          cnt[d] += dg == d ? 1 : 0;
          smf[d] += dg == d ? x[i] : 0.f;
        }
      }
#pragma unroll
      for (int d = 0; d < kDigits / 2; ++d) {
        const int n = wave_sum_i(cnt[d]);
        const double a = wave_sum_d((double)smf[d]);
        if (lane == 0) {
          sh.hn[w][half * (kDigits / 2) + d] = n;
          sh.hs[w][half * (kDigits / 2) + d] = a;
        }
      }
    }
    __syncthreads();
    if (tid < kDigits) {
      int n = 0;
      double a = 0.0;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) { n += sh.hn[ww][tid]; a += sh.hs[ww][tid]; }
      sh.hn[0][tid] = n;
      sh.hs[0][tid] = a;
    }
    __syncthreads();
    // the digit holding the boundary, scanned from the top
    int run_n = above_n, sel = 0;
    double run_s = above_s;
    bool pc = false;
    for (int d = kDigits - 1; d >= 0; --d) {
      const int n = sh.hn[0][d];
      if (n == 0) continue;
      const double a = sh.hs[0][d];
      pc = use_p && run_s + a >= (double)top_p;
      if (run_n + n >= kcap || pc) { sel = d; gcnt = n; break; }
      run_n += n;
      run_s += a;
    }
    above_n = run_n;
    above_s = run_s;
    p_cut = pc;
    prefix = (prefix << 4) | (uint32_t)sel;
  }
  // entries equal to tau: how many the rule keeps
  const float tf = __uint_as_float(prefix);
  int m = kcap - above_n;
  if (p_cut && tf > 0.f) {
    const double need = ((double)top_p - above_s) / (double)tf;
    const int mp = max(1, (int)ceil(need));
    m = min(m, mp);
  }
  int tix = 0x7fffffff;
  if (m < gcnt) {
    // the m-th index (in index order) of the group: bisection on the index
    int lo = 0, hi = V - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      int c = 0;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int v = tid + i * kThreads;
        c += (v <= mid && v < V && __float_as_uint(x[i]) == prefix) ? 1 : 0;
      }
      c = wave_sum_i(c);
      __syncthreads();
      if (lane == 0) sh.i[w] = c;
      __syncthreads();
      int tot = 0;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) tot += sh.i[ww];
      if (tot >= m) hi = mid; else lo = mid + 1;
    }
    tix = lo;
  }
  st.tau = prefix;
  st.tix = tix;
  __syncthreads();
}

// The row is held in registers (entry v = tid + kThreads i); p goes to sh.prow
// when `to_lds`, and to gout when given.
template <bool FILT, class SH>
__device__ __forceinline__ RowStats row_pass(const float *__restrict__ row, int V, float T,
                             SH &sh, bool to_lds,
                             float *__restrict__ gout, int top_k = 0,
                             float top_p = 1.f) {
  float x[kPer];
  load_row(row, V, -INFINITY, x);
  if (T != 1.0f) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) x[i] = x[i] / T;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) mx = fmaxf(mx, x[i]);
  mx = block_max(mx, sh);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int v = threadIdx.x + i * kThreads;
    x[i] = v < V ? expf(x[i] - mx) : 0.f;
    s += x[i];
  }
  const float rs = 1.0f / block_sum(s, sh);
#pragma unroll
  for (int i = 0; i < kPer; ++i) x[i] = x[i] * rs;
  RowStats st = mk_stats(mx, rs, 1.f);
  if constexpr (FILT) block_filter(x, V, top_k, top_p, sh, st);
  float f = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (FILT && !kept(x[i], (int)threadIdx.x + i * kThreads, st)) x[i] = 0.f;
    f += x[i];
  }
  st.rfs = 1.0f / block_sum(f, sh);
  if (to_lds || gout) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int v = threadIdx.x + i * kThreads;
      if (v < V) {
        const float p = x[i] * st.rfs;
        if constexpr (std::is_same_v<SH, Shared>) {
          if (to_lds) sh.prow[la(v)] = p;
        }
        if (gout) gout[v] = p;
      }
    }
    __syncthreads();
  }
  return st;
}

// FILT: the row is filtered by top_k / top_p (block_filter)
template <bool FILT = false>
__device__ __forceinline__ RowStats row_probs(const float *__restrict__ row,
                                              int V, float T, Shared &sh,
                                              float *__restrict__ gout = nullptr,
                                              int top_k = 0, float top_p = 1.f) {
  return row_pass<FILT>(row, V, T, sh, true, gout, top_k, top_p);
}

template <bool FILT = false, class SH>
__device__ __forceinline__ RowStats row_stats(const float *__restrict__ row,
                                              int V, float T, SH &sh,
                                              int top_k = 0, float top_p = 1.f) {
  return row_pass<FILT>(row, V, T, sh, false, nullptr, top_k, top_p);
}

// sh.prow = p recomputed from a row's statistics
__device__ __forceinline__ void fill_probs(const float *__restrict__ row,
                                           int V, float T, RowStats st,
                                           Shared &sh) {
  float x[kPer];
  load_row(row, V, 0.f, x);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int v = (int)threadIdx.x + i * kThreads;
    if (v < V) sh.prow[la(v)] = prob_of(x[i], v, T, st);
  }
  __syncthreads();
}

// sample_token (layer.cpp:1493-1498): std::discrete_distribution over
// sh.prow widened to double (weights w = p / S, S = sum p, running sum, last
// entry 1.0): the first v whose running sum of p reaches u * S.  Each thread
// owns a contiguous chunk; a chunk is scanned only when the crossing can lie
// in it or before it.
__device__ __forceinline__ int block_sample(int V, double u, Shared &sh) {
  // the thread's chunk [b0, b0 + C) (C <= kPer), read from LDS once
  const int C = (V + kThreads - 1) / kThreads;
  const int b0 = threadIdx.x * C;
  float pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    pv[i] = (i < C && b0 + i < V) ? sh.prow[la(min(b0 + i, V - 1))] : 0.f;
  double loc = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) loc += (double)pv[i];
  double S;
  double c = block_excl_scan_d(loc, sh, &S);
  const double target = u * S;
  int found = 0x7fffffff;
  if (c + loc >= target - 1e-12 * S) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int v = b0 + i;
      c += (double)pv[i];
      if (found == 0x7fffffff && i < C && v < V - 1 && c >= target) found = v;
    }
  }
  const int r = block_min_i(found, sh);
  return r == 0x7fffffff ? V - 1 : r;
}

template <bool FILT>
__device__ __forceinline__ int draw_row(const float *row, int V, float T, double u,
                        Shared &sh, int top_k = 0, float top_p = 1.f) {
  if (T <= 0.f) return block_argmax(row, V, sh);
  row_probs<FILT>(row, V, T, sh, nullptr, top_k, top_p);
  return block_sample(V, u, sh);
}

// ---------------------------------------------------------------------------
// Sampling from the lm head's tile statistics (TileStatsArgs: per 128-column
// tile of a row, (max s, sum exp(s - max)) for T > 0, (max l, first index of
// the max) for T <= 0).  The row's get_probs statistics are recombined from
// the tiles -- max over the tiles, sum_t e_t exp(m_t - max) -- instead of a
// pass over every logit, and the inverse CDF runs over the tiles' masses
// before it scans the one tile where the running sum reaches u * S, with the
// probabilities of that tile recomputed exactly as prob_at does.  The sums
// are formed in another order than a full pass, so p and S differ from the
// full pass in the last bits; a draw differs only if u * S falls within
// that difference of a CDF step (a tie).
// ---------------------------------------------------------------------------
constexpr int kTileMax = 16;   // tiles per lane of one wave: rows <= 1024 tiles
constexpr int kTileW = 128;    // columns of a tile (the lm head's column block)

// RowStats (T > 0) of a row from its nt tile statistics, by one wave
__device__ __forceinline__ RowStats wave_tiles_stats(const float2 *__restrict__ tl,
                                                     int nt) {
  const int lane = threadIdx.x & 63;
  float2 v[kTileMax];
#pragma unroll
  for (int i = 0; i < kTileMax; ++i) v[i] = tl[min(lane + 64 * i, nt - 1)];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kTileMax; ++i)
    if (lane + 64 * i < nt) mx = fmaxf(mx, v[i].x);
  mx = wave_max_all(mx);
  float e = 0.f;
#pragma unroll
  for (int i = 0; i < kTileMax; ++i)
    if (lane + 64 * i < nt && v[i].x > -INFINITY) e += v[i].y * expf(v[i].x - mx);
  e = wave_sum_all(e);
  const float rs = 1.0f / e;
  return mk_stats(mx, rs, 1.0f / (e * rs));
}

// first index of a row's maximum from its tile statistics (T <= 0), one wave
__device__ __forceinline__ int wave_tiles_argmax(const float2 *__restrict__ tl,
                                                 int nt) {
  const int lane = threadIdx.x & 63;
  float2 v[kTileMax];
#pragma unroll
  for (int i = 0; i < kTileMax; ++i) v[i] = tl[min(lane + 64 * i, nt - 1)];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kTileMax; ++i)
    if (lane + 64 * i < nt) mx = fmaxf(mx, v[i].x);
  mx = wave_max_all(mx);
  int ix = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < kTileMax; ++i)
    if (lane + 64 * i < nt && v[i].x == mx) ix = min(ix, __float_as_int(v[i].y));
  ix = wave_min_all(ix);
  return ix == 0x7fffffff ? 0 : ix;
}

// sample_token over p = prob_at(row, ., T, st) from the row's tile
// statistics: the tile where the running sum of the tile masses reaches
// u * S, then the first entry of it (entries in order, exact p) whose running
// sum reaches u * S; the next tile if rounding left the crossing short.
template <class SH>
__device__ __forceinline__ int tiles_sample(const float *__restrict__ row,
                                            const float2 *__restrict__ tl,
                                            int nt, int tw, int V, float T,
                                            RowStats st, double u, SH &sh) {
  const int t = threadIdx.x;
  double P = 0.0;
  if (t < nt) {
    const float2 v = tl[t];
    if (v.x > -INFINITY)
      P = (double)(v.y * expf(v.x - st.mx)) * (double)st.rsum * (double)st.rfs;
  }
  double S;
  const double c = block_excl_scan_d(P, sh, &S);
  const double target = u * S;
  int ts = block_min_i(t < nt && P > 0.0 && c + P >= target ? t : 0x7fffffff, sh);
  if (ts == 0x7fffffff) return V - 1;
  // running sum before tile ts, broadcast
  if (t == ts) sh.xd = c;
  __syncthreads();
  double before = sh.xd;
  for (; ts < nt; ++ts) {
    const int v = ts * tw + t;
    const bool in = t < tw && v < V;
    const double p = in ? (double)((expf(scaled(row[v], T) - st.mx) * st.rsum) * st.rfs) : 0.0;
    double tot;
    const double ex = block_excl_scan_d(p, sh, &tot);
    const int found = block_min_i(in && v < V - 1 && before + ex + p >= target ? v : 0x7fffffff, sh);
    if (found != 0x7fffffff) return found;
    before += tot;
  }
  return V - 1;
}

// One drafting step j (layer.cpp:1541-1558) from the draft lm head's tile
// statistics: q_j's statistics recombined from the tiles, q_j written in one
// pass over the row by kQParts workgroups per sequence (the accept step's
// candidate and residual read it; the pass is VALU-bound on expf, so it is
// spread over CUs), and the candidate drawn by tiles_sample in the first of
// them.  Greedy: the argmax of the tiles.
constexpr int kQParts = 8;
constexpr int kQPer = (kMaxV / kQParts + kThreads - 1) / kThreads;

// After drafting step j < k - 1 picked `tok` for sequence b (block-uniform):
// row b of the next draft forward, embedded here instead of by a gather
// launch of its own (SpecState::nd).  srow: kMaxEmbed floats of LDS, sred:
// kWaves floats.
constexpr int kMaxEmbed = 4096;
__device__ void embed_row(const NextRows &n, int64_t row, int id, float *srow,
                          float *sred) {
  if (id < 0 || id >= n.vocab) id = 0;
  const float *src = n.emb + (int64_t)id * n.d;
  float *dst = n.x + row * n.d;
  float mx = 0.f;
  for (int i = threadIdx.x; i < n.d; i += kThreads) {
    const float v = src[i];
    dst[i] = v;
    srow[i] = v;
    mx = fmaxf(mx, fabsf(v));
  }
  if (n.limbs) store_row_digits<kThreads>(srow, n.d, mx, row, n.limbs, n.mpad, n.rexp, sred);
  __syncthreads();   // srow free for the next row
}
__device__ void embed_next(const SpecState &s, int b, int j, int tok,
                           float *srow, float *sred) {
  if (j < s.k - 1 && s.nd.x) embed_row(s.nd, b, tok, srow, sred);
}

__global__ __launch_bounds__(kThreads) void draft_sample_tiles_kernel(
    SpecState s, int j, const float *__restrict__ logits, int64_t ldl) {
  __shared__ SmallShared sh;
  __shared__ RowStats rst;
  __shared__ float s_emb[kMaxEmbed], s_red[kWaves];
  __shared__ int s_tok;
  const int b = blockIdx.x, part = blockIdx.y;
  if (!s.active[b]) return;
  const float2 *tl = s.dtiles + ((int64_t)b * s.k + j) * s.nt;
  if (s.T <= 0.f) {
    if (part != 0) return;
    if (threadIdx.x < 64) {
      const int a = wave_tiles_argmax(tl, s.nt);
      if (threadIdx.x == 0) { s.cand[b * s.k + j] = a; s_tok = a; }
    }
    __syncthreads();
    embed_next(s, b, j, s_tok, s_emb, s_red);
    return;
  }
  const float *row = logits + b * ldl;
  if (s.qlog) {
    // the probabilities stay implicit in the logits: only the draw
    if (threadIdx.x < 64) {
      const RowStats st = wave_tiles_stats(tl, s.nt);
      if (threadIdx.x == 0) rst = st;
    }
    __syncthreads();
    const int tok = tiles_sample(row, tl, s.nt, s.tw, s.V, s.T, rst,
                                 draw_u(s, b, 2 * j, s.cyc[b], j), sh);
    if (threadIdx.x == 0) s.cand[b * s.k + j] = tok;
    embed_next(s, b, j, tok, s_emb, s_red);
    return;
  }
  // this part's entries requested while the statistics are formed
  const int chunk = (s.V + kQParts - 1) / kQParts;
  const int v0 = part * chunk, v1 = min(s.V, v0 + chunk);
  float x[kQPer];
#pragma unroll
  for (int i = 0; i < kQPer; ++i)
    x[i] = row[min(v0 + (int)threadIdx.x + i * kThreads, s.V - 1)];
  if (threadIdx.x < 64) {
    const RowStats st = wave_tiles_stats(tl, s.nt);
    if (threadIdx.x == 0) rst = st;
  }
  __syncthreads();
  const RowStats st = rst;
  float *q = s.qprob + ((int64_t)b * s.k + j) * s.V;
#pragma unroll
  for (int i = 0; i < kQPer; ++i) {
    const int v = v0 + (int)threadIdx.x + i * kThreads;
    if (v < v1) q[v] = (expf(scaled(x[i], s.T) - st.mx) * st.rsum) * st.rfs;
  }
  if (part != 0) return;
  const int tok = tiles_sample(row, tl, s.nt, s.tw, s.V, s.T, st,
                               draw_u(s, b, 2 * j, s.cyc[b], j), sh);
  if (threadIdx.x == 0) s.cand[b * s.k + j] = tok;
  embed_next(s, b, j, tok, s_emb, s_red);
}

// Tile statistics of rows of logits (launch_row_tile_stats): per 128-column
// tile, two columns a lane, the same operations in the same order as the LDS
// GEMM's lm-head epilogue, so a row gives the same statistics whether they
// come from there or from here.  A wave takes kTileRun consecutive tiles of
// one row and requests all of their logits (one 8-byte load a lane per tile,
// read once: non-temporal) before it reduces the first.
constexpr int kTileRun = 8;
constexpr int kTileThreads = 256;

// One tile's statistics from a wave holding its columns n, n + 1 (n = tile
// start + 2 lane) in l0, l1: T > 0 (max s, sum exp(s - max)) with s = l / T,
// else (max l, first index of the max as int bits); every lane gets them.
__device__ __forceinline__ float2 tile_stat(float l0, float l1, int n, int V, float T) {
  if (T > 0.f) {
    const float s0 = n < V ? scaled(l0, T) : -INFINITY;
    const float s1 = n + 1 < V ? scaled(l1, T) : -INFINITY;
    const float mx = wave_max_all(fmaxf(s0, s1));
    const float e = wave_sum_all((n < V ? expf(s0 - mx) : 0.f) +
                                 (n + 1 < V ? expf(s1 - mx) : 0.f));
    return make_float2(mx, e);
  }
  const float a0 = n < V ? l0 : -INFINITY, a1 = n + 1 < V ? l1 : -INFINITY;
  const float mx = wave_max_all(fmaxf(a0, a1));
  const int ix = wave_min_all(a0 == mx ? n : (a1 == mx ? n + 1 : 0x7fffffff));
  return make_float2(mx, __int_as_float(ix));
}

template <bool PAIRS>
__global__ __launch_bounds__(kTileThreads) void row_tile_stats_kernel(
    const float *__restrict__ logits, int64_t ldl, int V, float T, int nt,
    float2 *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * (kTileThreads / 64) + (threadIdx.x >> 6)) * kTileRun;
  const int64_t r = blockIdx.y;
  if (t0 >= nt) return;                       // whole wave
  const float *row = logits + r * ldl;
  // PAIRS: ldl and the base are even, so a pair of columns is one aligned
  // 8-byte word
  typedef float pair_t __attribute__((ext_vector_type(2)));
  pair_t v[kTileRun];
  if (PAIRS && (t0 + kTileRun) * kTileW <= V) {   // whole run inside the row
#pragma unroll
    for (int i = 0; i < kTileRun; ++i)
      v[i] = __builtin_nontemporal_load(
          reinterpret_cast<const pair_t *>(row + (t0 + i) * kTileW + 2 * lane));
  } else {
#pragma unroll
    for (int i = 0; i < kTileRun; ++i) {
      const int n = (t0 + i) * kTileW + 2 * lane;
      v[i].x = n < V ? row[n] : 0.f;
      v[i].y = n + 1 < V ? row[n + 1] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < kTileRun; ++i) {
    const int tn = t0 + i;
    if (tn >= nt) break;                      // whole wave
    const float2 ts = tile_stat(v[i].x, v[i].y, tn * kTileW + 2 * lane, V, T);
    if (lane == 0) out[r * nt + tn] = ts;
  }
}

// ---------------------------------------------------------------------------
// First token after the prefill (layer.cpp:1500-1510): Philox cycle 0, slot
// 2k, or the mt19937 stream's first double.
// ---------------------------------------------------------------------------
template <bool FILT>
__global__ __launch_bounds__(kThreads) void first_token_kernel(
    SpecState s, const float *__restrict__ logits, int64_t ldl) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  const double u = draw_u(s, b, 0, 0, 2 * s.k);
  const int tok = draw_row<FILT>(logits + b * ldl, s.V, s.T, u, sh, s.top_k, s.top_p);
  // the draw used one double of the mt19937 stream
  if (s.mt_ring && s.T > 0.f) mt_commit(s, b, 2);
  if (threadIdx.x == 0) {
    int32_t *out = s.out + (int64_t)b * s.out_stride;
    out[s.P] = tok;
    s.cur[b] = tok;
    s.gen[b] = 1;
    s.cyc[b] = 1;
    s.tlen[b] = s.P;
    // the draft prefill stops one token short: the last prompt token is the
    // pending catch-up token of the first cycle, dlen the length after it
    s.dlen[b] = s.P;
    s.catchup[b] = 1;
    s.catch_tok[b] = out[s.P - 1];
    s.pair[2 * b] = out[s.P - 1];
    s.pair[2 * b + 1] = tok;
    const int act = s.max_new > 1 ? 1 : 0;
    s.active[b] = act;
    if (act) atomicAdd(s.n_active, 1);
    if (act && s.n_far && s.max_new - 1 > s.k + 1) atomicAdd(s.n_far, 1);
  }
}

// One drafting step j (layer.cpp:1541-1558): q_j = get_probs(draft logits),
// candidate = sample_token(q_j) with u[seq][cycle][j] (Philox) or the
// double 2j outputs past the read counter (mt19937: step j's draw follows
// the j earlier ones of the cycle; steps j >= M draw but are not used).
template <bool FILT>
__global__ __launch_bounds__(kThreads) void draft_sample_kernel(
    SpecState s, int j, const float *__restrict__ logits, int64_t ldl) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  if (!s.active[b]) return;
  const float *row = logits + b * ldl;
  int tok;
  if (s.T <= 0.f) {
    tok = block_argmax(row, s.V, sh);
  } else {
    row_probs<FILT>(row, s.V, s.T, sh, s.qprob + ((int64_t)b * s.k + j) * s.V,
                    s.top_k, s.top_p);
    tok = block_sample(s.V, draw_u(s, b, 2 * j, s.cyc[b], j), sh);
  }
  if (threadIdx.x == 0) s.cand[b * s.k + j] = tok;
  // the probability row is no longer needed: its LDS holds the embedded row
  __syncthreads();
  embed_next(s, b, j, tok, sh.prow, sh.f);
}

__device__ __forceinline__ int verify_rows(const SpecState &s) {
  return s.trows > 0 ? s.trows : s.k + 1;
}

// Per verify row (b, j <= M): argmax (greedy) or the get_probs statistics
// (sampled), for all rows of the cycle at once.  tstat[b][j] =
// {max, 1/sum, 1/sum(kept p1), argmax, tau, tix} (the last three as int
// bits).
template <bool FILT>
__global__ __launch_bounds__(kThreads, FILT ? 1 : 8) void target_stats_kernel(
    SpecState s, const float *__restrict__ tlogits) {
  // the row stays in registers: only the filter needs the LDS row, so the
  // unfiltered kernel leaves room for a second workgroup on the CU
  __shared__ std::conditional_t<FILT, Shared, SmallShared> sh;
  const int j = blockIdx.x, b = blockIdx.y;
  if (!s.active[b]) return;
  const int gen0 = s.gen[b];
  const int M = min(s.k, s.max_new - gen0);
  // row M serves only the bonus sample, which needs room for one more token
  if (j > M || (j == M && gen0 + M >= s.max_new)) return;
  const int64_t r = (int64_t)b * (s.k + 1) + j;
  const float *row = tlogits + ((int64_t)b * verify_rows(s) + j) * s.V;
  float *ts = s.tstat + r * kTstat;
  if (s.T <= 0.f) {
    const int a = block_argmax(row, s.V, sh);
    if (threadIdx.x == 0) ts[3] = __int_as_float(a);
  } else {
    const RowStats st = row_stats<FILT>(row, s.V, s.T, sh, s.top_k, s.top_p);
    if (threadIdx.x == 0) {
      ts[0] = st.mx; ts[1] = st.rsum; ts[2] = st.rfs;
      ts[4] = __uint_as_float(st.tau); ts[5] = __int_as_float(st.tix);
    }
  }
}

// Residual max(0, p - q) (layer.cpp:1611-1630), p from the target row's
// statistics, q from the stored draft probabilities; then sample it, or p
// when the residual sums to zero.  The residual is sampled unnormalised:
// the discrete distribution normalises it.
// qrow: the draft probabilities, or with qlrow set the draft logits whose
// probabilities are (exp(l / T - qs.mx) * qs.rsum) * qs.rfs, the values the
// drafting step would have written
__device__ __forceinline__ int residual_sample(
    const float *__restrict__ qrow, const float *__restrict__ tlog_row,
    RowStats tst, int V, float T, double u, Shared &sh,
    const float *__restrict__ qlrow = nullptr, RowStats qs = RowStats{}) {
  // two halves of the thread's entries, each with its loads in flight
  constexpr int kHalf = kPer / 2;
  float loc = 0.f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    float xt[kHalf], xq[kHalf];
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int v = min((int)threadIdx.x + (hf * kHalf + i) * kThreads, V - 1);
      xt[i] = tlog_row[v];
      xq[i] = qlrow ? qlrow[v] : qrow[v];
    }
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int v = (int)threadIdx.x + (hf * kHalf + i) * kThreads;
      if (v < V) {
        const float p = prob_of(xt[i], v, T, tst);
        const float q = qlrow ? (expf(scaled(xq[i], T) - qs.mx) * qs.rsum) * qs.rfs : xq[i];
        const float r = fmaxf(0.0f, p - q);
        sh.prow[la(v)] = r;
        loc += r;
      }
    }
  }
  const float sr = block_sum(loc, sh);
  if (sr <= 0.0f) fill_probs(tlog_row, V, T, tst, sh);
  return block_sample(V, u, sh);
}

// The statistics of the accept step from logits (AcceptRows::launch_logits,
// T > 0 without top-k / top-p), rows decided in order.  Workgroups are
// numbered row-major (every sequence's row 0, then every row 1, ...); each
// takes a chunk of tiles of one verify row j of one sequence b, and forms
// for every tile of the chunk the target row's tile statistics (max, sum of
// exp) and, for a drafted position, the draft row's.  The last workgroup of
// (b, j) to
// finish (a counter per row) combines all of the row's tiles, as the accept
// step combines a draft row's (wave_tiles_stats): the target row's
// statistics go to tstat, and the candidate is tested; when it is rejected
// by a margin no rounding difference between this kernel and the accept step
// can cross (r * q >= p * (1 + 1e-5)), minrej[b] is lowered to j.  A
// workgroup whose sequence already has a smaller minrej returns at once: the
// accept step, which decides every position again from these statistics,
// stops at or before that rejection and never reads rows after it
// (layer.cpp:1581-1630 computes p_j only until the first rejection).
// Tile statistics cross workgroups through agent-scope atomic stores and
// loads; a workgroup's stores are complete (s_waitcnt) before it counts
// itself, and the counting workgroups never wait for one another.  The
// tiles here are kWideTile columns wide (one wave's: 16 logits a lane, one
// pair of wave reductions each), and a workgroup takes kStatWaves of them.
constexpr int kWideTile = 1024;
constexpr int kStatWaves = 4;
constexpr int kStatThreads = 64 * kStatWaves;

// RowStats of a row from nt <= 64 tile statistics, by one wave: the
// operations of wave_tiles_stats with one tile a lane
__device__ __forceinline__ RowStats wave_few_tiles_stats(const float2 *tl, int nt) {
  const int lane = threadIdx.x & 63;
  const float2 v = tl[min(lane, nt - 1)];
  const float mx = wave_max_all(lane < nt ? v.x : -INFINITY);
  float e = 0.f;
  if (lane < nt && v.x > -INFINITY) e += v.y * expf(v.x - mx);
  e = wave_sum_all(e);
  const float rs = 1.0f / e;
  return mk_stats(mx, rs, 1.0f / (e * rs));
}

// (max s, sum exp(s - max)), s = l / T, of one wave's wide tile: lane l holds
// columns n0 + 128 i + {0, 1}, n0 = tile start + 2 l, i < 8
__device__ __forceinline__ float2 wide_stat(const float2 (&v)[kTileRun], int n0,
                                            int V, float T) {
  float mxl = -INFINITY;
#pragma unroll
  for (int i = 0; i < kTileRun; ++i) {
    const int n = n0 + i * kTileW;
    if (n < V) mxl = fmaxf(mxl, scaled(v[i].x, T));
    if (n + 1 < V) mxl = fmaxf(mxl, scaled(v[i].y, T));
  }
  const float mx = wave_max_all(mxl);
  float e = 0.f;
#pragma unroll
  for (int i = 0; i < kTileRun; ++i) {
    const int n = n0 + i * kTileW;
    if (n < V) e += expf(scaled(v[i].x, T) - mx);
    if (n + 1 < V) e += expf(scaled(v[i].y, T) - mx);
  }
  return make_float2(mx, wave_sum_all(e));
}

__device__ __forceinline__ void st_pair(float2 *p, float2 v) {
  const uint64_t bits =
      ((uint64_t)__float_as_uint(v.y) << 32) | (uint64_t)__float_as_uint(v.x);
  __hip_atomic_store(reinterpret_cast<uint64_t *>(p), bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_pair(const float2 *p) {
  const uint64_t bits = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
}

template <bool PAIRS>
__device__ __forceinline__ void load_tile_run(const float *row, int t0, int V, int lane,
                                              float2 (&v)[kTileRun]) {
#pragma unroll
  for (int i = 0; i < kTileRun; ++i) {
    const int n = (t0 + i) * kTileW + 2 * lane;
    if (PAIRS && n + 1 < V) {
      v[i] = *reinterpret_cast<const float2 *>(row + n);
    } else {
      v[i].x = n < V ? row[n] : 0.f;
      v[i].y = n + 1 < V ? row[n + 1] : 0.f;
    }
  }
}

template <bool PAIRS>
__global__ __launch_bounds__(kStatThreads, 8) void accept_tiles_kernel(
    SpecState s, const float *__restrict__ tlogits, int nch) {
  __shared__ float2 s_t[kMaxV / kWideTile], s_d[kMaxV / kWideTile];
  __shared__ RowStats s_st[2];
  __shared__ int s_last;
  const int per_row = s.B * nch;
  const int j = blockIdx.x / per_row, rem = blockIdx.x % per_row;
  const int b = rem / nch, ch = rem % nch;
  // the first certain rejection first: most workgroups of rows j >= 2 end
  // here after one load
  if (j > 0 && __hip_atomic_load(s.minrej + b, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) < j)
    return;
  if (!s.active[b]) return;
  const int gen0 = s.gen[b];
  const int M = min(s.k, s.max_new - gen0);
  if (j > M || (j == M && gen0 + M >= s.max_new)) return;
  const bool drafted = j < M;                 // else the bonus row
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int V = s.V, nt = s.nt;
  const float *trow = tlogits + ((int64_t)b * verify_rows(s) + j) * V;
  const float *drow = s.qlog + j * s.qlog_js + b * s.qlog_bs;
  float2 *tt = s.ttiles + ((int64_t)b * (s.k + 1) + j) * nt;
  float2 *dt = const_cast<float2 *>(s.dtiles) + ((int64_t)b * s.k + j) * nt;
  const int wt = ch * kStatWaves + w;         // the wave's wide tile
  if (wt < nt) {
    static_assert(kWideTile == kTileRun * kTileW, "a wide tile is one run of 128-column tiles");
    float2 tv[kTileRun], dv[kTileRun];
    load_tile_run<PAIRS>(trow, wt * kTileRun, V, lane, tv);
    if (drafted) load_tile_run<PAIRS>(drow, wt * kTileRun, V, lane, dv);
    const int n0 = wt * kWideTile + 2 * lane;
    const float2 a = wide_stat(tv, n0, V, s.T);
    if (lane == 0) st_pair(tt + wt, a);
    if (drafted) {
      const float2 d = wide_stat(dv, n0, V, s.T);
      if (lane == 0) st_pair(dt + wt, d);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = atomicAdd(s.rowcnt + (int64_t)b * (s.k + 1) + j, 1) == nch - 1;
  __syncthreads();
  if (!s_last) return;
  // the last workgroup of the row: every tile, then the row's statistics
  for (int t = threadIdx.x; t < nt; t += kStatThreads) {
    s_t[t] = ld_pair(tt + t);
    if (drafted) s_d[t] = ld_pair(dt + t);
  }
  __syncthreads();
  if (w == 0) {
    const RowStats st = wave_few_tiles_stats(s_t, nt);
    if (lane == 0) s_st[0] = st;
  } else if (w == 1 && drafted) {
    const RowStats qs = wave_few_tiles_stats(s_d, nt);
    if (lane == 0) s_st[1] = qs;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const RowStats st = s_st[0];
    float *ts = s.tstat + ((int64_t)b * (s.k + 1) + j) * kTstat;
    ts[0] = st.mx; ts[1] = st.rsum; ts[2] = st.rfs;
    ts[4] = __uint_as_float(st.tau); ts[5] = __int_as_float(st.tix);
    if (drafted) {
      const RowStats qs = s_st[1];
      // (a candidate outside the vocabulary reads the last column)
      const int c = min(max(s.cand[b * s.k + j], 0), V - 1);
      const float pc = prob_of(trow[c], c, s.T, st);
      const float qc = (expf(scaled(drow[c], s.T) - qs.mx) * qs.rsum) * qs.rfs;
      const int M = min(s.k, s.max_new - s.gen[b]);
      const float u = s.ua ? s.ua[(int64_t)b * s.k + j]
                           : test_u(s, b, 2 * M + j, (uint32_t)s.cyc[b], s.k + j);
      if (u * qc >= pc * (1.0f + 1e-5f)) atomicMin(s.minrej + b, j);
    }
  }
}

// Accept / reject, resample or bonus, rollback (layer.cpp:1581-1655), from
// the verify rows' statistics (target_stats_kernel).  tlogits: [B][k+1][V],
// row i = verify position i.
__global__ __launch_bounds__(kThreads) void accept_kernel(
    SpecState s, const float *__restrict__ tlogits) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  if (!s.active[b]) return;
  const int V = s.V, k = s.k;
  const bool greedy = s.T <= 0.f;
  const int gen0 = s.gen[b];
  const int M = min(k, s.max_new - gen0);
  const uint32_t cyc = (uint32_t)s.cyc[b];
  const int tstart = s.tlen[b], dstart = s.dlen[b];
  const int tr = verify_rows(s);
  int32_t *out = s.out + (int64_t)b * s.out_stride;
  int nout = s.P + gen0;
  int rej = -1;
  int64_t ties = 0;
  auto stats_of = [&](int j) {
    const float *ts = s.tstat + ((int64_t)b * (k + 1) + j) * kTstat;
    RowStats st = mk_stats(ts[0], ts[1], ts[2]);
    st.tau = __float_as_uint(ts[4]);
    st.tix = __float_as_int(ts[5]);
    return st;
  };
  auto argmax_of = [&](int j) {
    return __float_as_int(s.tstat[((int64_t)b * (k + 1) + j) * kTstat + 3]);
  };
  // implicit draft probabilities (s.qlog): each drafting step's statistics
  // from its lm-head tiles, one wave a step, as the drafting step formed them
  __shared__ RowStats qst[kMaxLookahead];
  const bool qimp = s.qlog != nullptr && !greedy;
  if (qimp) {
    const int w = threadIdx.x >> 6;
    for (int j = w; j < M; j += kWaves) {
      const RowStats st = wave_tiles_stats(s.dtiles + ((int64_t)b * k + j) * s.nt, s.nt);
      if ((threadIdx.x & 63) == 0) qst[j] = st;
    }
    __syncthreads();
  }
  const int64_t qjs = s.qlog_js ? s.qlog_js : (int64_t)s.B * V;
  const int64_t qbs = s.qlog_bs ? s.qlog_bs : (int64_t)V;
  auto qlrow = [&](int j) { return s.qlog + j * qjs + b * qbs; };
  auto q_of = [&](float l, int j) {
    return (expf(scaled(l, s.T) - qst[j].mx) * qst[j].rsum) * qst[j].rfs;
  };
  // the candidates' target logits and draft probabilities, the first kPre
  // positions requested at once (their loop is unrolled so that the
  // prefetched values stay in registers)
  constexpr int kPre = 8;
  float lc[kPre], qcp[kPre];
  if (!greedy) {
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      if (j < M) {
        // reads clamped to the row: a candidate outside the vocabulary
        // (only from nnhip_spec_accept's caller) reads the last column
        const int c = min(max(s.cand[b * k + j], 0), V - 1);
        lc[j] = tlogits[((int64_t)b * tr + j) * V + c];
        qcp[j] = qimp ? qlrow(j)[c] : s.qprob[((int64_t)b * k + j) * V + c];
      }
    }
    if (qimp) {
#pragma unroll
      for (int j = 0; j < kPre; ++j)
        if (j < M) qcp[j] = q_of(qcp[j], j);
    }
  }
  // accept test of position j given its candidate's p and q
  auto test = [&](int j, int c, float lj, float qc) {
    if (greedy) return c == argmax_of(j);
    const RowStats st = stats_of(j);
    const float pc = prob_of(lj, c, s.T, st);
    const float r = s.ua ? s.ua[(int64_t)b * k + j] : test_u(s, b, 2 * M + j, cyc, k + j);
    if (fabs((double)r - (double)pc / (double)qc) < 1e-6) ++ties;
    return __fmul_rn(r, qc) < pc;
  };
#pragma unroll
  for (int j = 0; j < kPre; ++j) {
    if (j >= M || rej >= 0) break;
    const int c = s.cand[b * k + j];
    if (!test(j, c, lc[j], qcp[j])) { rej = j; break; }
    if (threadIdx.x == 0) out[nout] = c;
    ++nout;
  }
  for (int j = kPre; j < M && rej < 0; ++j) {
    const int c = s.cand[b * k + j];
    const int cr = min(max(c, 0), V - 1);
    const float lj = greedy ? 0.f : tlogits[((int64_t)b * tr + j) * V + cr];
    const float qc = greedy ? 0.f
                     : qimp ? q_of(qlrow(j)[cr], j)
                            : s.qprob[((int64_t)b * k + j) * V + cr];
    if (!test(j, c, lj, qc)) { rej = j; break; }
    if (threadIdx.x == 0) out[nout] = c;
    ++nout;
  }
  int gen = gen0 + (rej < 0 ? M : rej);
  int tok = -1, catch_tok = -1;
  // the resample / bonus draw follows the tests up to the first rejection
  const double u = s.ur ? (double)s.ur[b]
                        : draw_u(s, b, 2 * M + (rej >= 0 ? rej + 1 : M), cyc, 2 * k);
  if (rej >= 0) {
    const float *row = tlogits + ((int64_t)b * tr + rej) * V;
    if (greedy) {
      tok = argmax_of(rej);
    } else {
      tok = qimp ? residual_sample(nullptr, row, stats_of(rej), V, s.T, u, sh,
                                   qlrow(rej), qst[rej])
                 : residual_sample(s.qprob + ((int64_t)b * k + rej) * V, row,
                                   stats_of(rej), V, s.T, u, sh);
    }
    catch_tok = tok;
  } else if (gen < s.max_new) {
    const float *row = tlogits + ((int64_t)b * tr + M) * V;
    if (greedy) {
      tok = argmax_of(M);
    } else {
      fill_probs(row, V, s.T, stats_of(M), sh);
      tok = block_sample(V, u, sh);
    }
    catch_tok = s.cand[b * k + M - 1];
  }
  if (threadIdx.x == 0) {
    int64_t *st = s.stats + (int64_t)b * kSpecStats;
    st[0] += 1;
    st[1] += M;
    st[2] += (rej < 0 ? M : rej);
    st[3] += ties;
    if (s.n_acc_out) {
      s.n_acc_out[b] = rej < 0 ? M : rej;
      s.tok_out[b] = tok;
    }
    if (tok >= 0) {
      out[nout] = tok;
      ++gen;
      s.cur[b] = tok;
      if (rej >= 0) st[4] += 1; else st[5] += 1;
    }
    const int keep = rej >= 0 ? rej : M;
    s.tlen[b] = tstart + keep + 1;
    // The draft cache keeps [generated.back(), c_0 .. c_{rej-1}] after a
    // rejection (layer.cpp:1636) or [generated.back(), c_0 .. c_{M-2}] after
    // full acceptance, then takes the catch-up token (layer.cpp:1639-1653);
    // dlen is the length after that catch-up, which writes at dlen - 1.
    if (tok >= 0) s.dlen[b] = dstart + keep + (rej >= 0 ? 2 : 1);
    // lengths the reference's forwards reach this cycle: the verify forward
    // of M + 1 ids, the M drafting steps, the catch-up
    st[6] = max(st[6], (int64_t)(tstart + M + 1));
    st[7] = max(st[7], (int64_t)max(dstart + M, tok >= 0 ? s.dlen[b] : 0));
    s.catchup[b] = tok >= 0 ? 1 : 0;
    s.catch_tok[b] = catch_tok;
    s.pair[2 * b] = catch_tok;
    s.pair[2 * b + 1] = tok;
    s.gen[b] = gen;
    s.cyc[b] = (int)cyc + 1;
    if (gen >= s.max_new) {
      s.active[b] = 0;
      s.catchup[b] = 0;
      atomicSub(s.n_active, 1);
    }
    // no longer sure to need more than the next cycle
    if (s.n_far && s.max_new - gen0 > k + 1 && s.max_new - gen <= k + 1)
      atomicSub(s.n_far, 1);
  }
  // the mt19937 outputs of the cycle: M drafting draws, the tests up to the
  // first rejection, the resample or bonus draw
  if (s.mt_ring && !greedy)
    mt_commit(s, b, 2 * M + (rej >= 0 ? rej + 1 : M) + (tok >= 0 ? 2 : 0));
}

// generate_advanced sampling step (layer.cpp:1294-1373): u[seq][step][0]
// (Philox) or the mt19937 stream's next double.
template <bool FILT>
__global__ __launch_bounds__(kThreads) void ar_sample_kernel(
    SpecState s, int step, const float *__restrict__ logits, int64_t ldl) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  const double u = draw_u(s, b, 0, (uint32_t)step, 0);
  const int tok = draw_row<FILT>(logits + b * ldl, s.V, s.T, u, sh, s.top_k, s.top_p);
  if (threadIdx.x == 0) {
    s.out[(int64_t)b * s.out_stride + s.P + step] = tok;
    s.cur[b] = tok;
  }
  // one double of the mt19937 stream per sampled token
  if (s.mt_ring && s.T > 0.f) mt_commit(s, b, 2);
}

// State of the accept step run on given rows (AcceptRows): every sequence
// drafted k candidates (gen 0 of max_new = k, so no bonus row), at cycle 1.
// The accept step split over three launches (launch_accept with
// g_accept_split), so that the draw from the residual (or from p for the
// bonus) runs on many CUs instead of one per sequence:
//  1. accept_decide_kernel (one workgroup per sequence): the accept tests of
//     accept_kernel, the accepted candidates written out, and a record of
//     what remains to draw;
//  2. draw_chunks_kernel (kDrawChunks workgroups per sequence): over its
//     chunk of the vocabulary, the double sums of the residual
//     max(0, p - q) and of p (the weights residual_sample and fill_probs
//     form, the same expressions);
//  3. accept_final_kernel (one workgroup per sequence): the chunk in which
//     u * S falls, then block_sample's crossing rule inside it (running
//     double sums over the chunk prefix), and accept_kernel's state update.
// Record per sequence: kind (-1 inactive, 0 nothing to draw, 1 residual,
// 2 p of the bonus row), the rejected position (-1 none), ties, the greedy
// token, and the implicit draft statistics of the rejected row.
constexpr int kRec = kAcceptRec;

__global__ __launch_bounds__(kThreads) void accept_decide_kernel(
    SpecState s, const float *__restrict__ tlogits) {
  const int b = blockIdx.x;
  int32_t *rec = s.rec + (int64_t)b * kRec;
  if (!s.active[b]) {
    if (threadIdx.x == 0) rec[0] = -1;
    return;
  }
  const int V = s.V, k = s.k;
  const bool greedy = s.T <= 0.f;
  const int gen0 = s.gen[b];
  const int M = min(k, s.max_new - gen0);
  const uint32_t cyc = (uint32_t)s.cyc[b];
  const int tr = verify_rows(s);
  int32_t *out = s.out + (int64_t)b * s.out_stride;
  int nout = s.P + gen0;
  int rej = -1;
  int64_t ties = 0;
  auto stats_of = [&](int j) {
    const float *ts = s.tstat + ((int64_t)b * (k + 1) + j) * kTstat;
    RowStats st = mk_stats(ts[0], ts[1], ts[2]);
    st.tau = __float_as_uint(ts[4]);
    st.tix = __float_as_int(ts[5]);
    return st;
  };
  auto argmax_of = [&](int j) {
    return __float_as_int(s.tstat[((int64_t)b * (k + 1) + j) * kTstat + 3]);
  };
  // implicit draft probabilities (s.qlog): each drafting step's statistics
  // from its lm-head tiles, one wave a step, as the drafting step formed them
  __shared__ RowStats qst[kMaxLookahead];
  const bool qimp = s.qlog != nullptr && !greedy;
  if (qimp) {
    const int w = threadIdx.x >> 6;
    for (int j = w; j < M; j += kWaves) {
      const RowStats st = wave_tiles_stats(s.dtiles + ((int64_t)b * k + j) * s.nt, s.nt);
      if ((threadIdx.x & 63) == 0) qst[j] = st;
    }
    __syncthreads();
  }
  const int64_t qjs = s.qlog_js ? s.qlog_js : (int64_t)s.B * V;
  const int64_t qbs = s.qlog_bs ? s.qlog_bs : (int64_t)V;
  auto qlrow = [&](int j) { return s.qlog + j * qjs + b * qbs; };
  auto q_of = [&](float l, int j) {
    return (expf(scaled(l, s.T) - qst[j].mx) * qst[j].rsum) * qst[j].rfs;
  };
  // the candidates' target logits and draft probabilities, the first kPre
  // positions requested at once (their loop is unrolled so that the
  // prefetched values stay in registers)
  constexpr int kPre = 8;
  float lc[kPre], qcp[kPre];
  if (!greedy) {
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      if (j < M) {
        // reads clamped to the row: a candidate outside the vocabulary
        // (only from nnhip_spec_accept's caller) reads the last column
        const int c = min(max(s.cand[b * k + j], 0), V - 1);
        lc[j] = tlogits[((int64_t)b * tr + j) * V + c];
        qcp[j] = qimp ? qlrow(j)[c] : s.qprob[((int64_t)b * k + j) * V + c];
      }
    }
    if (qimp) {
#pragma unroll
      for (int j = 0; j < kPre; ++j)
        if (j < M) qcp[j] = q_of(qcp[j], j);
    }
  }
  // accept test of position j given its candidate's p and q
  auto test = [&](int j, int c, float lj, float qc) {
    if (greedy) return c == argmax_of(j);
    const RowStats st = stats_of(j);
    const float pc = prob_of(lj, c, s.T, st);
    const float r = s.ua ? s.ua[(int64_t)b * k + j] : test_u(s, b, 2 * M + j, cyc, k + j);
    if (fabs((double)r - (double)pc / (double)qc) < 1e-6) ++ties;
    return __fmul_rn(r, qc) < pc;
  };
#pragma unroll
  for (int j = 0; j < kPre; ++j) {
    if (j >= M || rej >= 0) break;
    const int c = s.cand[b * k + j];
    if (!test(j, c, lc[j], qcp[j])) { rej = j; break; }
    if (threadIdx.x == 0) out[nout] = c;
    ++nout;
  }
  for (int j = kPre; j < M && rej < 0; ++j) {
    const int c = s.cand[b * k + j];
    const int cr = min(max(c, 0), V - 1);
    const float lj = greedy ? 0.f : tlogits[((int64_t)b * tr + j) * V + cr];
    const float qc = greedy ? 0.f
                     : qimp ? q_of(qlrow(j)[cr], j)
                            : s.qprob[((int64_t)b * k + j) * V + cr];
    if (!test(j, c, lj, qc)) { rej = j; break; }
    if (threadIdx.x == 0) out[nout] = c;
    ++nout;
  }
  const int gen = gen0 + (rej < 0 ? M : rej);
  if (threadIdx.x == 0) {
    int kind = 0, tok = -1;
    if (rej >= 0) {
      if (greedy) tok = argmax_of(rej);
      else kind = 1;
    } else if (gen < s.max_new) {
      if (greedy) tok = argmax_of(M);
      else kind = 2;
    }
    rec[0] = kind;
    rec[1] = rej;
    rec[2] = (int)ties;
    rec[3] = tok;
    if (kind == 1 && qimp) {
      rec[5] = __float_as_int(qst[rej].mx);
      rec[6] = __float_as_int(qst[rej].rsum);
      rec[7] = __float_as_int(qst[rej].rfs);
    }
  }
}

// weight of entry v of the row to draw from: the residual max(0, p - q)
// (residual_sample's expressions) and p (fill_probs')
__device__ __forceinline__ void draw_weights(float xt, float xq, int v, float T,
                                             const RowStats &tst, bool implicit_q,
                                             const RowStats &qs, float &r, float &p) {
  p = prob_of(xt, v, T, tst);
  const float q = implicit_q ? (expf(scaled(xq, T) - qs.mx) * qs.rsum) * qs.rfs : xq;
  r = fmaxf(0.0f, p - q);
}

struct DrawRow {
  const float *trow, *qrow;   // target logits; draft logits or probabilities
  bool implicit_q;
  RowStats tst, qs;
};

__device__ __forceinline__ DrawRow draw_row(const SpecState &s, const float *tlogits,
                                            int b, const int32_t *rec) {
  const int kind = rec[0], rej = rec[1];
  const int k = s.k, V = s.V;
  const int gen0 = s.gen[b];
  const int M = min(k, s.max_new - gen0);
  const int j = kind == 1 ? rej : M;
  DrawRow d;
  d.trow = tlogits + ((int64_t)b * verify_rows(s) + j) * V;
  const float *ts = s.tstat + ((int64_t)b * (k + 1) + j) * kTstat;
  d.tst = mk_stats(ts[0], ts[1], ts[2]);
  d.tst.tau = __float_as_uint(ts[4]);
  d.tst.tix = __float_as_int(ts[5]);
  d.implicit_q = s.qlog != nullptr;
  d.qrow = nullptr;
  d.qs = mk_stats(0.f, 0.f, 0.f);
  if (kind == 1) {
    if (d.implicit_q) {
      const int64_t qjs = s.qlog_js ? s.qlog_js : (int64_t)s.B * V;
      const int64_t qbs = s.qlog_bs ? s.qlog_bs : (int64_t)V;
      d.qrow = s.qlog + j * qjs + b * qbs;
      d.qs = mk_stats(__int_as_float(rec[5]), __int_as_float(rec[6]), __int_as_float(rec[7]));
    } else {
      d.qrow = s.qprob + ((int64_t)b * k + j) * V;
    }
  }
  return d;
}

constexpr int kDrawThreads = 256;

__global__ __launch_bounds__(kDrawThreads) void draw_chunks_kernel(
    SpecState s, const float *__restrict__ tlogits) {
  __shared__ double s_red[2][kDrawThreads / 64];
  const int c = blockIdx.x, b = blockIdx.y;
  const int32_t *rec = s.rec + (int64_t)b * kRec;
  const int kind = rec[0];
  if (kind <= 0) return;
  const DrawRow d = draw_row(s, tlogits, b, rec);
  const int V = s.V, CH = (V + kDrawChunks - 1) / kDrawChunks;
  const int v0 = c * CH, v1 = min(V, v0 + CH);
  constexpr int kPerT = (kMaxV / kDrawChunks + kDrawThreads - 1) / kDrawThreads;
  float xt[kPerT], xq[kPerT];
#pragma unroll
  for (int i = 0; i < kPerT; ++i) {
    const int v = min(v0 + (int)threadIdx.x + i * kDrawThreads, V - 1);
    xt[i] = d.trow[v];
    xq[i] = kind == 1 ? d.qrow[v] : 0.f;
  }
  double rs = 0.0, ps = 0.0;
#pragma unroll
  for (int i = 0; i < kPerT; ++i) {
    const int v = v0 + (int)threadIdx.x + i * kDrawThreads;
    if (v < v1) {
      float r, p;
      draw_weights(xt[i], xq[i], v, s.T, d.tst, d.implicit_q, d.qs, r, p);
      rs += (double)r;
      ps += (double)p;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    rs += __shfl_xor(rs, o, 64);
    ps += __shfl_xor(ps, o, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { s_red[0][w] = rs; s_red[1][w] = ps; }
  __syncthreads();
  if (threadIdx.x == 0) {
    double tr = 0.0, tp = 0.0;
#pragma unroll
    for (int i = 0; i < kDrawThreads / 64; ++i) { tr += s_red[0][i]; tp += s_red[1][i]; }
    double *out = s.chunks + ((int64_t)b * kDrawChunks + c) * 2;
    out[0] = tr;
    out[1] = tp;
  }
}

__global__ __launch_bounds__(kThreads) void accept_final_kernel(
    SpecState s, const float *__restrict__ tlogits) {
  __shared__ SmallShared sh;
  const int b = blockIdx.x;
  const int32_t *rec = s.rec + (int64_t)b * kRec;
  const int kind = rec[0];
  if (kind < 0) return;
  const int V = s.V, k = s.k;
  const int gen0 = s.gen[b];
  const int M = min(k, s.max_new - gen0);
  const uint32_t cyc = (uint32_t)s.cyc[b];
  const int tstart = s.tlen[b], dstart = s.dlen[b];
  const int rej = rec[1];
  int32_t *out = s.out + (int64_t)b * s.out_stride;
  const int nout = s.P + gen0 + (rej < 0 ? M : rej);
  int gen = gen0 + (rej < 0 ? M : rej);
  int tok = rec[3], catch_tok = -1;
  if (kind > 0) {
    const double u = s.ur ? (double)s.ur[b]
                          : draw_u(s, b, 2 * M + (rej >= 0 ? rej + 1 : M), cyc, 2 * k);
    // the draw's weights: the residual, or p where the residual is all zero
    // (residual_sample) and for the bonus row
    const double *ch = s.chunks + (int64_t)b * kDrawChunks * 2;
    double rtot = 0.0;
    if (kind == 1) {
      for (int c = 0; c < kDrawChunks; ++c) rtot += ch[2 * c];
    }
    const int sel = (kind == 1 && rtot > 0.0) ? 0 : 1;
    double S = 0.0;
    for (int c = 0; c < kDrawChunks; ++c) S += ch[2 * c + sel];
    const double target = (double)u * S;
    // the chunk in which the running sum reaches the target
    int kc = kDrawChunks - 1;
    double pre = 0.0, pk = 0.0;
    for (int c = 0; c < kDrawChunks; ++c) {
      const double x = ch[2 * c + sel];
      if (pre + x >= target - 1e-12 * S) { kc = c; pk = pre; break; }
      pre += x;
    }
    // block_sample inside that chunk: contiguous runs per thread, running
    // double sums from the chunk's prefix
    const DrawRow d = draw_row(s, tlogits, b, rec);
    const int CH = (V + kDrawChunks - 1) / kDrawChunks;
    const int v0 = kc * CH, v1 = min(V, v0 + CH);
    constexpr int E = (kMaxV / kDrawChunks + kThreads - 1) / kThreads;
    const int E_ = (CH + kThreads - 1) / kThreads;
    const int b0 = v0 + (int)threadIdx.x * E_;
    float wv[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int v = b0 + i;
      wv[i] = 0.f;
      if (i < E_ && v < v1) {
        float r, p;
        draw_weights(d.trow[v], kind == 1 ? d.qrow[v] : 0.f, v, s.T, d.tst,
                     d.implicit_q, d.qs, r, p);
        wv[i] = sel == 0 ? r : p;
      }
    }
    double loc = 0.0;
#pragma unroll
    for (int i = 0; i < E; ++i) loc += (double)wv[i];
    double St;
    double c = pk + block_excl_scan_d(loc, sh, &St);
    int found = 0x7fffffff;
    if (c + loc >= target - 1e-12 * S) {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int v = b0 + i;
        c += (double)wv[i];
        if (found == 0x7fffffff && i < E_ && v < v1 && v < V - 1 && c >= target) found = v;
      }
    }
    const int r = block_min_i(found, sh);
    tok = r != 0x7fffffff ? r : min(v1, V - 1);
    catch_tok = kind == 1 ? tok : s.cand[b * k + M - 1];
  } else if (tok >= 0) {
    catch_tok = rej >= 0 ? tok : s.cand[b * k + M - 1];
  }
  if (threadIdx.x == 0) {
    const int64_t ties = rec[2];
    int64_t *st = s.stats + (int64_t)b * kSpecStats;
    st[0] += 1;
    st[1] += M;
    st[2] += (rej < 0 ? M : rej);
    st[3] += ties;
    if (s.n_acc_out) {
      s.n_acc_out[b] = rej < 0 ? M : rej;
      s.tok_out[b] = tok;
    }
    if (tok >= 0) {
      out[nout] = tok;
      ++gen;
      s.cur[b] = tok;
      if (rej >= 0) st[4] += 1; else st[5] += 1;
    }
    const int keep = rej >= 0 ? rej : M;
    s.tlen[b] = tstart + keep + 1;
    // The draft cache keeps [generated.back(), c_0 .. c_{rej-1}] after a
    // rejection (layer.cpp:1636) or [generated.back(), c_0 .. c_{M-2}] after
    // full acceptance, then takes the catch-up token (layer.cpp:1639-1653);
    // dlen is the length after that catch-up, which writes at dlen - 1.
    if (tok >= 0) s.dlen[b] = dstart + keep + (rej >= 0 ? 2 : 1);
    st[6] = max(st[6], (int64_t)(tstart + M + 1));
    st[7] = max(st[7], (int64_t)max(dstart + M, tok >= 0 ? s.dlen[b] : 0));
    s.catchup[b] = tok >= 0 ? 1 : 0;
    s.catch_tok[b] = catch_tok;
    s.pair[2 * b] = catch_tok;
    s.pair[2 * b + 1] = tok;
    s.gen[b] = gen;
    s.cyc[b] = (int)cyc + 1;
    if (gen >= s.max_new) {
      s.active[b] = 0;
      s.catchup[b] = 0;
      atomicSub(s.n_active, 1);
    }
    if (s.n_far && s.max_new - gen0 > k + 1 && s.max_new - gen <= k + 1)
      atomicSub(s.n_far, 1);
  }
  // the mt19937 outputs of the cycle (accept_kernel)
  if (s.mt_ring && s.T > 0.f)
    mt_commit(s, b, 2 * M + (rej >= 0 ? rej + 1 : M) + (kind > 0 ? 2 : 0));
}

__global__ void accept_rows_reset_kernel(SpecState s) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b == 0) *s.n_active = s.B;
  if (b >= s.B) return;
  s.cur[b] = -1; s.tlen[b] = 0; s.dlen[b] = 0; s.gen[b] = 0; s.cyc[b] = 1;
  s.active[b] = 1; s.catchup[b] = 0; s.catch_tok[b] = -1;
  if (s.minrej) s.minrej[b] = 0x7fffffff;
  if (s.rowcnt)
    for (int j = 0; j <= s.k; ++j) s.rowcnt[(int64_t)b * (s.k + 1) + j] = 0;
  for (int i = 0; i < kSpecStats; ++i) s.stats[(int64_t)b * kSpecStats + i] = 0;
}

// get_probs + sample_token on independent rows with explicit uniforms.
template <bool FILT>
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(
    const float *__restrict__ logits, int V, float T, int top_k, float top_p,
    const float *__restrict__ u, int32_t *__restrict__ tok,
    float *__restrict__ probs) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  const float *row = logits + (int64_t)b * V;
  int t;
  if (T <= 0.f) {
    t = block_argmax(row, V, sh);
  } else {
    row_probs<FILT>(row, V, T, sh, probs ? probs + (int64_t)b * V : nullptr,
                    top_k, top_p);
    t = block_sample(V, u[b], sh);
  }
  if (threadIdx.x == 0) tok[b] = t;
}

// whether a loop's sampling passes filter by top_k / top_p
bool filtered(const SpecState &s) {
  return s.T > 0.f && sampling_filtered(s.V, s.top_k, s.top_p);
}

}  // namespace

int g_accept_early = 1;
int g_accept_split = 1;

void launch_mt_seed(hipStream_t st, const SpecState &s) {
  NNHIP_REQUIRE(s.mt && s.mt_ring && s.mt_rw && s.B > 0, kErrArg,
                "mt19937 stream: buffers not set");
  hipLaunchKernelGGL(mt_seed_kernel, dim3(s.B), dim3(1024), 0, st, s);
  NNHIP_CHECK(hipGetLastError());
}

void launch_first_token(hipStream_t st, const SpecState &s,
                        const float *logits, int64_t ldl) {
  NNHIP_REQUIRE(s.V <= kMaxV, kErrUnsupported,
                "sampling: vocabulary above 32768");
  if (filtered(s))
    hipLaunchKernelGGL(first_token_kernel<true>, dim3(s.B), dim3(kThreads), 0,
                       st, s, logits, ldl);
  else
    hipLaunchKernelGGL(first_token_kernel<false>, dim3(s.B), dim3(kThreads), 0,
                       st, s, logits, ldl);
  NNHIP_CHECK(hipGetLastError());
}

void launch_draft_sample(hipStream_t st, const SpecState &s, int j,
                         const float *logits, int64_t ldl) {
  if (filtered(s))
    hipLaunchKernelGGL(draft_sample_kernel<true>, dim3(s.B), dim3(kThreads), 0,
                       st, s, j, logits, ldl);
  else
    hipLaunchKernelGGL(draft_sample_kernel<false>, dim3(s.B), dim3(kThreads), 0,
                       st, s, j, logits, ldl);
  NNHIP_CHECK(hipGetLastError());
}

// the accept step after the row statistics: accept_kernel, or its split
// form when the state carries the split's scratch
void launch_accept_step(hipStream_t st, const SpecState &s, const float *tlogits) {
  // greedy decoding draws nothing: the one-launch accept step (the split
  // form's chunk sums serve only the residual / bonus draw)
  if (s.rec && s.chunks && s.T > 0.f) {
    hipLaunchKernelGGL(accept_decide_kernel, dim3(s.B), dim3(kThreads), 0, st, s,
                       tlogits);
    NNHIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(draw_chunks_kernel, dim3(kDrawChunks, s.B), dim3(kDrawThreads),
                       0, st, s, tlogits);
    NNHIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(accept_final_kernel, dim3(s.B), dim3(kThreads), 0, st, s,
                       tlogits);
  } else {
    hipLaunchKernelGGL(accept_kernel, dim3(s.B), dim3(kThreads), 0, st, s,
                       tlogits);
  }
  NNHIP_CHECK(hipGetLastError());
}

void launch_accept(hipStream_t st, const SpecState &s, const float *tlogits) {
  NNHIP_REQUIRE(s.tstat != nullptr, kErrArg, "accept: no row statistics");
  if (filtered(s))
    hipLaunchKernelGGL(target_stats_kernel<true>, dim3(s.k + 1, s.B),
                       dim3(kThreads), 0, st, s, tlogits);
  else
    hipLaunchKernelGGL(target_stats_kernel<false>, dim3(s.k + 1, s.B),
                       dim3(kThreads), 0, st, s, tlogits);
  NNHIP_CHECK(hipGetLastError());
  launch_accept_step(st, s, tlogits);
}

void launch_draft_sample_tiles(hipStream_t st, const SpecState &s, int j,
                               const float *logits, int64_t ldl) {
  NNHIP_REQUIRE(s.dtiles && (s.T <= 0.f || s.qprob || s.qlog) && s.nt <= kThreads &&
                    s.tw <= kThreads && s.V <= kMaxV,
                kErrArg, "draft sample: tile statistics missing or too many tiles");
  NNHIP_REQUIRE(s.T <= 0.f || !sampling_filtered(s.V, s.top_k, s.top_p), kErrArg,
                "draft sample: tile statistics cannot apply top-k / top-p");
  hipLaunchKernelGGL(draft_sample_tiles_kernel, dim3(s.B, s.qlog ? 1 : kQParts),
                     dim3(kThreads), 0, st, s, j, logits, ldl);
  NNHIP_CHECK(hipGetLastError());
}

void launch_ar_sample(hipStream_t st, const SpecState &s, int step,
                      const float *logits, int64_t ldl) {
  NNHIP_REQUIRE(s.V <= kMaxV, kErrUnsupported,
                "sampling: vocabulary above 32768");
  if (filtered(s))
    hipLaunchKernelGGL(ar_sample_kernel<true>, dim3(s.B), dim3(kThreads), 0, st,
                       s, step, logits, ldl);
  else
    hipLaunchKernelGGL(ar_sample_kernel<false>, dim3(s.B), dim3(kThreads), 0,
                       st, s, step, logits, ldl);
  NNHIP_CHECK(hipGetLastError());
}

void launch_sample_rows(hipStream_t st, const float *logits, int B, int V,
                        float T, const float *u, int32_t *tok, float *probs,
                        int top_k, float top_p) {
  NNHIP_REQUIRE(V <= kMaxV, kErrUnsupported,
                "sampling: vocabulary above 32768");
  if (T > 0.f && sampling_filtered(V, top_k, top_p))
    hipLaunchKernelGGL(sample_rows_kernel<true>, dim3(B), dim3(kThreads), 0, st,
                       logits, V, T, top_k, top_p, u, tok, probs);
  else
    hipLaunchKernelGGL(sample_rows_kernel<false>, dim3(B), dim3(kThreads), 0,
                       st, logits, V, T, top_k, top_p, u, tok, probs);
  NNHIP_CHECK(hipGetLastError());
}

AcceptRows::AcceptRows(int B, int k, int V, float T) {
  NNHIP_REQUIRE(B > 0 && k > 0 && V > 0, kErrArg, "accept: bad sizes");
  NNHIP_REQUIRE(V <= kMaxV, kErrUnsupported, "sampling: vocabulary above 32768");
  cur.alloc(B); tlen.alloc(B); dlen.alloc(B); gen.alloc(B); cyc.alloc(B);
  active.alloc(B); catchup.alloc(B); catch_tok.alloc(B);
  pair.alloc((size_t)2 * B); out.alloc((size_t)B * (k + 1)); n_active.alloc(1);
  tstat.alloc((size_t)B * (k + 1) * kTstat);
  stats.alloc((size_t)B * kSpecStats);
  s = SpecState{};
  s.cur = cur.p; s.tstat = tstat.p; s.tlen = tlen.p; s.dlen = dlen.p;
  s.gen = gen.p; s.cyc = cyc.p; s.active = active.p; s.catchup = catchup.p;
  s.catch_tok = catch_tok.p; s.pair = pair.p; s.out = out.p;
  s.n_active = n_active.p; s.stats = stats.p;
  s.B = B; s.out_stride = k + 1; s.P = 0; s.max_new = k; s.k = k; s.V = V;
  s.T = T; s.trows = k; s.top_k = 0; s.top_p = 1.f;
}

void launch_row_tile_stats(hipStream_t st, const float *logits, int64_t ldl,
                           int rows, int V, float T, float2 *out) {
  NNHIP_REQUIRE(rows > 0 && V > 0 && ldl >= V && rows <= 65535, kErrArg,
                "row tile statistics: bad sizes");
  const int nt = (V + kTileW - 1) / kTileW;
  const int per_block = (kTileThreads / 64) * kTileRun;
  const dim3 grid((nt + per_block - 1) / per_block, rows);
  if (ldl % 2 == 0 && reinterpret_cast<uintptr_t>(logits) % 8 == 0)
    hipLaunchKernelGGL(row_tile_stats_kernel<true>, grid, dim3(kTileThreads), 0, st,
                       logits, ldl, V, T, nt, out);
  else
    hipLaunchKernelGGL(row_tile_stats_kernel<false>, grid, dim3(kTileThreads), 0, st,
                       logits, ldl, V, T, nt, out);
  NNHIP_CHECK(hipGetLastError());
}

void AcceptRows::launch_logits(hipStream_t st, const float *tlogits,
                               const float *dlogits, const int32_t *cand,
                               const float *ua, const float *ur, int32_t *n_acc,
                               int32_t *tok) {
  if (s.T <= 0.f) {   // greedy: the draft probabilities are not read
    launch(st, tlogits, nullptr, cand, ua, ur, n_acc, tok);
    return;
  }
  const int nt = (s.V + kTileW - 1) / kTileW;
  NNHIP_REQUIRE(nt <= kTileMax * 64, kErrUnsupported,
                "accept: more than 1024 tiles of draft statistics");
  if (!dtiles.p) dtiles.alloc((size_t)s.B * s.k * nt);
  const bool early = g_accept_early && !filtered(s);
  if (!early) launch_row_tile_stats(st, dlogits, s.V, s.B * s.k, s.V, s.T, dtiles.p);
  SpecState a = s;
  a.qlog = dlogits;
  a.qlog_js = s.V;
  a.qlog_bs = (int64_t)s.k * s.V;
  a.dtiles = dtiles.p;
  a.nt = nt;
  a.tw = kTileW;
  a.cand = const_cast<int32_t *>(cand);
  a.ua = ua; a.ur = ur; a.n_acc_out = n_acc; a.tok_out = tok;
  attach_split(a);
  if (early) {
    if (!minrej.p) {
      minrej.alloc(s.B);
      rowcnt.alloc((size_t)s.B * (s.k + 1));
      ttiles.alloc((size_t)s.B * (s.k + 1) * nt);
    }
    a.minrej = minrej.p;
    a.rowcnt = rowcnt.p;
    a.ttiles = ttiles.p;
    // wide tiles: the draft probabilities the accept step forms come from
    // these statistics
    a.nt = (s.V + kWideTile - 1) / kWideTile;
    a.tw = kWideTile;
  }
  hipLaunchKernelGGL(accept_rows_reset_kernel, dim3((s.B + 255) / 256),
                     dim3(256), 0, st, a);
  NNHIP_CHECK(hipGetLastError());
  if (!early) {
    launch_accept(st, a, tlogits);
    return;
  }
  // rows decided in order: the statistics of the rows up to each
  // sequence's first rejection, then the accept step
  const int nch = (a.nt + kStatWaves - 1) / kStatWaves;
  NNHIP_REQUIRE((int64_t)s.B * (s.k + 1) * nch <= 0x7fffffff, kErrArg, "accept: too many rows");
  const dim3 grid(s.B * (s.k + 1) * nch);
  if (s.V % 2 == 0 && reinterpret_cast<uintptr_t>(tlogits) % 8 == 0 &&
      reinterpret_cast<uintptr_t>(dlogits) % 8 == 0)
    hipLaunchKernelGGL(accept_tiles_kernel<true>, grid, dim3(kStatThreads), 0, st, a,
                       tlogits, nch);
  else
    hipLaunchKernelGGL(accept_tiles_kernel<false>, grid, dim3(kStatThreads), 0, st, a,
                       tlogits, nch);
  NNHIP_CHECK(hipGetLastError());
  launch_accept_step(st, a, tlogits);
}

void AcceptRows::launch(hipStream_t st, const float *tlogits, const float *qprob,
                        const int32_t *cand, const float *ua, const float *ur,
                        int32_t *n_acc, int32_t *tok) {
  SpecState a = s;
  a.qprob = const_cast<float *>(qprob);
  a.cand = const_cast<int32_t *>(cand);
  a.ua = ua; a.ur = ur; a.n_acc_out = n_acc; a.tok_out = tok;
  attach_split(a);
  hipLaunchKernelGGL(accept_rows_reset_kernel, dim3((s.B + 255) / 256),
                     dim3(256), 0, st, a);
  NNHIP_CHECK(hipGetLastError());
  launch_accept(st, a, tlogits);
}

void AcceptRows::attach_split(SpecState &a) {
  if (!g_accept_split) return;
  if (!rec.p) {
    rec.alloc((size_t)s.B * kAcceptRec);
    chunks.alloc((size_t)s.B * kDrawChunks * 2);
  }
  a.rec = rec.p;
  a.chunks = chunks.p;
}

}  // namespace nnhip

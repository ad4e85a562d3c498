// Internal declarations shared by the HIP kernels and the host engine of
// libnnhip.so.  Nothing here is part of the C ABI (include/nnhip.h is).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace nnhip {

// ---------------------------------------------------------------------------
// Errors: every failure becomes a std::runtime_error carrying the message
// that nnhip_last_error() returns at the C boundary.
// ---------------------------------------------------------------------------
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

#define NNHIP_CHECK(expr)                                                     \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess)                                                     \
      throw ::nnhip::Error(-3, std::string(#expr) + ": " +                    \
                                   hipGetErrorString(e_));                    \
  } while (0)

#define NNHIP_REQUIRE(cond, code, msg)                                        \
  do {                                                                        \
    if (!(cond)) throw ::nnhip::Error((code), (msg));                         \
  } while (0)

// Status codes of the C ABI.
enum : int {
  kOk = 0,
  kErrArg = -1,        // bad argument / shape
  kErrCapacity = -2,   // sequence would exceed max_seq_len
  kErrHip = -3,        // HIP runtime failure
  kErrUnsupported = -4, // option the device path does not implement
  kErrIO = -5          // a file could not be opened or written
};

// ---------------------------------------------------------------------------
// Device buffers
// ---------------------------------------------------------------------------
template <typename T>
struct DevBuf {
  T *p = nullptr;
  size_t n = 0;
  DevBuf() = default;
  explicit DevBuf(size_t count) { alloc(count); }
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  DevBuf(DevBuf &&o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
  DevBuf &operator=(DevBuf &&o) noexcept {
    if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
    return *this;
  }
  ~DevBuf() { release(); }
  void alloc(size_t count) {
    release();
    if (count) NNHIP_CHECK(hipMalloc(&p, count * sizeof(T)));
    n = count;
  }
  void ensure(size_t count) { if (count > n) alloc(count); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr; n = 0;
  }
  size_t bytes() const { return n * sizeof(T); }
};

// ---------------------------------------------------------------------------
// Kernel launch wrappers (defined in the .hip files).
// ---------------------------------------------------------------------------
enum Epi : int {
  kEpiBias = 0,    // y = acc*s + b
  kEpiResid = 1,   // y = resid + (acc*s + b)
  kEpiSwiGLU = 2,  // columns (2n, 2n+1) = (gate n, up n): y[n] = silu(g)*u
  kEpiTotals = 3,  // limb GEMM only: write the exact int64 dot totals
  kEpiRope = 4     // QKV projection: RoPE on q and k, k and v into the cache
};

// Arguments of the kEpiRope epilogue: row m = b*S + s sits at position
// base[b] + off + s; columns [0, E) are q (rotated into qrot [rows][E]),
// [E, 2E) are k (rotated into the cache), [2E, 3E) are v (into the cache),
// E = H*D; cache rows [b][h][pos][D] with seq_stride floats per sequence.
// With an int8 cache (KVCache(true)) kq / vq / ks / vs are set instead of
// kc / vc: codes [b][h][pos][D] (seq_stride per sequence) and one scale per
// row [b][h][pos] (sc_stride per sequence); see rope_store_pair_q8.
struct RopeArgs {
  int S = 1, H = 1, D = 2, off = 0, cap = 0;
  const int32_t *base = nullptr, *active = nullptr;
  const float *cosb = nullptr, *sinb = nullptr;
  float *qrot = nullptr, *kc = nullptr, *vc = nullptr;
  int64_t seq_stride = 0;
  int8_t *kq = nullptr, *vq = nullptr;
  float *ks = nullptr, *vs = nullptr;
  int64_t sc_stride = 0;
};

// Cache position of row m of a RoPE epilogue: base[b] + off + s for row
// m = b*S + s, or -1 when the row is not written (inactive sequence,
// position outside the cache).
// The two reads (base[b], active[b]) and the arithmetic are separate steps
// so that a kernel can issue the reads early and form the position late.
struct RopeRow { int base, act, s; };
__device__ inline RopeRow rope_row_read(const RopeArgs &ra, int64_t m) {
  const int b = (int)(m / ra.S);
  // without an active mask base[b] is read twice, unconditionally, so that
  // nothing waits for the reads here
  const int32_t *ap = ra.active ? ra.active : ra.base;
  return RopeRow{ra.base[b], ap[b], (int)(m % ra.S)};
}
__device__ inline int rope_row_pos(const RopeArgs &ra, const RopeRow &r) {
  const int pos = r.base + ra.off + r.s;
  const bool act = !ra.active || r.act != 0;
  return !act || pos < 0 || pos >= ra.cap ? -1 : pos;
}
__device__ inline int rope_row_pos(const RopeArgs &ra, int64_t m) {
  return rope_row_pos(ra, rope_row_read(ra, m));
}

// Tensor::rope (tensor.cpp:1141-1173) on one pair (x_2j, x_2j+1) of output
// column n (even) of row m at cache position pos (>= 0), with the pair's
// cos / sin already read (unused for the v part), then the KV append of
// layer.cpp:758-807.  Each product and the sum are rounded on their own, as
// the reference's scalar code does (no fused multiply-add).
__device__ inline void rope_store_pair_at(const RopeArgs &ra, int64_t m,
                                          int pos, int n, float xe, float xo,
                                          float c, float sn) {
#pragma clang fp contract(off)
  const int b = (int)(m / ra.S);
  const int E = ra.H * ra.D;
  const int part = n / E, nn = n % E;
  const int h = nn / ra.D, j = (nn % ra.D) >> 1;
  if (part == 2) {
    float *vd = ra.vc + b * ra.seq_stride + ((int64_t)h * ra.cap + pos) * ra.D + 2 * j;
    vd[0] = xe; vd[1] = xo;
    return;
  }
  // (plain operators under contract(off): the _rn helpers are header
  // functions whose operations the compiler may still fuse)
  const float r0 = xe * c - xo * sn;
  const float r1 = xe * sn + xo * c;
  float *dst = part == 0
                   ? ra.qrot + m * E + nn
                   : ra.kc + b * ra.seq_stride + ((int64_t)h * ra.cap + pos) * ra.D + 2 * j;
  dst[0] = r0; dst[1] = r1;
}

// cos / sin of column n's pair at position pos (>= 0)
__device__ inline float2 rope_cos_sin(const RopeArgs &ra, int pos, int n) {
  const int nn = n % (ra.H * ra.D), j = (nn % ra.D) >> 1, half = ra.D >> 1;
  return make_float2(ra.cosb[(int64_t)pos * half + j], ra.sinb[(int64_t)pos * half + j]);
}

// rope_store_pair_at for row m, reading the row's position and the pair's
// cos / sin itself.
__device__ inline void rope_store_pair(const RopeArgs &ra, int64_t m, int n,
                                       float xe, float xo) {
  const int pos = rope_row_pos(ra, m);
  if (pos < 0) return;
  const bool vpart = n / (ra.H * ra.D) == 2;
  const float2 cs = vpart ? make_float2(0.f, 0.f) : rope_cos_sin(ra, pos, n);
  rope_store_pair_at(ra, m, pos, n, xe, xo, cs.x, cs.y);
}

// The KV append into an int8 cache from an epilogue whose lanes hold the
// D/2 pairs of one (row, head) on D/2 consecutive lanes, aligned (D a power
// of two <= 64); every lane of such a group calls this together.  q pairs
// are rotated and stored as rope_store_pair does; k pairs (after RoPE) and
// v pairs are quantised as quantize_kv does (layer.cpp:635-657): scale =
// max|x| over the row / 127 (1 when 0), code = clamp(round(x * (1 /
// scale)), +-127), the same operations as rope_kv_q8_kernel.
__device__ inline void rope_store_pair_q8(const RopeArgs &ra, int64_t m, int n,
                                          float xe, float xo) {
#pragma clang fp contract(off)
  const int pos = rope_row_pos(ra, m);
  const int E = ra.H * ra.D;
  const int part = n / E, nn = n % E;
  const int h = nn / ra.D, j = (nn % ra.D) >> 1;
  float a = xe, b = xo;
  if (part != 2) {
    const float2 cs = pos >= 0 ? rope_cos_sin(ra, pos, n) : make_float2(0.f, 0.f);
    a = xe * cs.x - xo * cs.y;
    b = xe * cs.y + xo * cs.x;
  }
  if (part == 0) {
    if (pos >= 0) { float *q = ra.qrot + m * E + nn; q[0] = a; q[1] = b; }
    return;
  }
  float mx = fmaxf(fabsf(a), fabsf(b));
  for (int o = 1; o < ra.D / 2; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (pos < 0) return;
  float scale = mx / 127.0f;
  if (scale == 0.0f) scale = 1.0f;
  const float inv = 1.0f / scale;
  const float ca = fmaxf(-127.0f, fminf(127.0f, roundf(__fmul_rn(a, inv))));
  const float cb = fmaxf(-127.0f, fminf(127.0f, roundf(__fmul_rn(b, inv))));
  const int bq = (int)(m / ra.S);
  int8_t *dst = (part == 1 ? ra.kq : ra.vq) + bq * ra.seq_stride +
                ((int64_t)h * ra.cap + pos) * ra.D + 2 * j;
  dst[0] = (int8_t)ca;
  dst[1] = (int8_t)cb;
  if (j == 0)
    (part == 1 ? ra.ks : ra.vs)[bq * ra.sc_stride + (int64_t)h * ra.cap + pos] = scale;
}

// whether an epilogue can append to an int8 cache in place: each head's
// pairs on an aligned group of D/2 lanes, within a wave
__host__ __device__ inline bool rope_q8_head_dim_ok(int D) {
  return D >= 2 && D <= 64 && (D & (D - 1)) == 0;
}

// Activation limbs for the int8 MFMA GEMM: x[m][k] ~= X[m][k] * 2^-e[m] with
// X = hi*65536 + mid*256 + lo, each digit an int8.
static constexpr int kLimbs = 3;
static constexpr int kLimbBits = 22;  // |X| < 2^22

// The MFMA GEMMs' common epilogue steps, shared so that every kernel that
// forms the same integer total writes the same float.
// Dequantisation of an exact dot total of row digits (exponent e) and int8
// codes: tot * 2^-e * scale + bias, product and sum in one rounding.
__device__ inline float dequant_epilogue(long long tot, int e, float sc, float bi) {
  return fmaf(ldexpf((float)tot, -e), sc, bi);
}
// SwiGLU::forward (layer.cpp:1704-1710) on one (gate, up) pair:
// (g * sigmoid(g)) * u, sigmoid = 1 / (1 + exp(-g)) (cpu_backend.cpp:483-489).
__device__ inline float swiglu_pair(float g, float u) {
  const float sg = 1.0f / (1.0f + expf(-g));
  const float a = __fmul_rn(g, sg);
  return __fmul_rn(a, u);
}

// MFMA operand layout of an int8 [R][K] matrix (R % 32 == 0, K % 128 == 0):
// element (m, k) lives at
//   [m/32][k/128][(k%128)/32][lane = ((k%32)/16)*32 + m%32][k%16],
// so the 16 bytes one lane feeds to one v_mfma_i32_32x32x32_i8 step are
// contiguous, a wave's 64 lanes read one contiguous 1 KB block, and step s
// of a 128-wide chunk contracts the 32 consecutive k of [32 s, 32 s + 32)
// (two steps cover one 64-wide attention head).  Used for the weight codes
// of the MFMA path and for the activation digits (one plane of R*K bytes
// per digit).
__host__ __device__ inline int64_t mfma_operand_offset(int m, int k, int K) {
  const int nch = K / 128;
  const int c = k >> 7, kk = k & 127;
  const int h = (kk >> 4) & 1, s = kk >> 5, byte = kk & 15;
  const int lane = h * 32 + (m & 31);
  return ((((int64_t)(m >> 5) * nch + c) * 4 + s) * 64 + lane) * 16 + byte;
}

// X = rint(x * 2^e) split into balanced base-256 digits, returned packed
// four per int for 4 consecutive x as (hi, mid, lo).
__device__ inline int3 digits4(const float *x, int e) {
  int hi = 0, mid = 0, lo = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int X = (int)rintf(ldexpf(x[i], e));
    const int l = (int)(int8_t)(X & 0xff);
    const int t = (X - l) >> 8;
    const int md = (int)(int8_t)(t & 0xff);
    const int h = (t - md) >> 8;
    lo |= (l & 0xff) << (8 * i);
    mid |= (md & 0xff) << (8 * i);
    hi |= (h & 0xff) << (8 * i);
  }
  return make_int3(hi, mid, lo);
}

// Row exponent e = 22 - exponent(max|x|) (0 for an all-zero row).
__device__ inline int digit_exponent(float mx) {
  int e = 0;
  if (mx > 0.f) {
    int ex;
    (void)frexpf(mx, &ex);
    e = kLimbBits - ex;
  }
  return e;
}

// linear.hip
extern int g_accept_split;  // 1 = the accept step's draw spread over
                            // kDrawChunks workgroups per sequence
extern int g_accept_early;  // 1 = nnhip_spec_accept forms row statistics only up
                            // to each sequence's first rejection
extern int g_gemv16;     // 1 = int8 GEMVs with 128-bit code loads (gemv16_kernel)
extern int g_gemm_wide;  // GEMM tile choice (1 = 32x64 tiles allowed)
extern int g_limb_k8;    // digit-plane GEMM: 8 waves split K from this K on
// engine.hip
extern int g_lds_min_rows;  // the LDS-resident GEMM from this many rows on
// workgroups of the LDS GEMM resident at once (one per CU of an MI355X)
constexpr int kGemmSlots = 256;
extern int g_attn_waves; // attention: waves one launch aims for
extern int g_ln_split;   // LayerNorm rows of 512 / 1024 over 2 / 4 waves
extern int g_attn_short_q; // attention: queries per workgroup in a launch of
                           // few (sequence, head) pairs (1, 2, 4 or 8)
extern int g_attn_w4;    // attention: 4-wave merged workgroups for 4+ queries
                         // (1: launches of >= 128 workgroups, 2: always)
extern int g_persistent_draft; // 1 = short batches run their decoder layers as
                               // one persistent kernel (draft_layers.hip);
                               // 0 (default): the per-kernel path
extern int g_gemv_down_rows; // down projection on the GEMV up to this many rows
extern int g_gemv_ln;    // a GEMV over LN(h) of up to this many rows (default
                         // 2) forms the LayerNorm in its prologue; more rows
                         // get a LayerNorm launch before it
extern int g_o_head_digits; // 1 = the merged attention writes the output
                            // projection's digits per head (64-wide heads)
extern int g_o_limb_rows; // output projection after merged attention: digit
                          // planes + digit-plane GEMM up to this many rows
extern int g_kv_stream;  // attention: non-temporal fp32 KV loads (0 never,
                         // 1 when a launch reads more than the L2s hold, 2 always)
// workgroups of one LDS-GEMM launch (32-row tiles x column blocks of
// 32 * 16 / min(4, K/128) columns)
inline int64_t gemm_lds_workgroups(int rows, int K, int N) {
  const int nch = K / 128, nc = 32 * 16 / (nch < 4 ? nch : 4);
  return (int64_t)((rows + 31) / 32) * ((N + nc - 1) / nc);
}
// Source of the activation digits of the LDS-resident GEMM.
enum AFrom { kAFromDigits = 0, kAFromRows = 1, kAFromLayerNorm = 2 };
inline bool gemm_lds_supports(int rows, int K, int N) {
  return rows > 0 && (K == 128 || K == 256 || K == 512 || K == 1024) &&
         N >= 32 && N % 32 == 0;
}
// Reductions over a whole wave that every lane receives: DPP row rotations
// by 1, 2, 4, 8 within each row of 16 lanes, then the four rows' values read
// from lanes 0, 16, 32, 48 (no LDS permutes).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_max_all(float v) {
  v = fmaxf(v, dpp_f<0x121>(v));
  v = fmaxf(v, dpp_f<0x122>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x128>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum_all(float v) {
  v += dpp_f<0x121>(v);
  v += dpp_f<0x122>(v);
  v += dpp_f<0x124>(v);
  v += dpp_f<0x128>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ int wave_min_all(int v) {
  v = min(v, dpp_i<0x121>(v));
  v = min(v, dpp_i<0x122>(v));
  v = min(v, dpp_i<0x124>(v));
  v = min(v, dpp_i<0x128>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Softmax statistics of the lm head's logits per (row, column tile), written
// by the LDS GEMM's epilogue: for T > 0 tile t of row m gets
// out[m * ld + t] = (max_i s_i, sum_i exp(s_i - max)) with s = l / T (l when
// T == 1); for T <= 0 (max_i l_i, first index of the max as int bits).
// Tiles are the GEMM's column blocks, gemm_lds_tile_width(K) wide.
struct TileStatsArgs {
  float2 *out = nullptr;
  int64_t ld = 0;
  float T = 1.f;
};
// Column width of a tile of statistics, or 0 when the LDS GEMM cannot form
// them for this K (its column block must be one wave's 128 columns).
int gemm_lds_tile_width(int K);
void launch_gemm_lds(hipStream_t st, int mode, const int8_t *limbs, int mpad,
                     const int *rexp, const float *x, int64_t ldx,
                     const float *lng, const float *lnb, float *ln_out,
                     int64_t ldo, int rows, int K, int N, const int8_t *wq,
                     const float *scale, const float *bias,
                     const float *resid, int64_t ldr, float *y, int64_t ldy,
                     int epi, const RopeArgs *ra = nullptr,
                     const TileStatsArgs *ts = nullptr);
// A LayerNorm folded into the GEMV's input rows (launch_gemv): gamma g,
// beta b over the K entries of each row; the normalised rows go to out
// (stride ldo) when out is set.
struct GemvLn {
  const float *g = nullptr, *b = nullptr;
  float *out = nullptr;
  int64_t ldo = 0;
};
void launch_gemv(hipStream_t st, const float *x, int64_t ldx, int rows, int K,
                 int N, const int8_t *wq, const float *wf, const float *scale,
                 const float *bias, const float *resid, int64_t ldr, float *y,
                 int64_t ldy, int epi, const RopeArgs *ra = nullptr,
                 const GemvLn *ln = nullptr);
void launch_act_quant(hipStream_t st, const float *x, int64_t ldx, int rows,
                      int K, int8_t *limbs, int mpad, int *rexp);
bool gemm_limb_q8_ok(int D);
void launch_gemm_limb(hipStream_t st, const int8_t *limbs, int mpad,
                      const int *rexp, int rows, int K, int N,
                      const int8_t *wq, const float *scale, const float *bias,
                      const float *resid, int64_t ldr, float *y, int64_t ldy,
                      int epi, const RopeArgs *ra = nullptr);
// the same GEMM over digit planes with one exponent per 64-wide K chunk
// (hexp [rows][K/64], as the merged attention writes them; K <= 2048), bias
// or residual epilogue
constexpr int kMaxHxChunks = 32;
void launch_gemm_limb_hx(hipStream_t st, const int8_t *limbs, int mpad,
                         const int *hexp, int rows, int K, int N,
                         const int8_t *wq, const float *scale, const float *bias,
                         const float *resid, int64_t ldr, float *y, int64_t ldy,
                         int epi);
// QuantizedDense ctor (quantization.cpp:36-86) on rows of w [N][K]: one
// scale per row = max|w| / max_q (1 when 0), codes clamp(round(w / scale),
// +-max_q) one per byte; max_q 127 (bits 8, INT8) or 7 (bits 4, INT4)
void launch_quantize_w8(hipStream_t st, const float *w_nk, int N, int K,
                        int8_t *q_nk, float *scales, int bits = 8);
// row-major int8 [R][K] <-> MFMA operand layout (R % 32, K % 128 == 0)
void launch_swizzle_rows(hipStream_t st, const int8_t *src, int R, int K,
                         int8_t *dst, bool inverse);
void launch_transpose_into(hipStream_t st, const float *src_kn, int K, int N,
                           float *dst, int64_t row_base, int64_t row_stride);
void launch_transpose_out(hipStream_t st, const float *src, int K, int N,
                          int64_t row_base, int64_t row_stride, float *dst_kn);
void launch_init_normal(hipStream_t st, float *dst, int K, int N,
                        int64_t row_base, int64_t row_stride, uint64_t seed,
                        uint32_t param, float stdv, int transposed);
void launch_fill(hipStream_t st, float *p, int64_t n, float v);

// attention.hip
void launch_embed(hipStream_t st, const float *emb, int vocab, int d,
                  const int32_t *ids, int rows, float *x);
// row (b, s) takes ids[b*stride_b + s]; with lead, lead[b] for s = 0 and
// ids[b*stride_b + s - 1] after it
void launch_embed_strided(hipStream_t st, const float *emb, int vocab, int d,
                          const int32_t *ids, int B, int S, int stride_b,
                          float *x, int8_t *limbs = nullptr, int mpad = 0,
                          int *rexp = nullptr, const int32_t *lead = nullptr);
// qkv rows [q: H heads | k: Hkv heads | v: Hkv heads] (Hkv 0: H); the
// cache holds Hkv heads per sequence
void launch_rope_kv(hipStream_t st, const float *qkv, int B, int S, int H,
                    int D, const int32_t *base, int off, const int32_t *active,
                    const float *cosb, const float *sinb, float *qrot,
                    float *kc, float *vc, int cap, int64_t seq_stride,
                    int Hkv = 0);
// RoPE on q and k, then the append into an int8 cache: each new k / v row
// (one head, one position) is quantised as quantize_kv does
// (layer.cpp:635-657); codes [B][H][cap][D] (seq_stride codes per
// sequence), scales [B][H][cap] (sc_stride per sequence).
void launch_rope_kv_q8(hipStream_t st, const float *qkv, int B, int S, int H,
                       int D, const int32_t *base, int off,
                       const int32_t *active, const float *cosb,
                       const float *sinb, float *qrot, int8_t *kq, float *ks,
                       int8_t *vq, float *vs, int cap, int64_t seq_stride,
                       int64_t sc_stride);
// K / V rows an attention launch reads: fp32 rows, or int8 codes with one
// fp32 scale per (head, position) row (KVCache(quantized=true),
// layer.hpp:212-230).  Rows [B][Hkv][cap][D], seq_stride elements apart
// per sequence; scales [B][Hkv][cap], sc_stride apart.
struct KvSrc {
  const void *k = nullptr, *v = nullptr;
  const float *ks = nullptr, *vs = nullptr;
  int64_t seq_stride = 0, sc_stride = 0;
  bool q8 = false;
};
// true when launch_attention writes the context rows without the combine
// kernel (and so without digit planes)
bool attention_merged(int D, int max_keys);
// returns whether the digit planes (one exponent per row, rexp) were
// written; with hexp the merged attention writes the rows' digit planes with
// one exponent per (row, head) instead, hexp [rows][H] (D == 64)
bool launch_attention(hipStream_t st, const float *q, const KvSrc &kv, int B,
                      int S, int H, int Hkv, int D, int cap,
                      const int32_t *base, int off, const int32_t *active,
                      int max_keys, float *part, int64_t part_elems,
                      float *out, int8_t *limbs = nullptr, int mpad = 0,
                      int *rexp = nullptr, int *hexp = nullptr);
int64_t attention_partial_elems(int B, int S, int H, int D, int max_keys);
void launch_layernorm(hipStream_t st, const float *h, int rows, int d,
                      const float *g, const float *b, float *y,
                      int8_t *limbs, int mpad, int *rexp);

// tensor_ops.hip: strided fp32 operands of the ExecutionBackend ops
// (include/backend/backend.hpp:35-206): element offset, shape and strides
// in elements, up to kMaxRank dimensions.
constexpr int kMaxRank = 8;
struct TensorView {
  void *data = nullptr;
  int64_t offset = 0;
  int rank = 0;
  int64_t shape[kMaxRank] = {};
  int64_t strides[kMaxRank] = {};
};
enum TensorOp : int {
  // binary: out = f(a, b)
  kOpAdd = 0, kOpSub = 1, kOpMul = 2, kOpDiv = 3,
  // binary backward: grad_in = f(forward input or output, grad_out)
  kOpReluBack = 4, kOpSigmoidBack = 5, kOpTanhBack = 6, kOpSqrtBack = 7,
  kOpLogBack = 8,
  // unary: out = f(in)
  kOpRelu = 16, kOpSigmoid = 17, kOpTanh = 18, kOpSqrt = 19, kOpLog = 20
};
void launch_binary(hipStream_t st, int op, const TensorView &a,
                   const TensorView &b, const TensorView &out);
void launch_unary(hipStream_t st, int op, const TensorView &in,
                  const TensorView &out);
void launch_matmul(hipStream_t st, const TensorView &a, const TensorView &b,
                   const TensorView &out);
void launch_sum(hipStream_t st, const TensorView &in, const TensorView &out,
                const int64_t *axes, int naxes);
void launch_softmax(hipStream_t st, const TensorView &in, const TensorView &out,
                    int axis);
void launch_softmax_backward(hipStream_t st, const TensorView &y,
                             const TensorView &dy, const TensorView &dx,
                             int axis);
void launch_embedding(hipStream_t st, const TensorView &w, const TensorView &ids,
                      const TensorView &out);
void launch_slice_backward(hipStream_t st, const TensorView &gs,
                           const TensorView &gp, int axis, int64_t index);

// sampling.hip
// floats per verify row of SpecState::tstat
constexpr int kTstat = 6;
// int64 counters per sequence of SpecState::stats
constexpr int kSpecStats = 8;
// the split accept step (launch_accept with g_accept_split): int32 words of
// a sequence's record, and vocabulary chunks of the draw
constexpr int kAcceptRec = 8;
constexpr int kDrawChunks = 16;
// largest lookahead k of the speculative loop
constexpr int kMaxLookahead = 63;
// std::mt19937 streams (SpecState::mt): words of the engine's state, outputs
// a sequence's ring holds, and the fewest unread outputs a launch leaves
// before it appends the next 624 (a cycle reads at most 3k + 2 <= 191)
constexpr int kMtN = 624;
constexpr int kMtRing = 1024;
constexpr int kMtLow = kMtRing - kMtN;
// whether get_probs filters with these options (layer.cpp:1452-1472)
inline bool sampling_filtered(int V, int top_k, float top_p) {
  return (top_k > 0 && top_k < V) || (top_p > 0.0f && top_p < 1.0f);
}
// Rows of the next forward that a sampling kernel embeds itself (the gather
// of embed_kernel, cpu_backend.cpp:1020-1025, with the rows' digits for the
// first q/k/v GEMM when limbs is set): row r of x takes emb[id] (ids outside
// [0, vocab) read row 0).  Unset (x null): the forward gathers them.
struct NextRows {
  const float *emb = nullptr;
  int vocab = 0, d = 0;
  float *x = nullptr;
  int8_t *limbs = nullptr;
  int mpad = 0;
  int *rexp = nullptr;
};
struct SpecState {
  int32_t *cur;        // [B] last committed token (generated.back())
  int32_t *cand;       // [B][k] draft candidates of this cycle
  float *qprob;        // [B][k][V] draft probabilities (sampled mode), or
                       // null when qlog is set
  // the drafting steps' logits [k][B][V] (step j, sequence b at row
  // j*B + b): with the lm head's tile statistics (dtiles) they give every
  // draft probability, which is then computed where it is needed instead
  // of being written out at each step (sampled mode without top-k / top-p)
  const float *qlog = nullptr;
  // row of step j, sequence b in qlog: qlog + j*qlog_js + b*qlog_bs (0: the
  // loop's [k][B][V] layout, js = B*V, bs = V)
  int64_t qlog_js = 0, qlog_bs = 0;
  float *tstat;        // [B][k+1][kTstat] verify-row statistics (accept)
  int32_t *tlen;       // [B] target cache length
  int32_t *dlen;       // [B] draft cache length
  int32_t *gen;        // [B] tokens generated so far
  int32_t *cyc;        // [B] cycle counter (1-based) for the uniform stream
  int32_t *active;     // [B] 1 while gen < max_new
  int32_t *catchup;    // [B] 1 when the draft needs a catch-up forward
  int32_t *catch_tok;  // [B] token of that catch-up forward
  int32_t *pair;       // [B][2] {catch_tok, cur}: ids of the next cycle's
                       // first draft forward
  int32_t *out;        // [B][out_stride] prompt + generated ids
  int32_t *n_active;   // [1]
  // [1] active sequences that cannot finish within one more cycle (more than
  // k + 1 tokens to go), or null: the host stops launching cycles once the
  // ones it has launched are sure to finish every sequence
  int32_t *n_far = nullptr;
  int64_t *stats;      // [B][kSpecStats] cycles, drafted, accepted, ties,
                       // resampled, bonus, and the largest target / draft
                       // cache lengths the reference's forwards reach
                       // (S_past + S of layer.cpp:1171-1179)
  const float2 *dtiles;  // [B][k][nt] draft lm-head tile statistics
                         // (TileStatsArgs) of the cycle's steps, or null
  int nt, tw;            // tiles per row, tile width
  int B, out_stride, P, max_new, k, V;
  float T;
  int top_k;             // get_probs filters (layer.cpp:1447-1489): top_k in
  float top_p;           // (0, V) and top_p in (0, 1) are active
  uint64_t seed;
  uint32_t seq0;       // global index of sequence 0 (Philox key part)
  int trows = 0;       // verify rows per sequence in tlogits (0: k + 1)
  // explicit accept / final uniforms ([B][k] and [B]) instead of the
  // Philox slots k + j and 2k (nnhip_spec_accept); null in the loop
  const float *ua = nullptr, *ur = nullptr;
  // when set, accept_kernel also writes each sequence's accepted count and
  // its resampled / bonus token (-1 when none)
  int32_t *n_acc_out = nullptr, *tok_out = nullptr;
  // [B] lowest position whose candidate is certainly rejected, or null: the
  // row statistics skip the rows after it (accept_rows_stats_kernel)
  int32_t *minrej = nullptr;
  // with minrej: [B][k+1] workgroups of a row done, and the verify rows'
  // tile statistics [B][k+1][nt] (accept_tiles_kernel)
  int32_t *rowcnt = nullptr;
  float2 *ttiles = nullptr;
  // the split accept step's scratch: [B][kAcceptRec] records and
  // [B][kDrawChunks][2] chunk sums (null: one accept_kernel per sequence)
  int32_t *rec = nullptr;
  double *chunks = nullptr;
  // The reference's generator (layer.cpp:1249, 1394: one std::mt19937 per
  // call, seeded with the seed; here sequence b's engine is seeded with
  // seed + seq0 + b): per sequence the engine's state [B][kMtN], a ring of
  // its tempered outputs [B][kMtRing] and the {read, write} counters
  // [B][2].  A cycle's launches read ahead of the read counter in the
  // reference's order -- the M drafting draws (two outputs each), the
  // accept tests up to the first rejection (one each), then the resample or
  // bonus draw (two) -- and the accept step advances it by what was used.
  // Null: the Philox stream (uniform()).
  uint32_t *mt = nullptr, *mt_ring = nullptr, *mt_rw = nullptr;
  // when nd is set, drafting steps j < k - 1 embed their token as row b of
  // the next draft forward
  NextRows nd;
};
// seeds SpecState::mt of every sequence and fills its ring with the first
// 624 outputs (read counter 0)
void launch_mt_seed(hipStream_t st, const SpecState &s);
void launch_first_token(hipStream_t st, const SpecState &s,
                        const float *logits, int64_t ldl);
void launch_draft_sample(hipStream_t st, const SpecState &s, int j,
                         const float *logits, int64_t ldl);
void launch_accept(hipStream_t st, const SpecState &s, const float *tlogits);
// drafting step j from the draft lm head's tile statistics (s.dtiles)
void launch_draft_sample_tiles(hipStream_t st, const SpecState &s, int j,
                               const float *logits, int64_t ldl);
void launch_ar_sample(hipStream_t st, const SpecState &s, int step,
                      const float *logits, int64_t ldl);
void launch_sample_rows(hipStream_t st, const float *logits, int B, int V,
                        float T, const float *u, int32_t *tok, float *probs,
                        int top_k = 0, float top_p = 1.f);
void launch_add_scalar(hipStream_t st, int32_t *p, int n, int v);
// The speculative loop's accept step (target_stats_kernel + accept_kernel)
// over given rows: B sequences that each drafted k candidates, target
// logits [B][k][V] (no bonus row), draft probabilities [B][k][V] as the
// drafting steps form them (get_probs), explicit uniforms ua [B][k] and
// ur [B].  Writes n_acc [B] and tok [B] (resampled id, or -1 when all k
// are accepted).  The sequence state is reset by each launch.
struct AcceptRows {
  DevBuf<int32_t> cur, tlen, dlen, gen, cyc, active, catchup, catch_tok, pair,
      out, n_active;
  DevBuf<float> tstat;
  DevBuf<float2> dtiles;   // [B][k][nt] draft-row tile statistics
  DevBuf<int32_t> minrej;  // [B] first certain rejection (early exit)
  DevBuf<int32_t> rowcnt;  // [B][k+1] workgroups done per row (early exit)
  DevBuf<float2> ttiles;   // [B][k+1][nt] verify-row tile statistics
  DevBuf<int32_t> rec;     // split accept step: records and chunk sums
  DevBuf<double> chunks;
  DevBuf<int64_t> stats;
  SpecState s;
  AcceptRows(int B, int k, int V, float T);
  // from draft probabilities qprob [B][k][V] (null in greedy mode)
  void launch(hipStream_t st, const float *tlogits, const float *qprob,
              const int32_t *cand, const float *ua, const float *ur,
              int32_t *n_acc, int32_t *tok);
  // from draft logits dlogits [B][k][V]: their 128-column tile statistics
  // (launch_row_tile_stats), then the accept step forms each draft
  // probability it reads from the logit and the row's statistics, as the
  // loop's drafting steps leave them (SpecState::qlog)
  void launch_logits(hipStream_t st, const float *tlogits,
                     const float *dlogits, const int32_t *cand, const float *ua,
                     const float *ur, int32_t *n_acc, int32_t *tok);
  // the split accept step's scratch into a (g_accept_split)
  void attach_split(SpecState &a);
};
// Softmax statistics per 128-column tile of each row of logits [rows][V]
// (rows ldl apart), the TileStatsArgs values the LDS GEMM's lm-head epilogue
// forms: out[r * nt + t] = (max s, sum exp(s - max)) over the tile's
// columns, s = l / T (T > 0), or (max l, first index of the max) (T <= 0);
// nt = ceil(V / 128).
void launch_row_tile_stats(hipStream_t st, const float *logits, int64_t ldl,
                           int rows, int V, float T, float2 *out);

// ---------------------------------------------------------------------------
// The decoder layers of a short batch as one persistent kernel
// (draft_layers.hip): per-layer weights and caches, the forward's rows and
// positions, and the kernel's own state (a ring of stage outputs, one flag
// word per workgroup, an error word).
// ---------------------------------------------------------------------------
constexpr int kPdMaxLayers = 8;
constexpr int kPdFlagSlot = 1024;       // tile flags per (layer, step)
struct PdLayer {
  const int8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wdn = nullptr;  // codes [N][K]
  const float *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sdn = nullptr;   // scales [N]
  const float *bqkv = nullptr, *bo = nullptr, *bgu = nullptr, *bdn = nullptr;   // biases [N]
  const float *g1 = nullptr, *b1 = nullptr, *g2 = nullptr, *b2 = nullptr;       // LayerNorms
  float *kc = nullptr, *vc = nullptr;   // fp32 cache of the layer, [B][H][cap][D]
};
struct PdArgs {
  int R = 0, S = 1, B = 0, d = 0, H = 0, D = 0, F = 0, L = 0, cap = 0, off = 0;
  int64_t seq_stride = 0;               // H * cap * D
  const float *x0 = nullptr;            // [R][d] the layer-0 input rows
  const int32_t *base = nullptr;        // [B] position of row (b, 0) is base[b] + off
  const int32_t *active = nullptr;      // [B] or null: 0 = the sequence is skipped
  const float *cosb = nullptr, *sinb = nullptr;  // RoPE tables [rope_len][D/2]
  float *out = nullptr;                 // [R][d] the last layer's output before LN2
  float *ring = nullptr;                // L * pd_ring_layer_floats floats
  unsigned *flags = nullptr;            // one word per workgroup: its launches
  unsigned *tflags = nullptr;           // [L][5][kPdFlagSlot] tile done flags
  int *err = nullptr;                   // set when a wait timed out
  PdLayer ly[kPdMaxLayers];
};
__host__ __device__ inline int64_t pd_ring_layer_floats(int R, int d, int F) {
  return (int64_t)R * (6 * d + F);
}
bool draft_layers_supported(int d, int H, int F, int L, int R, int cap);
void launch_draft_layers(hipStream_t st, const PdArgs &a, int nwg);

}  // namespace nnhip

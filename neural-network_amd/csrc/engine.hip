// Host engine of libnnhip.so (see engine.hpp).
#include "engine.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>

namespace nnhip {

int g_lds_min_rows = 128;
int g_o_limb_rows = 256;
int g_persistent_draft = 0;
int g_gemv_down_rows = 64;
int g_o_head_digits = 1;
int g_gemv_ln = 2;

namespace {

constexpr int kLimbMinRows = 16;
constexpr int64_t kFusedNormMaxBlocks = 768;

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Table of RoPE factors for positions [0, max_seq) by the float formula of
// Tensor::rope (tensor.cpp:1147-1153): theta = pow(10000, -2j/D),
// omega = pos * theta, cos/sin(omega).
void rope_tables(int max_seq, int D, std::vector<float> &c,
                 std::vector<float> &s) {
  const int half = D / 2;
  c.resize((size_t)max_seq * half);
  s.resize((size_t)max_seq * half);
  for (int p = 0; p < max_seq; ++p) {
    const float m = (float)p;
    for (int j = 0; j < half; ++j) {
      const float theta =
          std::pow(10000.0f, -2.0f * (float)j / (float)D);
      const float omega = m * theta;
      c[(size_t)p * half + j] = std::cos(omega);
      s[(size_t)p * half + j] = std::sin(omega);
    }
  }
}

struct ParamRef {
  enum Kind { kEmb, kWeight, kBias, kVec } kind;
  Linear *lin = nullptr;
  DevBuf<float> *vec = nullptr;
  int K = 0, N = 0;           // logical [K][N] (reference layout)
  int64_t row_base = 0, row_stride = 1;
};

}  // namespace

void Linear::init(int k, int n) {
  K = k; N = n;
  w.alloc((size_t)N * K);
  b.alloc(N);
  s.alloc(N);
  quant = false;
}

Model::Model(Ctx *c, int vocab, int d_model, int heads, int d_ff,
             int n_layers, int max_seq_len)
    : ctx(c), V(vocab), d(d_model), H(heads), D(d_model / heads), F(d_ff),
      L(n_layers), max_seq(max_seq_len) {
  NNHIP_REQUIRE(vocab > 0 && d_model > 0 && heads > 0 && d_ff > 0 &&
                    n_layers > 0 && max_seq_len > 0,
                kErrArg, "decoder: sizes must be positive");
  NNHIP_REQUIRE(d_model % heads == 0, kErrArg,
                "embed_dim must be divisible by num_heads");
  NNHIP_REQUIRE(D % 8 == 0 && D <= 64, kErrUnsupported,
                "head dim must be a multiple of 8 and at most 64");
  NNHIP_REQUIRE(d % 4 == 0 && F % 4 == 0 && d <= 4096 && F <= 4096, kErrUnsupported,
                "d_model and d_ff must be multiples of 4 and at most 4096");
  hipStream_t st = ctx->stream;
  emb.alloc((size_t)V * d);
  layers.resize(L);
  for (auto &ly : layers) {
    ly.qkv.init(d, 3 * d);
    ly.o.init(d, d);
    ly.gu.init(d, 2 * F);
    ly.down.init(F, d);
    ly.g1.alloc(d); ly.b1.alloc(d); ly.g2.alloc(d); ly.b2.alloc(d);
  }
  lm.init(d, V);
  init_normal(0, 0.0f);  // zero weights, zero biases, gamma 1, beta 0
  ensure_rope(max_seq);
  NNHIP_CHECK(hipStreamSynchronize(st));
}

void Model::ensure_rope(int n) {
  if (n <= rope_len) return;
  std::vector<float> hc, hs;
  rope_tables(n, D, hc, hs);
  hipStream_t st = ctx->stream;
  NNHIP_CHECK(hipStreamSynchronize(st));
  cosb.alloc(hc.size());
  sinb.alloc(hs.size());
  NNHIP_CHECK(hipMemcpyAsync(cosb.p, hc.data(), hc.size() * 4,
                             hipMemcpyHostToDevice, st));
  NNHIP_CHECK(hipMemcpyAsync(sinb.p, hs.data(), hs.size() * 4,
                             hipMemcpyHostToDevice, st));
  NNHIP_CHECK(hipStreamSynchronize(st));
  rope_len = n;
}

static ParamRef param_ref(Model &m, int idx) {
  ParamRef r{};
  const int last = 1 + 18 * m.L;
  NNHIP_REQUIRE(idx >= 0 && idx <= last + 1, kErrArg, "parameter index out of range");
  if (idx == 0) { r.kind = ParamRef::kEmb; r.K = m.V; r.N = m.d; return r; }
  if (idx == last) { r.kind = ParamRef::kWeight; r.lin = &m.lm; r.K = m.d; r.N = m.V; return r; }
  if (idx == last + 1) { r.kind = ParamRef::kBias; r.lin = &m.lm; r.K = 1; r.N = m.V; return r; }
  LayerW &ly = m.layers[(idx - 1) / 18];
  const int j = (idx - 1) % 18;
  const int d = m.d, F = m.F;
  switch (j / 2) {
    case 0: case 1: case 2:
      r.lin = &ly.qkv; r.K = d; r.N = d; r.row_base = (int64_t)(j / 2) * d; break;
    case 3: r.lin = &ly.o; r.K = d; r.N = d; break;
    case 4: r.lin = &ly.gu; r.K = d; r.N = F; r.row_base = 0; r.row_stride = 2; break;
    case 5: r.lin = &ly.gu; r.K = d; r.N = F; r.row_base = 1; r.row_stride = 2; break;
    case 6: r.lin = &ly.down; r.K = F; r.N = d; break;
    default: {
      DevBuf<float> *v4[4] = {&ly.g1, &ly.b1, &ly.g2, &ly.b2};
      r.kind = ParamRef::kVec; r.vec = v4[j - 14]; r.K = 1; r.N = d;
      return r;
    }
  }
  if (j % 2 == 0) r.kind = ParamRef::kWeight;
  else { r.kind = ParamRef::kBias; r.K = 1; }
  return r;
}

void Model::param_shape(int idx, int64_t *rows, int64_t *cols) const {
  ParamRef r = param_ref(const_cast<Model &>(*this), idx);
  *rows = r.K; *cols = r.N;
}

void Model::set_param(int idx, const float *host) {
  hipStream_t st = ctx->stream;
  ParamRef r = param_ref(*this, idx);
  const size_t n = (size_t)r.K * r.N;
  if (r.kind == ParamRef::kEmb || r.kind == ParamRef::kVec) {
    float *dst = r.kind == ParamRef::kEmb ? emb.p : r.vec->p;
    NNHIP_CHECK(hipMemcpyAsync(dst, host, n * 4, hipMemcpyHostToDevice, st));
    NNHIP_CHECK(hipStreamSynchronize(st));
    return;
  }
  DevBuf<float> stage(n);
  NNHIP_CHECK(hipMemcpyAsync(stage.p, host, n * 4, hipMemcpyHostToDevice, st));
  if (r.kind == ParamRef::kWeight)
    launch_transpose_into(st, stage.p, r.K, r.N, r.lin->w.p, r.row_base,
                          r.row_stride);
  else
    launch_transpose_into(st, stage.p, 1, r.N, r.lin->b.p, r.row_base,
                          r.row_stride);
  if (r.kind == ParamRef::kWeight && r.lin->quant) {
    launch_quantize_w8(st, r.lin->w.p, r.lin->N, r.lin->K, r.lin->q.p,
                       r.lin->s.p, bits);
    if (r.lin->qs.p)
      launch_swizzle_rows(st, r.lin->q.p, r.lin->N, r.lin->K, r.lin->qs.p,
                          false);
  }
  NNHIP_CHECK(hipStreamSynchronize(st));
}

void Model::get_param(int idx, float *host) const {
  hipStream_t st = ctx->stream;
  ParamRef r = param_ref(const_cast<Model &>(*this), idx);
  const size_t n = (size_t)r.K * r.N;
  if (r.kind == ParamRef::kEmb || r.kind == ParamRef::kVec) {
    const float *src = r.kind == ParamRef::kEmb ? emb.p : r.vec->p;
    NNHIP_CHECK(hipMemcpyAsync(host, src, n * 4, hipMemcpyDeviceToHost, st));
    NNHIP_CHECK(hipStreamSynchronize(st));
    return;
  }
  DevBuf<float> stage(n);
  if (r.kind == ParamRef::kWeight)
    launch_transpose_out(st, r.lin->w.p, r.K, r.N, r.row_base, r.row_stride,
                         stage.p);
  else
    launch_transpose_out(st, r.lin->b.p, 1, r.N, r.row_base, r.row_stride,
                         stage.p);
  NNHIP_CHECK(hipMemcpyAsync(host, stage.p, n * 4, hipMemcpyDeviceToHost, st));
  NNHIP_CHECK(hipStreamSynchronize(st));
}

// Seeded weights: Dense weights and the embedding N(0, std) (element (k, n)
// of parameter idx is a function of (seed, idx, k*N + n) only), biases 0,
// LayerNorm gamma 1 and beta 0 (layer.cpp:157-159, 203-209).
void Model::init_normal(uint64_t seed, float stdv) {
  hipStream_t st = ctx->stream;
  for (int idx = 0; idx < num_params(); ++idx) {
    ParamRef r = param_ref(*this, idx);
    switch (r.kind) {
      case ParamRef::kEmb:
        launch_init_normal(st, emb.p, r.K, r.N, 0, 1, seed, idx, stdv, 0);
        break;
      case ParamRef::kWeight:
        launch_init_normal(st, r.lin->w.p, r.K, r.N, r.row_base, r.row_stride,
                           seed, idx, stdv, 1);
        break;
      case ParamRef::kBias:
        launch_fill(st, r.lin->b.p, r.lin->N, 0.0f);
        break;
      case ParamRef::kVec: {
        const int j = (idx - 1) % 18;
        launch_fill(st, r.vec->p, r.N, (j == 14 || j == 16) ? 1.0f : 0.0f);
        break;
      }
    }
  }
  if (quantized) quantize(bits);
  NNHIP_CHECK(hipStreamSynchronize(st));
}

// quantize_model / MultiHeadAttention::quantize extended to the whole
// decoder: every Dense (q, k, v, o, gate, up, down, lm_head) becomes a
// symmetric per-output-channel QuantizedDense (quantization.cpp:7-87), INT8
// or INT4; the embedding stays fp32.  INT4 codes are held one per byte, as
// INT8 codes are: dequantize_weight gives both the same values (code *
// scale), so every kernel serves both.
void Model::quantize(int b) {
  hipStream_t st = ctx->stream;
  NNHIP_REQUIRE(b == 8 || b == 4, kErrUnsupported,
                "weight quantization: INT8 or INT4 only");
  bits = b;
  auto q = [&](Linear &ln) {
    if (!ln.q.p) ln.q.alloc((size_t)ln.N * ln.K);
    launch_quantize_w8(st, ln.w.p, ln.N, ln.K, ln.q.p, ln.s.p, bits);
    if (ln.K % 128 == 0 && ln.N % 64 == 0) {
      if (!ln.qs.p) ln.qs.alloc((size_t)ln.N * ln.K);
      launch_swizzle_rows(st, ln.q.p, ln.N, ln.K, ln.qs.p, false);
    }
    ln.quant = true;
  };
  for (auto &ly : layers) { q(ly.qkv); q(ly.o); q(ly.gu); q(ly.down); }
  q(lm);
  quantized = true;
  NNHIP_CHECK(hipStreamSynchronize(st));
}

void Model::get_quantized(int layer, int which, int8_t *codes_kn,
                          float *scales) const {
  NNHIP_REQUIRE(quantized, kErrArg, "model is not quantized");
  const Linear *ln;
  int64_t base = 0, stride = 1;
  int K = d, N = d;
  if (which == 7) { ln = &lm; N = V; }
  else {
    NNHIP_REQUIRE(layer >= 0 && layer < L && which >= 0 && which < 7, kErrArg,
                  "get_quantized: bad layer or index");
    const LayerW &ly = layers[layer];
    switch (which) {
      case 0: case 1: case 2: ln = &ly.qkv; base = (int64_t)which * d; break;
      case 3: ln = &ly.o; break;
      case 4: ln = &ly.gu; N = F; base = 0; stride = 2; break;
      case 5: ln = &ly.gu; N = F; base = 1; stride = 2; break;
      default: ln = &ly.down; K = F; break;
    }
  }
  std::vector<int8_t> all((size_t)ln->N * ln->K);
  std::vector<float> sc(ln->N);
  NNHIP_CHECK(hipMemcpy(all.data(), ln->q.p, all.size(), hipMemcpyDeviceToHost));
  NNHIP_CHECK(hipMemcpy(sc.data(), ln->s.p, sc.size() * 4, hipMemcpyDeviceToHost));
  for (int n = 0; n < N; ++n) {
    const int64_t row = base + (int64_t)n * stride;
    scales[n] = sc[row];
    for (int k = 0; k < K; ++k) codes_kn[(int64_t)k * N + n] = all[row * ln->K + k];
  }
}

void Model::reserve(int rows, int lrows, int max_keys) {
  Workspace &ws = wsp;
  if (rows > ws.rows) {
    const int r = std::max(rows, 64);
    ws.rows = r;
    ws.x.alloc((size_t)r * d); ws.qrot.alloc((size_t)r * d);
    ws.ctx.alloc((size_t)r * d); ws.h.alloc((size_t)r * d);
    ws.x1.alloc((size_t)r * d);
    ws.qkv.alloc((size_t)r * 3 * d);
    ws.ff.alloc((size_t)r * F);
    ws.mpad = round_up(r, 64);
    ws.limbs.alloc((size_t)kLimbs * ws.mpad * std::max(d, F));
    ws.rexp.alloc(ws.mpad);
    ws.hexp.alloc((size_t)ws.mpad * H);
    NNHIP_CHECK(hipMemsetAsync(ws.hexp.p, 0, ws.hexp.bytes(), ctx->stream));
    ws.ids.alloc(r);
    ws.zeros.alloc(r);
    NNHIP_CHECK(hipMemsetAsync(ws.zeros.p, 0, (size_t)r * 4, ctx->stream));
  }
  if (lrows > ws.lrows) {
    ws.lrows = lrows;
    ws.logits.alloc((size_t)lrows * V);
  }
  const int64_t pe = attention_partial_elems(1, rows, H, D, max_keys);
  if (pe > ws.part_elems) {
    ws.part.alloc(pe);
    ws.part_elems = pe;
  }
  // the persistent layer kernel's state for short batches, once the option
  // is on
  if (g_persistent_draft && rows > pd_rows && rows <= 64 &&
      draft_layers_supported(d, H, F, L, rows, 1)) {
    if (!pd_nwg) {
      int dev = 0, ncu = 0;
      NNHIP_CHECK(hipGetDevice(&dev));
      NNHIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
      pd_nwg = std::max(1, ncu);
      pd_flags.alloc(pd_nwg);
      pd_tflags.alloc((size_t)L * 5 * kPdFlagSlot);
      pd_err.alloc(1);
      NNHIP_CHECK(hipMemsetAsync(pd_flags.p, 0, pd_flags.bytes(), ctx->stream));
      NNHIP_CHECK(hipMemsetAsync(pd_tflags.p, 0, pd_tflags.bytes(), ctx->stream));
      NNHIP_CHECK(hipMemsetAsync(pd_err.p, 0, pd_err.bytes(), ctx->stream));
    }
    pd_rows = std::max(rows, 32);
    pd_ring.alloc((size_t)L * pd_ring_layer_floats(pd_rows, d, F));
  }
}

bool Model::use_pd(int rows, int S, const KVCache *kv) const {
  if (!(g_persistent_draft && quantized && kv && !kv->q8 && S >= 1 && S <= 2 &&
        rows <= pd_rows && pd_ring.p &&
        draft_layers_supported(d, H, F, L, rows, kv->cap)))
    return false;
  for (const auto &ly : layers)
    if (!ly.qkv.q.p || !ly.o.q.p || !ly.gu.q.p || !ly.down.q.p) return false;
  return true;
}

void Model::check_pd() {
  if (!pd_err.p) return;
  int e = 0;
  NNHIP_CHECK(hipMemcpy(&e, pd_err.p, 4, hipMemcpyDeviceToHost));
  if (!e) return;
  NNHIP_CHECK(hipMemset(pd_flags.p, 0, pd_flags.bytes()));
  NNHIP_CHECK(hipMemset(pd_tflags.p, 0, pd_tflags.bytes()));
  NNHIP_CHECK(hipMemset(pd_err.p, 0, pd_err.bytes()));
  NNHIP_CHECK(hipDeviceSynchronize());
  throw Error(kErrHip, "persistent decoder-layer kernel: a wait for another "
                       "workgroup's tile timed out (results of that forward are invalid)");
}

bool Model::use_limbs(const Linear &ln, int rows) const {
  return ln.quant && ln.qs.p && rows >= kLimbMinRows && ln.K % 128 == 0 &&
         ln.N % 64 == 0;
}

// Where the LDS-resident GEMM is used (measured on the batch-32 decode
// shapes): the lm head, and every projection with K <= 1024 on tall inputs
// (>= 128 rows: the verify batch), where one digit tile per 32 rows serves
// 128 columns.  Short inputs (the draft's 32 and 64 rows) run faster on the
// digit-plane GEMM.  A pending LayerNorm is folded into the GEMM prologue
// only for the lm head of a short batch; elsewhere the prologue's repeated
// per-column-block normalisation costs more than a LayerNorm launch.
bool Model::use_lds(const Linear &ln, int rows) const {
  if (!(ln.quant && ln.qs.p && rows >= kLimbMinRows &&
        gemm_lds_supports(rows, ln.K, ln.N)))
    return false;
  return &ln == &lm || rows >= g_lds_min_rows;
}

// whether linear_in folds a pending LayerNorm into the LDS GEMM's prologue
bool Model::norm_folds(const Linear &ln, int rows) const {
  return use_lds(ln, rows) && &ln == &lm && rows < g_lds_min_rows &&
         gemm_lds_workgroups(rows, ln.K, ln.N) <= kFusedNormMaxBlocks;
}

bool Model::lm_tiles(int rows) const {
  return use_lds(lm, rows) && gemm_lds_tile_width(lm.K) > 0;
}

void Model::linear_in(const Linear &ln, const float *x, int64_t ldx,
                      const PendingNorm *pn, int rows, bool limbs_ready,
                      const float *resid, int64_t ldr, float *y, int64_t ldy,
                      int epi, const RopeArgs *ra, const TileStatsArgs *ts) {
  hipStream_t st = ctx->stream;
  Workspace &ws = wsp;
  if (use_lds(ln, rows)) {
    // Each column block of a fused GEMM normalises and digitises its rows
    // again: only the short-batch lm head folds the norm in; elsewhere one
    // LayerNorm launch writes digit planes for the GEMM to copy.
    const bool fold = norm_folds(ln, rows);
    if (pn && !fold && pn->ldh == ln.K) {
      launch_layernorm(st, pn->h, rows, ln.K, pn->g, pn->b,
                       pn->out ? pn->out : ws.x.p, ws.limbs.p, ws.mpad,
                       ws.rexp.p);
      launch_gemm_lds(st, kAFromDigits, ws.limbs.p, ws.mpad, ws.rexp.p,
                      nullptr, 0, nullptr, nullptr, nullptr, 0, rows, ln.K,
                      ln.N, ln.qs.p, ln.s.p, ln.b.p, resid, ldr, y, ldy, epi,
                      ra, ts);
      return;
    }
    const int mode = pn ? kAFromLayerNorm
                        : (limbs_ready ? kAFromDigits : kAFromRows);
    launch_gemm_lds(st, mode, ws.limbs.p, ws.mpad, ws.rexp.p,
                    pn ? pn->h : x, pn ? pn->ldh : ldx, pn ? pn->g : nullptr,
                    pn ? pn->b : nullptr, pn ? pn->out : nullptr,
                    pn ? pn->ldo : 0, rows, ln.K, ln.N, ln.qs.p, ln.s.p,
                    ln.b.p, resid, ldr, y, ldy, epi, ra, ts);
    return;
  }
  NNHIP_REQUIRE(!ts || !ts->out, kErrArg,
                "linear_in: tile statistics need the LDS-resident GEMM");
  // short rows: the LayerNorm in the GEMV's prologue only up to g_gemv_ln
  // rows (every workgroup of the GEMV forms the rows' statistics again: for
  // the batch-1 draft's one or two rows that costs less than a launch, for
  // the verify step's five a LayerNorm launch before a plain GEMV measured
  // faster)
  if (pn && rows <= g_gemv_ln && !use_limbs(ln, rows) && ln.K <= 1024 &&
      ln.K % 4 == 0 && pn->ldh % 4 == 0 && (!pn->out || pn->ldo % 4 == 0)) {
    // short rows on the GEMV: the LayerNorm is its prologue
    GemvLn lf;
    lf.g = pn->g; lf.b = pn->b; lf.out = pn->out; lf.ldo = pn->ldo;
    launch_gemv(st, pn->h, pn->ldh, rows, ln.K, ln.N, ln.quant ? ln.q.p : nullptr,
                ln.quant ? nullptr : ln.w.p, ln.s.p, ln.b.p, resid, ldr, y, ldy,
                epi, ra, &lf);
    return;
  }
  if (pn) {
    // the normalisation as its own kernel, then the linear over its output
    NNHIP_REQUIRE(pn->out && pn->ldh == ln.K && pn->ldo == ln.K, kErrArg,
                  "linear_in: unfused LayerNorm needs contiguous rows");
    const bool lr = use_limbs(ln, rows);
    launch_layernorm(st, pn->h, rows, ln.K, pn->g, pn->b, pn->out,
                     lr ? ws.limbs.p : nullptr, ws.mpad, ws.rexp.p);
    linear(ln, pn->out, pn->ldo, rows, lr, resid, ldr, y, ldy, epi, ra);
    return;
  }
  linear(ln, x, ldx, rows, limbs_ready, resid, ldr, y, ldy, epi, ra);
}

void Model::linear(const Linear &ln, const float *x, int64_t ldx,
                   int rows, bool limbs_ready, const float *resid, int64_t ldr,
                   float *y, int64_t ldy, int epi, const RopeArgs *ra) {
  hipStream_t st = ctx->stream;
  Workspace &ws = wsp;
  if (use_limbs(ln, rows)) {
    if (!limbs_ready)
      launch_act_quant(st, x, ldx, rows, ln.K, ws.limbs.p, ws.mpad, ws.rexp.p);
    launch_gemm_limb(st, ws.limbs.p, ws.mpad, ws.rexp.p, rows, ln.K, ln.N,
                     ln.qs.p, ln.s.p, ln.b.p, resid, ldr, y, ldy, epi, ra);
  } else {
    launch_gemv(st, x, ldx, rows, ln.K, ln.N, ln.quant ? ln.q.p : nullptr,
                ln.quant ? nullptr : ln.w.p, ln.s.p, ln.b.p, resid, ldr, y,
                ldy, epi, ra);
  }
}

bool Model::emb_digits(int rows) const {
  return use_lds(layers[0].qkv, rows) || use_limbs(layers[0].qkv, rows);
}

NextRows Model::next_rows(int rows) const {
  NNHIP_REQUIRE(wsp.rows >= rows && d <= 4096, kErrArg,
                "next_rows: workspace not reserved, or d above 4096");
  NextRows n;
  n.emb = emb.p; n.vocab = V; n.d = d; n.x = wsp.x.p;
  n.limbs = emb_digits(rows) ? wsp.limbs.p : nullptr;
  n.mpad = wsp.mpad; n.rexp = wsp.rexp.p;
  return n;
}

void Model::forward(KVCache *cache, int b_off, const int32_t *ids,
                    int ids_stride, int B, int S, const int32_t *base, int off,
                    const int32_t *active, int max_keys, float *logits,
                    bool last_only, int64_t ldl, const TileStatsArgs *ts,
                    bool embedded, const int32_t *lead) {
  if (ldl == 0) ldl = V;
  hipStream_t st = ctx->stream;
  const int R = B * S;
  std::unique_ptr<KVCache> tmp;
  KVCache *kv = cache;
  if (!kv) {
    tmp.reset(new KVCache(this, B, S));
    kv = tmp.get();
    b_off = 0; base = nullptr; off = 0; active = nullptr; max_keys = S;
  }
  NNHIP_REQUIRE(b_off >= 0 && b_off + B <= kv->B, kErrArg,
                "forward: sequence range outside the cache");
  reserve(R, logits ? (last_only ? B : R) : 0, max_keys);
  Workspace &ws = wsp;
  const int32_t *bp = base ? base : ws.zeros.p;
  // Post-norm blocks (layer.cpp:1098-1113): each LayerNorm is applied by the
  // linear that consumes it (norm1 -> ffn gate/up, norm2 -> next q/k/v or
  // the lm head), which also writes the normalised rows for the residual.
  PendingNorm norm2;            // norm2 of the previous layer, if any
  bool have_norm2 = false;
  const bool pd = use_pd(R, S, kv);
  // the embedding kernel also writes the rows' digits for the first q/k/v
  // GEMM when that is an MFMA GEMM
  const bool emb_digits = !pd && this->emb_digits(R);
  if (!embedded)
    launch_embed_strided(st, emb.p, V, d, ids, B, S, ids_stride, ws.x.p,
                         emb_digits ? ws.limbs.p : nullptr, ws.mpad, ws.rexp.p,
                         lead);
  if (pd) {
    // every layer in one persistent kernel; its output is the last layer's
    // t2 before LN2, which the lm head applies
    PdArgs pa;
    pa.R = R; pa.S = S; pa.B = B; pa.d = d; pa.H = H; pa.D = D; pa.F = F;
    pa.L = L; pa.cap = kv->cap; pa.off = off;
    pa.seq_stride = kv->seq_stride();
    pa.x0 = ws.x.p; pa.base = bp; pa.active = active;
    pa.cosb = cosb.p; pa.sinb = sinb.p;
    pa.out = ws.h.p; pa.ring = pd_ring.p;
    pa.flags = pd_flags.p; pa.tflags = pd_tflags.p; pa.err = pd_err.p;
    for (int l = 0; l < L; ++l) {
      const LayerW &ly = layers[l];
      const KvSrc kvs = kv->src(l, b_off);
      PdLayer &p = pa.ly[l];
      p.wqkv = ly.qkv.q.p; p.wo = ly.o.q.p; p.wgu = ly.gu.q.p; p.wdn = ly.down.q.p;
      p.sqkv = ly.qkv.s.p; p.so = ly.o.s.p; p.sgu = ly.gu.s.p; p.sdn = ly.down.s.p;
      p.bqkv = ly.qkv.b.p; p.bo = ly.o.b.p; p.bgu = ly.gu.b.p; p.bdn = ly.down.b.p;
      p.g1 = ly.g1.p; p.b1 = ly.b1.p; p.g2 = ly.g2.p; p.b2 = ly.b2.p;
      p.kc = (float *)kvs.k; p.vc = (float *)kvs.v;
    }
    launch_draft_layers(st, pa, pd_nwg);
    norm2.h = ws.h.p; norm2.ldh = d;
    norm2.g = layers[L - 1].g2.p; norm2.b = layers[L - 1].b2.p;
    norm2.out = ws.x.p; norm2.ldo = d;
    have_norm2 = true;
  }
  for (int l = 0; l < (pd ? 0 : L); ++l) {
    LayerW &ly = layers[l];
    const KvSrc kvs = kv->src(l, b_off);
    // the int8 append runs in the LDS GEMM's epilogue (each head's pairs on
    // one group of lanes), or the digit-plane GEMM's for heads of <= 32;
    // otherwise (GEMV rows, 64-wide heads on 32-column tiles) it is a
    // kernel of its own
    const bool q8_epi = kv->q8 && rope_q8_head_dim_ok(D) &&
                        (use_lds(ly.qkv, R) ||
                         (use_limbs(ly.qkv, R) && gemm_limb_q8_ok(D)));
    if (kv->q8 && !q8_epi) {
      // q, k, v rows, then RoPE and the quantised append
      linear_in(ly.qkv, ws.x.p, d, have_norm2 ? &norm2 : nullptr, R,
                l == 0 && emb_digits, nullptr, 0, ws.qkv.p, 3 * d, kEpiBias);
      launch_rope_kv_q8(st, ws.qkv.p, B, S, H, D, bp, off, active, cosb.p,
                        sinb.p, ws.qrot.p, (int8_t *)kvs.k, (float *)kvs.ks,
                        (int8_t *)kvs.v, (float *)kvs.vs, kv->cap,
                        kvs.seq_stride, kvs.sc_stride);
    } else {
      // q, k, v projection with RoPE and the KV append in its epilogue
      RopeArgs ra;
      ra.S = S; ra.H = H; ra.D = D; ra.off = off; ra.cap = kv->cap;
      ra.base = bp; ra.active = active; ra.cosb = cosb.p; ra.sinb = sinb.p;
      ra.qrot = ws.qrot.p;
      ra.seq_stride = kvs.seq_stride;
      if (kv->q8) {
        ra.kq = (int8_t *)kvs.k; ra.vq = (int8_t *)kvs.v;
        ra.ks = (float *)kvs.ks; ra.vs = (float *)kvs.vs;
        ra.sc_stride = kvs.sc_stride;
      } else {
        ra.kc = (float *)kvs.k; ra.vc = (float *)kvs.v;
      }
      linear_in(ly.qkv, ws.x.p, d, have_norm2 ? &norm2 : nullptr, R,
                l == 0 && emb_digits, nullptr, 0, nullptr, 3 * d, kEpiRope, &ra);
    }
    // short contexts: the attention workgroups merge their key splits and
    // write ctx; up to g_o_limb_rows rows ctx is then digitised by act_quant
    // for the digit-plane GEMM (two launches, measured faster than the LDS
    // GEMM digitising ctx in its prologue), taller inputs (prefill) use the
    // latter.  Long contexts: split attention + combine, which also writes
    // ctx's digits.
    // Short contexts with 64-wide heads: the merged attention writes the
    // output projection's digits itself, one exponent per (row, head), and
    // the digit-plane GEMM scales each head's exact total by its own
    // exponent (no act_quant launch).
    const bool merged = attention_merged(D, max_keys);
    const bool lo = !merged && (use_lds(ly.o, R) || use_limbs(ly.o, R));
    const bool hd = merged && g_o_head_digits && R <= g_o_limb_rows &&
                    use_limbs(ly.o, R) && D == 64 && d % 128 == 0 &&
                    d / 64 <= kMaxHxChunks;
    launch_attention(st, ws.qrot.p, kvs, B, S, H, H, D, kv->cap, bp, off,
                     active, max_keys, ws.part.p, ws.part_elems, ws.ctx.p,
                     lo || hd ? ws.limbs.p : nullptr, ws.mpad, ws.rexp.p,
                     hd ? ws.hexp.p : nullptr);
    if (hd)
      launch_gemm_limb_hx(st, ws.limbs.p, ws.mpad, ws.hexp.p, R, d, d, ly.o.qs.p,
                          ly.o.s.p, ly.o.b.p, ws.x.p, d, ws.h.p, d, kEpiResid);
    else if (merged && R <= g_o_limb_rows && use_limbs(ly.o, R))
      linear(ly.o, ws.ctx.p, d, R, false, ws.x.p, d, ws.h.p, d, kEpiResid);
    else if (merged && ly.o.quant && ly.o.qs.p && R >= kLimbMinRows &&
             gemm_lds_supports(R, d, d))
      launch_gemm_lds(st, kAFromRows, nullptr, 0, nullptr, ws.ctx.p, d,
                      nullptr, nullptr, nullptr, 0, R, d, d, ly.o.qs.p,
                      ly.o.s.p, ly.o.b.p, ws.x.p, d, ws.h.p, d, kEpiResid);
    else
      linear_in(ly.o, ws.ctx.p, d, nullptr, R, lo, ws.x.p, d, ws.h.p, d,
                kEpiResid);
    PendingNorm norm1;
    norm1.h = ws.h.p; norm1.ldh = d; norm1.g = ly.g1.p; norm1.b = ly.b1.p;
    norm1.out = ws.x1.p; norm1.ldo = d;
    linear_in(ly.gu, nullptr, 0, &norm1, R, false, nullptr, 0, ws.ff.p, F,
              kEpiSwiGLU);
    // short batches (the draft's): the down projection on the GEMV over the
    // fp32 SwiGLU rows, which needs no digit planes (one launch instead of
    // act_quant + digit-plane GEMM; measured faster at 32 and 64 rows)
    if (R <= g_gemv_down_rows && ly.down.quant && ly.down.q.p)
      launch_gemv(st, ws.ff.p, F, R, F, d, ly.down.q.p, nullptr, ly.down.s.p,
                  ly.down.b.p, ws.x1.p, d, ws.h.p, d, kEpiResid);
    else
      linear_in(ly.down, ws.ff.p, F, nullptr, R, false, ws.x1.p, d, ws.h.p, d,
                kEpiResid);
    norm2.h = ws.h.p; norm2.ldh = d; norm2.g = ly.g2.p; norm2.b = ly.b2.p;
    norm2.out = ws.x.p; norm2.ldo = d;
    have_norm2 = true;
  }
  if (logits) {
    // norm2 of the last layer feeds the lm head only
    const int rows = last_only ? B : R;
    if (use_lds(lm, rows)) {
      PendingNorm pn = norm2;
      pn.out = nullptr;
      if (last_only) { pn.h = ws.h.p + (int64_t)(S - 1) * d; pn.ldh = (int64_t)S * d; }
      linear_in(lm, nullptr, 0, &pn, rows, false, nullptr, 0, logits, ldl,
                kEpiBias, nullptr, ts);
    } else if (rows <= g_gemv_ln && !use_limbs(lm, rows) && d <= 1024 &&
               d % 4 == 0) {
      // short rows on the GEMV: the last norm2 is its prologue
      NNHIP_REQUIRE(!ts || !ts->out, kErrArg,
                    "forward: tile statistics need the LDS-resident lm head");
      GemvLn lf;
      lf.g = norm2.g; lf.b = norm2.b;
      const float *hx = last_only ? ws.h.p + (int64_t)(S - 1) * d : ws.h.p;
      const int64_t ldh = last_only ? (int64_t)S * d : d;
      launch_gemv(st, hx, ldh, rows, d, V, lm.quant ? lm.q.p : nullptr,
                  lm.quant ? nullptr : lm.w.p, lm.s.p, lm.b.p, nullptr, 0,
                  logits, ldl, kEpiBias, nullptr, &lf);
    } else {
      NNHIP_REQUIRE(!ts || !ts->out, kErrArg,
                    "forward: tile statistics need the LDS-resident lm head");
      launch_layernorm(st, ws.h.p, R, d, norm2.g, norm2.b, ws.x.p, nullptr,
                       ws.mpad, ws.rexp.p);
      if (last_only)
        linear(lm, ws.x.p + (int64_t)(S - 1) * d, (int64_t)S * d, B, false,
               nullptr, 0, logits, ldl, kEpiBias);
      else
        linear(lm, ws.x.p, d, R, false, nullptr, 0, logits, ldl, kEpiBias);
    }
  }
  if (tmp) NNHIP_CHECK(hipStreamSynchronize(st));
}

KVCache::KVCache(Model *model, int batch, int capacity, bool quantized)
    : m(model), B(batch), cap(capacity), q8(quantized) {
  NNHIP_REQUIRE(batch > 0 && capacity > 0, kErrArg, "kvcache: bad size");
  NNHIP_REQUIRE(!q8 || (m->D % 2 == 0 && m->D <= 64), kErrUnsupported,
                "kvcache: the int8 cache needs an even head dim <= 64");
  const size_t n = (size_t)m->L * B * m->H * cap * m->D;
  if (q8) {
    const size_t ns = (size_t)m->L * B * m->H * cap;
    kq.alloc(n);
    vq.alloc(n);
    ks.alloc(ns);
    vs.alloc(ns);
  } else {
    k.alloc(n);
    v.alloc(n);
  }
  len.alloc(B);
  host_len.assign(B, 0);
  sync_len_to_device();
}

KvSrc KVCache::src(int l, int b_off) const {
  KvSrc s;
  s.q8 = q8;
  s.seq_stride = seq_stride();
  s.sc_stride = sc_seq_stride();
  const int64_t o = (int64_t)l * layer_stride() + b_off * seq_stride();
  if (q8) {
    const int64_t so = (int64_t)l * sc_layer_stride() + b_off * sc_seq_stride();
    s.k = kq.p + o; s.v = vq.p + o;
    s.ks = ks.p + so; s.vs = vs.p + so;
  } else {
    s.k = k.p + o; s.v = v.p + o;
  }
  return s;
}

void KVCache::sync_len_to_device() {
  NNHIP_CHECK(hipMemcpyAsync(len.p, host_len.data(), (size_t)B * 4,
                             hipMemcpyHostToDevice, m->ctx->stream));
  NNHIP_CHECK(hipStreamSynchronize(m->ctx->stream));
}

// ---------------------------------------------------------------------------
// Speculative decoding for B independent sequences, entirely on the device
// after the prompt upload: per cycle k draft forwards + k draft samplings,
// one verify forward of k+1 tokens and the accept step.  The draft's
// catch-up token (layer.cpp:1639-1653) is not given a forward of its own:
// it is the first of two rows of the next cycle's first draft forward
// (positions dlen-1 and dlen), which writes the same cache entries; the
// draft prefill stops one token short so that the first cycle has the last
// prompt token in that place.  The per-sequence state (lengths, counters, candidates) stays in
// device memory, so the cycle is a fixed kernel sequence that is captured
// once into a HIP graph and replayed; the host only polls the count of
// active sequences one cycle behind.
// ---------------------------------------------------------------------------
namespace {

struct SpecBuffers {
  DevBuf<int32_t> cur, cand, tlen, dlen, gen, cyc, active, catchup, catch_tok, pair,
      out, n_active, prompts;
  DevBuf<float> qprob, dlog, tlog, tstat;
  DevBuf<float2> dtiles;
  DevBuf<int64_t> stats;
  DevBuf<int32_t> rec;    // the split accept step's records and chunk sums
  DevBuf<double> chunks;
  DevBuf<uint32_t> mt, mt_ring, mt_rw;   // mt19937 streams (SpecState::mt)
};

// The mt19937 streams of B sequences when the context asks for them and
// the loop samples (greedy decoding draws nothing), seeded on the stream.
void attach_mt(Ctx *ctx, hipStream_t st, int B, float T, SpecState &s,
               DevBuf<uint32_t> &mt, DevBuf<uint32_t> &ring,
               DevBuf<uint32_t> &rw) {
  if (ctx->rng != 1 || T <= 0.f) return;
  mt.alloc((size_t)B * kMtN);
  ring.alloc((size_t)B * kMtRing);
  rw.alloc((size_t)B * 2);
  s.mt = mt.p; s.mt_ring = ring.p; s.mt_rw = rw.p;
  launch_mt_seed(st, s);
}

void check_sampling_options(int V, int top_k, float top_p) {
  NNHIP_REQUIRE(V > 0 && V <= 32768, kErrUnsupported,
                "sampling: vocabulary above 32768");
  (void)top_k; (void)top_p;
}

}  // namespace

void generate_speculative_batch(Model &t, Model &dm, int B,
                                const int32_t *prompts, int P, int max_new,
                                int k, float T, int top_k, float top_p,
                                uint64_t seed, uint32_t seq0,
                                bool quantized_cache, int32_t *out,
                                SpecStats *stats, SpecTiming *timing) {
  NNHIP_REQUIRE(t.ctx == dm.ctx, kErrArg, "target and draft need one context");
  NNHIP_REQUIRE(t.V == dm.V, kErrArg, "target and draft vocabularies differ");
  NNHIP_REQUIRE(B > 0 && P > 0 && k > 0 && max_new >= 0, kErrArg,
                "generate_speculative: bad sizes");
  NNHIP_REQUIRE(k <= kMaxLookahead, kErrUnsupported,
                "generate_speculative: lookahead above 63");
  check_sampling_options(t.V, top_k, top_p);
  // The reference throws when a forward's S_past + S exceeds max_seq_len
  // (layer.cpp:1171-1179); with an int8 cache it never checks (the length
  // is read from caches[0].k, which is null).  The prefill is checked here;
  // the cycles' lengths depend on acceptance and are checked after the run
  // from the largest lengths the device recorded.
  NNHIP_REQUIRE(quantized_cache || (P <= t.max_seq && P <= dm.max_seq),
                kErrCapacity,
                "Sequence length S plus past cached length exceeds max_seq_len");
  // Cache capacities cover every row the device writes: the verify step
  // always runs k + 1 rows, and the draft cache keeps a duplicate of every
  // recovered token (layer.cpp:1639-1642 then :1542), up to one per
  // generated token.
  const int t_need = P + max_new + k + 1;
  const int d_need = P + 2 * max_new + k + 2;
  t.ensure_rope(t_need);
  dm.ensure_rope(d_need);
  Ctx *ctx = t.ctx;
  hipStream_t st = ctx->stream;
  const int V = t.V;
  const int out_stride = P + std::max(max_new, 1);

  // KVCache(quantized_cache) for both models (layer.cpp:1396-1398)
  KVCache tc(&t, B, t_need, quantized_cache), dc(&dm, B, d_need, quantized_cache);
  SpecBuffers bf;
  bf.cur.alloc(B); bf.cand.alloc((size_t)B * k); bf.tlen.alloc(B);
  bf.dlen.alloc(B); bf.gen.alloc(B); bf.cyc.alloc(B); bf.active.alloc(B);
  bf.catchup.alloc(B); bf.catch_tok.alloc(B); bf.pair.alloc((size_t)2 * B);
  bf.out.alloc((size_t)B * out_stride);
  bf.n_active.alloc(2);   // n_active, n_far
  bf.prompts.alloc((size_t)B * P);
  // Drafting samples from the draft lm head's tile statistics when that lm
  // head forms them for the batch's row count; otherwise from full passes
  // over the logits.  (The verify rows keep full passes: tile statistics in
  // the target lm head, six row tiles per workgroup, cost about what
  // target_stats_kernel does.)
  const int tw = gemm_lds_tile_width(dm.lm.K);
  const int nt = tw > 0 ? (V + tw - 1) / tw : 0;
  // (tile statistics carry no top-k / top-p: filtered rows take full passes)
  const bool tiles = tw > 0 && nt <= 1024 &&
                     (T <= 0.f || !sampling_filtered(V, top_k, top_p)) &&
                     dm.lm_tiles(B);
  if (tiles) bf.dtiles.alloc((size_t)B * k * nt);
  // sampled drafting from tile statistics keeps each step's logits; the
  // draft probabilities are then formed where the accept step needs them
  // (s.qlog) instead of written out at every step
  const bool qlog = tiles && T > 0.f;
  if (T > 0.f && !qlog) bf.qprob.alloc((size_t)B * k * V);
  bf.tstat.alloc((size_t)B * (k + 1) * kTstat);
  bf.dlog.alloc((size_t)(qlog ? k : 1) * B * V);
  bf.tlog.alloc((size_t)B * (k + 1) * V);
  bf.stats.alloc((size_t)B * kSpecStats);
  NNHIP_CHECK(hipMemsetAsync(bf.stats.p, 0, bf.stats.bytes(), st));
  NNHIP_CHECK(hipMemsetAsync(bf.n_active.p, 0, 8, st));
  NNHIP_CHECK(hipMemsetAsync(bf.cand.p, 0, bf.cand.bytes(), st));
  NNHIP_CHECK(hipMemsetAsync(bf.out.p, 0, bf.out.bytes(), st));
  NNHIP_CHECK(hipMemcpyAsync(bf.prompts.p, prompts, (size_t)B * P * 4,
                             hipMemcpyHostToDevice, st));
  NNHIP_CHECK(hipMemcpy2DAsync(bf.out.p, (size_t)out_stride * 4, prompts,
                               (size_t)P * 4, (size_t)P * 4, B,
                               hipMemcpyHostToDevice, st));

  SpecState s{};
  s.cur = bf.cur.p; s.cand = bf.cand.p; s.qprob = bf.qprob.p;
  if (qlog) s.qlog = bf.dlog.p;
  s.tstat = bf.tstat.p;
  if (tiles) { s.dtiles = bf.dtiles.p; s.nt = nt; s.tw = tw; }
  s.tlen = bf.tlen.p; s.dlen = bf.dlen.p; s.gen = bf.gen.p; s.cyc = bf.cyc.p;
  s.active = bf.active.p; s.catchup = bf.catchup.p;
  s.catch_tok = bf.catch_tok.p; s.pair = bf.pair.p; s.out = bf.out.p;
  s.n_active = bf.n_active.p; s.n_far = bf.n_active.p + 1;
  if (g_accept_split) {
    bf.rec.alloc((size_t)B * kAcceptRec);
    bf.chunks.alloc((size_t)B * kDrawChunks * 2);
    s.rec = bf.rec.p;
    s.chunks = bf.chunks.p;
  }
  s.stats = bf.stats.p;
  s.B = B; s.out_stride = out_stride; s.P = P; s.max_new = max_new;
  s.k = k; s.V = V; s.T = T; s.seed = seed; s.seq0 = seq0;
  s.top_k = top_k; s.top_p = top_p;
  attach_mt(ctx, st, B, T, s, bf.mt, bf.mt_ring, bf.mt_rw);
  // workspace for every shape the loop uses, before any graph capture
  t.reserve(B * P, B * (k + 1), t_need);
  t.reserve(B * (k + 1), B * (k + 1), t_need);
  dm.reserve(B * P, B, d_need);
  dm.reserve(2 * B, B, d_need);

  hipEvent_t e0, e1, e2;
  NNHIP_CHECK(hipEventCreate(&e0));
  NNHIP_CHECK(hipEventCreate(&e1));
  NNHIP_CHECK(hipEventCreate(&e2));
  NNHIP_CHECK(hipEventRecord(e0, st));
  // prefill (layer.cpp:1400-1408); the draft's prefill logits are unused
  t.forward(&tc, 0, bf.prompts.p, P, B, P, nullptr, 0, nullptr, P, bf.dlog.p,
            true);
  launch_first_token(st, s, bf.dlog.p, V);
  if (P > 1)
    dm.forward(&dc, 0, bf.prompts.p, P, B, P - 1, nullptr, 0, nullptr, P - 1,
               nullptr, true);
  NNHIP_CHECK(hipEventRecord(e1, st));

  // Drafting steps j < k - 1 embed the next draft step's row themselves
  // (s.nd), so those forwards gather nothing; the verify forward gathers
  // [cur, c_0 .. c_{k-1}] straight from the last tokens and the candidates.
  // (The last drafting step embedding the verify rows itself, k + 1 rows of
  // one workgroup, measured no faster than the gather launch.)
  s.nd = dm.next_rows(B);
  auto cycle = [&]() {
    for (int j = 0; j < k; ++j) {
      TileStatsArgs dts;
      if (tiles) {
        dts.out = bf.dtiles.p + (size_t)j * nt;
        dts.ld = (int64_t)k * nt;
        dts.T = T;
      }
      float *dl = bf.dlog.p + (qlog ? (size_t)j * B * V : 0);
      if (j == 0)   // {catch-up token, cur} at dlen - 1, dlen
        dm.forward(&dc, 0, bf.pair.p, 2, B, 2, bf.dlen.p, -1, bf.active.p,
                   d_need, dl, true, 0, &dts);
      else
        dm.forward(&dc, 0, bf.cand.p + (j - 1), k, B, 1, bf.dlen.p, j,
                   bf.active.p, d_need, dl, false, 0, &dts, true);
      if (tiles) launch_draft_sample_tiles(st, s, j, dl, V);
      else launch_draft_sample(st, s, j, dl, V);
    }
    t.forward(&tc, 0, bf.cand.p, k, B, k + 1, bf.tlen.p, 0, bf.active.p,
              t_need, bf.tlog.p, false, 0, nullptr, false, bf.cur.p);
    launch_accept(st, s, bf.tlog.p);
  };

  // per cycle parity: {n_active, n_far} after that cycle
  int32_t *h_nact = nullptr;
  NNHIP_CHECK(hipHostMalloc((void **)&h_nact, 4 * sizeof(int32_t)));
  hipEvent_t ev[2];
  NNHIP_CHECK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
  NNHIP_CHECK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming));
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int64_t launched = 0;
  try {
    if (max_new > 1) {
      if (ctx->use_graphs) {
        NNHIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        try {
          cycle();
        } catch (...) {
          hipGraph_t g2 = nullptr;
          (void)hipStreamEndCapture(st, &g2);
          if (g2) (void)hipGraphDestroy(g2);
          throw;
        }
        NNHIP_CHECK(hipStreamEndCapture(st, &graph));
        NNHIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
      }
      // Each cycle commits at least one and at most k + 1 tokens per active
      // sequence.  The host reads the counts one cycle behind, so that the
      // device never waits for it; once no sequence had more than k + 1
      // tokens to go after cycle c - 1, cycle c may finish them all, and
      // the host waits for its counts before it launches another (no cycle
      // runs after the last sequence finished).
      const int max_cycles = max_new - 1;
      for (int c = 0; c < max_cycles; ++c) {
        if (exec) NNHIP_CHECK(hipGraphLaunch(exec, st));
        else cycle();
        ++launched;
        int32_t *hc = &h_nact[2 * (c & 1)];
        NNHIP_CHECK(hipMemcpyAsync(hc, bf.n_active.p, 8,
                                   hipMemcpyDeviceToHost, st));
        NNHIP_CHECK(hipEventRecord(ev[c & 1], st));
        // after the first token every active sequence has max_new - 1 to go
        bool near = c == 0 && max_new - 1 <= k + 1;
        if (c >= 1) {
          const int32_t *hp = &h_nact[2 * ((c - 1) & 1)];
          NNHIP_CHECK(hipEventSynchronize(ev[(c - 1) & 1]));
          if (hp[0] == 0) break;
          near = hp[1] == 0;
        }
        if (near) {
          NNHIP_CHECK(hipEventSynchronize(ev[c & 1]));
          if (hc[0] == 0) break;
        }
      }
    }
    NNHIP_CHECK(hipEventRecord(e2, st));
    NNHIP_CHECK(hipStreamSynchronize(st));
  } catch (...) {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipHostFree(h_nact);
    (void)hipEventDestroy(ev[0]); (void)hipEventDestroy(ev[1]);
    (void)hipEventDestroy(e0); (void)hipEventDestroy(e1); (void)hipEventDestroy(e2);
    throw;
  }
  if (exec) NNHIP_CHECK(hipGraphExecDestroy(exec));
  if (graph) NNHIP_CHECK(hipGraphDestroy(graph));
  NNHIP_CHECK(hipHostFree(h_nact));
  NNHIP_CHECK(hipEventDestroy(ev[0]));
  NNHIP_CHECK(hipEventDestroy(ev[1]));
  float ms_pre = 0.f, ms_dec = 0.f;
  NNHIP_CHECK(hipEventElapsedTime(&ms_pre, e0, e1));
  NNHIP_CHECK(hipEventElapsedTime(&ms_dec, e1, e2));
  NNHIP_CHECK(hipEventDestroy(e0));
  NNHIP_CHECK(hipEventDestroy(e1));
  NNHIP_CHECK(hipEventDestroy(e2));
  if (timing) {
    timing->prefill_ms = ms_pre;
    timing->decode_ms = ms_dec;
    timing->cycles_launched = launched;
  }
  t.check_pd();
  dm.check_pd();
  std::vector<int64_t> hs((size_t)B * kSpecStats);
  NNHIP_CHECK(hipMemcpy(hs.data(), bf.stats.p, hs.size() * 8,
                        hipMemcpyDeviceToHost));
  if (!quantized_cache) {
    for (int b = 0; b < B; ++b) {
      const int64_t *x = &hs[(size_t)b * kSpecStats];
      NNHIP_REQUIRE(x[6] <= t.max_seq && x[7] <= dm.max_seq, kErrCapacity,
                    "Sequence length S plus past cached length exceeds max_seq_len");
    }
  }
  NNHIP_CHECK(hipMemcpy(out, bf.out.p, bf.out.bytes(), hipMemcpyDeviceToHost));
  if (stats) {
    for (int b = 0; b < B; ++b) {
      const int64_t *x = &hs[(size_t)b * kSpecStats];
      stats[b] = SpecStats{x[0], x[1], x[2], x[3], x[4], x[5]};
    }
  }
}

void generate_advanced_batch(Model &m, int B, const int32_t *prompts, int P,
                             int max_new, float T, int top_k, float top_p,
                             uint64_t seed, uint32_t seq0, bool use_cache,
                             int32_t *out) {
  NNHIP_REQUIRE(B > 0 && P > 0 && max_new >= 0, kErrArg,
                "generate_advanced: bad sizes");
  check_sampling_options(m.V, top_k, top_p);
  hipStream_t st = m.ctx->stream;
  const int total = P + max_new;
  if (use_cache)
    NNHIP_REQUIRE(total <= m.max_seq + 1, kErrCapacity,
                  "Sequence length S plus past cached length exceeds max_seq_len");
  DevBuf<int32_t> dout((size_t)B * std::max(total, 1)), cur(B), len(B);
  DevBuf<float> lg((size_t)B * m.V);
  NNHIP_CHECK(hipMemcpy(dout.p, prompts, (size_t)B * P * 4, hipMemcpyHostToDevice));
  // prompts are [B][P]; re-lay them with stride `total`
  if (total != P) {
    std::vector<int32_t> h((size_t)B * total, 0);
    for (int b = 0; b < B; ++b)
      std::memcpy(&h[(size_t)b * total], prompts + (size_t)b * P, (size_t)P * 4);
    NNHIP_CHECK(hipMemcpy(dout.p, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  }
  NNHIP_CHECK(hipMemset(len.p, 0, (size_t)B * 4));
  SpecState s{};
  s.cur = cur.p; s.out = dout.p; s.B = B; s.out_stride = total; s.P = P;
  s.max_new = max_new; s.k = 0; s.V = m.V; s.T = T; s.seed = seed;
  s.seq0 = seq0; s.top_k = top_k; s.top_p = top_p;
  DevBuf<uint32_t> mt, mt_ring, mt_rw;
  attach_mt(m.ctx, st, B, T, s, mt, mt_ring, mt_rw);
  std::unique_ptr<KVCache> cache;
  if (use_cache) cache.reset(new KVCache(&m, B, std::max(total, 1)));
  for (int step = 0; step < max_new; ++step) {
    const int n = P + step;
    if (use_cache && step > 0) {
      m.forward(cache.get(), 0, cur.p, 1, B, 1, len.p, 0, nullptr, n, lg.p,
                true);
      launch_add_scalar(st, len.p, B, 1);
    } else {
      // the reference keeps the last max_seq_len tokens (layer.cpp:1271-1277)
      int S = n, start = 0;
      if (S > m.max_seq) { start = S - m.max_seq; S = m.max_seq; }
      m.forward(cache.get(), 0, dout.p + start, total, B, S,
                use_cache ? len.p : nullptr, 0, nullptr, S, lg.p, true);
      if (use_cache) launch_add_scalar(st, len.p, B, S);
    }
    launch_ar_sample(st, s, step, lg.p, m.V);
  }
  NNHIP_CHECK(hipStreamSynchronize(st));
  NNHIP_CHECK(hipMemcpy(out, dout.p, (size_t)B * total * 4, hipMemcpyDeviceToHost));
}

}  // namespace nnhip

// Host engine of libnnhip.so: device-resident TransformerDecoder, ragged KV
// caches, the forward pass and the on-device speculative loop.  Mirrors the
// reference's TransformerDecoder / KVCache / QuantizedDense objects
// (include/nn/layer.hpp:212-330, include/nn/quantization.hpp:15-43).
#pragma once

#include "nnhip_internal.hpp"

#include <memory>
#include <string>

namespace nnhip {

// A context owns one HIP stream at the default priority; every launch of the
// library is ordered on it.
struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool use_graphs = true;
  // uniforms of the generate loops: 0 the Philox counter stream, 1 the
  // reference's std::mt19937 per sequence (SpecState::mt)
  int rng = 0;
};

// One Dense on the device, weight transposed to [N][K].  Fused layouts:
// QKV rows [q | k | v]; gate/up interleaved (row 2n = gate n, 2n+1 = up n).
struct Linear {
  int K = 0, N = 0;
  DevBuf<float> w;      // [N][K] fp32 master weight
  DevBuf<int8_t> q;     // [N][K] int8 codes (after quantize)
  DevBuf<int8_t> qs;    // the same codes in the MFMA operand layout
  DevBuf<float> s;      // [N] per-channel scales
  DevBuf<float> b;      // [N] bias
  bool quant = false;
  void init(int k, int n);
};

struct LayerW {
  Linear qkv, o, gu, down;
  DevBuf<float> g1, b1, g2, b2;
};

struct Workspace {
  int rows = 0, lrows = 0;
  DevBuf<float> x, qkv, qrot, ctx, h, x1, ff, logits, part;
  DevBuf<int8_t> limbs;
  DevBuf<int> rexp;
  DevBuf<int> hexp;        // [mpad][H] per-(row, head) digit exponents
  DevBuf<int32_t> ids, zeros;
  int mpad = 0;
  int64_t part_elems = 0;
};

struct KVCache;

struct Model {
  Ctx *ctx = nullptr;
  int V = 0, d = 0, H = 0, D = 0, F = 0, L = 0, max_seq = 0;
  bool quantized = false;
  int bits = 8;       // weight code width once quantized (8 or 4)
  DevBuf<float> emb;  // [V][d]
  std::vector<LayerW> layers;
  Linear lm;
  DevBuf<float> cosb, sinb;  // [rope_len][D/2], rope_len >= max_seq
  int rope_len = 0;
  // RoPE tables for positions [0, n): the speculative loop writes rows past
  // max_seq_len (its verify step always runs k + 1 rows, and an int8 cache
  // has no length check in the reference)
  void ensure_rope(int n);
  Workspace wsp;  // activations of the current forward
  // state of the persistent decoder-layer kernel (draft_layers.hip): its
  // ring of stage outputs for up to pd_rows rows, one flag word per
  // workgroup (pd_nwg of them, one per CU) and the error word
  DevBuf<float> pd_ring;
  DevBuf<unsigned> pd_flags, pd_tflags;
  DevBuf<int> pd_err;
  int pd_rows = 0, pd_nwg = 0;
  // whether a forward of `rows` rows (S per sequence) over `kv` runs its
  // layers as that one kernel
  bool use_pd(int rows, int S, const KVCache *kv) const;
  // throws if a wait of that kernel timed out (and resets its state)
  void check_pd();

  Model(Ctx *c, int vocab, int d_model, int heads, int d_ff, int n_layers,
        int max_seq_len);
  int num_params() const { return 1 + 18 * L + 2; }
  void param_shape(int idx, int64_t *rows, int64_t *cols) const;
  void set_param(int idx, const float *host);
  void get_param(int idx, float *host) const;
  void init_normal(uint64_t seed, float stdv);
  void quantize(int bits = 8);
  void get_quantized(int layer, int which, int8_t *codes_kn,
                     float *scales) const;

  // Ensures the workspace for `rows` rows of which `lrows` need logits.
  void reserve(int rows, int lrows, int max_keys);

  // TransformerDecoder::forward for B sequences of S new tokens each, using
  // cache sequences [b_off, b_off + B).
  // Token of row (b, s): ids[b*ids_stride + s].  Positions start at
  // base[b] + off (device array; nullptr = 0).  Sequences with
  // active[b] == 0 neither write nor read the cache.  logits: nullptr (not
  // needed), or [B*S][V] (all rows) or [B][V] (last_only), rows ldl apart
  // (0 = V).  ts: the lm head's tile statistics as well (lm_tiles(rows)).
  // embedded: the rows (and their digits, when emb_digits(B * S)) are
  // already in the workspace (next_rows), ids are not read.  lead: row
  // (b, 0) takes lead[b] and row (b, s) ids[b*ids_stride + s - 1].
  void forward(KVCache *cache, int b_off, const int32_t *ids,
               int ids_stride, int B, int S, const int32_t *base, int off,
               const int32_t *active, int max_keys, float *logits,
               bool last_only, int64_t ldl = 0,
               const TileStatsArgs *ts = nullptr, bool embedded = false,
               const int32_t *lead = nullptr);
  // whether the embedding step also writes the rows' digits (the first
  // q/k/v projection of `rows` rows is an MFMA GEMM)
  bool emb_digits(int rows) const;
  // where a kernel other than the embedding writes the input rows of a
  // forward of `rows` rows (the workspace must be reserved for them)
  NextRows next_rows(int rows) const;
  // whether the lm head on `rows` rows can form tile statistics
  bool lm_tiles(int rows) const;

  void linear(const Linear &ln, const float *x, int64_t ldx, int rows,
              bool limbs_ready, const float *resid, int64_t ldr, float *y,
              int64_t ldy, int epi, const RopeArgs *ra = nullptr);
  // A LayerNorm of h (rows of stride ldh) that the next linear applies to
  // its input; the normalised rows go to out (stride ldo) when out is set.
  struct PendingNorm {
    const float *h = nullptr, *g = nullptr, *b = nullptr;
    int64_t ldh = 0;
    float *out = nullptr;
    int64_t ldo = 0;
  };
  // linear over x, or over LN(h) when pn is given (x is then ignored)
  void linear_in(const Linear &ln, const float *x, int64_t ldx,
                 const PendingNorm *pn, int rows, bool limbs_ready,
                 const float *resid, int64_t ldr, float *y, int64_t ldy,
                 int epi, const RopeArgs *ra = nullptr,
                 const TileStatsArgs *ts = nullptr);
  bool use_limbs(const Linear &ln, int rows) const;
  bool norm_folds(const Linear &ln, int rows) const;
  bool use_lds(const Linear &ln, int rows) const;
};

// Ragged KV cache for B sequences: per layer [B][H][cap][D], one length per
// sequence (KVCache, layer.hpp:212-230, with per-sequence lengths).  A
// quantised cache (KVCache(true)) holds int8 codes in the same layout and one
// fp32 scale per (sequence, head, position) for k and for v.
struct KVCache {
  Model *m = nullptr;
  int B = 0, cap = 0;
  bool q8 = false;
  DevBuf<float> k, v;          // fp32 cache
  DevBuf<int8_t> kq, vq;       // int8 cache: codes
  DevBuf<float> ks, vs;        //             scales [L][B][H][cap]
  DevBuf<int32_t> len;
  std::vector<int32_t> host_len;
  KVCache(Model *model, int batch, int capacity, bool quantized = false);
  int64_t seq_stride() const { return (int64_t)m->H * cap * m->D; }
  int64_t layer_stride() const { return (int64_t)B * seq_stride(); }
  int64_t sc_seq_stride() const { return (int64_t)m->H * cap; }
  int64_t sc_layer_stride() const { return (int64_t)B * sc_seq_stride(); }
  // the rows layer l's attention reads for sequences [b_off, B)
  KvSrc src(int l, int b_off) const;
  void sync_len_to_device();
};

struct SpecStats {
  int64_t cycles, drafted, accepted, ties, resampled, bonus;
};

struct SpecTiming {
  double prefill_ms, decode_ms;
  int64_t cycles_launched;
};

// Layer::save_weights / load_weights (layer.cpp:463-470): NETW v1 files of
// the decoder's parameters() (netw.hip).
void save_weights(const Model &m, const std::string &path);
void load_weights(Model &m, const std::string &path);

// generate_speculative (layer.cpp:1382-1661) for B independent sequences.
void generate_speculative_batch(Model &target, Model &draft, int B,
                                const int32_t *prompts, int P, int max_new,
                                int k, float T, int top_k, float top_p,
                                uint64_t seed, uint32_t seq0,
                                bool quantized_cache, int32_t *out,
                                SpecStats *stats, SpecTiming *timing);

// generate_advanced (layer.cpp:1240-1380) for B independent sequences.
void generate_advanced_batch(Model &m, int B, const int32_t *prompts, int P,
                             int max_new, float T, int top_k, float top_p,
                             uint64_t seed, uint32_t seq0, bool use_cache,
                             int32_t *out);

}  // namespace nnhip

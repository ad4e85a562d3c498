// Microbenchmark entry points: time one kernel of the decode path on the
// context's stream with HIP events, over `nbuf` rotating input sets so that
// the timed bytes come from HBM rather than from the 256 MB Infinity Cache.
// Inputs are generated on the device (seeded Philox normals).
#include "api_common.hpp"

#include <functional>
#include <vector>

using nnhip::guard;

namespace {

float time_loop(nnhip_ctx *ctx, int iters, const std::function<void(int)> &f) {
  hipStream_t st = ctx->c.stream;
  f(0);  // warm-up launch
  NNHIP_CHECK(hipEventRecord(ctx->t0, st));
  for (int i = 0; i < iters; ++i) f(i);
  NNHIP_CHECK(hipEventRecord(ctx->t1, st));
  NNHIP_CHECK(hipEventSynchronize(ctx->t1));
  float ms = 0.f;
  NNHIP_CHECK(hipEventElapsedTime(&ms, ctx->t0, ctx->t1));
  return ms / iters;
}

}  // namespace

extern "C" {

// Verify-step attention: B sequences x H heads, S new queries per sequence
// attending causally among themselves and fully to n_cached cached
// positions (keys n_cached + S), K/V entries N(0, 1); quantized != 0 reads
// an int8 cache instead (constant codes and scales: the timing does not
// depend on the values).
int nnhip_bench_attention(nnhip_ctx *ctx, int B, int S, int H, int D,
                          int n_cached, int iters, int nbuf, int quantized,
                          float *ms) {
  return guard([&] {
    NNHIP_REQUIRE(ctx && ms && B > 0 && S > 0 && H > 0 && D > 0 &&
                      n_cached >= 0 && iters > 0 && nbuf > 0,
                  nnhip::kErrArg, "nnhip_bench_attention: bad argument");
    hipStream_t st = ctx->c.stream;
    const int cap = n_cached + S;
    const int64_t kv = (int64_t)B * H * cap * D;
    const int64_t ns = (int64_t)B * H * cap;
    std::vector<nnhip::DevBuf<float>> K(nbuf), Vv(nbuf), Q(nbuf), O(nbuf);
    std::vector<nnhip::DevBuf<int8_t>> Kq(nbuf), Vq(nbuf);
    std::vector<nnhip::DevBuf<float>> Ks(nbuf), Vs(nbuf);
    for (int i = 0; i < nbuf; ++i) {
      Q[i].alloc((size_t)B * S * H * D); O[i].alloc((size_t)B * S * H * D);
      nnhip::launch_init_normal(st, Q[i].p, 1, B * S * H * D, 0, 1, 3000 + i, 0, 1.f, 0);
      if (quantized) {
        Kq[i].alloc(kv); Vq[i].alloc(kv); Ks[i].alloc(ns); Vs[i].alloc(ns);
        NNHIP_CHECK(hipMemsetAsync(Kq[i].p, 0x25, (size_t)kv, st));
        NNHIP_CHECK(hipMemsetAsync(Vq[i].p, 0x1b, (size_t)kv, st));
        nnhip::launch_fill(st, Ks[i].p, ns, 0.02f);
        nnhip::launch_fill(st, Vs[i].p, ns, 0.02f);
      } else {
        K[i].alloc(kv); Vv[i].alloc(kv);
        nnhip::launch_init_normal(st, K[i].p, 1, (int)kv, 0, 1, 1000 + i, 0, 1.f, 0);
        nnhip::launch_init_normal(st, Vv[i].p, 1, (int)kv, 0, 1, 2000 + i, 0, 1.f, 0);
      }
    }
    std::vector<int32_t> hpos(B, n_cached);
    nnhip::DevBuf<int32_t> pos(B);
    NNHIP_CHECK(hipMemcpyAsync(pos.p, hpos.data(), (size_t)B * 4, hipMemcpyHostToDevice, st));
    const int64_t pe = nnhip::attention_partial_elems(B, S, H, D, cap);
    nnhip::DevBuf<float> part(pe > 0 ? pe : 1);
    *ms = time_loop(ctx, iters, [&](int i) {
      const int j = i % nbuf;
      nnhip::KvSrc src;
      src.seq_stride = (int64_t)H * cap * D;
      if (quantized) {
        src.q8 = true;
        src.k = Kq[j].p; src.v = Vq[j].p; src.ks = Ks[j].p; src.vs = Vs[j].p;
        src.sc_stride = (int64_t)H * cap;
      } else {
        src.k = K[j].p; src.v = Vv[j].p;
      }
      nnhip::launch_attention(st, Q[j].p, src, B, S, H, H, D, cap, pos.p, 0,
                              nullptr, cap, part.p, pe, O[j].p);
    });
  });
}

// Acceptance step of the speculative loop from logits, as
// nnhip_spec_accept runs it (AcceptRows::launch_logits: the state reset, the
// rows' statistics up to each sequence's first rejection, the accept
// step), timed together.  B sequences
// x k positions x V, target and draft logits N(0, 2) (nbuf sets of each),
// each set's draft ids drawn from its draft probabilities with a separate
// stream beforehand (fixture preparation, not timed), one accept uniform per
// position and one resample uniform per sequence.  n_accept (host, [B])
// receives the accepted counts of input set 0.
int nnhip_bench_spec_accept(nnhip_ctx *ctx, int B, int k, int V, float T,
                            int iters, int nbuf, float *ms,
                            int32_t *n_accept) {
  return guard([&] {
    NNHIP_REQUIRE(ctx && ms && B > 0 && k > 0 && V > 0 && iters > 0 && nbuf > 0,
                  nnhip::kErrArg, "nnhip_bench_spec_accept: bad argument");
    hipStream_t st = ctx->c.stream;
    const int64_t n = (int64_t)B * k * V;
    std::vector<nnhip::DevBuf<float>> TL(nbuf), DL(nbuf);
    std::vector<nnhip::DevBuf<int32_t>> dtok(nbuf);
    nnhip::DevBuf<float> q0(n);
    nnhip::DevBuf<int32_t> nacc(B), next(B);
    nnhip::DevBuf<float> ua((size_t)B * k), ur(B), us((size_t)B * k);
    // uniforms in [0, 1) from a fixed host xorshift stream
    std::vector<float> hu((size_t)B * k * 2 + B);
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (auto &u : hu) {
      x ^= x << 13; x ^= x >> 7; x ^= x << 17;
      u = (float)(x >> 40) * (1.0f / 16777216.0f);
    }
    NNHIP_CHECK(hipMemcpyAsync(ua.p, hu.data(), (size_t)B * k * 4, hipMemcpyHostToDevice, st));
    NNHIP_CHECK(hipMemcpyAsync(us.p, hu.data() + B * k, (size_t)B * k * 4, hipMemcpyHostToDevice, st));
    NNHIP_CHECK(hipMemcpyAsync(ur.p, hu.data() + 2 * B * k, (size_t)B * 4, hipMemcpyHostToDevice, st));
    const float Tq = T > 0.f ? T : 1.f;
    for (int i = 0; i < nbuf; ++i) {
      TL[i].alloc(n); DL[i].alloc(n);
      nnhip::launch_init_normal(st, TL[i].p, 1, (int)n, 0, 1, 4000 + i, 0, 2.f, 0);
      nnhip::launch_init_normal(st, DL[i].p, 1, (int)n, 0, 1, 5000 + i, 0, 2.f, 0);
    }
    // each set's draft ids are draws from its own draft probabilities
    for (int i = 0; i < nbuf; ++i) {
      dtok[i].alloc((size_t)B * k);
      nnhip::launch_sample_rows(st, DL[i].p, B * k, V, Tq, us.p, dtok[i].p, q0.p);
    }
    nnhip::AcceptRows ar(B, k, V, T);
    *ms = time_loop(ctx, iters, [&](int i) {
      const int j = i % nbuf;
      ar.launch_logits(st, TL[j].p, DL[j].p, dtok[j].p, ua.p, ur.p, nacc.p, next.p);
    });
    if (n_accept) {
      ar.launch_logits(st, TL[0].p, DL[0].p, dtok[0].p, ua.p, ur.p, nacc.p, next.p);
      NNHIP_CHECK(hipMemcpyAsync(n_accept, nacc.p, (size_t)B * 4, hipMemcpyDeviceToHost, st));
      NNHIP_CHECK(hipStreamSynchronize(st));
    }
  });
}

// W8A32 Linear: rows x K activations N(0, 1) times an int8 [N][K] weight.
// path 1 = fp32 GEMV, 2 = int8-digit MFMA GEMM (digit split included),
// 3 = LDS GEMM from fp32 rows, 4 = LDS GEMM over digit planes (digit split
// included), 5 = LDS GEMM with LayerNorm (gamma 1, beta 0) in its prologue,
// 6 = LDS GEMM over digit planes made once, with tile statistics; over
// digit planes made once, the GEMM alone: 7 = LDS GEMM, 8 = digit-plane
// GEMM.
int nnhip_bench_linear(nnhip_ctx *ctx, int rows, int K, int N, int path,
                       int iters, int nbuf, float *ms) {
  return guard([&] {
    NNHIP_REQUIRE(ctx && ms && rows > 0 && K > 0 && N > 0 && iters > 0 && nbuf > 0,
                  nnhip::kErrArg, "nnhip_bench_linear: bad argument");
    hipStream_t st = ctx->c.stream;
    std::vector<nnhip::DevBuf<int8_t>> W(nbuf), WS(nbuf);
    std::vector<nnhip::DevBuf<float>> S(nbuf);
    nnhip::DevBuf<float> wf((size_t)N * K), x((size_t)rows * K), y((size_t)rows * N), b(N);
    nnhip::launch_init_normal(st, x.p, 1, rows * K, 0, 1, 11, 0, 1.f, 0);
    nnhip::launch_fill(st, b.p, N, 0.f);
    for (int i = 0; i < nbuf; ++i) {
      W[i].alloc((size_t)N * K); S[i].alloc(N);
      nnhip::launch_init_normal(st, wf.p, 1, N * K, 0, 1, 20 + i, 0, 0.02f, 0);
      nnhip::launch_quantize_w8(st, wf.p, N, K, W[i].p, S[i].p);
      if (path >= 2) {
        WS[i].alloc((size_t)N * K);
        nnhip::launch_swizzle_rows(st, W[i].p, N, K, WS[i].p, false);
      }
    }
    const int mpad = (rows + 63) / 64 * 64;
    nnhip::DevBuf<int8_t> limbs((size_t)3 * mpad * K);
    nnhip::DevBuf<int> rexp(mpad);
    nnhip::DevBuf<float> g1(K), b0(K);
    nnhip::launch_fill(st, g1.p, K, 1.f);
    nnhip::launch_fill(st, b0.p, K, 0.f);
    NNHIP_REQUIRE(path >= 1 && path <= 9, nnhip::kErrArg, "nnhip_bench_linear: unknown path");
    NNHIP_REQUIRE(path <= 2 || path >= 8 || nnhip::gemm_lds_supports(rows, K, N),
                  nnhip::kErrArg, "nnhip_bench_linear: shape not supported by the LDS GEMM");
    NNHIP_REQUIRE((path != 8 && path != 9) || (K % 128 == 0 && N % 64 == 0), nnhip::kErrArg,
                  "nnhip_bench_linear: the digit-plane GEMM needs K % 128 == 0, N % 64 == 0");
    NNHIP_REQUIRE(path != 9 || K / 64 <= nnhip::kMaxHxChunks, nnhip::kErrArg,
                  "nnhip_bench_linear: per-chunk exponents need K <= 2048");
    // path 6: digit planes prepared once, then the GEMM alone with the lm
    // head's tile statistics (T = 1)
    const int tw = nnhip::gemm_lds_tile_width(K);
    NNHIP_REQUIRE(path != 6 || tw > 0, nnhip::kErrArg,
                  "nnhip_bench_linear: tile statistics need K of 512 or 1024");
    const int ntile = tw > 0 ? (N + tw - 1) / tw : 0;
    nnhip::DevBuf<float2> tstat(path == 6 ? (size_t)rows * ntile : 0);
    nnhip::TileStatsArgs tsa;
    tsa.out = tstat.p; tsa.ld = ntile; tsa.T = 1.f;
    if (path >= 6)
      nnhip::launch_act_quant(st, x.p, K, rows, K, limbs.p, mpad, rexp.p);
    // path 9: the output projection's GEMM, one exponent per 64-wide K chunk
    // (each row's exponent repeated over its chunks)
    nnhip::DevBuf<int> hexp(path == 9 ? (size_t)mpad * (K / 64) : 0);
    if (path == 9) {
      std::vector<int> re(mpad), he((size_t)mpad * (K / 64));
      NNHIP_CHECK(hipMemcpyAsync(re.data(), rexp.p, (size_t)mpad * 4,
                                 hipMemcpyDeviceToHost, st));
      NNHIP_CHECK(hipStreamSynchronize(st));
      for (size_t i = 0; i < he.size(); ++i) he[i] = re[i / (K / 64)];
      NNHIP_CHECK(hipMemcpyAsync(hexp.p, he.data(), he.size() * 4,
                                 hipMemcpyHostToDevice, st));
      NNHIP_CHECK(hipStreamSynchronize(st));
    }
    *ms = time_loop(ctx, iters, [&](int i) {
      const int j = i % nbuf;
      if (path == 9) {
        nnhip::launch_gemm_limb_hx(st, limbs.p, mpad, hexp.p, rows, K, N, WS[j].p,
                                   S[j].p, b.p, nullptr, 0, y.p, N, nnhip::kEpiBias);
      } else if (path == 8) {
        nnhip::launch_gemm_limb(st, limbs.p, mpad, rexp.p, rows, K, N, WS[j].p,
                                S[j].p, b.p, nullptr, 0, y.p, N, nnhip::kEpiBias);
      } else if (path >= 3) {
        if (path == 4)
          nnhip::launch_act_quant(st, x.p, K, rows, K, limbs.p, mpad, rexp.p);
        const int mode = path == 3 ? nnhip::kAFromRows
                         : path == 4 || path >= 6 ? nnhip::kAFromDigits
                                                  : nnhip::kAFromLayerNorm;
        nnhip::launch_gemm_lds(st, mode, limbs.p, mpad, rexp.p, x.p, K, g1.p,
                               b0.p, nullptr, 0, rows, K, N, WS[j].p, S[j].p,
                               b.p, nullptr, 0, y.p, N, nnhip::kEpiBias,
                               nullptr, path == 6 ? &tsa : nullptr);
      } else if (path == 2) {
        nnhip::launch_act_quant(st, x.p, K, rows, K, limbs.p, mpad, rexp.p);
        nnhip::launch_gemm_limb(st, limbs.p, mpad, rexp.p, rows, K, N, WS[j].p,
                                S[j].p, b.p, nullptr, 0, y.p, N, nnhip::kEpiBias);
      } else {
        nnhip::launch_gemv(st, x.p, K, rows, K, N, W[j].p, nullptr, S[j].p,
                           b.p, nullptr, 0, y.p, N, nnhip::kEpiBias);
      }
    });
  });
}

// One forward of the model over B sequences x S new tokens after n_cached
// cached positions (the verify step of the speculative loop: S = k + 1),
// logits of every row written: TransformerDecoder::forward (layer.cpp:
// 1159-1216) with its KV cache.  The cache holds zeros; the forward writes
// positions [n_cached, n_cached + S) each time.  Captured once as a HIP
// graph and replayed, as the loop replays its cycle.
int nnhip_bench_forward(nnhip_model *mm, int B, int S, int n_cached,
                        int quantized, int iters, float *ms) {
  return guard([&] {
    NNHIP_REQUIRE(mm && ms && B > 0 && S > 0 && n_cached >= 0 && iters > 0,
                  nnhip::kErrArg, "nnhip_bench_forward: bad argument");
    nnhip::Model &m = *mm->m;
    NNHIP_REQUIRE(n_cached + S <= m.max_seq, nnhip::kErrCapacity,
                  "nnhip_bench_forward: n_cached + S exceeds max_seq_len");
    hipStream_t st = m.ctx->stream;
    nnhip::KVCache kv(&m, B, m.max_seq, quantized != 0);
    if (kv.q8) {
      NNHIP_CHECK(hipMemsetAsync(kv.kq.p, 0, kv.kq.bytes(), st));
      NNHIP_CHECK(hipMemsetAsync(kv.vq.p, 0, kv.vq.bytes(), st));
      nnhip::launch_fill(st, kv.ks.p, (int64_t)kv.ks.n, 1.f);
      nnhip::launch_fill(st, kv.vs.p, (int64_t)kv.vs.n, 1.f);
    } else {
      NNHIP_CHECK(hipMemsetAsync(kv.k.p, 0, kv.k.bytes(), st));
      NNHIP_CHECK(hipMemsetAsync(kv.v.p, 0, kv.v.bytes(), st));
    }
    std::vector<int32_t> lens(B, n_cached);
    NNHIP_CHECK(hipMemcpyAsync(kv.len.p, lens.data(), (size_t)B * 4,
                               hipMemcpyHostToDevice, st));
    nnhip::DevBuf<int32_t> ids((size_t)B * S);
    NNHIP_CHECK(hipMemsetAsync(ids.p, 0, ids.bytes(), st));
    nnhip::DevBuf<float> logits((size_t)B * S * m.V);
    auto fwd = [&] {
      m.forward(&kv, 0, ids.p, S, B, S, kv.len.p, 0, nullptr, n_cached + S,
                logits.p, false);
    };
    fwd();  // sizes the workspace outside the capture
    NNHIP_CHECK(hipStreamSynchronize(st));
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    NNHIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    try {
      fwd();
    } catch (...) {
      hipGraph_t g2 = nullptr;
      (void)hipStreamEndCapture(st, &g2);
      if (g2) (void)hipGraphDestroy(g2);
      throw;
    }
    NNHIP_CHECK(hipStreamEndCapture(st, &graph));
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    NNHIP_CHECK(ie);
    struct ExecGuard {
      hipGraphExec_t e;
      ~ExecGuard() { (void)hipGraphExecDestroy(e); }
    } eg{exec};
    struct Events {
      hipEvent_t e[2] = {nullptr, nullptr};
      ~Events() { for (hipEvent_t x : e) if (x) (void)hipEventDestroy(x); }
    } ev;
    NNHIP_CHECK(hipEventCreate(&ev.e[0]));
    NNHIP_CHECK(hipEventCreate(&ev.e[1]));
    NNHIP_CHECK(hipGraphLaunch(exec, st));  // warm-up replay
    NNHIP_CHECK(hipEventRecord(ev.e[0], st));
    for (int i = 0; i < iters; ++i) NNHIP_CHECK(hipGraphLaunch(exec, st));
    NNHIP_CHECK(hipEventRecord(ev.e[1], st));
    NNHIP_CHECK(hipEventSynchronize(ev.e[1]));
    float t = 0.f;
    NNHIP_CHECK(hipEventElapsedTime(&t, ev.e[0], ev.e[1]));
    *ms = t / iters;
  });
}

}  // extern "C"

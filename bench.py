#!/usr/bin/env python3
"""Speculative-decoding benchmark on one MI355X.

Workload (one "step"): sampled speculative decoding of 32 independent
sequences with an int8 weight-quantised target (12 layers, d_model 1024,
16 heads of 64, MLP 4096, vocab 32000) and draft (4 layers, d_model 512,
8 heads, MLP 2048), prompts of 256 uniform random ids, k = 5, temperature
1.0, 128 new tokens per sequence, Philox uniforms.  Weights are N(0, 0.02)
from a seeded generator (synthetic; no checkpoints).

value = committed tokens per second of the decode loop (accepted drafts plus
one resample or bonus per cycle, prefill excluded), timed by HIP events on
the library's stream around the cycle loop, with fp32 KV caches.  Also
reported: the same workload with int8 KV caches (kv_int8, the reference's
quantized_cache option), the batch-1 int8 greedy configuration (6L/512
target, 2L/256 draft, k=4, 256 new), the roofline of the dominant kernel,
and the oracle timed on the host as the CPU baseline.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neural-network_amd", "python"))

import nnhip  # noqa: E402

HBM_PEAK_GBS = 8000.0
TARGET = dict(vocab=32000, d=1024, H=16, F=4096, L=12)
DRAFT = dict(vocab=32000, d=512, H=8, F=2048, L=4)
B, P, K_LOOK, NEW, TEMP = 32, 256, 5, 128, 1.0
CFG2_T = dict(vocab=4096, d=512, H=8, F=2048, L=6)
CFG2_D = dict(vocab=4096, d=256, H=4, F=1024, L=2)
MAX_SEQ = 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_model(ctx, cfg, seed):
    m = nnhip.Decoder(ctx, cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                      cfg["L"], MAX_SEQ)
    m.init_normal(seed, 0.02)
    m.quantize()
    return m


def weight_bytes(cfg):
    """int8 codes + fp32 scales and biases of every Dense, per forward."""
    d, F, V, L = cfg["d"], cfg["F"], cfg["vocab"], cfg["L"]
    dense = L * (4 * d * d + 3 * d * F) + d * V
    outs = L * (4 * d + 2 * F + d) + V
    return dense + 8 * outs


def kv_bytes(cfg, n_keys, q8=False):
    """K and V read by one forward over n_keys cached positions: fp32 rows,
    or int8 codes plus one fp32 scale per (head, position) row."""
    if q8:
        H = cfg["H"]
        return cfg["L"] * 2 * n_keys * (cfg["d"] + 4 * H)
    return cfg["L"] * 2 * n_keys * cfg["d"] * 4


def cycle_bytes(ctx_len, k, Bn, q8=False, target=TARGET, draft=DRAFT):
    """Algorithmic HBM bytes of one cycle at mean context ctx_len: verify
    (weights once, k+1 rows of KV per sequence), k draft forwards (the
    catch-up token rides in the first of them) and the logits written and
    read by sampling."""
    v = weight_bytes(target) + Bn * kv_bytes(target, ctx_len + k + 1, q8)
    dr = k * (weight_bytes(draft) + Bn * kv_bytes(draft, ctx_len + k, q8))
    lg = Bn * (2 * k + 1) * target["vocab"] * 4 * 2
    return v + dr + lg


def attention_bytes(Bn, S, H, D, n_keys, q8=False):
    kv = 2 * Bn * H * n_keys * (D + 4 if q8 else D * 4)
    return kv + 2 * Bn * S * H * D * 4


def run_cfg4(ctx, steps, warmup, models=None, q8=False):
    if models is None:
        log("building cfg4 models (init + int8 quantisation on device)")
        t = make_model(ctx, TARGET, 1234)
        d = make_model(ctx, DRAFT, 5678)
        rng = np.random.default_rng(2024)
        prompts = rng.integers(0, TARGET["vocab"], (B, P)).astype(np.int32)
    else:
        t, d, prompts = models
    for i in range(warmup):
        log(f"warmup {i}" + (" (int8 KV cache)" if q8 else ""))
        t.generate_speculative_batch(d, prompts, NEW, K_LOOK, TEMP, 42,
                                     quantized_cache=q8)
    ctx.sync()
    dec_ms, wall, toks, stats_all = 0.0, 0.0, 0, []
    for i in range(steps):
        t0 = time.perf_counter()
        out, stats, tm = t.generate_speculative_batch(d, prompts, NEW, K_LOOK,
                                                      TEMP, 42,
                                                      quantized_cache=q8)
        ctx.sync()
        wall += time.perf_counter() - t0
        dec_ms += tm.decode_ms
        toks += B * (NEW - 1)
        stats_all = stats
        log(f"step {i}: decode {tm.decode_ms:.2f} ms prefill "
            f"{tm.prefill_ms:.2f} ms cycles {tm.cycles_launched}")
    cycles = max(s.cycles for s in stats_all)
    acc = sum(s.accepted for s in stats_all)
    drafted = sum(s.drafted for s in stats_all)
    ties = sum(s.ties for s in stats_all)
    res = dict(value=toks / (dec_ms / 1e3), wall_s=wall, decode_ms=dec_ms,
               steps=steps, cycles=cycles, accepted=acc, drafted=drafted,
               ties=ties, prefill_ms=tm.prefill_ms,
               tokens_per_cycle_per_seq=(NEW - 1) / max(cycles, 1))
    # algorithmic-byte roofline of the whole decode loop
    ctx_mid = P + NEW // 2
    bytes_total = cycles * cycle_bytes(ctx_mid, K_LOOK, B, q8)
    res["loop_bytes"] = bytes_total
    res["loop_GBs"] = bytes_total / (dec_ms / steps / 1e3) / 1e9
    res["models"] = (t, d, prompts)
    return res


def run_cfg2(ctx):
    log("batch-1 int8 greedy configuration")
    t = make_model(ctx, CFG2_T, 11)
    d = make_model(ctx, CFG2_D, 12)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, 4096, (1, 128)).astype(np.int32)
    t.generate_speculative_batch(d, prompt, 256, 4, 0.0, 42)
    out, stats, tm = t.generate_speculative_batch(d, prompt, 256, 4, 0.0, 42)
    # the same models and prompt at the headline's lookahead (k = 5)
    t.generate_speculative_batch(d, prompt, 256, 5, 0.0, 42)
    _, stats5, tm5 = t.generate_speculative_batch(d, prompt, 256, 5, 0.0, 42)
    # the target's GEMV at the verify shape (k + 1 = 5 rows): gate/up and
    # the lm head, int8 codes read once per launch
    gemv = {}
    for name, K_, N_ in (("gate/up", 512, 4096), ("lm head", 512, 4096)):
        ms = nnhip.bench_linear(ctx, 5, K_, N_, 1, iters=200, nbuf=4)
        byt = N_ * K_ + 8 * N_ + 5 * K_ * 4 + 5 * N_ * 4
        gemv[name] = dict(us=round(ms * 1e3, 2),
                          GBs=round(byt / (ms / 1e3) / 1e9, 1))
    t.free(); d.free()
    cyc = stats[0].cycles
    byt = cyc * cycle_bytes(128 + 128, 4, 1, target=CFG2_T, draft=CFG2_D)
    gbs = byt / (tm.decode_ms / 1e3) / 1e9
    cyc5 = stats5[0].cycles
    byt5 = cyc5 * cycle_bytes(128 + 128, 5, 1, target=CFG2_T, draft=CFG2_D)
    gbs5 = byt5 / (tm5.decode_ms / 1e3) / 1e9
    return dict(tokens_per_s=255 / (tm.decode_ms / 1e3),
                decode_ms=tm.decode_ms, cycles=cyc,
                ms_per_cycle=round(tm.decode_ms / max(cyc, 1), 4),
                accepted=stats[0].accepted,
                loop_roofline=dict(achieved_GBs=round(gbs, 1),
                                   frac=round(gbs / HBM_PEAK_GBS, 4)),
                gemv_verify=gemv,
                k5=dict(tokens_per_s=round(255 / (tm5.decode_ms / 1e3), 1),
                        decode_ms=round(tm5.decode_ms, 3), cycles=cyc5,
                        ms_per_cycle=round(tm5.decode_ms / max(cyc5, 1), 4),
                        accepted=stats5[0].accepted,
                        loop_roofline=dict(achieved_GBs=round(gbs5, 1),
                                           frac=round(gbs5 / HBM_PEAK_GBS, 4))))


ATTN_SHAPE = dict(B=B, S=K_LOOK + 1, H=16, D=64, n_cached=P + NEW // 2)
TRAFFIC_NOTE = os.path.join(ROOT, "profiles", "attention_verify_traffic.md")


GEMM_NOTE = os.path.join(ROOT, "profiles", "gemm_cycle_shapes.md")


def profile_value(note, key, kernel=None, cast=float):
    """A figure recorded in a profiles/ note as a `key: value` or
    `key[kernel]: value` line, or None."""
    key = (key if kernel is None else f"{key}[{kernel}]") + ":"
    try:
        with open(note) as f:
            for line in f:
                if line.startswith(key):
                    return cast(line.split(":")[1])
    except OSError:
        pass
    return None


def measured_traffic(note=TRAFFIC_NOTE, kernel=None):
    """HBM bytes per launch of a kernel as measured by the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs recorded in profiles/ (the note's
    traffic_bytes_per_launch line, or traffic_bytes_per_launch[kernel])."""
    return profile_value(note, "traffic_bytes_per_launch", kernel, int)


def roofline_attention(ctx, w4=True, q8=False):
    """Verify-step attention at the cfg4 mid-run shape: 32 sequences x 16
    heads, 6 queries, 320 cached keys (+6 new); one launch of the merged
    split kernel.  Algorithmic bytes: K and V of every visible key once
    (fp32 rows, or int8 codes and a scale per row), the queries read and
    the context rows written."""
    sh = ATTN_SHAPE
    ms = nnhip.bench_attention(ctx, sh["B"], sh["S"], sh["H"], sh["D"],
                               sh["n_cached"], iters=200, nbuf=4,
                               quantized=q8)
    byt = attention_bytes(sh["B"], sh["S"], sh["H"], sh["D"],
                          sh["n_cached"] + sh["S"], q8)
    ach = byt / (ms / 1e3) / 1e9
    if q8:
        return dict(achieved=round(ach, 1), frac=round(ach / HBM_PEAK_GBS, 4),
                    unit="GB/s", bytes_per_launch=byt,
                    us_per_launch=round(ms * 1e3, 2),
                    kernel="attn_kernel<8, 8, 4, int8 rows> (scores on the int8 MFMA)")
    return dict(bound="hbm", achieved=round(ach, 1), peak=HBM_PEAK_GBS,
                unit="GB/s", frac=round(ach / HBM_PEAK_GBS, 4),
                traffic=measured_traffic(),
                kernel=("attn_kernel<8, 8, 4> (verify, 4 key splits merged "
                        "in LDS, 2 workgroups per CU)" if w4 else
                        "attn_kernel<8, 8, 8> (verify, 8 key splits merged "
                        "in LDS)"),
                bytes_per_launch=byt, us_per_launch=round(ms * 1e3, 2))


INT8_PEAK_TOPS = 5000.0


def dense_shapes(cfg):
    """(K, N) of every Dense one forward runs, in the device's fused layout:
    q/k/v, output, gate/up (interleaved), down per layer, then the lm head."""
    d, F = cfg["d"], cfg["F"]
    return [(d, 3 * d), (d, d), (d, 2 * F), (F, d)] * cfg["L"] + \
        [(d, cfg["vocab"])]


def verify_step(ctx, t, q8=False):
    """One target forward at the verify shape (32 sequences x k+1 = 6 rows,
    320 cached positions), replayed as a HIP graph.  Algorithmic bytes:
    every int8 weight with its scales and biases once, the KV rows read,
    the logits written.  MFMA work: every projection as three int8 digit
    planes of the activations against the codes (3 x 2 x rows x K x N int8
    ops)."""
    S, n_cached = K_LOOK + 1, P + NEW // 2
    ms = nnhip.bench_forward(t, B, S, n_cached, quantized=q8, iters=50)
    rows = B * S
    byt = (weight_bytes(TARGET) + B * kv_bytes(TARGET, n_cached + S, q8) +
           rows * TARGET["vocab"] * 4)
    ops = sum(3 * 2 * rows * k_ * n_ for k_, n_ in dense_shapes(TARGET))
    gbs = byt / (ms / 1e3) / 1e9
    tops = ops / (ms / 1e3) / 1e12
    return dict(us=round(ms * 1e3, 1), bytes=byt, achieved_GBs=round(gbs, 1),
                frac_hbm=round(gbs / HBM_PEAK_GBS, 4),
                mfma_TOPS_3digit=round(tops, 1),
                frac_int8_peak=round(tops / INT8_PEAK_TOPS, 4),
                rows=rows, n_cached=n_cached,
                kv="int8" if q8 else "fp32")


# The cycle's GEMM launches (batch 32, k = 5): the 5 draft forwards on 32
# rows (d 512; the first also carries the catch-up row, 64 rows) and the
# verify forward on 192 rows (d 1024), with the kernel each runs in the
# library (nnhip_bench_linear path: 1 = GEMV over fp32 rows, 6 = LDS GEMM
# over digit planes with the lm head's tile statistics, 7 = LDS GEMM over
# digit planes, 8 = digit-plane GEMM; the digit planes of the output and
# down projections are made by act_quant_kernel, timed apart) and launches
# per cycle.
CYCLE_GEMMS = [
    # name, rows, K, N, path, kernel family, launches per cycle
    ("draft qkv", 32, 512, 1536, 8, "gemm_limb_kernel", 16),
    ("draft o", 32, 512, 512, 9, "gemm_limb_kernel", 16),
    ("draft gate/up", 32, 512, 4096, 8, "gemm_limb_kernel", 16),
    ("draft down", 32, 2048, 512, 1, "gemv16_kernel", 16),
    ("draft lm head", 32, 512, 32000, 6, "gemm_lds_kernel", 4),
    ("draft qkv (catch-up)", 64, 512, 1536, 8, "gemm_limb_kernel", 4),
    ("draft o (catch-up)", 64, 512, 512, 9, "gemm_limb_kernel", 4),
    ("draft gate/up (catch-up)", 64, 512, 4096, 8, "gemm_limb_kernel", 4),
    ("draft down (catch-up)", 64, 2048, 512, 1, "gemv16_kernel", 4),
    ("draft lm head (catch-up)", 32, 512, 32000, 6, "gemm_lds_kernel", 1),
    ("verify qkv", 192, 1024, 3072, 7, "gemm_lds_kernel", 12),
    ("verify o", 192, 1024, 1024, 9, "gemm_limb_kernel", 12),
    ("verify gate/up", 192, 1024, 8192, 7, "gemm_lds_kernel", 12),
    ("verify down", 192, 4096, 1024, 8, "gemm_limb_kernel", 12),
    ("verify lm head", 192, 1024, 32000, 6, "gemm_lds_kernel", 1),
]


def gemm_bytes(rows, K, N, path):
    """Algorithmic bytes of one GEMM launch: int8 codes, fp32 scale and bias
    per column, the activations as read (three int8 digit planes and an
    exponent per row -- per 64-wide K chunk for path 9, the output
    projection -- or fp32 rows for the GEMV), fp32 outputs written (tile
    statistics instead of logits are not counted: the logits are written
    too)."""
    exps = 4 * (K // 64) if path == 9 else 4
    act = rows * K * 4 if path in (1, 3) else rows * (3 * K + exps)
    return N * K + 8 * N + act + rows * N * 4


GEMM_LAUNCH_SCALE = 10


def gemm_table(ctx):
    """Each GEMM shape of the cycle timed alone (HIP events around
    GEMM_LAUNCH_SCALE x its launches per cycle, after one warm-up launch,
    over 4 weight sets), its bytes and int8 MFMA rate, then per kernel
    family the launch-weighted totals per cycle.  The launch counts follow
    the cycle's, so a kernel trace of `bench.py --gemm-probe` (which runs
    this table) averages each family over the same mix of shapes."""
    rows_out, fam = [], {}
    for name, rows, K, N, path, kern, n in CYCLE_GEMMS:
        ms = nnhip.bench_linear(ctx, rows, K, N, path,
                                iters=GEMM_LAUNCH_SCALE * n, nbuf=4)
        us = ms * 1e3
        byt = gemm_bytes(rows, K, N, path)
        ops = 3 * 2 * rows * K * N
        rows_out.append(dict(name=name, rows=rows, K=K, N=N, kernel=kern,
                             launches=n, us=round(us, 2),
                             GBs=round(byt / us / 1e3, 1),
                             TOPS_3digit=round(ops / us / 1e6, 1)))
        f = fam.setdefault(kern, dict(us=0.0, bytes=0, ops=0, launches=0))
        f["us"] += n * us
        f["bytes"] += n * byt
        f["ops"] += n * ops
        f["launches"] += n
    families = {k: dict(us_per_cycle=round(v["us"], 1), launches=v["launches"],
                        achieved_GBs=round(v["bytes"] / v["us"] / 1e3, 1),
                        TOPS_3digit=round(v["ops"] / v["us"] / 1e6, 1))
                for k, v in fam.items()}
    return rows_out, families, fam


DECODE_NOTE = os.path.join(ROOT, "profiles", "decode_b32_k5_kernel_stats.md")


def roofline_gemm(fam, kern):
    """HBM roofline of one GEMM kernel family over the cycle's launches:
    launch-weighted algorithmic bytes over launch-weighted time (HIP events,
    this run; `frac`).  Beside it, the same bytes over the family's mean
    kernel duration in two committed kernel traces: of `bench.py
    --gemm-probe`, which runs the same launches as this table
    (`profile_frac`), and of the decode loop itself, where each launch
    follows other kernels and finds less of its data in cache
    (`in_loop_frac`)."""
    f = fam[kern]
    ach = f["bytes"] / f["us"] / 1e3
    byt = f["bytes"] / f["launches"]
    out = dict(bound="hbm", achieved=round(ach, 1), peak=HBM_PEAK_GBS,
               unit="GB/s", frac=round(ach / HBM_PEAK_GBS, 4),
               traffic=measured_traffic(GEMM_NOTE, kern),
               kernel=kern, launches_per_cycle=f["launches"],
               us_per_launch=round(f["us"] / f["launches"], 3),
               bytes_per_launch=int(byt),
               mfma_TOPS_3digit=round(f["ops"] / f["us"] / 1e6, 1),
               mfma_frac=round(f["ops"] / f["us"] / 1e6 / INT8_PEAK_TOPS, 4))
    for tag, note, key in (("profile", GEMM_NOTE, "kernel_trace_us_per_launch"),
                           ("in_loop", DECODE_NOTE, "in_loop_us_per_launch")):
        us = profile_value(note, key, kern)
        out[f"{tag}_us_per_launch"] = us
        out[f"{tag}_frac"] = (round(byt / us / 1e3 / HBM_PEAK_GBS, 4)
                              if us else None)
    return out


def cfg3_cfg5(ctx):
    """The attention microbench (16 x 8 heads of 64, 2048 cached + 8 new
    queries, fp32) and the acceptance microbench (256 sequences x 8
    positions x vocab 32000, T = 1), 1000 timed launches each."""
    ms = nnhip.bench_attention(ctx, 16, 8, 8, 64, 2048, iters=1000, nbuf=4)
    byt = attention_bytes(16, 8, 8, 64, 2048 + 8)
    c3 = dict(us=round(ms * 1e3, 2), bytes=byt,
              achieved_GBs=round(byt / (ms / 1e3) / 1e9, 1),
              frac=round(byt / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4))
    c5 = cfg5_accept(ctx)
    return c3, c5


CFG5 = dict(B=256, k=8, V=32000)
CFG5_NOTE = os.path.join(ROOT, "profiles", "cfg5_accept_kernel_stats.md")


def cfg5_accept(ctx, iters=1000):
    """Logits in, (accepted count, resampled token) out, on
    nnhip_spec_accept's path: the state reset, the rows' statistics up to
    each sequence's first rejection (the reference forms p_j only until the
    first rejection, layer.cpp:1581-1630; rows after it are skipped), the
    accept decisions, the residual draw and the state update, per launch;
    1000 launches over 3 sets of logits, each set's draft ids drawn from its
    own draft probabilities.  Bytes: `bytes` counts what the algorithm must
    read, the target and draft rows up to and including each sequence's
    first rejection (all k when every draft is accepted), 2 x V x 4 B a row,
    from input set 0's accepted counts (the other sets are drawn the same
    way); `dense_bytes` is every logit once, 2 x 256 x 8 x 32000 x 4 =
    524,288,000 B, for comparison with a kernel that reads every row."""
    c = CFG5
    ms5, nacc = nnhip.bench_spec_accept(ctx, c["B"], c["k"], c["V"], 1.0,
                                        iters=iters, nbuf=3)
    rows = int(np.minimum(np.asarray(nacc) + 1, c["k"]).sum())
    b5 = rows * 2 * c["V"] * 4
    dense = 2 * c["B"] * c["k"] * c["V"] * 4
    # the kernel trace of `bench.py --cfg5-probe` (this function alone):
    # the mean durations of its kernels summed per launch
    us_prof = profile_value(CFG5_NOTE, "kernel_trace_us_per_launch")
    return dict(us=round(ms5 * 1e3, 2), bytes=b5, rows_read=rows,
                dense_bytes=dense, iters=iters,
                achieved_GBs=round(b5 / (ms5 / 1e3) / 1e9, 1),
                frac=round(b5 / (ms5 / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                dense_equivalent_GBs=round(dense / (ms5 / 1e3) / 1e9, 1),
                profile_us=us_prof,
                profile_frac=(round(b5 / us_prof / 1e3 / HBM_PEAK_GBS, 4)
                              if us_prof else None),
                mean_accepted=round(float(np.mean(nacc)), 3),
                timed="reset + row statistics up to the first rejection + "
                      "accept decisions + residual draw, logits in")


def cfg5_probe():
    """For rocprofv3 --kernel-trace: the acceptance microbench alone."""
    log(json.dumps(cfg5_accept(nnhip.Context(0))))


def traffic_probe():
    """For rocprofv3 --pmc runs: a plain device copy of 256 MiB (the
    calibration of FETCH_SIZE / WRITE_SIZE) followed by 20 launches of the
    verify attention kernel at the roofline shape."""
    copy_calibration()
    ctx = nnhip.Context(0)
    sh = ATTN_SHAPE
    ms = nnhip.bench_attention(ctx, sh["B"], sh["S"], sh["H"], sh["D"],
                               sh["n_cached"], iters=20, nbuf=4)
    log(f"attention: {ms * 1e3:.2f} us per launch, algorithmic bytes "
        f"{attention_bytes(sh['B'], sh['S'], sh['H'], sh['D'], sh['n_cached'] + sh['S'])}")


# the batch-32 cycle's attention launches at mid-run context: the verify
# step (16 heads, k + 1 = 6 queries) and a drafting step (8 heads, 1 query)
ATTN_PROBE_SHAPES = [("verify", B, K_LOOK + 1, 16, 64, P + NEW // 2),
                     ("draft", B, 1, 8, 64, P + NEW // 2 + 30)]


def attn_probe():
    """For rocprofv3 --pmc runs: the verify and drafting attention
    launches over fp32 and int8 KV rows, 50 launches each."""
    ctx = nnhip.Context(0)
    for name, b, s, h, d, n in ATTN_PROBE_SHAPES:
        for q8 in (False, True):
            ms = nnhip.bench_attention(ctx, b, s, h, d, n, iters=50, nbuf=4,
                                       quantized=q8)
            byt = attention_bytes(b, s, h, d, n + s, q8)
            log(f"{name} attention {'int8' if q8 else 'fp32'} rows: "
                f"{ms * 1e3:.2f} us, {byt} algorithmic bytes, "
                f"{byt / (ms / 1e3) / 1e9:.1f} GB/s")


def copy_calibration():
    """A plain device copy of 256 MiB, three times: the reference point for
    scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    b_ = torch.empty_like(a)
    for _ in range(3):
        b_.copy_(a)
    torch.cuda.synchronize()
    log(f"copied {a.numel() * 4} bytes x 3")


def gemm_probe():
    """For rocprofv3 runs: the copy calibration, then the GEMM table of
    the batch-32 cycle exactly as bench.py times it (gemm_table: one
    warm-up launch and GEMM_LAUNCH_SCALE x the cycle's launches per shape,
    the kernel alone over digit planes made once) and the prefill's gate/up
    projection (8192 rows = 32 prompts x 256, 21 launches)."""
    copy_calibration()
    ctx = nnhip.Context(0)
    rows_out, families, _ = gemm_table(ctx)
    for r in rows_out:
        log(f"{r['name']}: {r['rows']}x{r['K']}x{r['N']} {r['us']:.2f} us")
    log(json.dumps(families))
    ms = nnhip.bench_linear(ctx, B * P, 1024, 8192, 7, iters=20, nbuf=2)
    log(f"prefill gate/up: {B * P}x1024x8192 path 7 {ms * 1e3:.2f} us")


# batch-1 GEMV shapes of the target's verify step (k + 1 = 5 rows) and the
# draft's single row: q/k/v, gate/up and the lm head
GEMV_SHAPES = [(5, 512, 1536), (5, 512, 4096), (5, 512, 4096),
               (1, 256, 768), (1, 256, 2048), (1, 256, 4096)]


def gemv_probe():
    """For rocprofv3 --pmc runs: the copy calibration, then the batch-1
    GEMVs (fp32 rows x int8 codes), 20 launches each."""
    copy_calibration()
    ctx = nnhip.Context(0)
    for rows, K, N in GEMV_SHAPES:
        ms = nnhip.bench_linear(ctx, rows, K, N, 1, iters=20, nbuf=4)
        log(f"gemv {rows}x{K}x{N}: {ms * 1e3:.2f} us")


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(models, budget_s=20.0, sample_new=24):
    """The oracle -- the C restatement of the reference's CPU path: per-call
    dequantisation of every int8 weight (quantization.cpp:89-125) and the
    fp32 product in column blocks, attention heads in parallel, as the
    reference's ThreadPool splits them -- on the same workload's weights
    and prompts, one thread per core available to this process (the
    reference's hardware_concurrency rule, thread_pool.cpp:9-10).  The
    reference is batch-1, so sequences run one after another, as many as
    fit in about budget_s seconds of decode (at least one)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py as O
    t, d, prompts = models
    threads = len(os.sched_getaffinity(0))
    log("cpu baseline: copying weights to the host")
    ot = O.Model(TARGET["vocab"], TARGET["d"], TARGET["H"], TARGET["F"],
                 TARGET["L"], MAX_SEQ,
                 [t.get_param(i) for i in range(t.num_params())], True)
    od = O.Model(DRAFT["vocab"], DRAFT["d"], DRAFT["H"], DRAFT["F"],
                 DRAFT["L"], MAX_SEQ,
                 [d.get_param(i) for i in range(d.num_params())], True)
    O.set_threads(threads)
    dec_ms, pre_ms, toks, seqs = 0.0, 0.0, 0, 0
    try:
        while seqs < len(prompts) and (seqs == 0 or dec_ms < budget_s * 1e3):
            log(f"cpu baseline: sequence {seqs} ({threads} threads)")
            _, st = O.generate_speculative(ot, od, prompts[seqs], sample_new,
                                           K_LOOK, TEMP, 42, seq=seqs)
            dec_ms += st.decode_ms
            pre_ms += st.prefill_ms
            toks += sample_new - 1
            seqs += 1
    finally:
        O.set_threads(1)
    return dict(value=round(toks / (dec_ms / 1e3), 3), unit="tokens/s",
                cores=threads, kind="port", cpu=cpu_model(),
                blas=("none: the port's own column-blocked fp32 loops (the "
                      "reference calls cblas_sgemm)"),
                sample=(f"sequences 0..{seqs - 1} of the workload one after "
                        f"another, {sample_new} new tokens each after the "
                        f"256-id prompt; decode loop only ({dec_ms / 1e3:.1f} "
                        f"s; prefill {pre_ms / 1e3:.1f} s excluded), "
                        f"{threads} threads"))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batch1", action="store_true")
    ap.add_argument("--no-mt19937", action="store_true",
                    help="skip the decode loop on the reference's "
                         "std::mt19937 generator")
    ap.add_argument("--no-kv-int8", action="store_true",
                    help="skip the secondary run with int8 KV caches "
                         "(generate_speculative(..., quantized_cache=true))")
    ap.add_argument("--batch1-only", action="store_true",
                    help="only run the batch-1 int8 greedy configuration "
                         "and print its figures (for profiling)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the copy calibration and the attention "
                         "kernel (for rocprofv3 --pmc)")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only run the copy calibration and the cycle's GEMM "
                         "shapes (for rocprofv3 --pmc)")
    ap.add_argument("--attn-probe", action="store_true",
                    help="only the attention launches of the cycle over fp32 "
                         "and int8 KV rows (for rocprofv3 --pmc)")
    ap.add_argument("--cfg5-probe", action="store_true",
                    help="only run the acceptance microbench (for "
                         "rocprofv3 --kernel-trace)")
    ap.add_argument("--gemv-probe", action="store_true",
                    help="only run the copy calibration and the batch-1 "
                         "GEMVs (for rocprofv3 --pmc)")
    ap.add_argument("--loop-only", action="store_true",
                    help="only the decode loop (no microbenchmarks): for "
                         "kernel traces of the cycle")
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch each kernel of a cycle separately instead "
                         "of replaying one HIP graph per cycle")
    ap.add_argument("--option", action="append", default=[],
                    metavar="KEY=VALUE",
                    help="nnhip_set_option before the run (repeatable)")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU only: the workload's sequences "
              "shard over GPUs with no exchange step (each GPU runs its own "
              "copy of this measurement on its share of the batch)",
              file=sys.stderr)
        sys.exit(2)
    if a.traffic_probe:
        traffic_probe()
        return
    if a.gemm_probe:
        gemm_probe()
        return
    if a.gemv_probe:
        gemv_probe()
        return
    if a.cfg5_probe:
        cfg5_probe()
        return
    if a.attn_probe:
        attn_probe()
        return
    ctx = nnhip.Context(0)
    if a.no_graphs:
        ctx.set_option("graphs", 0)
    for kv in a.option:
        key, val = kv.split("=")
        ctx.set_option(key, int(val))
    if a.batch1_only:
        print(json.dumps({"batch1": run_cfg2(ctx)}), flush=True)
        return
    r = run_cfg4(ctx, a.steps, a.warmup)
    if a.loop_only:
        print(json.dumps({"value": round(r["value"], 1), "unit": "tokens/s",
                          "decode_ms_per_step": round(r["decode_ms"] / a.steps, 2),
                          "cycles": r["cycles"]}), flush=True)
        return
    attn = roofline_attention(ctx, w4="attn_w4=0" not in a.option)
    log("verify step, GEMM shapes, attention and acceptance microbenches")
    ver = verify_step(ctx, r["models"][0])
    gemms, families, fam = gemm_table(ctx)
    dominant = max(fam, key=lambda k: fam[k]["us"])
    roof = roofline_gemm(fam, dominant)
    c3, c5 = cfg3_cfg5(ctx)
    kv8 = None
    if not a.no_kv_int8:
        r8 = run_cfg4(ctx, 1, 1, models=r["models"], q8=True)
        kv8 = {"value": round(r8["value"], 1), "unit": "tokens/s",
               "decode_ms": round(r8["decode_ms"], 2),
               "cycles": r8["cycles"],
               "acceptance": round(r8["accepted"] / max(r8["drafted"], 1), 4),
               "loop_roofline": {
                   "achieved_GBs": round(r8["loop_GBs"], 1),
                   "frac": round(r8["loop_GBs"] / HBM_PEAK_GBS, 4)},
               "attention": roofline_attention(ctx, q8=True),
               "verify_step": verify_step(ctx, r["models"][0], q8=True)}
    # the same loop on the reference's generator (option "rng" 1: one
    # std::mt19937 per sequence, drawn in the reference's order); its draws
    # differ from the Philox stream's, so do the cycle count and acceptance
    mt = None
    if not a.no_mt19937:
        ctx.set_option("rng", 1)
        try:
            rm = run_cfg4(ctx, 1, 1, models=r["models"])
        finally:
            ctx.set_option("rng", 0)
        mt = {"value": round(rm["value"], 1), "unit": "tokens/s",
              "decode_ms": round(rm["decode_ms"], 2), "cycles": rm["cycles"],
              "ms_per_cycle": round(rm["decode_ms"] / rm["cycles"], 4),
              "acceptance": round(rm["accepted"] / max(rm["drafted"], 1), 4)}
    b1 = None if a.no_batch1 else run_cfg2(ctx)
    cpu = None if a.no_cpu_baseline else cpu_baseline(r["models"])
    ms_step = r["wall_s"] / a.steps * 1e3
    line = {
        "metric": "accepted tokens/sec (batch 32, int8 target, k=5)",
        "value": round(r["value"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x fp32 activations (fp32 KV)",
        "data": "synthetic: seeded N(0,0.02) weights, uniform random prompts",
        "config": {"workload": "sampled speculative decode, 32 sequences, "
                               "target 12L/1024/16h/4096/V32000 int8, draft "
                               "4L/512/8h/2048 int8, prompt 256, k=5, T=1.0, "
                               "128 new", "batch": B, "lookahead": K_LOOK,
                   "new_tokens": NEW, "prompt": P},
        "decode_ms_per_step": round(r["decode_ms"] / a.steps, 2),
        "prefill_ms": round(r["prefill_ms"], 2),
        "cycles": r["cycles"],
        "ms_per_cycle": round(r["decode_ms"] / a.steps / r["cycles"], 4),
        "acceptance": round(r["accepted"] / max(r["drafted"], 1), 4),
        "ties": r["ties"],
        "loop_roofline": {"achieved_GBs": round(r["loop_GBs"], 1),
                          "frac": round(r["loop_GBs"] / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "attention_roofline": attn,
        "verify_step": ver,
        "gemm_families": families,
        "gemm_shapes": gemms,
        "cfg3_attention": c3,
        "cfg5_accept": c5,
        "kv_int8": kv8,
        "rng_mt19937": mt,
        "batch1": b1,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

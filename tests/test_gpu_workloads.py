"""The benchmark workloads themselves on the device, against the oracle (GPU).

* The batch-32 sampled speculative decode at full model size: target
  12L/1024/16h/4096/V32000 and draft 4L/512/8h/2048, int8 weights, prompts of
  256 ids, k = 5, T = 1.0, Philox uniforms.  The device runs all 32
  sequences in lockstep with the decode loop's own kernels (draft sampling
  from the draft lm head's tile statistics, the verify rows' statistics, the
  accept / residual kernel); a stated subset of sequences is compared with
  the oracle's single-sequence runs (sequence index b keys the uniforms).
  max_new is 24 instead of 128 to keep the oracle's run short; every kernel
  and shape of the loop is the same, the contexts are shorter.
* The acceptance microbenchmark at its full size: 256 sequences x k = 8 x
  V = 32000, target and draft logits N(0, 2), one accept uniform per
  position and one resample uniform per sequence, through nnhip_spec_accept
  (the loop's target_stats_kernel + accept_kernel).

Sampled decisions may differ from the oracle's only where the oracle's
closest random decision lies within 1e-5 of its boundary.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle_py as O
from gpu_util import nnhip
from test_gpu_decode import check_stream

pytestmark = pytest.mark.gpu

CFG4_T = dict(vocab=32000, d=1024, H=16, F=4096, L=12)
CFG4_D = dict(vocab=32000, d=512, H=8, F=2048, L=4)
THREADS = 16


def device_and_oracle(ctx, cfg, seed, max_seq=1024):
    """Seeded N(0, 0.02) weights made on the device, int8-quantised there;
    the oracle gets the same fp32 weights and quantises them itself (the
    int8 codes are bit-exact, test_params_roundtrip_and_quantized_codes)."""
    gm = nnhip.Decoder(ctx, cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                       cfg["L"], max_seq)
    gm.init_normal(seed, 0.02)
    gm.quantize()
    params = [gm.get_param(i) for i in range(gm.num_params())]
    om = O.Model(cfg["vocab"], cfg["d"], cfg["H"], cfg["F"], cfg["L"],
                 max_seq, params, True)
    return gm, om


def test_cfg4_sampled_batch32_matches_oracle(ctx):
    B, P, new, k, T, seed = 32, 256, 24, 5, 1.0, 42
    gt, ot = device_and_oracle(ctx, CFG4_T, 1234)
    gd, od = device_and_oracle(ctx, CFG4_D, 5678)
    rng = np.random.default_rng(2024)
    prompts = rng.integers(0, CFG4_T["vocab"], (B, P)).astype(np.int32)
    got, stats, tm = gt.generate_speculative_batch(gd, prompts, new, k, T,
                                                   seed)
    assert got.shape == (B, P + new)
    np.testing.assert_array_equal(got[:, :P], prompts)
    assert ((got >= 0) & (got < CFG4_T["vocab"])).all()
    for b in range(B):
        s = stats[b]
        # every cycle commits its accepted drafts plus one token
        assert s.accepted + s.resampled + s.bonus + 1 == new, b
        assert s.drafted >= s.accepted
    O.set_threads(THREADS)
    try:
        diverged = 0
        for b in (0, 13, 31):
            i = check_stream(ot, od, got[b], prompts[b], new, k, T, seed,
                             seq=b, dev=stats[b], what=f"cfg4 b={b}")
            diverged += i is not None
    finally:
        O.set_threads(1)
    # a divergence needs a decision within 1e-5 of its boundary: rare
    assert diverged <= 1
    gt.free(); gd.free()


def test_cfg4_greedy_batch32_matches_oracle(ctx):
    """The same models in greedy mode (T = 0): exact streams."""
    B, P, new, k = 32, 256, 12, 5
    gt, ot = device_and_oracle(ctx, CFG4_T, 1234)
    gd, od = device_and_oracle(ctx, CFG4_D, 5678)
    rng = np.random.default_rng(2025)
    prompts = rng.integers(0, CFG4_T["vocab"], (B, P)).astype(np.int32)
    got, stats, _ = gt.generate_speculative_batch(gd, prompts, new, k, 0.0, 42)
    O.set_threads(THREADS)
    try:
        for b in (0, 31):
            want, ost = O.generate_speculative(ot, od, prompts[b], new, k, 0.0,
                                               42, seq=b)
            np.testing.assert_array_equal(got[b], want)
            assert stats[b].accepted == ost.accepted
    finally:
        O.set_threads(1)
    gt.free(); gd.free()


def oracle_probs(rows, T):
    with ThreadPoolExecutor(THREADS) as ex:
        return np.stack(list(ex.map(lambda r: O.get_probs(r, T), rows)))


@pytest.mark.parametrize("T", [1.0, 0.0])
def test_cfg5_accept_batch256_matches_oracle(ctx, T):
    B, k, V = 256, 8, 32000
    rng = np.random.default_rng(505)
    tl = (rng.standard_normal((B, k, V), np.float32) * np.float32(2.0))
    dl = (rng.standard_normal((B, k, V), np.float32) * np.float32(2.0))
    ua = rng.random((B, k), np.float32)
    ur = rng.random(B, np.float32)
    ud = rng.random((B, k))
    Tq = T if T > 0 else 1.0
    q = oracle_probs(dl.reshape(-1, V), Tq).reshape(B, k, V)
    # draft ids drawn from the draft probabilities by a separate stream
    cand = np.array([[O.sample(q[b, j], ud[b, j]) for j in range(k)]
                     for b in range(B)], np.int32)
    dev = {}
    for name, a in (("tl", tl), ("dl", dl), ("cand", cand), ("ua", ua),
                    ("ur", ur)):
        dev[name] = ctx.array(np.ascontiguousarray(a))
    n_acc = ctx.array(shape=(B,), dtype=np.int32)
    tok = ctx.array(shape=(B,), dtype=np.int32)
    nnhip.call("nnhip_spec_accept", ctx.h, dev["tl"].p, dev["dl"].p,
               dev["cand"].p, dev["ua"].p, dev["ur"].p, B, k, V, T, n_acc.p,
               tok.p)
    g_n, g_tok = n_acc.numpy(), tok.numpy()
    # T <= 0: get_probs gives the one-hot of the first argmax (layer.cpp:
    # 1413-1424), the greedy accept test's target
    p = oracle_probs(tl.reshape(-1, V), T).reshape(B, k, V)
    mismatches = 0
    for b in range(B):
        if T > 0:
            O.decision_margin(reset=True)
            n, t, _ = O.accept_step(p[b], q[b], cand[b], False, False, ua[b],
                                    ur[b])
            margin = O.decision_margin(reset=True)
        else:
            n, t, _ = O.accept_step(p[b], q[b], cand[b], True, False, ua[b],
                                    ur[b])
            margin = 1.0
        if (g_n[b], g_tok[b]) != (n, t):
            assert margin < 1e-5, (b, g_n[b], n, g_tok[b], t, margin)
            mismatches += 1
    assert mismatches <= 2
    if T > 0:
        # random N(0, 2) rows: some sequences reject at 0, some accept
        assert (g_n == 0).any() and (g_n > 0).any()
        assert (g_tok >= 0).all() or (g_n == k).any()
    for a in list(dev.values()) + [n_acc, tok]:
        a.free()

"""The benchmark workloads themselves on the device, against the oracle (GPU).

* The batch-32 sampled speculative decode at full model size: target
  12L/1024/16h/4096/V32000 and draft 4L/512/8h/2048, int8 weights, prompts of
  256 ids, k = 5, T = 1.0, Philox uniforms (and once more on the
  reference's std::mt19937, two sequences compared).  The device runs all 32
  sequences in lockstep with the decode loop's own kernels (draft sampling
  from the draft lm head's tile statistics, the verify rows' statistics, the
  accept / residual kernel) over the full 128 new tokens; a stated subset
  of six sequences (the first and the last to finish, one of median length,
  and fixed indices) is compared with the oracle's single-sequence runs
  (sequence index b keys the uniforms), and two sequences in greedy mode.
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


@pytest.fixture(scope="module")
def cfg4(ctx):
    """The batch-32 workload as the benchmark runs it: both models, the 32
    prompts, and the device's sampled (T = 1) and greedy runs at the full
    128 new tokens per sequence."""
    B, P, new, k, seed = 32, 256, 128, 5, 42
    gt, ot = device_and_oracle(ctx, CFG4_T, 1234)
    gd, od = device_and_oracle(ctx, CFG4_D, 5678)
    rng = np.random.default_rng(2024)
    prompts = rng.integers(0, CFG4_T["vocab"], (B, P)).astype(np.int32)
    sampled = gt.generate_speculative_batch(gd, prompts, new, k, 1.0, seed)
    greedy = gt.generate_speculative_batch(gd, prompts, new, k, 0.0, seed)
    # the same sampled run on the reference's generator (std::mt19937 per
    # sequence, seeded seed + b)
    ctx.set_option("rng", 1)
    try:
        sampled_mt = gt.generate_speculative_batch(gd, prompts, new, k, 1.0,
                                                   seed)
    finally:
        ctx.set_option("rng", 0)
    yield dict(ot=ot, od=od, prompts=prompts, new=new, k=k, seed=seed,
               sampled=sampled, greedy=greedy, sampled_mt=sampled_mt)
    gt.free(); gd.free()


def sampled_subset(stats):
    """The sequences compared with the oracle: the one that finishes first
    (fewest cycles), the one that finishes last (most cycles; it runs the
    lockstep tail alone), one of median length, and sequences 0, 13, 31."""
    cyc = np.array([s.cycles for s in stats])
    order = np.argsort(cyc, kind="stable")
    first, last, mid = int(order[0]), int(order[-1]), int(order[len(order) // 2])
    seqs = [first, last, mid]
    for b in (0, 13, 31, 7, 22):
        if len(seqs) >= 6:
            break
        if b not in seqs:
            seqs.append(b)
    return seqs


def test_cfg4_sampled_batch32_device_invariants(cfg4):
    got, stats, _ = cfg4["sampled"]
    B, P, new = 32, 256, cfg4["new"]
    assert got.shape == (B, P + new)
    np.testing.assert_array_equal(got[:, :P], cfg4["prompts"])
    assert ((got >= 0) & (got < CFG4_T["vocab"])).all()
    for b in range(B):
        s = stats[b]
        # every cycle commits its accepted drafts plus one token
        assert s.accepted + s.resampled + s.bonus + 1 == new, b
        assert s.drafted >= s.accepted
    # the longest sequence reaches context 256 + 128 + k in the verify
    assert max(s.cycles for s in stats) > min(s.cycles for s in stats)
    # no cycle is launched after the last sequence finished
    assert cfg4["sampled"][2].cycles_launched == max(s.cycles for s in stats)
    assert cfg4["greedy"][2].cycles_launched == max(
        s.cycles for s in cfg4["greedy"][1])


@pytest.mark.parametrize("part", [0, 1])
def test_cfg4_sampled_batch32_full_length_matches_oracle(cfg4, part):
    """Six sequences over all 128 new tokens (contexts up to ~389 in the
    verify, the lockstep tail after the first sequence finishes), each
    against the oracle's single-sequence run keyed by its index; three per
    test to keep each test short."""
    got, stats, _ = cfg4["sampled"]
    seqs = sampled_subset(stats)[3 * part:3 * part + 3]
    O.set_threads(THREADS)
    diverged = 0
    try:
        for b in seqs:
            print(f"cfg4 sampled: sequence {b} ({stats[b].cycles} cycles)",
                  flush=True)
            i = check_stream(cfg4["ot"], cfg4["od"], got[b], cfg4["prompts"][b],
                             cfg4["new"], cfg4["k"], 1.0, cfg4["seed"], seq=b,
                             dev=stats[b], what=f"cfg4 b={b}")
            diverged += i is not None
    finally:
        O.set_threads(1)
    # a divergence needs a decision within 1e-5 of its boundary: rare
    assert diverged <= 1


def test_cfg4_mt19937_batch32_matches_oracle(cfg4):
    """The batch-32 workload with the context option "rng" 1 (the
    reference's std::mt19937, layer.cpp:1394): the first and the last
    sequence to finish over all 128 new tokens against the oracle's
    mt19937 runs (or_set_rng(1)), up to a recorded tie; the streams differ
    from the Philox run's."""
    got, stats, _ = cfg4["sampled_mt"]
    assert not np.array_equal(got, cfg4["sampled"][0])
    cyc = np.array([s.cycles for s in stats])
    seqs = [int(np.argmin(cyc)), int(np.argmax(cyc))]
    O.set_threads(THREADS)
    O.set_rng(1)
    try:
        for b in seqs:
            print(f"cfg4 mt19937: sequence {b} ({stats[b].cycles} cycles)",
                  flush=True)
            check_stream(cfg4["ot"], cfg4["od"], got[b], cfg4["prompts"][b],
                         cfg4["new"], cfg4["k"], 1.0, cfg4["seed"], seq=b,
                         dev=stats[b], what=f"cfg4 mt19937 b={b}")
    finally:
        O.set_rng(0)
        O.set_threads(1)


def test_cfg4_greedy_batch32_full_length_matches_oracle(cfg4):
    """The same models in greedy mode (T = 0), 128 new tokens: exact
    streams and acceptance counts for the first and last sequence."""
    got, stats, _ = cfg4["greedy"]
    O.set_threads(THREADS)
    try:
        for b in (0, 31):
            print(f"cfg4 greedy: sequence {b}", flush=True)
            want, ost = O.generate_speculative(
                cfg4["ot"], cfg4["od"], cfg4["prompts"][b], cfg4["new"],
                cfg4["k"], 0.0, cfg4["seed"], seq=b)
            np.testing.assert_array_equal(got[b], want)
            assert stats[b].accepted == ost.accepted
    finally:
        O.set_threads(1)


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

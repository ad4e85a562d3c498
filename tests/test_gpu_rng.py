"""The reference's std::mt19937 stream on the device (GPU).

generate_speculative and generate_advanced seed one std::mt19937 with the
caller's seed (layer.cpp:1249, 1394) and draw, in this order per cycle, the
M drafting samples (std::discrete_distribution, generate_canonical<double,
53>: two outputs each, layer.cpp:1493-1498, 1541-1558), the accept tests up
to the first rejection (uniform_real_distribution<float>: one output each,
layer.cpp:1596-1597), then the resample or the bonus sample (two outputs,
layer.cpp:1611-1630, 1643-1647); the first token and every
generate_advanced token take one double.  With the context option "rng" 1
the library does the same per sequence (seed + seq0 + b), and its streams
equal the oracle's run with or_set_rng(1) -- whose engine and draws are
pinned to libstdc++'s outputs (test_oracle_rng.py) -- exactly in
generate_advanced, and in the speculative loop up to a divergence inside a
cycle whose closest random decision lies within 1e-5 of its boundary.
Streams long enough to cross several 624-output refills of the device's
per-sequence ring.
"""
import numpy as np
import pytest

import oracle_py as O
from gpu_util import nnhip
from test_gpu_decode import TILE_D, TILE_T, TOY_D, TOY_T, check_stream, spec_pair

pytestmark = pytest.mark.gpu


@pytest.fixture
def mt_mode(ctx):
    ctx.set_option("rng", 1)
    O.set_rng(1)
    try:
        yield
    finally:
        ctx.set_option("rng", 0)
        O.set_rng(0)


@pytest.mark.parametrize("split", [0, 1])
def test_mt_speculative_batch_matches_oracle(ctx, mt_mode, split):
    """Batch of 4 at seq0 = 3, k = 4, T = 1, 260 new tokens each, with the
    accept step in one launch (split 0) and in three (split 1)."""
    ctx.set_option("accept_split", split)
    try:
        ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 40, False, std=0.3)
        rng = np.random.default_rng(41)
        prompts = rng.integers(0, 256, (4, 16)).astype(np.int32)
        got, stats, _ = gt.generate_speculative_batch(gd, prompts, 260, 4,
                                                      1.0, 123, seq0=3)
        parted = [check_stream(ot, od, got[b], prompts[b], 260, 4, 1.0, 123,
                               seq=3 + b, dev=stats[b],
                               what=f"split={split} b={b}")
                  for b in range(4)]
        # a tie is rare: most streams are equal to the end
        assert sum(i is None for i in parted) >= 3, parted
    finally:
        ctx.set_option("accept_split", 1)
    gt.free(); gd.free()


def test_mt_single_sequence_is_the_reference_seeding(ctx, mt_mode):
    """nnhip_generate_speculative (one sequence, seq 0): the engine seeded
    with the seed itself, as std::mt19937 gen(seed); a seed above 2^32 is
    taken mod 2^32, as the reference's unsigned int seed is."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 42, True, std=0.3)
    rng = np.random.default_rng(43)
    prompt = rng.integers(0, 256, 24).astype(np.int32)
    got, st = gt.generate_speculative(gd, prompt, 120, 3, 0.9, seed=2024)
    check_stream(ot, od, got, prompt, 120, 3, 0.9, 2024, dev=st)
    big, _ = gt.generate_speculative(gd, prompt, 120, 3, 0.9,
                                     seed=2024 + (1 << 32))
    np.testing.assert_array_equal(big, got)
    gt.free(); gd.free()


@pytest.mark.parametrize("max_new", [1, 2, 3, 7])
def test_mt_edge_lengths_filtered_quantized(ctx, mt_mode, max_new):
    """M = min(k, remaining) < k, no bonus draw when no room is left, the
    top-k / top-p filter on every draw, the int8 cache, no graphs."""
    ctx.set_option("graphs", 0)
    try:
        ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 44, True, std=0.3)
        rng = np.random.default_rng(45)
        prompts = rng.integers(0, 256, (3, 9)).astype(np.int32)
        got, stats, _ = gt.generate_speculative_batch(
            gd, prompts, max_new, 4, 0.8, 6, top_k=6, top_p=0.9,
            quantized_cache=True)
        for b in range(3):
            check_stream(ot, od, got[b], prompts[b], max_new, 4, 0.8, 6,
                         seq=b, dev=stats[b], what=f"b={b}", top_k=6,
                         top_p=0.9, quantized_cache=True)
    finally:
        ctx.set_option("graphs", 1)
    gt.free(); gd.free()


def test_mt_tile_sampling_matches_oracle(ctx, mt_mode):
    """Drafting from the draft lm head's tile statistics (vocabulary 2000,
    batch 16) with the mt19937 draws."""
    ot, gt, od, gd = spec_pair(ctx, TILE_T, TILE_D, 46, True, std=0.1)
    rng = np.random.default_rng(47)
    prompts = rng.integers(0, 2000, (16, 12)).astype(np.int32)
    got, stats, _ = gt.generate_speculative_batch(gd, prompts, 40, 3, 0.7, 9)
    for b in (0, 7, 15):
        check_stream(ot, od, got[b], prompts[b], 40, 3, 0.7, 9, seq=b,
                     dev=stats[b], what=f"b={b}")
    gt.free(); gd.free()


def test_mt_generate_advanced_matches_oracle(ctx, mt_mode):
    """generate_advanced: one double per token, 300 tokens (several
    refills), batch of 3 at seq0 = 5 and one sequence at seq 0; exact."""
    ot, gt, _, gd = spec_pair(ctx, TOY_T, TOY_D, 48, False, std=0.3)
    rng = np.random.default_rng(49)
    prompts = rng.integers(0, 256, (3, 7)).astype(np.int32)
    got = gt.generate_advanced_batch(prompts, 300, 1.0, 77, seq0=5)
    for b in range(3):
        want = O.generate_advanced(ot, prompts[b], 300, 1.0, 77, seq=5 + b)
        np.testing.assert_array_equal(got[b], want, err_msg=f"b={b}")
    one = gt.generate_advanced(prompts[0], 40, 0.8, seed=9,
                               top_k=8, top_p=0.95)
    want = O.generate_advanced(ot, prompts[0], 40, 0.8, 9, top_k=8,
                               top_p=0.95)
    np.testing.assert_array_equal(one, want)
    gt.free(); gd.free()


def test_mt_mode_leaves_greedy_and_philox_streams(ctx):
    """Greedy decoding draws nothing: the same stream in both modes; with
    the option back at 0 the Philox stream returns."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 50, False, std=0.3)
    rng = np.random.default_rng(51)
    prompt = rng.integers(0, 256, 20).astype(np.int32)
    runs = {}
    for mode in (1, 0):
        ctx.set_option("rng", mode)
        try:
            runs[mode] = (gt.generate_speculative(gd, prompt, 48, 4, 0.0)[0],
                          gt.generate_speculative(gd, prompt, 48, 4, 1.0,
                                                  seed=3)[0])
        finally:
            ctx.set_option("rng", 0)
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    assert not np.array_equal(runs[0][1], runs[1][1])
    check_stream(ot, od, runs[0][1], prompt, 48, 4, 1.0, 3)
    gt.free(); gd.free()


def test_mt_generate_advanced_without_cache_and_bad_option(ctx):
    """generate_advanced(use_kv_cache = false) draws the same doubles in the
    same order (layer.cpp:1269-1372); an rng value other than 0 or 1 is
    refused with NNHIP_EARG and leaves the context's stream unchanged."""
    ot, gt, _, gd = spec_pair(ctx, TOY_T, TOY_D, 52, False, std=0.3)
    rng = np.random.default_rng(53)
    prompt = rng.integers(0, 256, 9).astype(np.int32)
    ctx.set_option("rng", 1)
    O.set_rng(1)
    try:
        got = gt.generate_advanced(prompt, 30, 1.0, seed=11, use_kv_cache=False)
        want = O.generate_advanced(ot, prompt, 30, 1.0, 11, use_cache=False)
        np.testing.assert_array_equal(got, want)
        with pytest.raises(nnhip.NNHipError) as e:
            ctx.set_option("rng", 2)
        assert e.value.code == -1
        again = gt.generate_advanced(prompt, 30, 1.0, seed=11, use_kv_cache=False)
        np.testing.assert_array_equal(again, got)
    finally:
        ctx.set_option("rng", 0)
        O.set_rng(0)
    gt.free(); gd.free()


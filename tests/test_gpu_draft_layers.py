"""The persistent decoder-layer kernel (draft_layers.hip) against the oracle
and against the per-kernel path (GPU).

Forwards of up to 64 rows with one or two new positions per sequence over a
KV cache run every decoder layer (layer.cpp:1097-1114) as one kernel whose
workgroups wait on per-tile flags between its steps.  Its logits must be within 1e-4 of a row
of the oracle's cached forward (layer.cpp:1161-1193) and of the same
forward with the option off (the per-kernel MFMA / GEMV path); its cache
entries within 1e-5 of that path's.  Shapes: the batch-32 workload's draft
(4 layers, d 512, 8 heads, MLP 2048) and the batch-1 workload's draft
(2 layers, d 256, 4 heads, MLP 1024), batches that are not a multiple of
the kernel's 8-row tiles, finished sequences in the speculative loop.
"""
import numpy as np
import pytest

import oracle_py as O
from gpu_util import assert_rows_close, nnhip
from test_gpu_decode import check_stream

# The kernel is off by default (option persistent_draft = 0) and these tests
# are not run.  This kernel passed them in two GPU runs; two later variants
# of it (V rows requested before the softmax; the tile products on MFMA)
# each made a GPU memory fault on the first test, and no out-of-bounds
# access or missing wait was found in them.  Both variants are taken out,
# and the kernel stays off until such a cause is shown.
pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="persistent decoder-layer kernel is off: two of its "
                            "variants faulted the GPU with no cause found"),
]

DRAFT4 = dict(vocab=4096, d=512, H=8, F=2048, L=4)
DRAFT2 = dict(vocab=4096, d=256, H=4, F=1024, L=2)


def models(ctx, cfg, seed, max_seq=256):
    params = O.make_params(cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                           cfg["L"], seed, std=0.03)
    om = O.Model(cfg["vocab"], cfg["d"], cfg["H"], cfg["F"], cfg["L"],
                 max_seq, params, True)
    gm = nnhip.Decoder(ctx, cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                       cfg["L"], max_seq)
    gm.set_params(params)
    gm.quantize()
    return om, gm


def run_steps(ctx, gm, prompts, steps, pd):
    """Prefill (per-kernel path: many rows), then `steps` cached forwards
    of [B][S] ids each; returns the logits of every step and the cache."""
    ctx.set_option("persistent_draft", pd)
    try:
        cache = nnhip.KVCache(gm, batch=prompts.shape[0])
        gm.forward(prompts, cache)
        outs = [gm.forward(ids, cache) for ids in steps]
    finally:
        ctx.set_option("persistent_draft", 0)
    return outs, cache


@pytest.mark.parametrize("cfg,B", [(DRAFT4, 32), (DRAFT4, 3), (DRAFT2, 1),
                                   (DRAFT2, 5)])
def test_draft_layers_forward(ctx, cfg, B):
    om, gm = models(ctx, cfg, 70 + B)
    rng = np.random.default_rng(B)
    V = cfg["vocab"]
    P = 19
    prompts = rng.integers(0, V, (B, P)).astype(np.int32)
    # one position, then two, then one (the drafting steps' shapes)
    steps = [rng.integers(0, V, (B, S)).astype(np.int32) for S in (1, 2, 1)]
    got, cache = run_steps(ctx, gm, prompts, steps, 1)
    ref, cache0 = run_steps(ctx, gm, prompts, steps, 0)
    D = cfg["d"] // cfg["H"]
    for i, ids in enumerate(steps):
        for b in range(B):
            assert_rows_close(got[i][b], ref[i][b], 1e-4, f"step {i} b={b} vs per-kernel")
    for b in range(min(B, 4)):
        oc = O.Cache(om)
        om.forward(prompts[b], oc)
        for i, ids in enumerate(steps):
            want = om.forward(ids[b], oc)
            assert_rows_close(got[i][b], want, 1e-4, f"step {i} b={b} vs oracle")
    # the appended keys and values (RoPE'd k) agree with the per-kernel path
    for layer in range(cfg["L"]):
        for b in (0, B - 1):
            k1, v1 = cache.read(layer, b, cfg["H"], D)
            k0, v0 = cache0.read(layer, b, cfg["H"], D)
            assert k1.shape == k0.shape == (cfg["H"], P + 4, D)
            np.testing.assert_array_equal(k1[:, :P], k0[:, :P])
            np.testing.assert_allclose(k1, k0, atol=1e-5 * np.abs(k0).max())
            np.testing.assert_allclose(v1, v0, atol=1e-5 * np.abs(v0).max())
    cache.free(); cache0.free()
    gm.free()


def test_draft_layers_in_the_speculative_loop(ctx):
    """Speculative decoding with the draft's layers on the persistent
    kernel.  Greedy: the token streams equal the oracle's and the
    per-kernel path's.  Sampled (T = 1): sequences accept different numbers
    of drafts and finish at different cycles, so later drafting steps run
    with finished sequences; each stream equals the oracle's up to a
    decision within 1e-5 of its boundary."""
    tcfg = dict(vocab=4096, d=512, H=8, F=2048, L=2)
    ot, gt = models(ctx, tcfg, 90, max_seq=512)
    od, gd = models(ctx, DRAFT2, 91, max_seq=512)
    rng = np.random.default_rng(92)
    B, P, new, k = 8, 24, 40, 4
    prompts = rng.integers(0, 4096, (B, P)).astype(np.int32)
    ctx.set_option("persistent_draft", 1)
    try:
        got, stats, _ = gt.generate_speculative_batch(gd, prompts, new, k, 0.0, 42)
    finally:
        ctx.set_option("persistent_draft", 0)
    ref, _, _ = gt.generate_speculative_batch(gd, prompts, new, k, 0.0, 42)
    np.testing.assert_array_equal(got, ref)
    for b in (0, 5):
        want, _ = O.generate_speculative(ot, od, prompts[b], new, k, 0.0, 42,
                                         seq=b)
        np.testing.assert_array_equal(got[b], want)
    ctx.set_option("persistent_draft", 1)
    try:
        got, stats, _ = gt.generate_speculative_batch(gd, prompts, new, k, 1.0, 7)
    finally:
        ctx.set_option("persistent_draft", 0)
    assert len({s.cycles for s in stats}) > 1
    for b in range(B):
        check_stream(ot, od, got[b], prompts[b], new, k, 1.0, 7, seq=b,
                     dev=stats[b], what=f"sampled b={b}")
    gt.free(); gd.free()

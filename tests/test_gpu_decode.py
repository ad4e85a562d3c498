"""Whole-path parity of libnnhip.so against the oracle (GPU).

Forward logits within 1e-4 (row-relative) of the oracle, the reference's
integration invariants on the device (greedy speculative == greedy
autoregressive, cache == no cache, causal independence), and token streams
identical to the oracle's generate_speculative given the same Philox
uniforms: exactly in greedy mode, and in sampled mode up to a divergence
inside a cycle whose closest random decision lies within 1e-5 of its
boundary (the oracle's record of that cycle says so).
"""
import numpy as np
import pytest

import oracle_py as O
from gpu_util import assert_rows_close, nnhip

pytestmark = pytest.mark.gpu

# Toy greedy configuration (target 2L/128/4h/512, draft 1L/64/2h/256, V 256)
TOY_T = dict(vocab=256, d=128, H=4, F=512, L=2)
TOY_D = dict(vocab=256, d=64, H=2, F=256, L=1)
# int8 batch-1 configuration (target 6L/512/8h/2048, draft 2L/256/4h/1024)
CFG2_T = dict(vocab=4096, d=512, H=8, F=2048, L=6)
CFG2_D = dict(vocab=4096, d=256, H=4, F=1024, L=2)


def build(ctx, cfg, seed, quantize, max_seq=1024, std=0.02, bits=8):
    params = O.make_params(cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                           cfg["L"], seed, std=std)
    om = O.Model(cfg["vocab"], cfg["d"], cfg["H"], cfg["F"], cfg["L"],
                 max_seq, params, quantize, bits=bits)
    gm = nnhip.Decoder(ctx, cfg["vocab"], cfg["d"], cfg["H"], cfg["F"],
                       cfg["L"], max_seq)
    gm.set_params(params)
    if quantize:
        gm.quantize(bits)
    return om, gm, params


def test_params_roundtrip_and_quantized_codes(ctx):
    om, gm, params = build(ctx, TOY_T, 1, True)
    for i in (0, 1, 2, 9, 10, 15, 16, len(params) - 2, len(params) - 1):
        np.testing.assert_array_equal(gm.get_param(i).ravel(),
                                      params[i].ravel())
    d, F, V = TOY_T["d"], TOY_T["F"], TOY_T["vocab"]
    for layer, which, n_in, n_out in ((0, 0, d, d), (1, 2, d, d),
                                      (0, 4, d, F), (1, 5, d, F),
                                      (0, 6, F, d), (0, 7, d, V)):
        gc, gs = gm.get_quantized(layer, which, n_in, n_out)
        oc, os_ = om.quantized(layer, which, n_in, n_out)
        np.testing.assert_array_equal(gc, oc)
        np.testing.assert_array_equal(gs, os_)
    gm.free()


def test_int4_decoder_matches_oracle(ctx):
    """INT4 QuantizedDense (quantization.cpp:38-86) for every Dense of the
    decoder: codes and scales bit-exact with the oracle's, forward logits
    within 1e-4, greedy speculative stream equal; nnhip_quantize_w4 on a
    single weight equals the oracle's quantize_w(w, 4)."""
    om, gm, params = build(ctx, TOY_T, 61, True, std=0.05, bits=4)
    d, F, V = TOY_T["d"], TOY_T["F"], TOY_T["vocab"]
    for layer, which, n_in, n_out in ((0, 0, d, d), (1, 4, d, F),
                                      (0, 6, F, d), (0, 7, d, V)):
        gc, gs = gm.get_quantized(layer, which, n_in, n_out)
        oc, os_ = om.quantized(layer, which, n_in, n_out)
        np.testing.assert_array_equal(gc, oc)
        np.testing.assert_array_equal(gs, os_)
        assert np.abs(gc).max() <= 7
    rng = np.random.default_rng(62)
    ids = rng.integers(0, V, (2, 9)).astype(np.int32)
    got = gm.forward(ids)
    for b in range(2):
        assert_rows_close(got[b], om.forward(ids[b]), 1e-4, f"int4 b={b}")
    od, gd, _ = build(ctx, TOY_D, 63, True, std=0.05, bits=4)
    prompt = rng.integers(0, V, 20).astype(np.int32)
    spec, _ = gm.generate_speculative(gd, prompt, 24, 4, 0.0)
    want, _ = O.generate_speculative(om, od, prompt, 24, 4, 0.0, 42)
    np.testing.assert_array_equal(spec, want)
    w = (rng.standard_normal((96, 64)) * 0.1).astype(np.float32)
    dw = ctx.array(w)
    dc = ctx.array(shape=(64, 96), dtype=np.int8)
    ds = ctx.array(shape=(64,))
    nnhip.call("nnhip_quantize_w4", ctx.h, dw.p, 96, 64, dc.p, ds.p)
    oc, os_ = O.quantize_w(w, 4)
    np.testing.assert_array_equal(dc.numpy().T, oc)
    np.testing.assert_array_equal(ds.numpy(), os_)
    gm.free(); gd.free()


def test_init_normal_rules(ctx):
    gm = nnhip.Decoder(ctx, 512, 128, 4, 256, 2, 64)
    gm.init_normal(7, 0.02)
    a = gm.get_param(1)                      # q.w
    assert abs(a.mean()) < 2e-3 and abs(a.std() - 0.02) < 1e-3
    assert not gm.get_param(2).any()         # q.b = 0
    assert (gm.get_param(15) == 1).all()     # ln1.gamma = 1
    assert not gm.get_param(16).any()        # ln1.beta = 0
    gm2 = nnhip.Decoder(ctx, 512, 128, 4, 256, 2, 64)
    gm2.init_normal(7, 0.02)
    np.testing.assert_array_equal(gm2.get_param(9), gm.get_param(9))
    gm.free(); gm2.free()


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("S", [1, 7, 40])
def test_forward_vs_oracle(ctx, quant, S):
    om, gm, _ = build(ctx, TOY_T, 3, quant, std=0.05)
    rng = np.random.default_rng(S)
    ids = rng.integers(0, 256, (2, S)).astype(np.int32)
    ids[1, 0] = 999                          # out of range -> row 0
    got = gm.forward(ids)
    for b in range(2):
        want = om.forward(ids[b])
        assert_rows_close(got[b], want, 1e-4, f"forward b={b}")
    gm.free()


@pytest.mark.parametrize("quant", [False, True])
def test_forward_gemv_layernorm_forms(ctx, quant):
    """Rows on the GEMV (1, 2 and 5 rows a sequence): the LayerNorms as
    launches of their own before plain GEMVs (option gemv_ln = 0) and in
    the GEMVs' prologues (gemv_ln = 16), both within 1e-4 of a row of the
    oracle's forward and within 1e-5 of each other."""
    om, gm, _ = build(ctx, TOY_T, 21, quant, std=0.05)
    rng = np.random.default_rng(22)
    for S in (1, 2, 5):
        ids = rng.integers(0, 256, (1, S)).astype(np.int32)
        try:
            ctx.set_option("gemv_ln", 0)
            sep = gm.forward(ids)
            ctx.set_option("gemv_ln", 16)
            pro = gm.forward(ids)
        finally:
            ctx.set_option("gemv_ln", 2)
        want = om.forward(ids[0])
        assert_rows_close(sep[0], want, 1e-4, f"separate S={S}")
        assert_rows_close(pro[0], want, 1e-4, f"prologue S={S}")
        assert_rows_close(sep[0], pro[0], 1e-5, f"forms S={S}")
    gm.free()


# one layer at the batch-32 config's width (d 1024, 16 heads, MLP 4096)
WIDE = dict(vocab=512, d=1024, H=16, F=4096, L=1)


def test_forward_wide_vs_oracle(ctx):
    """80 rows through a d = 1024 layer: q/k/v with RoPE, the output
    projection with its residual, gate/up with SwiGLU on the LDS-resident
    GEMMs, the down projection (K = 4096) on the digit-plane GEMM."""
    om, gm, _ = build(ctx, WIDE, 8, True, std=0.03)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 512, (2, 40)).astype(np.int32)
    got = gm.forward(ids)
    for b in range(2):
        assert_rows_close(got[b], om.forward(ids[b]), 1e-4, f"forward b={b}")
    gm.free()


# 64-wide heads, the width the output projection's per-head digits need
HEADS = dict(vocab=512, d=512, H=8, F=1024, L=2)


@pytest.mark.parametrize("B,S", [(32, 1), (32, 6), (4, 40), (4, 6)])
def test_forward_head_digits_vs_oracle(ctx, B, S):
    """Rows of 64-wide heads after the merged attention (the drafting and
    verify shapes; (4, 6) a launch of few (sequence, head) pairs, one query
    per workgroup): the attention writes the output projection's digit
    planes with one exponent per (row, head) and the digit-plane GEMM scales
    each head's exact total by its own exponent.  Against the oracle's
    forward (layer.cpp:1159-1216) within 1e-4 of a row, and against the
    path with one exponent per row (act_quant; option o_head_digits = 0)."""
    om, gm, _ = build(ctx, HEADS, 11, True, std=0.03)
    rng = np.random.default_rng(B * 100 + S)
    ids = rng.integers(0, 512, (B, S)).astype(np.int32)
    got = gm.forward(ids)
    ctx.set_option("o_head_digits", 0)
    try:
        per_row = gm.forward(ids)
    finally:
        ctx.set_option("o_head_digits", 1)
    for b in range(B):
        assert_rows_close(got[b], om.forward(ids[b]), 1e-4, f"forward b={b}")
        assert_rows_close(got[b], per_row[b], 1e-5, f"per-row digits b={b}")
    gm.free()


@pytest.mark.parametrize("B,S", [(1, 5), (32, 1), (32, 6)])
def test_fused_rope_append_bit_exact(ctx, B, S):
    """The q/k/v epilogue's RoPE and KV append (tensor.cpp:1141-1173,
    layer.cpp:758-807) bit for bit, on the GEMV (5 rows), the digit-plane
    GEMM (32) and the LDS GEMM (192): after a forward, layer 0's cached keys
    equal the device's own q/k/v projection of the embedded rows (the same
    kernels with a bias epilogue, nnhip_linear_w8a32) rotated by the
    oracle's or_rope, which rounds every product and sum on its own; the
    cached values equal that projection."""
    om, gm, params = build(ctx, HEADS, 13, True, std=0.03)
    d, H = HEADS["d"], HEADS["H"]
    D = d // H
    rng = np.random.default_rng(B * 10 + S)
    ids = rng.integers(0, HEADS["vocab"], (B, S)).astype(np.int32)
    gc = nnhip.KVCache(gm, B)
    gm.forward(ids, gc)
    # the fused q/k/v weight of layer 0 as the forward holds it
    parts = [gm.get_quantized(0, which, d, d) for which in (0, 1, 2)]
    codes = np.ascontiguousarray(np.concatenate([c for c, _ in parts], axis=1).T)
    scales = np.concatenate([sc for _, sc in parts])
    bias = np.concatenate([params[i].ravel() for i in (2, 4, 6)])
    x = gm.get_param(0)[ids.ravel()]
    R = B * S
    dx, dc = ctx.array(x), ctx.array(codes)
    ds, db = ctx.array(scales), ctx.array(bias)
    dy = ctx.array(shape=(R, 3 * d))
    call = nnhip.call
    call("nnhip_linear_w8a32", ctx.h, dx.p, R, d, dc.p, ds.p, db.p, 3 * d,
         dy.p, 1 if R < 16 else 2)
    y = dy.numpy()
    for b in range(B):
        kg, vg = gc.read(0, b, heads=H, head_dim=D)
        rows = y[b * S:(b + 1) * S]
        k = np.ascontiguousarray(rows[:, d:2 * d].reshape(S, H, D).transpose(1, 0, 2))
        O.lib().or_rope(O.fptr(k), H, S, D, 0)
        np.testing.assert_array_equal(kg, k, err_msg=f"keys b={b}")
        v = rows[:, 2 * d:].reshape(S, H, D).transpose(1, 0, 2)
        np.testing.assert_array_equal(vg, v, err_msg=f"values b={b}")
    gc.free()
    gm.free()


@pytest.mark.parametrize("quant", [False, True])
def test_forward_cache_truncate_vs_oracle(ctx, quant):
    om, gm, _ = build(ctx, TOY_T, 4, quant, std=0.05)
    rng = np.random.default_rng(5)
    seq = rng.integers(0, 256, 30).astype(np.int32)
    gc = nnhip.KVCache(gm, 1)
    oc = O.Cache(om)
    for lo, hi in ((0, 20), (20, 21), (21, 26)):
        g = gm.forward(seq[None, lo:hi], gc)[0]
        o = om.forward(seq[lo:hi], oc)
        assert_rows_close(g, o, 1e-4, f"cached [{lo},{hi})")
    assert gc.length() == 26
    gc.truncate(22)
    oc.truncate(22)
    g = gm.forward(seq[None, 26:30], gc)[0]
    o = om.forward(seq[26:30], oc)
    assert_rows_close(g, o, 1e-4, "after truncate")
    gc.free()
    gm.free()


def test_netw_weights_files(ctx, tmp_path):
    """Layer::save_weights / load_weights (layer.cpp:463-470) through the
    device decoder: its NETW file is byte-identical to the oracle's
    (serialization.cpp:8-47) for the same parameters; a device decoder
    loaded from the oracle's file holds the same parameters and gives the
    oracle's logits (1e-4), quantised too (the Dense layers re-quantised from
    the loaded weights); bad files are rejected with the reference's
    messages."""
    cfg = TOY_T
    args = (cfg["vocab"], cfg["d"], cfg["H"], cfg["F"], cfg["L"])
    params = O.make_params(*args, 31, std=0.05, bias_std=0.02)
    om = O.Model(*args, 256, params)
    gm = nnhip.Decoder(ctx, *args, 256)
    gm.set_params(params)
    pd, po = tmp_path / "dev.netw", tmp_path / "oracle.netw"
    gm.save_weights(pd)
    om.save_weights(po)
    assert pd.read_bytes() == po.read_bytes()
    ids = np.array([[5, 17, 200, 3, 99, 42]], np.int32)
    for quant in (False, True):
        g2 = nnhip.Decoder(ctx, *args, 256)
        g2.init_normal(9, 0.02)
        if quant:
            g2.quantize()
        g2.load_weights(po)
        for i in (0, 1, 2, 9, 15, len(params) - 1):
            np.testing.assert_array_equal(g2.get_param(i).ravel(),
                                          params[i].ravel())
        want = O.Model(*args, 256, params, quant).forward(ids[0])
        assert_rows_close(g2.forward(ids)[0], want, 1e-4, f"loaded q={quant}")
        g2.free()
    wide = nnhip.Decoder(ctx, cfg["vocab"], 2 * cfg["d"], cfg["H"], cfg["F"],
                         cfg["L"], 256)
    with pytest.raises(nnhip.NNHipError) as e:
        wide.load_weights(po)
    assert e.value.code == nnhip.EARG and "shape mismatch" in str(e.value)
    bad = tmp_path / "bad.netw"
    bad.write_bytes(b"NETX" + po.read_bytes()[4:])
    with pytest.raises(nnhip.NNHipError) as e:
        gm.load_weights(bad)
    assert "Invalid file format signature" in str(e.value)
    with pytest.raises(nnhip.NNHipError) as e:
        gm.load_weights(tmp_path / "missing.netw")
    assert e.value.code == nnhip.EIO
    wide.free()
    gm.free()


def test_causal_independence(ctx):
    """transformer_test.cpp:153-176 on the device."""
    _, gm, _ = build(ctx, TOY_T, 6, True)
    a = gm.forward(np.array([[1, 2, 3, 4, 5]], np.int32))
    b = gm.forward(np.array([[1, 2, 3, 4, 9]], np.int32))
    np.testing.assert_array_equal(a[0, :4], b[0, :4])
    gm.free()


@pytest.mark.parametrize("quant_cache", [False, True])
def test_capacity_rule_matches_oracle(ctx, quant_cache):
    """The reference throws when a forward's S_past + S exceeds max_seq_len
    (layer.cpp:1171-1179), except with int8 caches, whose length it never
    reads (caches[0].k is null there).  Around the boundary max_seq = P + max_new -- where
    the target fits and the draft cache, which gains one duplicate per
    rejection, may not -- the device fails (ECAPACITY) exactly when the
    oracle does, and otherwise returns the oracle's stream."""
    P, new, k = 30, 20, 4
    for max_seq in (P + new - 1, P + new, P + new + 8, 2 * (P + new)):
        ot, gt, _ = build(ctx, TOY_T, 7, False, max_seq=max_seq, std=0.3)
        od, gd, _ = build(ctx, TOY_D, 8, False, max_seq=max_seq, std=0.3)
        prompt = np.arange(P, dtype=np.int32) * 3 % 256
        try:
            want, _ = O.generate_speculative(ot, od, prompt, new, k, 0.0, 42,
                                             quantized_cache=quant_cache)
        except RuntimeError:
            want = None
        try:
            got, _ = gt.generate_speculative(gd, prompt, new, k, 0.0,
                                             quantized_cache=quant_cache)
        except nnhip.NNHipError as e:
            assert e.code == nnhip.ECAPACITY, e
            got = None
        assert (got is None) == (want is None), (max_seq, quant_cache)
        if got is not None:
            np.testing.assert_array_equal(got, want)
        if quant_cache:
            assert got is not None
        gt.free(); gd.free()
    # the prompt alone over max_seq_len: the prefill throws (fp32 caches)
    _, gt, _ = build(ctx, TOY_T, 7, False, max_seq=16)
    _, gd, _ = build(ctx, TOY_D, 8, False, max_seq=16)
    if not quant_cache:
        with pytest.raises(nnhip.NNHipError) as e:
            gt.generate_speculative(gd, np.arange(20), 4, 4, 0.0)
        assert e.value.code == nnhip.ECAPACITY
    gt.free(); gd.free()


def check_on_device_codes(om, gc, cfg, b, n_before, ids, got, what):
    """One forward of `ids` (sequence b, positions n_before..) over an int8
    cache, checked against the oracle given the same cache:
    (a) the oracle's forward over a cache holding the device's codes and
        scales for every position (the new ones included) gives the device's
        logits within 1e-4 (row-relative);
    (b) the device's codes at the new positions are the oracle's quantize_kv
        of the fp32 k / v rows that forward computed, except by one where the
        oracle's x * (1 / scale) lies within 2e-3 of a rounding boundary (the
        rows differ from the device's in their last bits, and the quantiser is
        exact on either side: see test_rope_kv_append_q8); scales within
        1e-5.
    Chained over forwards, (a) and (b) pin the whole int8-cache path; the
    oracle's own int8 run is not compared code by code, because one code
    rounded the other way at a boundary moves every later row of the
    layers above it."""
    H, D, L = cfg["H"], cfg["d"] // cfg["H"], cfg["L"]
    dev = [gc.read_q8(layer, b, H, D) for layer in range(L)]
    oc = O.Cache(om, quantized=True)
    for layer in range(L):
        oc.write_q8(layer, *dev[layer])
    oc.set_len(n_before)
    oc.freeze()
    want = om.forward(ids, oc)
    assert_rows_close(got, want, 1e-4, what)
    new = slice(n_before, n_before + len(ids))
    for layer in range(L):
        kr, vr = oc.read_raw(layer)
        dk, dks, dv, dvs = dev[layer]
        for raw, dq, ds in ((kr, dk, dks), (vr, dv, dvs)):
            oq, os_ = O.quantize_kv(raw[:, new])
            np.testing.assert_allclose(ds[:, new], os_, rtol=1e-5)
            d = dq[:, new].astype(np.int32) - oq.astype(np.int32)
            assert np.abs(d).max() <= 1, (what, layer)
            off = d != 0
            if off.any():
                t = np.abs(raw[:, new] * (np.float32(1.0) / os_)[..., None])
                frac = t - np.floor(t)
                assert (np.abs(frac[off] - 0.5) < 2e-3).all(), (what, layer)


@pytest.mark.parametrize("quant", [False, True])
def test_forward_int8_cache_vs_oracle(ctx, quant):
    """KVCache(quantized=true) through prefill, single steps, a multi-token
    step and a truncation, each forward checked by check_on_device_codes."""
    om, gm, _ = build(ctx, TOY_T, 14, quant, std=0.05)
    rng = np.random.default_rng(15)
    seq = rng.integers(0, 256, 40).astype(np.int32)
    gc = nnhip.KVCache(gm, 1, quantized=True)
    n = 0
    for lo, hi in [(0, 20), (20, 21), (21, 27), ("truncate", 23), (27, 35)]:
        if lo == "truncate":
            gc.truncate(hi)
            n = hi
            continue
        g = gm.forward(seq[None, lo:hi], gc)[0]
        check_on_device_codes(om, gc, TOY_T, 0, n, seq[lo:hi], g,
                              f"int8 cache [{lo},{hi})")
        n += hi - lo
    assert gc.length() == 31
    gc.free()
    gm.free()


@pytest.mark.parametrize("S", [1, 2, 4, 6])
def test_forward_int8_cache_ragged_batch(ctx, S):
    """The verify / draft shapes on an int8 cache: 5 sequences at different
    lengths (prefill, then per-sequence truncation) take S rows each; each
    sequence's forwards checked by check_on_device_codes."""
    om, gm, _ = build(ctx, TOY_T, 18, True, std=0.2)
    B = 5
    rng = np.random.default_rng(19 + S)
    seqs = rng.integers(0, 256, (B, 40)).astype(np.int32)
    gc = nnhip.KVCache(gm, B, quantized=True)
    pre = gm.forward(seqs[:, :24], gc)
    for b in range(B):
        check_on_device_codes(om, gc, TOY_T, b, 0, seqs[b, :24], pre[b],
                              f"prefill seq {b}")
    keeps = [24 - 3 * b for b in range(B)]
    for b in range(B):
        gc.truncate(keeps[b], b)
    ids = np.stack([seqs[b, keeps[b]:keeps[b] + S] for b in range(B)])
    got = gm.forward(ids, gc)
    for b in range(B):
        check_on_device_codes(om, gc, TOY_T, b, keeps[b], ids[b], got[b],
                              f"ragged int8 seq {b}")
    gc.free()
    gm.free()


@pytest.mark.parametrize("T", [0.0, 1.0])
def test_int8_cache_spec_matches_oracle(ctx, T):
    """generate_speculative(..., quantized_cache=true): batch-1 and a batch
    of 5 in lockstep against the oracle with int8 caches; greedy streams
    exact, sampled ones up to a recorded tie.  Weights N(0, 0.05): a code
    that rounds the other way at a boundary (see assert_q8_cache_matches)
    moves the logits by ~1e-6 here, far below the streams' argmax margins,
    whereas with large weights (N(0, 0.3)) one such code can move a logit by
    1e-2 and legitimately change a greedy stream."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 16, True, std=0.05)
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, 256, 32).astype(np.int32)
    got, st = gt.generate_speculative(gd, prompt, 48, 4, T, seed=3,
                                      quantized_cache=True)
    check_stream(ot, od, got, prompt, 48, 4, T, 3, dev=st,
                 quantized_cache=True)
    B = 5
    prompts = rng.integers(0, 256, (B, 20)).astype(np.int32)
    gotb, stats, _ = gt.generate_speculative_batch(gd, prompts, 30, 3, T, 8,
                                                   quantized_cache=True)
    for b in range(B):
        check_stream(ot, od, gotb[b], prompts[b], 30, 3, T, 8, seq=b,
                     dev=stats[b], what=f"b={b}", quantized_cache=True)
    gt.free(); gd.free()


def check_stream(ot, od, got, prompt, max_new, k, T, seed, seq=0, dev=None,
                 what="", **kw):
    """The device stream `got` against the oracle's run of the same
    sequence: equal in greedy mode; in sampled mode equal, or first
    different inside a cycle whose closest random decision the oracle made
    within 1e-5 of its boundary (O.assert_same_stream).  When the streams
    are equal the device's counters (`dev`, SpecStats) equal the oracle's."""
    want, ost, cyc, fm = O.generate_speculative_traced(
        ot, od, prompt, max_new, k, T, seed, seq=seq, **kw)
    i = O.assert_same_stream(got, want, cyc, fm, len(prompt), what=what)
    if T <= 0:
        assert i is None, what
    if i is None and dev is not None:
        assert (dev.cycles, dev.accepted, dev.resampled, dev.bonus) == (
            ost.cycles, ost.accepted, ost.resampled, ost.bonus), what
    return i


def spec_pair(ctx, tcfg, dcfg, seed, quant, std=0.02):
    ot, gt, _ = build(ctx, tcfg, seed, quant, std=std)
    od, gd, _ = build(ctx, dcfg, seed + 1, quant, std=std)
    return ot, gt, od, gd


@pytest.mark.parametrize("k", [1, 4])
@pytest.mark.parametrize("graphs", [0, 1])
def test_toy_greedy_matches_oracle_and_ar(ctx, k, graphs):
    """Config: toy fp32 greedy (B=1, prompt 32, 64 new): the device token
    stream equals the oracle's and the device greedy autoregressive one."""
    ctx.set_option("graphs", graphs)
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 10, False, std=0.3)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, 256, 32).astype(np.int32)
    got, st = gt.generate_speculative(gd, prompt, 64, k, 0.0)
    want, ost = O.generate_speculative(ot, od, prompt, 64, k, 0.0, 42)
    np.testing.assert_array_equal(got, want)
    assert (st.cycles, st.accepted) == (ost.cycles, ost.accepted)
    ar = gt.generate_advanced(prompt, 64, 0.0)
    np.testing.assert_array_equal(got, ar)
    ctx.set_option("graphs", 1)
    gt.free(); gd.free()


def test_toy_sampled_matches_oracle(ctx):
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 20, False, std=0.3)
    rng = np.random.default_rng(21)
    for seed in (1, 2, 3):
        prompt = rng.integers(0, 256, 32).astype(np.int32)
        got, st = gt.generate_speculative(gd, prompt, 64, 4, 1.0, seed=seed)
        check_stream(ot, od, got, prompt, 64, 4, 1.0, seed, dev=st,
                     what=f"seed {seed}")
    gt.free(); gd.free()


@pytest.mark.parametrize("T", [0.0, 1.0])
def test_spec_edge_lengths_match_oracle(ctx, T):
    """Lengths at the edges of the loop (layer.cpp:1508-1518): max_new 0 and
    1 (the first token only: the reference always appends it), 2 and 3 with
    k = 4 > max_new - 1 (M = min(k, remaining)), a one-token prompt, in a
    batch of 3 and alone; streams equal to the oracle's (sampled: up to a
    recorded tie)."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 24, True, std=0.3)
    rng = np.random.default_rng(25)
    for P in (1, 5):
        prompts = rng.integers(0, 256, (3, P)).astype(np.int32)
        for max_new in (0, 1, 2, 3):
            got, stats, _ = gt.generate_speculative_batch(gd, prompts, max_new,
                                                          4, T, 11)
            assert got.shape == (3, P + max(max_new, 1))
            for b in range(3):
                check_stream(ot, od, got[b], prompts[b], max_new, 4, T, 11,
                             seq=b, dev=stats[b], what=f"P={P} new={max_new}")
            one, _ = gt.generate_speculative(gd, prompts[0], max_new, 4, T,
                                             seed=11)
            np.testing.assert_array_equal(one, got[0])
    gt.free(); gd.free()


@pytest.mark.parametrize("top_k,top_p", [(4, 0.9), (0, 0.8), (6, 1.0)])
def test_spec_top_k_top_p_matches_oracle(ctx, top_k, top_p):
    """transformer_test.cpp:340-345 runs generate_speculative with top_k 4,
    top_p 0.9, T 1.0: every get_probs of the loop filtered (draft, verify,
    residual, bonus).  Batch-1 and a batch of 5 against the oracle: equal
    streams up to a recorded tie (vocabularies of 256 keep the top-p running
    sums far from their rounding error)."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 22, True, std=0.3)
    rng = np.random.default_rng(23)
    prompt = rng.integers(0, 256, 32).astype(np.int32)
    got, st = gt.generate_speculative(gd, prompt, 40, 3, 1.0, top_k=top_k,
                                      top_p=top_p, seed=5)
    check_stream(ot, od, got, prompt, 40, 3, 1.0, 5, dev=st, top_k=top_k,
                 top_p=top_p)
    B = 5
    prompts = rng.integers(0, 256, (B, 20)).astype(np.int32)
    gotb, stats, _ = gt.generate_speculative_batch(gd, prompts, 30, 4, 0.8, 6,
                                                   top_k=top_k, top_p=top_p)
    for b in range(B):
        check_stream(ot, od, gotb[b], prompts[b], 30, 4, 0.8, 6, seq=b,
                     dev=stats[b], what=f"b={b}", top_k=top_k, top_p=top_p)
    ar = gt.generate_advanced_batch(prompts, 12, 1.0, 7, top_k=top_k,
                                    top_p=top_p)
    for b in range(B):
        want = O.generate_advanced(ot, prompts[b], 12, 1.0, 7, seq=b,
                                   top_k=top_k, top_p=top_p)
        np.testing.assert_array_equal(ar[b], want)
    gt.free(); gd.free()


@pytest.mark.parametrize("T", [0.0, 1.0])
def test_batch_matches_oracle_per_sequence(ctx, T):
    """B independent sequences in lockstep = B oracle runs (seq index b)."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 30, True, std=0.2)
    B = 6
    rng = np.random.default_rng(31)
    prompts = rng.integers(0, 256, (B, 24)).astype(np.int32)
    got, stats, tm = gt.generate_speculative_batch(gd, prompts, 40, 3, T, 77)
    assert tm.decode_ms > 0
    for b in range(B):
        check_stream(ot, od, got[b], prompts[b], 40, 3, T, 77, seq=b,
                     dev=stats[b], what=f"b={b}")
    gt.free(); gd.free()


def test_batch_mfma_rows_match_oracle(ctx):
    """B = 20 rows of drafting use the MFMA digit GEMM (rows >= 16); the
    100-row verify and the 320-row prefill use the LDS-resident GEMMs."""
    ot, gt, od, gd = spec_pair(ctx, TOY_T, TOY_D, 40, True, std=0.2)
    B = 20
    rng = np.random.default_rng(41)
    prompts = rng.integers(0, 256, (B, 16)).astype(np.int32)
    got, stats, _ = gt.generate_speculative_batch(gd, prompts, 24, 4, 0.0, 5)
    for b in (0, 7, 19):
        want, _ = O.generate_speculative(ot, od, prompts[b], 24, 4, 0.0, 5,
                                         seq=b)
        np.testing.assert_array_equal(got[b], want)
    gt.free(); gd.free()


# d = 512 draft at batch 16: the draft lm head runs on the LDS-resident GEMM
# with 128-column blocks, so drafting samples from its tile statistics
TILE_T = dict(vocab=2000, d=512, H=8, F=1024, L=1)
TILE_D = dict(vocab=2000, d=512, H=8, F=512, L=1)


@pytest.mark.parametrize("T", [0.0, 1.0, 0.7])
def test_batch_tile_sampling_matches_oracle(ctx, T):
    """Drafting from the draft lm head's tile statistics: greedy streams
    exact, sampled streams equal to the oracle's up to a recorded tie; the
    last tile is ragged (vocabulary 2000 = 15 x 128 + 80)."""
    ot, gt, od, gd = spec_pair(ctx, TILE_T, TILE_D, 70, True, std=0.1)
    B = 16
    rng = np.random.default_rng(71)
    prompts = rng.integers(0, 2000, (B, 12)).astype(np.int32)
    got, stats, _ = gt.generate_speculative_batch(gd, prompts, 20, 3, T, 9)
    for b in (0, 5, 15):
        check_stream(ot, od, got[b], prompts[b], 20, 3, T, 9, seq=b,
                     dev=stats[b], what=f"b={b}")
    gt.free(); gd.free()


def test_cfg2_int8_greedy_full_size(ctx):
    """int8 greedy at full size: target 6L/512/8h/2048/V4096, draft
    2L/256/4h/1024, prompt 128, k=4, 256 new tokens; exact token stream."""
    ot, gt, od, gd = spec_pair(ctx, CFG2_T, CFG2_D, 50, True)
    rng = np.random.default_rng(51)
    prompt = rng.integers(0, 4096, 128).astype(np.int32)
    got, st = gt.generate_speculative(gd, prompt, 256, 4, 0.0)
    want, ost = O.generate_speculative(ot, od, prompt, 256, 4, 0.0, 42)
    np.testing.assert_array_equal(got, want)
    assert st.accepted == ost.accepted and st.cycles == ost.cycles
    gt.free(); gd.free()

"""Pins the oracle (oracle/liboracle.so) before it is trusted as the checker.

Each test anchors one oracle function on something outside the oracle: the
reference's own known-answer tests (file:line under tests/ of the reference),
the Random123 known-answer vectors, closed forms, float64 brute force, and
the reference's integration invariants.  The reference itself cannot be built
here (its CPU backend needs an external BLAS), so no output of it is used.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_py as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# --------------------------------------------------------------------------
# Philox4x32-10 -- Random123 known-answer vectors
# --------------------------------------------------------------------------
def test_philox_kat():
    for case in golden("philox4x32_10_kat.json")["vectors"]:
        ctr = [int(x, 16) for x in case["ctr"]]
        key = [int(x, 16) for x in case["key"]]
        want = [int(x, 16) for x in case["out"]]
        assert O.philox(ctr, key) == want


def test_uniform_layout():
    # u = top 24 bits of word 0 of Philox(ctr = {slot, cycle, seq, 0},
    # key = {seed_lo, seed_hi}) times 2^-24
    seed = 0x1234_5678_9ABC_DEF0
    for seq, cyc, slot in [(0, 0, 0), (3, 7, 2), (31, 200, 10)]:
        w = O.philox([slot, cyc, seq, 0], [seed & 0xFFFFFFFF, seed >> 32])[0]
        assert O.uniform(seed, seq, cyc, slot) == np.float32((w >> 8) / 2**24)
    us = np.array([O.uniform(7, s, 1, 0) for s in range(4000)])
    assert 0.0 <= us.min() and us.max() < 1.0
    assert abs(us.mean() - 0.5) < 0.02


# --------------------------------------------------------------------------
# int8 quantisation -- quantization_test.cpp:6-26 and the closed form
# --------------------------------------------------------------------------
def quantize(w):
    w = np.ascontiguousarray(w, np.float32)
    codes = np.zeros(w.shape, np.int8)
    scales = np.zeros(w.shape[1], np.float32)
    O.lib().or_quantize_w8(O.fptr(w), w.shape[0], w.shape[1], O.i8ptr(codes),
                           O.fptr(scales))
    return codes, scales


def test_quantize_kat_reference():
    kat = golden("reference_kats.json")["quantize_int8"]
    codes, scales = quantize(np.array(kat["weight"], np.float32).reshape(2, 2))
    np.testing.assert_allclose(scales, kat["scales"], atol=1e-5)
    deq = codes.astype(np.float32) * scales[None, :]
    np.testing.assert_allclose(deq.ravel()[0], kat["dequant"][0], atol=0.05)
    np.testing.assert_allclose(deq.ravel()[1:], kat["dequant"][1:], atol=1e-5)


def test_quantize_closed_form():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((37, 19)) * 0.02).astype(np.float32)
    w[:, 4] = 0.0                      # all-zero column -> scale 1
    w[5, 7] = 0.5 * (np.abs(w[:, 7]).max() * 2)  # force a new max
    codes, scales = quantize(w)
    for c in range(w.shape[1]):
        mx = np.float32(np.abs(w[:, c]).max())
        s = np.float32(mx / np.float32(127.0))
        assert scales[c] == (np.float32(1.0) if s == 0 else s)
        q = np.trunc(w[:, c] / scales[c] + np.copysign(np.float32(0.5),
                                                        w[:, c]))
        np.testing.assert_array_equal(codes[:, c], np.clip(q, -127, 127))
    assert np.abs(codes).max() == 127
    # round half away from zero: 2.5 -> 3, -2.5 -> -3
    w2 = np.array([[2.5, -2.5], [127.0, 127.0]], np.float32)
    c2, s2 = quantize(w2)
    assert list(s2) == [1.0, 1.0] and list(c2[0]) == [3, -3]


def test_quantized_dense_forward_reference():
    """quantization_test.cpp:47-87: int8 forward within 5% of fp32."""
    kat = golden("reference_kats.json")["quantized_dense_forward"]
    w = np.array(kat["weight"], np.float32).reshape(4, 3)
    b = np.array(kat["bias"], np.float32)
    x = np.array(kat["x"], np.float32).reshape(2, 4)
    codes, scales = quantize(w)
    y = np.zeros((2, 3), np.float32)
    yq = np.zeros((2, 3), np.float32)
    O.lib().or_dense(O.fptr(x), 2, 4, 3, O.fptr(w), None, None, O.fptr(b),
                     O.fptr(y))
    O.lib().or_dense(O.fptr(x), 2, 4, 3, None, O.i8ptr(codes), O.fptr(scales),
                     O.fptr(b), O.fptr(yq))
    np.testing.assert_allclose(y, x.astype(np.float64) @ w + b, rtol=1e-6)
    rel = np.abs(y - yq) / np.maximum(1.0, np.abs(y))
    assert rel.max() < 0.05


def test_quantize_int4_reference_kat_and_packing():
    """QuantizationTest.Int4Packing (quantization_test.cpp:28-45): scale
    7 / 7 = 1, dequantised -7, 3, 0, 5.  Packing (quantization.cpp:68-86):
    two codes a byte, the even flat index in the low nibble, so -7 (0x9)
    and 3 give 0x39, 0 and 5 give 0x50; unpacking sign-extends
    (quantization.cpp:106-122) back to the codes."""
    kat = golden("reference_kats.json")["quantize_int4"]
    w = np.array(kat["weight"], np.float32).reshape(kat["shape"])
    codes, scales = O.quantize_w(w, 4)
    np.testing.assert_array_equal(scales, kat["scales"])
    np.testing.assert_array_equal((codes * scales[None, :]).ravel(),
                                  kat["dequant"])
    packed = O.pack_int4(codes)
    assert packed.tolist() == [0x39, 0x50]
    np.testing.assert_array_equal(O.unpack_int4(packed, 4), codes.ravel())
    # every code value survives a round trip; an odd count leaves the last
    # high nibble zero
    allc = np.arange(-7, 8, dtype=np.int8)
    p2 = O.pack_int4(allc)
    assert len(p2) == 8 and p2[-1] >> 4 == 0
    np.testing.assert_array_equal(O.unpack_int4(p2, 15), allc)


def test_quantize_int4_closed_form_and_forward():
    """INT4 codes: scale = max|w| / 7 per output column (1 when 0), codes
    round-half-away-from-zero clamped to +-7, the column maximum at +-7;
    QuantizedDenseForward's INT4 case (quantization_test.cpp:76-86) within
    70% of the fp32 forward."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((33, 12)) * 0.02).astype(np.float32)
    w[:, 3] = 0.0
    codes, scales = O.quantize_w(w, 4)
    for c in range(w.shape[1]):
        mx = np.float32(np.abs(w[:, c]).max())
        s = np.float32(mx / np.float32(7.0))
        assert scales[c] == (np.float32(1.0) if s == 0 else s)
        q = np.trunc(w[:, c] / scales[c] + np.copysign(np.float32(0.5), w[:, c]))
        np.testing.assert_array_equal(codes[:, c], np.clip(q, -7, 7))
    assert np.abs(codes).max() == 7
    kat = golden("reference_kats.json")["quantized_dense_forward"]
    wk = np.array(kat["weight"], np.float32).reshape(4, 3)
    b = np.array(kat["bias"], np.float32)
    x = np.array(kat["x"], np.float32).reshape(2, 4)
    c4, s4 = O.quantize_w(wk, 4)
    y = np.zeros((2, 3), np.float32)
    y4 = np.zeros((2, 3), np.float32)
    O.lib().or_dense(O.fptr(x), 2, 4, 3, O.fptr(wk), None, None, O.fptr(b),
                     O.fptr(y))
    O.lib().or_dense(O.fptr(x), 2, 4, 3, None, O.i8ptr(c4), O.fptr(s4),
                     O.fptr(b), O.fptr(y4))
    rel = np.abs(y - y4) / np.maximum(1.0, np.abs(y))
    assert rel.max() < kat["max_rel_err_int4"]


def test_matmul_kat_reference():
    """tensor_test.cpp:82-94: [[1,2,3],[4,5,6]] . [[7,8],[9,10],[11,12]]."""
    kat = golden("reference_kats.json")["matmul"]
    a = np.array(kat["a"], np.float32).reshape(2, 3)
    b = np.array(kat["b"], np.float32).reshape(3, 2)
    y = np.zeros((2, 2), np.float32)
    O.lib().or_dense(O.fptr(a), 2, 3, 2, O.fptr(b), None, None, None,
                     O.fptr(y))
    assert y.ravel().tolist() == kat["out"]


def test_dense_w8_vs_float64():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 96)).astype(np.float32)
    w = (rng.standard_normal((96, 40)) * 0.02).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    codes, scales = quantize(w)
    y = np.zeros((6, 40), np.float32)
    O.lib().or_dense(O.fptr(x), 6, 96, 40, None, O.i8ptr(codes),
                     O.fptr(scales), O.fptr(b), O.fptr(y))
    ref = x.astype(np.float64) @ (codes.astype(np.float64) *
                                  scales.astype(np.float64)) + b
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------
# RoPE -- rope_swiglu_test.cpp:10-48 and the rotation invariants
# --------------------------------------------------------------------------
def test_rope_kat_reference():
    kat = golden("reference_kats.json")["rope"]
    x = np.array(kat["x"], np.float32)
    O.lib().or_rope(O.fptr(x), 1, 2, 4, 0)
    np.testing.assert_allclose(x[:4], kat["x"][:4], atol=1e-5)
    np.testing.assert_allclose(x[4:6], kat["out_s1_pair0"], atol=1e-4)


def test_rope_closed_form():
    rng = np.random.default_rng(9)
    H, S, D, past = 3, 5, 16, 11
    x = rng.standard_normal((H, S, D)).astype(np.float32)
    y = x.copy()
    O.lib().or_rope(O.fptr(y), H, S, D, past)
    j = np.arange(D // 2)
    theta = 10000.0 ** (-2.0 * j / D)
    for s in range(S):
        ang = (past + s) * theta
        c, sn = np.cos(ang), np.sin(ang)
        xe, xo = x[:, s, 0::2].astype(np.float64), x[:, s, 1::2]
        np.testing.assert_allclose(y[:, s, 0::2], xe * c - xo * sn, atol=2e-5)
        np.testing.assert_allclose(y[:, s, 1::2], xe * sn + xo * c, atol=2e-5)
    # rotation preserves each pair's norm
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-4)


# --------------------------------------------------------------------------
# LayerNorm -- layer_test.cpp:56-80
# --------------------------------------------------------------------------
def test_layernorm_kat_reference():
    kat = golden("reference_kats.json")["layernorm"]
    x = np.array(kat["x"], np.float32)
    y = np.zeros_like(x)
    g = np.ones(3, np.float32)
    b = np.zeros(3, np.float32)
    O.lib().or_layernorm(O.fptr(x), 2, 3, O.fptr(g), O.fptr(b), 1e-5,
                         O.fptr(y))
    np.testing.assert_allclose(y[:3], kat["out_row0"], atol=1e-3)
    np.testing.assert_allclose(y[3:], kat["out_row0"], atol=1e-3)


def test_layernorm_vs_float64():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((4, 200)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(200).astype(np.float32)
    b = rng.standard_normal(200).astype(np.float32)
    y = np.zeros_like(x)
    O.lib().or_layernorm(O.fptr(x), 4, 200, O.fptr(g), O.fptr(b), 1e-5,
                         O.fptr(y))
    xd = x.astype(np.float64)
    m = xd.mean(1, keepdims=True)
    v = ((xd - m) ** 2).mean(1, keepdims=True)
    np.testing.assert_allclose(y, (xd - m) / np.sqrt(v + 1e-5) * g + b,
                               rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------
# Attention -- float64 brute force with causal mask
# --------------------------------------------------------------------------
def attn_f64(q, k, v, causal):
    H, S, D = q.shape
    St = k.shape[1]
    out = np.zeros((S, H, D))
    for h in range(H):
        sc = q[h].astype(np.float64) @ k[h].T.astype(np.float64) / math.sqrt(D)
        if causal:
            for i in range(S):
                sc[i, St - S + i + 1:] = -np.inf
        p = np.exp(sc - sc.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[:, h] = p @ v[h].astype(np.float64)
    return out


@pytest.mark.parametrize("S,St", [(1, 1), (1, 9), (4, 4), (5, 37)])
def test_attention_vs_float64(S, St):
    rng = np.random.default_rng(S * 100 + St)
    H, D = 3, 16
    q = rng.standard_normal((H, S, D)).astype(np.float32)
    k = rng.standard_normal((H, St, D)).astype(np.float32)
    v = rng.standard_normal((H, St, D)).astype(np.float32)
    out = np.zeros((S, H, D), np.float32)
    O.lib().or_attention(O.fptr(q), O.fptr(k), O.fptr(v), H, H, S, St, D, 1,
                         O.fptr(out))
    np.testing.assert_allclose(out, attn_f64(q, k, v, True), rtol=1e-5,
                               atol=1e-5)


@pytest.mark.parametrize("H,Hkv", [(4, 2), (8, 1), (6, 3)])
def test_attention_gqa_equals_repeated_kv_heads(H, Hkv):
    """Grouped-query attention (layer.cpp:862-864, h_kv = h / (H / H_kv)):
    equal, bit for bit, to full multi-head attention over the kv heads
    repeated H / H_kv times each (head h reading copy h); the modular
    mapping h % H_kv would fail this."""
    rng = np.random.default_rng(H * 10 + Hkv)
    S, St, D = 3, 11, 8
    q = rng.standard_normal((H, S, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, St, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, St, D)).astype(np.float32)
    out = np.zeros((S, H, D), np.float32)
    O.lib().or_attention(O.fptr(q), O.fptr(k), O.fptr(v), H, Hkv, S, St, D, 1,
                         O.fptr(out))
    kr = np.ascontiguousarray(np.repeat(k, H // Hkv, axis=0))
    vr = np.ascontiguousarray(np.repeat(v, H // Hkv, axis=0))
    full = np.zeros((S, H, D), np.float32)
    O.lib().or_attention(O.fptr(q), O.fptr(kr), O.fptr(vr), H, H, S, St, D, 1,
                         O.fptr(full))
    np.testing.assert_array_equal(out, full)
    np.testing.assert_allclose(out, attn_f64(q, kr, vr, True), rtol=1e-5,
                               atol=1e-5)


# --------------------------------------------------------------------------
# get_probs / sample_token
# --------------------------------------------------------------------------
def test_get_probs_closed_form():
    rng = np.random.default_rng(2)
    lg = (rng.standard_normal(500) * 2).astype(np.float32)
    for T in (1.0, 0.7, 2.5):
        p = O.get_probs(lg, T)
        z = lg.astype(np.float64) / T
        ref = np.exp(z - z.max())
        ref /= ref.sum()
        np.testing.assert_allclose(p, ref, rtol=2e-6, atol=1e-12)
    g = O.get_probs(lg, 0.0)
    assert g.sum() == 1.0 and g[int(np.argmax(lg))] == 1.0
    tie = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    assert O.get_probs(tie, 0.0)[1] == 1.0          # first index wins ties


def test_get_probs_top_k_top_p():
    lg = np.log(np.array([0.1, 0.4, 0.2, 0.3], np.float32))
    p = O.get_probs(lg, 1.0, top_k=2)
    np.testing.assert_allclose(p, [0, 4 / 7, 0, 3 / 7], rtol=1e-6)
    p = O.get_probs(lg, 1.0, top_p=0.65)        # 0.4 + 0.3 >= 0.65 -> cut
    np.testing.assert_allclose(p, [0, 4 / 7, 0, 3 / 7], rtol=1e-6)
    p = O.get_probs(lg, 1.0, top_p=0.75)        # 0.4 + 0.3 + 0.2
    np.testing.assert_allclose(p, [0, 4 / 9, 2 / 9, 3 / 9], rtol=1e-6)


def test_sample_inverse_cdf_brute_force():
    rng = np.random.default_rng(4)
    p = rng.random(50).astype(np.float32)
    p[[3, 17]] = 0
    cdf = np.cumsum(p.astype(np.float64) / p.astype(np.float64).sum())
    cdf[-1] = 1.0
    for u in list(rng.random(300)) + [0.0, 1 - 2**-24]:
        want = int(np.searchsorted(cdf, u, side="left"))
        assert O.sample(p, u) == want
    # a boundary value picks the first index whose cdf reaches it
    q = np.array([0.25, 0.25, 0.5], np.float32)
    assert O.sample(q, 0.25) == 0 and O.sample(q, 0.2500001) == 1


# --------------------------------------------------------------------------
# Whole-path invariants (transformer_test.cpp)
# --------------------------------------------------------------------------
def tiny_models(vocab=8, quantize=False, seed=11):
    tp = O.make_params(vocab, 16, 2, 32, 2, seed, std=0.3)
    dp = O.make_params(vocab, 16, 2, 32, 1, seed + 1, std=0.3)
    return (O.Model(vocab, 16, 2, 32, 2, 64, tp, quantize),
            O.Model(vocab, 16, 2, 32, 1, 64, dp, quantize))


def test_causal_independence():
    """transformer_test.cpp:153-176: a later token leaves earlier rows
    bit-equal."""
    t, _ = tiny_models()
    a = t.forward([1, 2, 3, 4])
    b = t.forward([1, 2, 3, 7])
    np.testing.assert_array_equal(a[:3], b[:3])
    assert not np.array_equal(a[3], b[3])


def test_kv_cache_equals_no_cache():
    """transformer_test.cpp:250-273 and cached vs uncached logits."""
    t, _ = tiny_models(quantize=True)
    full = t.forward([5, 1, 2, 7, 3, 0])
    c = O.Cache(t)
    parts = [t.forward([5, 1, 2], c), t.forward([7], c), t.forward([3, 0], c)]
    np.testing.assert_allclose(np.concatenate(parts), full, rtol=1e-5,
                               atol=1e-6)
    assert len(c) == 6
    c.truncate(4)
    again = t.forward([3, 0], c)
    np.testing.assert_array_equal(again, parts[2])
    a = O.generate_advanced(t, [1, 2, 3], 6, 0.0, 42, use_cache=False)
    b = O.generate_advanced(t, [1, 2, 3], 6, 0.0, 42, use_cache=True)
    np.testing.assert_array_equal(a, b)


def test_max_seq_len_throws():
    t, _ = tiny_models()
    with pytest.raises(RuntimeError):
        t.forward(list(range(8)) * 9)


def test_int8_cache_skips_the_length_check():
    """layer.cpp:1171-1179 reads S_past from caches[0].k, which an int8
    cache leaves null: the check never fires and the cache grows past
    max_seq_len, while an fp32 cache throws at the same length.
    Past max_seq_len the int8-cache forward equals a no-cache forward of
    the same ids on a model with room (attention over the dequantised
    rows within 0.08, gqa_test.cpp:213-265's bound)."""
    vocab = 8
    tp = O.make_params(vocab, 16, 2, 32, 2, 11, std=0.3)
    small = O.Model(vocab, 16, 2, 32, 2, 16, tp)
    big = O.Model(vocab, 16, 2, 32, 2, 64, tp)
    ids = [i * 5 % vocab for i in range(24)]
    c8 = O.Cache(small, quantized=True)
    parts = [small.forward(ids[:10], c8), small.forward(ids[10:20], c8),
             small.forward(ids[20:], c8)]
    assert len(c8) == 24
    np.testing.assert_allclose(np.concatenate(parts), big.forward(ids),
                               atol=0.08)
    c32 = O.Cache(small)
    small.forward(ids[:10], c32)
    with pytest.raises(RuntimeError):
        small.forward(ids[10:20], c32)
    # the speculative loop: the int8 run completes, the fp32 one fails
    d = O.Model(vocab, 16, 2, 32, 1, 16,
                O.make_params(vocab, 16, 2, 32, 1, 12, std=0.3))
    out, _ = O.generate_speculative(small, d, [1, 2, 3], 20, 3, 0.0, 42,
                                    quantized_cache=True)
    assert len(out) == 23
    with pytest.raises(RuntimeError):
        O.generate_speculative(small, d, [1, 2, 3], 20, 3, 0.0, 42)


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("k", [1, 3, 4])
def test_greedy_spec_equals_ar(quant, k):
    """transformer_test.cpp:307-346: greedy speculative == greedy AR."""
    t, d = tiny_models(quantize=quant)
    for prompt in ([1, 2, 3], [7, 0, 5, 5, 2]):
        ar = O.generate_advanced(t, prompt, 12, 0.0, 42)
        sp, st = O.generate_speculative(t, d, prompt, 12, k, 0.0, 42)
        np.testing.assert_array_equal(sp, ar)
        assert len(sp) == len(prompt) + 12
        assert st.accepted + st.resampled + st.bonus + 1 == 12


def _trace_draft_cache(prompt, first, cycles, draft, what):
    """Hand trace of the reference's draft cache (layer.cpp:1541-1545,
    1632-1653), written as the explicit token sequence it holds: the draft
    prefill holds the prompt; drafting step j of a cycle appends
    generated.back() (j = 0) or c_{j-1}; a rejection at r truncates it to
    dstart + r + 1 and appends the recovered token, which the next cycle
    appends again as generated.back(); full acceptance with a bonus appends
    c_{M-1}.  Each drafting step's logits must be those of a no-cache
    forward over that sequence (positions = indices).  Returns what kinds of
    cycle ends were seen and how far the duplicate moved the logits."""
    dseq = list(prompt)
    gen = list(prompt) + [first]
    kinds, dup_effect = set(), 0.0
    prev_rej = None
    for ci, cyc in enumerate(cycles):
        assert cyc["dstart"] == len(dseq), (what, ci)
        assert cyc["tstart"] == len(gen) - 1, (what, ci)
        if prev_rej is not None:
            # after a rejection at r: dstart' = dstart + r + 2, and the
            # recovered token is fed again at the next position
            dstart0, r, rec = prev_rej
            assert cyc["dstart"] == dstart0 + r + 2, (what, ci)
            assert dseq[-1] == rec and gen[-1] == rec
        for j in range(cyc["M"]):
            dseq.append(gen[-1] if j == 0 else int(cyc["cand"][j - 1]))
            want = draft.forward(dseq)[-1]
            np.testing.assert_allclose(cyc["dlogits"][j], want, rtol=1e-5,
                                       atol=1e-6, err_msg=f"{what} {ci} {j}")
            if j == 0 and prev_rej is not None:
                # the sequence without the duplicate gives other logits
                alt = draft.forward(dseq[:-2] + dseq[-1:])[-1]
                dup_effect = max(dup_effect, float(np.abs(alt - want).max()))
        acc, tok, M = cyc["acc"], cyc["tok"], cyc["M"]
        gen += [int(c) for c in cyc["cand"][:acc]]
        prev_rej = None
        if acc < M:
            dseq = dseq[:cyc["dstart"] + acc + 1] + [tok]
            gen.append(tok)
            kinds.add("reject@0" if acc == 0 else "reject@j")
            prev_rej = (cyc["dstart"], acc, tok)
        elif tok >= 0:
            dseq.append(int(cyc["cand"][M - 1]))
            gen.append(tok)
            kinds.add("bonus")
    return gen, kinds, dup_effect


@pytest.mark.parametrize("T", [1.0, 0.0])
def test_draft_cache_duplicate_rule_hand_traced(T):
    """The oracle's draft-side state (the draft cache after each cycle's
    rollback and catch-up) pinned by a hand trace of
    the reference: after a rejection the draft cache holds the recovered
    token twice and later draft positions drift by one
    (layer.cpp:1541-1545, 1632-1642); after full acceptance it does not
    (layer.cpp:1649-1653).  A draft close to the target (its weights the
    target's plus noise) gives rejections at j = 0 and j > 0 and full
    acceptances in one run."""
    vocab, d_, H, F = 16, 16, 2, 32
    tp = O.make_params(vocab, d_, H, F, 2, 31, std=0.3)
    rng = np.random.default_rng(5)
    dp = [p + (rng.standard_normal(p.shape).astype(np.float32) *
               np.float32(0.05) if p.ndim == 2 and p.shape[0] > 1 else 0)
          for p in tp]
    dp = [np.ascontiguousarray(p, np.float32) for p in dp]
    t = O.Model(vocab, d_, H, F, 2, 256, tp)
    dm = O.Model(vocab, d_, H, F, 2, 256, dp)
    prompt = [3, 1, 4, 1, 5]
    kinds_all, effect = set(), 0.0
    for seed in (42, 7, 99):
        out, st, cycles, _ = O.generate_speculative_traced(t, dm, prompt, 40,
                                                           3, T, seed)
        gen, kinds, eff = _trace_draft_cache(prompt, int(out[len(prompt)]),
                                             cycles, dm, f"seed {seed}")
        np.testing.assert_array_equal(gen, out)
        assert len(cycles) == st.cycles
        kinds_all |= kinds
        effect = max(effect, eff)
    want = {"reject@0", "reject@j", "bonus"} if T > 0 else {"reject@0"}
    assert want <= kinds_all, kinds_all
    # a restatement without the duplicate would fail the check above
    assert effect > 1e-3, effect


def test_threads_do_not_change_results():
    """or_set_threads splits only independent outputs: logits and a sampled
    run are bit-identical for 1 and 4 threads."""
    t, d = tiny_models(vocab=64)
    try:
        O.set_threads(1)
        a = t.forward(list(range(20)))
        sa, _ = O.generate_speculative(t, d, [1, 2, 3], 10, 3, 1.0, 42)
        O.set_threads(4)
        b = t.forward(list(range(20)))
        sb, _ = O.generate_speculative(t, d, [1, 2, 3], 10, 3, 1.0, 42)
    finally:
        O.set_threads(1)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(sa, sb)


def test_sampled_same_seed_same_output():
    """transformer_test.cpp:275-305 (same seed => same tokens)."""
    t, d = tiny_models()
    a, sa = O.generate_speculative(t, d, [1, 2, 3], 10, 3, 1.0, 42)
    b, sb = O.generate_speculative(t, d, [1, 2, 3], 10, 3, 1.0, 42)
    np.testing.assert_array_equal(a, b)
    assert (sa.cycles, sa.accepted) == (sb.cycles, sb.accepted)
    assert ((a >= 0) & (a < 8)).all()


def test_speculative_sampling_preserves_target_distribution():
    """Accept-with-r*q<p plus the max(0, p-q) residual must emit tokens
    distributed as the target's p (the speculative-sampling theorem).  With
    k=1 and max_new=2 the second token comes from one verify cycle; its
    empirical law, conditioned on the first token, is compared with the
    target softmax by a chi-square bound."""
    t, d = tiny_models(vocab=6, seed=23)
    prompt = [1, 4, 2]
    counts = {}
    n = 6000
    for s in range(n):
        out, _ = O.generate_speculative(t, d, prompt, 2, 1, 1.0, 1000 + s)
        counts.setdefault(int(out[3]), np.zeros(6))[int(out[4])] += 1
    worst = 0.0
    for first, cnt in counts.items():
        if cnt.sum() < 300:
            continue
        p = O.get_probs(t.forward(prompt + [first])[-1], 1.0).astype(
            np.float64)
        exp = p * cnt.sum()
        keep = exp > 5
        chi2 = (((cnt - exp) ** 2 / exp)[keep]).sum()
        worst = max(worst, chi2)
        # 5 degrees of freedom: P(chi2 > 25) ~ 1.4e-4
        assert chi2 < 25.0, (first, cnt, exp)
    # the draft must differ from the target for the test to mean anything
    q = O.get_probs(d.forward(prompt + [3])[-1], 1.0)
    p = O.get_probs(t.forward(prompt + [3])[-1], 1.0)
    assert np.abs(p - q).sum() > 0.2


# --------------------------------------------------------------------------
# int8 KV cache (KVCache(quantized=true), layer.cpp:635-757, 878-938)
# --------------------------------------------------------------------------
def test_quantize_kv_known_answers():
    """quantize_kv on rows whose answers are fixed by hand: max 127 gives
    scale 1 exactly, so the codes are round-half-away-from-zero of the
    values themselves (2.5 -> 3, -2.5 -> -3, 1.5 -> 2, -0.5 -> -1, where
    round-half-even would give 2, -2, 2, 0); an all-zero row gets scale 1
    and zero codes; a row led by a negative maximum maps it to -127."""
    rows = np.array([[127.0, -63.5, 2.5, -2.5, 0.49, 0.0, 1.5, -0.5],
                     [0.0] * 8,
                     [-3.0, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 1.5]], np.float32)
    codes, scales = O.quantize_kv(rows)
    np.testing.assert_array_equal(codes[0], [127, -64, 3, -3, 0, 0, 2, -1])
    np.testing.assert_array_equal(codes[1], np.zeros(8))
    s = np.float32(3.0) / np.float32(127.0)
    inv = np.float32(1.0) / s
    assert scales[0] == 1.0 and scales[1] == 1.0 and scales[2] == s
    assert codes[2, 0] == -127
    assert codes[2, 1] == int(np.round(np.float32(1.0) * inv))     # 42
    assert codes[2, 7] == 64                                        # 63.5 -> 64


def test_quantize_kv_error_bound():
    """|code * scale - x| <= scale / 2 (plus one rounding of x / scale) for
    every element; the largest |x| of a row maps to +-127."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((300, 64)) * rng.random((300, 1)) * 5).astype(np.float32)
    codes, scales = O.quantize_kv(x)
    deq = codes.astype(np.float64) * scales[:, None]
    err = np.abs(deq - x.astype(np.float64))
    assert (err <= scales[:, None] * (0.5 + 1e-5)).all()
    top = np.abs(x).argmax(1)
    np.testing.assert_array_equal(np.abs(codes[np.arange(300), top]), 127)
    assert np.abs(codes).max() <= 127


def test_attention_q8_equals_dequantised_fp32_path():
    """The quantized fused path equals the fp32 fused path run on the
    dequantised cache (layer.cpp:826-831 dequantize_k / _v then the same
    per-element products): bit-exact, since both form (float)code * scale
    and then the same fp32 operations in the same order."""
    rng = np.random.default_rng(4)
    H, Hkv, S, St, D = 4, 2, 3, 21, 16
    q = rng.standard_normal((H, S, D)).astype(np.float32)
    kq = rng.integers(-127, 128, (Hkv, St, D)).astype(np.int8)
    vq = rng.integers(-127, 128, (Hkv, St, D)).astype(np.int8)
    ks = (rng.random((Hkv, St)) * 0.05 + 1e-3).astype(np.float32)
    vs = (rng.random((Hkv, St)) * 0.05 + 1e-3).astype(np.float32)
    got = O.attention_q8(q, kq, ks, vq, vs)
    k = (kq.astype(np.float32) * ks[:, :, None]).astype(np.float32)
    v = (vq.astype(np.float32) * vs[:, :, None]).astype(np.float32)
    want = np.zeros((S, H, D), np.float32)
    O.lib().or_attention(O.fptr(q), O.fptr(np.ascontiguousarray(k)),
                         O.fptr(np.ascontiguousarray(v)), H, Hkv, S, St, D, 1,
                         O.fptr(want))
    np.testing.assert_array_equal(got, want)
    # and both agree with the float64 softmax attention over the same rows
    kk = np.repeat(k, H // Hkv, 0)
    vv = np.repeat(v, H // Hkv, 0)
    np.testing.assert_allclose(got, attn_f64(q, kk, vv, True), rtol=1e-5,
                               atol=1e-5)


def test_int8_cache_close_to_fp32_cache():
    """gqa_test.cpp:213-265 (KVQuantizationVerification): the int8-cache
    outputs stay within 0.08 of the fp32-cache ones, step by step; here on
    whole-model logits with the cache's codes checked against a fresh
    quantisation of the fp32 cache's rows."""
    t, _ = tiny_models(quantize=True)
    cf, cq = O.Cache(t), O.Cache(t, quantized=True)
    for ids in ([5, 1, 2], [7], [3, 0]):
        a = t.forward(ids, cf)
        b = t.forward(ids, cq)
        assert np.abs(a - b).max() <= 0.08
        assert not np.array_equal(a, b) or len(ids) == 0
    kq, ks, vq, vs = cq.read_q8(1)
    assert kq.shape == (2, 6, 8) and ks.shape == (2, 6)
    assert (np.abs(kq).max(2) == 127).all() and (np.abs(vq).max(2) == 127).all()


def test_spec_quantized_reference_case():
    """transformer_test.cpp:348-371 (SpeculativeDecodingQuantized): vocab 6,
    embed 8, 2 heads, MLP 16, target 2 layers, draft 1, max_seq 32, prompt
    {2, 4, 1}, 5 new, k = 2, greedy, quantized cache: 8 ids, all < 6."""
    tp = O.make_params(6, 8, 2, 16, 2, 5, std=0.3)
    dp = O.make_params(6, 8, 2, 16, 1, 6, std=0.3)
    t = O.Model(6, 8, 2, 16, 2, 32, tp)
    d = O.Model(6, 8, 2, 16, 1, 32, dp)
    out, st = O.generate_speculative(t, d, [2, 4, 1], 5, 2, 0.0, 42,
                                     quantized_cache=True)
    assert len(out) == 8 and ((out >= 0) & (out < 6)).all()
    assert list(out[:3]) == [2, 4, 1]


@pytest.mark.parametrize("k", [1, 3])
def test_greedy_spec_int8_cache_equals_ar_int8_cache(k):
    """Greedy speculative decoding with int8 caches equals greedy
    autoregressive decoding through an int8 cache: every cached row is
    quantised from the same token prefix however the cycles batch and
    roll back the positions (transformer_test.cpp:307-346 with
    KVCache(true))."""
    t, d = tiny_models(quantize=True)
    for prompt in ([1, 2, 3], [7, 0, 5, 5, 2]):
        c = O.Cache(t, quantized=True)
        seq = list(prompt)
        lg = t.forward(np.array(seq, np.int32), c)
        for _ in range(12):
            seq.append(int(np.argmax(lg[-1])))
            lg = t.forward(np.array(seq[-1:], np.int32), c)
        sp, st = O.generate_speculative(t, d, prompt, 12, k, 0.0, 42,
                                        quantized_cache=True)
        np.testing.assert_array_equal(sp, seq)
        assert st.accepted + st.resampled + st.bonus + 1 == 12


def test_frozen_cache_recomputes_forward():
    """The checker hook: a forward over a cache that was given another
    cache's codes (new positions included) and frozen reproduces that
    cache's own forward bit for bit."""
    t, _ = tiny_models(quantize=True)
    a = O.Cache(t, quantized=True)
    t.forward([5, 1, 2, 6], a)
    want = t.forward([7, 3], a)
    b = O.Cache(t, quantized=True)
    for layer in range(2):
        b.write_q8(layer, *a.read_q8(layer))
    b.set_len(4)
    b.freeze()
    np.testing.assert_array_equal(t.forward([7, 3], b), want)
    kr, vr = a.read_raw(0)
    kq, ks, vq, vs = a.read_q8(0)
    for raw, codes, scales in ((kr, kq, ks), (vr, vq, vs)):
        c, sc = O.quantize_kv(raw)
        np.testing.assert_array_equal(c, codes)
        np.testing.assert_array_equal(sc, scales)


# --------------------------------------------------------------------------
# NETW weight files (serialization.cpp:8-109; serialization_test.cpp)
# --------------------------------------------------------------------------
def reference_shapes(vocab, d, F, L):
    """parameters() shapes as the reference constructs them: Embedding
    [V][d] (layer.cpp:267-268); Dense weight [in][out] and bias [1][out]
    (layer.cpp:153-157); LayerNorm gamma / beta [d] (layer.cpp:1063-1064)."""
    dense = lambda i, o: [(i, o), (1, o)]
    shapes = [(vocab, d)]
    for _ in range(L):
        for _ in range(4):
            shapes += dense(d, d)                     # q, k, v, o
        shapes += dense(d, F) + dense(d, F) + dense(F, d)   # gate, up, down
        shapes += [(d,), (d,), (d,), (d,)]
    return shapes + dense(d, vocab)


def parse_netw(blob):
    import struct
    assert blob[:4] == b"NETW"
    version, count = struct.unpack_from("<HI", blob, 4)
    off, out = 10, []
    for _ in range(count):
        (rank,) = struct.unpack_from("<I", blob, off); off += 4
        dims = struct.unpack_from("<%dQ" % rank, blob, off); off += 8 * rank
        (n,) = struct.unpack_from("<Q", blob, off); off += 8
        data = np.frombuffer(blob, np.float32, n, off); off += 4 * n
        out.append((dims, data))
    assert off == len(blob)
    return version, out


def test_netw_layout(tmp_path):
    """The file bytes follow save_parameters field by field: magic, uint16
    version 1, uint32 count, then rank / extents / count / fp32 data per
    tensor in parameters() order with the reference's shapes."""
    V, d, H, F, L = 5, 4, 2, 8, 2
    params = O.make_params(V, d, H, F, L, 3, std=0.5, bias_std=0.1)
    m = O.Model(V, d, H, F, L, 16, params)
    path = tmp_path / "w.netw"
    m.save_weights(path)
    version, tensors = parse_netw(path.read_bytes())
    assert version == 1
    shapes = reference_shapes(V, d, F, L)
    assert len(tensors) == len(shapes) == len(params)
    for (dims, data), shape, p in zip(tensors, shapes, params):
        assert dims == shape
        np.testing.assert_array_equal(data, p.ravel())


def test_netw_round_trip(tmp_path):
    """serialization_test.cpp SaveAndLoadConsistency: a model loaded from
    another's file has its parameters and gives its outputs (bit-equal);
    a quantised model re-quantises from the loaded weights."""
    V, d, H, F, L = 12, 8, 2, 16, 2
    pa = O.make_params(V, d, H, F, L, 4, std=0.3)
    pb = O.make_params(V, d, H, F, L, 5, std=0.3)
    a = O.Model(V, d, H, F, L, 32, pa)
    path = tmp_path / "a.netw"
    a.save_weights(path)
    ids = [3, 1, 4, 1, 5]
    for quant in (False, True):
        b = O.Model(V, d, H, F, L, 32, pb, quantize=quant)
        assert b.load_weights(path) == 0
        want = O.Model(V, d, H, F, L, 32, pa, quantize=quant).forward(ids)
        np.testing.assert_array_equal(b.forward(ids), want)


def test_netw_errors(tmp_path):
    """serialization_test.cpp ShapeMismatchAssertion and the other checks of
    load_parameters: wrong extent, tensor count, rank, signature, version,
    a missing file and a truncated one are all rejected."""
    import struct
    V, d, H, F = 6, 4, 2, 8
    a = O.Model(V, d, H, F, 1, 16, O.make_params(V, d, H, F, 1, 1))
    path = tmp_path / "a.netw"
    a.save_weights(path)
    blob = path.read_bytes()
    wide = O.Model(V, 8, H, F, 1, 16, O.make_params(V, 8, H, F, 1, 1))
    assert wide.load_weights(path) == -6                  # extent
    deep = O.Model(V, d, H, F, 2, 16, O.make_params(V, d, H, F, 2, 1))
    assert deep.load_weights(path) == -4                  # tensor count
    fresh = O.Model(V, d, H, F, 1, 16, O.make_params(V, d, H, F, 1, 2))
    for name, data, code in (
            ("magic", b"NETX" + blob[4:], -2),
            ("version", blob[:4] + struct.pack("<H", 2) + blob[6:], -3),
            ("rank", blob[:10] + struct.pack("<I", 3) + blob[14:], -5),
            ("short", blob[:-3], -8)):
        p = tmp_path / name
        p.write_bytes(data)
        assert fresh.load_weights(p) == code, name
    assert fresh.load_weights(tmp_path / "missing") == -1

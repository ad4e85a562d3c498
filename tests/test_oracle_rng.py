"""Pins the oracle's std::mt19937 stream (or_mt_*) and the order in which
or_generate_speculative / or_generate_advanced consume it (CPU).

generate_speculative and generate_advanced seed one std::mt19937 with the
caller's seed (layer.cpp:1249, 1394) and draw from it with
std::discrete_distribution<size_t> (layer.cpp:1369-1371, 1493-1498) and
std::uniform_real_distribution<float>(0, 1) (layer.cpp:1596-1597).  The
fixture tests/golden/mt19937_kat.json holds what the C++ standard library
(libstdc++ of this image, tests/golden/make_mt19937_kat.sh) returns for
those calls: raw outputs at the twist boundaries, the standard's check
value (the 10000th output of a default-seeded engine is 4123659995), and
streams that interleave the float draw, generate_canonical<double, 53> and
discrete_distribution draws.
"""
import json
import os
import struct

import numpy as np

import oracle_py as O

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                  "mt19937_kat.json")))


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def dbits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def discrete(weights, u):
    """std::discrete_distribution over double weights: divide by the
    left-to-right double sum, left-to-right partial sums, the last set to
    1.0, the first index whose partial sum is not below u."""
    total = 0.0
    for w in weights:
        total += w
    cp, acc = [], 0.0
    for w in weights:
        acc += w / total
        cp.append(acc)
    cp[-1] = 1.0
    for i, c in enumerate(cp):
        if c >= u:
            return i
    return len(cp) - 1


def test_raw_outputs_and_the_standard_check_value():
    for rec in KAT["raw"]:
        g = O.MT19937(rec["seed"])
        want = dict(rec["out"])
        for i in range(max(want) + 1):
            v = g.next()
            if i in want:
                assert v == want[i], (rec["seed"], i)
    g = O.MT19937(5489)
    for _ in range(9999):
        g.next()
    assert g.next() == KAT["default_10000th"] == 4123659995


def test_interleaved_float_double_and_discrete_draws():
    w = [0.1, 0.0, 0.25, 0.05, 0.3, 0.0, 0.2, 0.1]
    for rec in KAT["mixed"]:
        g = O.MT19937(rec["seed"])
        for i, (kind, val) in enumerate(rec["draws"]):
            if kind == 0:
                assert fbits(g.f()) == val, (rec["seed"], i)
            elif kind == 1:
                assert dbits(g.d()) == val, (rec["seed"], i)
            else:
                assert discrete(w, g.d()) == val, (rec["seed"], i)


def test_discrete_lower_bound_rule_over_many_draws():
    rec = KAT["discrete"]
    g = O.MT19937(rec["seed"])
    got = [discrete(rec["weights"], g.d()) for _ in rec["draws"]]
    assert got == rec["draws"]
    # zero-weight entries are never drawn
    assert all(rec["weights"][i] > 0 for i in got)


def test_float_draw_stays_below_one():
    """(float)x rounds x >= 2^32 - 128 up to 2^32: the draw is then the
    float just below 1 (nextafter), as libstdc++ returns."""
    g = O.MT19937(0)
    for _ in range(5000):
        assert 0.0 <= g.f() < 1.0


def tiny_models():
    vocab = 24
    tp = O.make_params(vocab, 16, 2, 32, 2, 5, std=0.3)
    dp = O.make_params(vocab, 16, 2, 32, 1, 6, std=0.3)
    return (O.Model(vocab, 16, 2, 32, 2, 96, tp),
            O.Model(vocab, 16, 2, 32, 1, 96, dp))


def test_speculative_loop_consumes_the_stream_in_the_reference_order():
    """With or_set_rng(1) the draft candidates of every cycle are the
    draws of get_probs(draft logits) from the next doubles of the stream
    seeded seed + seq, after the first token's double and, per earlier
    cycle, 2 outputs a draft sample, one a test up to the first rejection
    and 2 for the resample or bonus (layer.cpp:1493-1498, 1541-1558,
    1581-1630, 1643-1647).  A plausible mistake -- tests drawn before the
    draft samples, one output per double, drawing all k tests -- moves the
    candidates off these draws."""
    t, d = tiny_models()
    prompt = np.array([3, 7, 1, 19, 4], np.int32)
    seed, seq, k, new = 77, 3, 4, 30
    O.set_rng(1)
    try:
        out, st, cycles, _ = O.generate_speculative_traced(
            t, d, prompt, new, k, 1.0, seed, seq=seq)
    finally:
        O.set_rng(0)
    g = O.MT19937(seed + seq)
    g.d()                                  # the first token
    ngen = 1
    for c in cycles:
        M = c["M"]
        for j in range(M):
            q = O.get_probs(c["dlogits"][j], 1.0)
            assert O.sample(q, g.d()) == c["cand"][j]
        tests = c["acc"] + 1 if c["acc"] < M else M
        for _ in range(tests):
            g.next()
        if c["acc"] < M or ngen + M < new:
            g.d()
        ngen += c["acc"] + (1 if c["tok"] >= 0 else 0)
    assert len(out) == len(prompt) + new and st.cycles == len(cycles)


def test_mt_stream_changes_sampled_outputs_not_greedy_ones():
    t, d = tiny_models()
    prompt = np.array([3, 7, 1, 19, 4], np.int32)
    runs = {}
    for mode in (0, 1):
        O.set_rng(mode)
        try:
            runs[mode] = (O.generate_speculative(t, d, prompt, 24, 3, 1.0, 5)[0],
                          O.generate_speculative(t, d, prompt, 24, 3, 0.0, 5)[0],
                          O.generate_advanced(t, prompt, 24, 1.0, 5))
        finally:
            O.set_rng(0)
    assert not np.array_equal(runs[0][0], runs[1][0])
    np.testing.assert_array_equal(runs[0][1], runs[1][1])
    assert not np.array_equal(runs[0][2], runs[1][2])


def test_generate_advanced_draws_one_double_per_token():
    """Sampled generate_advanced (layer.cpp:1249-1372): token i is the draw of
    get_probs(last logits) from the i-th double of the stream."""
    t, _ = tiny_models()
    prompt = np.array([2, 9, 14], np.int32)
    O.set_rng(1)
    try:
        out = O.generate_advanced(t, prompt, 12, 0.8, 31, seq=2)
    finally:
        O.set_rng(0)
    g = O.MT19937(33)
    seqn = list(prompt)
    for i in range(12):
        lg = t.forward(np.array(seqn, np.int32))[-1]
        tok = O.sample(O.get_probs(lg, 0.8), g.d())
        assert tok == out[len(prompt) + i]
        seqn.append(tok)

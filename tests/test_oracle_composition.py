"""Pins how or_forward composes a decoder (CPU).

The oracle's parts (Dense, RoPE, LayerNorm, attention) are pinned one by one
in test_oracle.py; these tests pin the way the reference puts them together
in TransformerDecoder::forward (layer.cpp:1161-1193) and
TransformerDecoderLayer::forward (layer.cpp:1097-1114), with weights built so
that the whole forward reduces to a short float64 closed form
(tests/composition.py):

* post-LN order x1 = LN1(x + MHA(x)), y = LN2(x1 + SwiGLU(x1))
  (layer.cpp:1097-1114) and no final LayerNorm before lm_head
  (layer.cpp:1189-1192);
* SwiGLU's roles (g * sigmoid(g)) * u with g the gate Dense and u the up
  Dense (layer.cpp:1704-1710);
* RoPE on q and k only (layer.cpp:629-630), at absolute positions
  S_past + s with the pair angles of the head width (tensor.cpp:1126-1226),
  scores scaled by 1/sqrt(D), causal mask j <= S_past + i
  (layer.cpp:842-952).

Every case also evaluates its closed form under the plausible mistakes it is
meant to catch and requires each of them to lie far outside the tolerance,
so a case that could not tell a mistake apart fails here rather than
passing silently.
"""
import numpy as np
import pytest

import composition as CP
import oracle_py as O

TOL = 2e-5          # fp32 oracle vs float64 closed form, O(1) activations
FAR = 100 * TOL     # a mistaken composition must miss by at least this


def oracle_model(P, max_seq=64):
    c = CP.CFG
    return O.Model(c["vocab"], c["d"], c["H"], c["F"], P.L, max_seq,
                   P.flat())


def check(got, want, mistakes, what):
    err = CP.max_abs(got, want(None))
    assert err <= TOL, f"{what}: |oracle - closed form| = {err:.3g}"
    for m in mistakes:
        miss = CP.max_abs(got, want(m))
        assert miss >= FAR, f"{what}: the case cannot tell '{m}' apart ({miss:.3g})"


IDS = [5, 17, 3, 40, 17, 127, 0, 29, 8, 51]


@pytest.mark.parametrize("L", [1, 2])
def test_post_ln_output_and_no_final_layernorm(L):
    """lm_head a permutation, lm bias random: (logits - b)[perm[j]] undone
    through the last layer's LN2 gamma and beta is a normalised row (mean 0,
    mean square v / (v + 1e-5)).  A pre-LN layer, a final LayerNorm after the
    last layer (which would renormalise gamma2 * xhat + beta2) or a
    transposed lm head leaves rows that are not normalised."""
    P, perm = CP.case_post_ln(seed=10 + L, L=L)
    logits = oracle_model(P).forward(IDS)
    z = CP.post_ln_residual(P, perm, logits)
    assert np.abs(z.mean(1)).max() < 1e-5
    ms = (z * z).mean(1)
    assert ms.max() <= 1.0 + 1e-5 and ms.min() >= 1.0 - 1e-3
    # the same undo with the transposed permutation or with a final
    # gamma = 1, beta = 0 normalisation is not a normalised row
    zt = CP.post_ln_residual(P, np.argsort(perm), logits)
    assert np.abs(zt.mean(1)).max() > 1e-2
    renorm = CP.ln(np.asarray(logits, np.float64), 1.0, 0.0)
    zf = CP.post_ln_residual(P, perm, renorm)
    assert np.abs(zf.mean(1)).max() > 1e-2


@pytest.mark.parametrize("L", [1, 2])
def test_layer_composition_closed_form(L):
    """W_v = 0 (attention adds only b_o) and W_gate = 0 (the gate is its
    bias c): each layer is x1 = LN1(x + b_o),
    y = LN2(x1 + ((c sigmoid c) (x1 W_up + b_up)) W_down + b_down), logits =
    y + b_lm (lm_head = I).  Rejects pre-LN, a gate/up swap
    (u sigmoid(u) c), a dropped residual on either sublayer and a final
    LayerNorm; with L = 2 also layer 2 reading layer 1's parameters."""
    P = CP.case_layer(seed=20 + L, L=L)
    got = oracle_model(P).forward(IDS)
    check(got, lambda m: CP.layer_closed_form(P, IDS, m),
          CP.MISTAKES["layer"], f"layer L={L}")
    # every row depends on its own token only (attention adds a constant)
    np.testing.assert_array_equal(got[1], got[4])
    if L == 2:
        swapped = CP.case_layer(seed=22, L=2)
        swapped.layers = swapped.layers[::-1]
        assert CP.max_abs(got, CP.layer_closed_form(swapped, IDS)) >= FAR


def test_attention_is_causal_mean_of_unrotated_v():
    """W_q = W_k = 0: every score is 0, so row i's attention output is the
    mean of v_j over j <= i, with v not rotated.  RoPE applied to v or a
    missing causal mask fails; the cached forward (two calls) gives the
    same rows, so the cached keys sit at their absolute positions."""
    P = CP.case_mean_v(seed=30)
    m = oracle_model(P)
    got = m.forward(IDS)
    check(got, lambda mk: CP.mean_v_closed_form(P, IDS, mk),
          CP.MISTAKES["mean_v"], "mean of v")
    c = O.Cache(m)
    parts = np.concatenate([m.forward(IDS[:4], c), m.forward(IDS[4:], c)])
    assert CP.max_abs(parts, CP.mean_v_closed_form(P, IDS)) <= TOL


def test_rope_on_q_and_k_at_absolute_positions():
    """q and k inputs the same for every token: the scores are set by RoPE
    of q and k alone (complex rotation by p theta_m, theta_m =
    10000^(-2m / D) with D the head width), scaled by 1/sqrt(D).  No RoPE,
    angles from d_model instead of D, or no 1/sqrt(D) fails.  Split over
    three cached calls the rows are unchanged, which places the new rows at
    S_past + s."""
    P = CP.case_rope(seed=40)
    m = oracle_model(P)
    got = m.forward(IDS)
    check(got, lambda mk: CP.rope_closed_form(P, IDS, mk),
          CP.MISTAKES["rope"], "rope")
    c = O.Cache(m)
    parts = np.concatenate([m.forward(IDS[:3], c), m.forward(IDS[3:4], c),
                            m.forward(IDS[4:], c)])
    assert CP.max_abs(parts, CP.rope_closed_form(P, IDS)) <= TOL
    # positions restarting at 0 on each call would change the rows
    fresh = np.concatenate([m.forward(IDS[:3]), m.forward(IDS[3:4]),
                            m.forward(IDS[4:])])
    assert CP.max_abs(fresh, CP.rope_closed_form(P, IDS)) >= FAR


def test_int8_forward_is_the_composition_of_dequantised_dense():
    """The quantised decoder composes the same way: its forward equals the
    fp32 decoder built from the dequantised weights (codes * scale,
    quantization.cpp:88-147) within fp32 rounding."""
    P = CP.case_layer(seed=50, L=2)
    P.lm_w = P.rng.standard_normal((CP.CFG["d"], CP.CFG["vocab"])) * 0.2
    c = CP.CFG
    q = O.Model(c["vocab"], c["d"], c["H"], c["F"], P.L, 64, P.flat(), True)
    D = CP.dequantized(P, q.quantized)
    fp = O.Model(c["vocab"], c["d"], c["H"], c["F"], P.L, 64, D.flat())
    np.testing.assert_allclose(q.forward(IDS), fp.forward(IDS), atol=2e-5)

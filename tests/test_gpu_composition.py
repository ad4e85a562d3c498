"""The device decoder against the float64 closed forms of constructed
decoders (GPU).

The same constructed weights as test_oracle_composition.py
(tests/composition.py) pin the device's own composition directly, not only
through the oracle: post-LN order and no final LayerNorm
(layer.cpp:1097-1114, 1189-1192), SwiGLU's gate/up roles
(layer.cpp:1704-1710; the device interleaves gate and up columns in one
GEMM), RoPE on q and k only at absolute positions (layer.cpp:629-630; the
device applies it in the q/k/v GEMM epilogue), the causal mask and the
1/sqrt(D) scale (layer.cpp:842-952).  fp32 models run the fp32 Dense path;
int8 models run the GEMV (10 rows), the digit-plane MFMA GEMM (40 rows) and
the LDS MFMA GEMM (192 rows) and are compared with the closed form over
their dequantised weights.  Tolerance: 1e-4 of a row (row-relative, as the
other parity tests).
"""
import numpy as np
import pytest

import composition as CP
from gpu_util import assert_rows_close, nnhip

pytestmark = pytest.mark.gpu

SHAPES = [(1, 10), (4, 10), (32, 6)]


def device_model(ctx, P, quantize):
    c = CP.CFG
    gm = nnhip.Decoder(ctx, c["vocab"], c["d"], c["H"], c["F"], P.L, 64)
    gm.set_params(P.flat())
    if quantize:
        gm.quantize(8)
    return gm, (CP.dequantized(P, gm.get_quantized) if quantize else P)


def ids_for(B, S, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, CP.CFG["vocab"], (B, S)).astype(np.int32)


def check_rows(got, want, mistakes_want, what):
    assert_rows_close(got, want, 1e-4, what)
    for m, w in mistakes_want:
        err = float(np.abs(np.asarray(got, np.float64) - w).max() /
                    np.abs(w).max())
        assert err > 1e-2, f"{what}: indistinguishable from '{m}'"


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("B,S", SHAPES)
def test_device_layer_composition(ctx, quant, B, S):
    P = CP.case_layer(seed=60, L=2)
    gm, E = device_model(ctx, P, quant)
    ids = ids_for(B, S, 61)
    got = gm.forward(ids)
    for b in range(B):
        cf = lambda m: CP.layer_closed_form(E, ids[b], m)  # noqa: E731
        check_rows(got[b], cf(None),
                   [(m, cf(m)) for m in CP.MISTAKES["layer"]],
                   f"layer quant={quant} b={b}")
    gm.free()


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("B,S", SHAPES)
def test_device_attention_mean_of_unrotated_v(ctx, quant, B, S):
    P = CP.case_mean_v(seed=62)
    gm, E = device_model(ctx, P, quant)
    ids = ids_for(B, S, 63)
    got = gm.forward(ids)
    for b in range(B):
        cf = lambda m: CP.mean_v_closed_form(E, ids[b], m)  # noqa: E731
        check_rows(got[b], cf(None),
                   [(m, cf(m)) for m in CP.MISTAKES["mean_v"]],
                   f"mean_v quant={quant} b={b}")
    gm.free()


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("B,S", SHAPES)
def test_device_rope_positions(ctx, quant, B, S):
    """Whole-sequence forward and the same rows over a KV cache in two
    calls (the second at S_past = 4)."""
    P = CP.case_rope(seed=64)
    gm, E = device_model(ctx, P, quant)
    ids = ids_for(B, S, 65)
    got = gm.forward(ids)
    cache = nnhip.KVCache(gm, batch=B)
    cut = min(4, S - 1)
    parts = np.concatenate([gm.forward(ids[:, :cut], cache),
                            gm.forward(ids[:, cut:], cache)], axis=1)
    for b in range(B):
        cf = lambda m: CP.rope_closed_form(E, ids[b], m)  # noqa: E731
        check_rows(got[b], cf(None),
                   [(m, cf(m)) for m in CP.MISTAKES["rope"]],
                   f"rope quant={quant} b={b}")
        assert_rows_close(parts[b], cf(None), 1e-4, f"rope cached b={b}")
    cache.free()
    gm.free()


@pytest.mark.parametrize("quant", [False, True])
def test_device_post_ln_output(ctx, quant):
    P, perm = CP.case_post_ln(seed=66, L=2)
    gm, _ = device_model(ctx, P, quant)
    ids = ids_for(32, 6, 67)
    got = gm.forward(ids).reshape(-1, CP.CFG["vocab"])
    # int8: the lm head's codes are the permutation times 127 with scales
    # 1/127, so it stays a permutation to fp32 rounding
    z = CP.post_ln_residual(P, perm, got)
    assert np.abs(z.mean(1)).max() < 1e-4
    ms = (z * z).mean(1)
    assert ms.max() <= 1.0 + 2e-4 and ms.min() >= 1.0 - 2e-3
    gm.free()

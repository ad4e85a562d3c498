"""Constructed decoders whose forward has a short float64 closed form.

Each case zeroes or fixes a few weights of a TransformerDecoder so that the
forward collapses to a formula a reader can check against the reference's
layer code line by line, and each case is built so that one family of
plausible composition mistakes changes the result by orders of magnitude
more than fp32 rounding:

* ``case_post_ln``: the logits are the lm head applied to the last layer's
  LN2 output, with no final LayerNorm (``layer.cpp:1097-1114, 1189-1192``);
  the lm head is a permutation, so a transposed lm head also fails.
* ``case_layer``: W_v = 0 makes every attention output zero, so the MHA
  output is the out_proj bias b_o; W_gate = 0 makes the gate the constant
  bias c.  Each layer is then
  ``x1 = LN1(x + b_o)``, ``y = LN2(x1 + ((c*sigmoid(c)) * (x1 W_up + b_up)) W_down + b_down)``
  (post-LN order ``layer.cpp:1097-1114``, SwiGLU roles ``layer.cpp:1704-1710``).
* ``case_mean_v``: W_q = W_k = 0 makes every score zero, so each query
  attends uniformly to the keys at or before its own position: the
  attention output of row i is the mean of the unrotated v_j, j <= i
  (causal mask ``layer.cpp:842-952``, RoPE on q and k only
  ``layer.cpp:629-630``).
* ``case_rope``: the query and key inputs are the same for every token, so
  a score depends on the positions alone, through RoPE of q and k at their
  absolute positions S_past + s with the pair angles of the head width D
  (``tensor.cpp:1126-1226``), scaled by 1/sqrt(D).

The closed forms are float64.  RoPE is written as a complex rotation of the
pairs (x_2m + i x_2m+1) by exp(i p theta_m), theta_m = 10000^(-2m/D).
``MISTAKES`` lists, per case, the variants the case must reject; the tests
check that every variant lies far from the oracle's (and the device's)
result, so the case is shown to tell them apart.
"""
import numpy as np

EPS = 1e-5
# d = vocab so that an identity or permutation lm head is square; 8 heads
# of width 16 (the device needs a head width that is a multiple of 8, and
# K a multiple of 128 for its MFMA GEMMs)
CFG = dict(vocab=128, d=128, H=8, F=256)
NAMES = ("q.w", "q.b", "k.w", "k.b", "v.w", "v.b", "o.w", "o.b", "gate.w",
         "gate.b", "up.w", "up.b", "down.w", "down.b", "ln1.g", "ln1.b",
         "ln2.g", "ln2.b")


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def ln(x, g, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + EPS) * g + b


class Params:
    """Parameters in TransformerDecoder::parameters() order
    (layer.cpp:1140-1154): emb, per layer the 18 of NAMES, lm.w, lm.b."""

    def __init__(self, L, seed, std=0.3):
        c = CFG
        self.L = L
        rng = np.random.default_rng(seed)
        self.rng = rng
        d, F, V = c["d"], c["F"], c["vocab"]

        def r(*shape, s=std):
            return rng.standard_normal(shape) * s

        self.emb = r(V, d, s=1.0)
        self.layers = []
        for _ in range(L):
            p = {}
            for nm, (i, o) in (("q", (d, d)), ("k", (d, d)), ("v", (d, d)),
                               ("o", (d, d)), ("gate", (d, F)),
                               ("up", (d, F)), ("down", (F, d))):
                p[nm + ".w"] = r(i, o, s=std / np.sqrt(i / 16))
                p[nm + ".b"] = r(o, s=0.2)
            for nm in ("ln1", "ln2"):
                p[nm + ".g"] = rng.uniform(0.5, 1.5, d)
                p[nm + ".b"] = r(d, s=0.3)
            self.layers.append(p)
        self.lm_w = r(d, V, s=std / 2)
        self.lm_b = r(V, s=0.2)

    def flat(self):
        """float32 arrays in parameter order, each shaped as the reference's
        tensor ([in, out] Dense weights, [1, n] biases and LN vectors)."""
        out = [self.emb]
        for p in self.layers:
            for nm in NAMES:
                a = p[nm]
                out.append(a if a.ndim == 2 else a[None, :])
        out += [self.lm_w, self.lm_b[None, :]]
        return [np.ascontiguousarray(a, np.float32) for a in out]

    def f64(self):
        """The float64 values of the float32 parameters the models get."""
        q = Params.__new__(Params)
        q.L = self.L
        cast = lambda a: a.astype(np.float32).astype(np.float64)  # noqa: E731
        q.emb = cast(self.emb)
        q.layers = [{k: cast(v) for k, v in p.items()} for p in self.layers]
        q.lm_w, q.lm_b = cast(self.lm_w), cast(self.lm_b)
        return q


def dequantized(P, get_quantized):
    """A float64 copy of P whose Dense weights are the int8 (or INT4) codes
    times their per-channel scales (QuantizedDense::dequantize_weight,
    quantization.cpp:88-147); get_quantized(layer, which, n_in, n_out)
    returns (codes [in][out], scales [out]) with which = 0..6 for q, k, v,
    o, gate, up, down and 7 (layer 0) for the lm head."""
    D = P.f64()
    for l, p in enumerate(D.layers):
        for w, nm in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
            n_in, n_out = p[nm + ".w"].shape
            codes, scales = get_quantized(l, w, n_in, n_out)
            p[nm + ".w"] = codes.astype(np.float64) * scales
    codes, scales = get_quantized(0, 7, CFG["d"], CFG["vocab"])
    D.lm_w = codes.astype(np.float64) * scales
    return D


def rope_c(x, pos, D, D_theta=None):
    """RoPE of rows x [S][H*D] at positions pos [S], per head of width D,
    as a complex rotation of the pairs (2m, 2m+1) by pos * theta_m,
    theta_m = 10000^(-2m / D_theta) (D_theta = D unless a test asks for a
    mistaken width)."""
    S, W = x.shape
    z = x.reshape(S, W // D, D // 2, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    theta = 10000.0 ** (-2.0 * np.arange(D // 2) / (D_theta or D))
    zc = zc * np.exp(1j * np.asarray(pos, np.float64)[:, None, None] * theta)
    return np.stack([zc.real, zc.imag], -1).reshape(S, W)


def attention(q, k, v, pos_q, H, causal=True):
    """softmax(q k^T / sqrt(D)) v per head; a query at position p sees the
    keys at positions 0..p (all keys when not causal)."""
    S, d = q.shape
    D = d // H
    out = np.zeros((S, d))
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(D)
        if causal:
            j = np.arange(k.shape[0])
            s = np.where(j[None, :] > np.asarray(pos_q)[:, None], -np.inf, s)
        s = np.exp(s - s.max(1, keepdims=True))
        out[:, sl] = (s / s.sum(1, keepdims=True)) @ v[:, sl]
    return out


# ---------------------------------------------------------------------------
# case_post_ln: (logits - lm_b)[:, pi(j)] = gamma2_j * xhat_j + beta2_j
# ---------------------------------------------------------------------------
def case_post_ln(seed=1, L=2):
    P = Params(L, seed)
    V = CFG["vocab"]
    perm = P.rng.permutation(V)
    P.lm_w = np.zeros((CFG["d"], V))
    P.lm_w[np.arange(V), perm] = 1.0          # column perm[j] reads y_j
    return P, perm


def post_ln_residual(P, perm, logits):
    """z_j = (logits[perm[j]] - lm_b[perm[j]] - beta2_j) / gamma2_j, which is
    the normalised LN2 input x-hat when the logits are the permuted LN2
    output: every row then has mean 0 and mean square v / (v + eps) ~ 1."""
    Q = P.f64()
    last = Q.layers[-1]
    y = (np.asarray(logits, np.float64) - Q.lm_b)[:, perm]
    return (y - last["ln2.b"]) / last["ln2.g"]


# ---------------------------------------------------------------------------
# case_layer: attention contributes b_o only; the gate is the constant c
# ---------------------------------------------------------------------------
def case_layer(seed=2, L=2):
    P = Params(L, seed)
    for p in P.layers:
        p["v.w"][:] = 0.0
        p["v.b"][:] = 0.0
        p["gate.w"][:] = 0.0
        p["gate.b"] = P.rng.standard_normal(CFG["F"]) * 1.5
    P.lm_w = np.eye(CFG["d"])
    return P


def layer_closed_form(P, ids, mistake=None):
    Q = P.f64()
    x = Q.emb[np.asarray(ids)]
    for p in Q.layers:
        c = p["gate.b"]
        if mistake == "pre_ln":
            # x + MHA(LN1 x) then + MLP(LN2 .), no norm on the stream
            x1 = x + p["o.b"]
            h = ln(x1, p["ln2.g"], p["ln2.b"])
            u = h @ p["up.w"] + p["up.b"]
            x = x1 + ((c * sigmoid(c)) * u) @ p["down.w"] + p["down.b"]
            continue
        r = p["o.b"] + (0.0 if mistake == "no_attn_residual" else x)
        x1 = ln(r, p["ln1.g"], p["ln1.b"])
        u = x1 @ p["up.w"] + p["up.b"]
        if mistake == "gate_up_swap":
            h = (u * sigmoid(u)) * c
        else:
            h = (c * sigmoid(c)) * u
        m = h @ p["down.w"] + p["down.b"]
        r = m + (0.0 if mistake == "no_mlp_residual" else x1)
        x = ln(r, p["ln2.g"], p["ln2.b"])
    if mistake == "final_ln":
        x = ln(x, 1.0, 0.0)
    return x @ Q.lm_w + Q.lm_b


# ---------------------------------------------------------------------------
# case_mean_v: zero scores, so each row averages v_j over j <= i
# ---------------------------------------------------------------------------
def case_mean_v(seed=3):
    P = Params(1, seed)
    p = P.layers[0]
    for nm in ("q.w", "q.b", "k.w", "k.b", "gate.w", "gate.b"):
        p[nm][:] = 0.0                         # gate 0: the MLP adds b_down
    P.lm_w = np.eye(CFG["d"])
    return P


def mean_v_closed_form(P, ids, mistake=None):
    Q = P.f64()
    p = Q.layers[0]
    x = Q.emb[np.asarray(ids)]
    S = len(ids)
    v = x @ p["v.w"] + p["v.b"]
    if mistake == "rope_on_v":
        v = rope_c(v, np.arange(S), CFG["d"] // CFG["H"])
    if mistake == "no_mask":
        a = np.repeat(v.mean(0, keepdims=True), S, 0)
    else:
        a = np.cumsum(v, 0) / np.arange(1, S + 1)[:, None]
    x1 = ln(x + a @ p["o.w"] + p["o.b"], p["ln1.g"], p["ln1.b"])
    y = ln(x1 + p["down.b"], p["ln2.g"], p["ln2.b"])
    return y @ Q.lm_w + Q.lm_b


# ---------------------------------------------------------------------------
# case_rope: token-independent q and k inputs; scores set by RoPE alone
# ---------------------------------------------------------------------------
def case_rope(seed=4):
    P = Params(1, seed)
    d = CFG["d"]
    half = d // 2
    P.emb[:, :half] = P.emb[0, :half]         # shared q/k block
    p = P.layers[0]
    p["q.w"][half:] = 0.0                      # q, k read the shared block
    p["k.w"][half:] = 0.0
    p["q.w"] *= 3.0                            # sharp enough scores
    p["k.w"] *= 3.0
    p["v.w"][:half] = 0.0                      # v reads the per-token block
    p["gate.w"][:] = 0.0
    p["gate.b"][:] = 0.0
    P.lm_w = np.eye(d)
    return P


def rope_closed_form(P, ids, mistake=None):
    """Forward of the whole sequence ids (positions 0..S-1)."""
    Q = P.f64()
    p = Q.layers[0]
    H, d = CFG["H"], CFG["d"]
    D = d // H
    x = Q.emb[np.asarray(ids)]
    S = len(ids)
    pos = np.arange(S)
    q = x @ p["q.w"] + p["q.b"]
    k = x @ p["k.w"] + p["k.b"]
    v = x @ p["v.w"] + p["v.b"]
    if mistake != "no_rope":
        # "theta_from_d_model": pair angles of the model width, not the head's
        Dt = d if mistake == "theta_from_d_model" else D
        q = rope_c(q, pos, D, Dt)
        k = rope_c(k, pos, D, Dt)
    if mistake == "no_scale":
        q = q * np.sqrt(D)
    a = attention(q, k, v, pos, H)
    x1 = ln(x + a @ p["o.w"] + p["o.b"], p["ln1.g"], p["ln1.b"])
    y = ln(x1 + p["down.b"], p["ln2.g"], p["ln2.b"])
    return y @ Q.lm_w + Q.lm_b


MISTAKES = {
    "layer": ("pre_ln", "gate_up_swap", "no_attn_residual", "no_mlp_residual",
              "final_ln"),
    "mean_v": ("rope_on_v", "no_mask"),
    "rope": ("no_rope", "theta_from_d_model", "no_scale"),
}


def max_abs(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max())

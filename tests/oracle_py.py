"""ctypes view of oracle/liboracle.so (the CPU checker) for the tests.

The oracle restates the reference's CPU path; see oracle/oracle.h.  This
module also generates the seeded synthetic weights the tests share between
the oracle and the device library.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None


class SpecTrace(C.Structure):
    _fields_ = [("max_cycles", C.c_int), ("k", C.c_int), ("V", C.c_int),
                ("n", C.c_int), ("dlogits", C.POINTER(C.c_float)),
                ("cand", C.POINTER(C.c_int32)), ("M", C.POINTER(C.c_int32)),
                ("acc", C.POINTER(C.c_int32)), ("tok", C.POINTER(C.c_int32)),
                ("dstart", C.POINTER(C.c_int32)),
                ("tstart", C.POINTER(C.c_int32)),
                ("margin", C.POINTER(C.c_double)),
                ("first_margin", C.c_double)]


class SpecStats(C.Structure):
    _fields_ = [("cycles", C.c_int64), ("drafted", C.c_int64),
                ("accepted", C.c_int64), ("ties", C.c_int64),
                ("resampled", C.c_int64), ("bonus", C.c_int64),
                ("prefill_ms", C.c_double), ("decode_ms", C.c_double)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.check_call(["make", "-s", "-C", ORACLE_DIR])
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, f32, u32, u64 = (C.c_void_p, C.c_int, C.c_int64,
                                       C.c_float, C.c_uint32, C.c_uint64)
        fp = C.POINTER(C.c_float)
        ip = C.POINTER(C.c_int32)
        L.or_philox4x32_10.argtypes = [C.POINTER(u32), C.POINTER(u32),
                                       C.POINTER(u32)]
        L.or_uniform.argtypes = [u64, u32, u32, u32]
        L.or_uniform.restype = f32
        L.or_model_create.argtypes = [i32] * 6
        L.or_model_create.restype = vp
        L.or_model_free.argtypes = [vp]
        L.or_model_num_params.argtypes = [vp]
        L.or_model_param_shape.argtypes = [vp, i32, C.POINTER(i64),
                                           C.POINTER(i64)]
        L.or_model_set_param.argtypes = [vp, i32, fp]
        L.or_model_quantize.argtypes = [vp]
        L.or_model_quantize_bits.argtypes = [vp, i32]
        L.or_quantize_w.argtypes = [fp, i64, i64, i32, C.POINTER(C.c_int8), fp]
        L.or_pack_int4.argtypes = [C.POINTER(C.c_int8), i64,
                                   C.POINTER(C.c_uint8)]
        L.or_unpack_int4.argtypes = [C.POINTER(C.c_uint8), i64,
                                     C.POINTER(C.c_int8)]
        L.or_model_get_quantized.argtypes = [vp, i32, i32,
                                             C.POINTER(C.c_int8), fp]
        L.or_cache_create.argtypes = [vp]
        L.or_cache_create.restype = vp
        L.or_cache_create_q.argtypes = [vp, i32]
        L.or_cache_create_q.restype = vp
        L.or_cache_read_q8.argtypes = [vp, i32, C.POINTER(C.c_int8), fp,
                                       C.POINTER(C.c_int8), fp]
        L.or_cache_read_raw.argtypes = [vp, i32, fp, fp]
        L.or_cache_write_q8.argtypes = [vp, i32, i32, C.POINTER(C.c_int8), fp,
                                        C.POINTER(C.c_int8), fp]
        L.or_cache_set_len.argtypes = [vp, i32]
        L.or_cache_freeze.argtypes = [vp, i32]
        L.or_model_save_weights.argtypes = [vp, C.c_char_p]
        L.or_model_load_weights.argtypes = [vp, C.c_char_p]
        L.or_quantize_kv.argtypes = [fp, i64, i64, C.POINTER(C.c_int8), fp]
        L.or_attention_q8.argtypes = [fp, C.POINTER(C.c_int8), fp,
                                      C.POINTER(C.c_int8), fp, i64, i64, i64,
                                      i64, i64, i32, fp]
        L.or_cache_free.argtypes = [vp]
        L.or_cache_len.argtypes = [vp]
        L.or_cache_truncate.argtypes = [vp, i32]
        L.or_forward.argtypes = [vp, vp, ip, i32, fp]
        L.or_quantize_w8.argtypes = [fp, i64, i64, C.POINTER(C.c_int8), fp]
        L.or_dense.argtypes = [fp, i64, i64, i64, fp, C.POINTER(C.c_int8),
                               fp, fp, fp]
        L.or_rope.argtypes = [fp, i64, i64, i64, i64]
        L.or_layernorm.argtypes = [fp, i64, i64, fp, fp, f32, fp]
        L.or_attention.argtypes = [fp, fp, fp, i64, i64, i64, i64, i64, i32,
                                   fp]
        L.or_get_probs.argtypes = [fp, i32, f32, i32, f32, fp]
        L.or_sample.argtypes = [fp, i32, C.c_double]
        L.or_argmax.argtypes = [fp, i32]
        L.or_accept_step.argtypes = [fp, fp, ip, i32, i32, i32, i32, fp, f32,
                                     C.POINTER(C.c_int),
                                     C.POINTER(C.c_int64)]
        L.or_generate_speculative.argtypes = [vp, vp, ip, i32, i32, i32, f32,
                                              i32, f32, u64, i32, u32, ip,
                                              C.POINTER(SpecStats)]
        L.or_set_spec_trace.argtypes = [C.POINTER(SpecTrace)]
        L.or_set_threads.argtypes = [i32]
        L.or_set_rng.argtypes = [i32]
        L.or_set_rng.restype = None
        L.or_mt_seed.argtypes = [C.c_void_p, u32]
        L.or_mt_seed.restype = None
        L.or_mt_next.argtypes = [C.c_void_p]
        L.or_mt_next.restype = u32
        L.or_mt_float.argtypes = [C.c_void_p]
        L.or_mt_float.restype = f32
        L.or_mt_double.argtypes = [C.c_void_p]
        L.or_mt_double.restype = C.c_double
        L.or_decision_margin.argtypes = [i32]
        L.or_decision_margin.restype = C.c_double
        L.or_generate_advanced.argtypes = [vp, ip, i32, i32, f32, i32, f32,
                                           u64, u32, i32, ip]
        _lib = L
    return _lib


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def iptr(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def i8ptr(a):
    assert a.dtype == np.int8 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_int8))


def philox(ctr, key):
    out = (C.c_uint32 * 4)()
    lib().or_philox4x32_10((C.c_uint32 * 4)(*ctr), (C.c_uint32 * 2)(*key), out)
    return list(out)


def uniform(seed, seq, cycle, slot):
    return lib().or_uniform(seed, seq, cycle, slot)


# ----------------------------------------------------------------------------
# Seeded synthetic decoder weights, TransformerDecoder::parameters() order:
# Dense weights and the embedding ~ N(0, std), biases 0, LayerNorm gamma 1,
# beta 0.  Shapes follow the reference ([in, out] Dense weights).
# ----------------------------------------------------------------------------
def param_shapes(vocab, d, H, F, L):
    shapes = [("emb", (vocab, d))]
    for l in range(L):
        for nm, (i, o) in (("q", (d, d)), ("k", (d, d)), ("v", (d, d)),
                           ("o", (d, d)), ("gate", (d, F)), ("up", (d, F)),
                           ("down", (F, d))):
            shapes.append((f"{nm}.w", (i, o)))
            shapes.append((f"{nm}.b", (1, o)))
        for nm in ("ln1.g", "ln1.b", "ln2.g", "ln2.b"):
            shapes.append((nm, (1, d)))
    shapes.append(("lm.w", (d, vocab)))
    shapes.append(("lm.b", (1, vocab)))
    return shapes


def make_params(vocab, d, H, F, L, seed, std=0.02, bias_std=0.0):
    rng = np.random.default_rng(seed)
    out = []
    for name, shp in param_shapes(vocab, d, H, F, L):
        if name.endswith(".w") or name == "emb":
            a = (rng.standard_normal(shp, dtype=np.float32) * np.float32(std))
        elif name.endswith(".g"):
            a = np.ones(shp, np.float32)
        else:
            a = (rng.standard_normal(shp, dtype=np.float32) *
                 np.float32(bias_std)) if bias_std else np.zeros(shp,
                                                                 np.float32)
        out.append(np.ascontiguousarray(a, dtype=np.float32))
    return out


class Model:
    """Oracle TransformerDecoder(vocab, d, heads, d_ff, layers, max_seq)."""

    def __init__(self, vocab, d, H, F, L, max_seq, params, quantize=False,
                 bits=8):
        self.vocab, self.d, self.H, self.F, self.L = vocab, d, H, F, L
        self.max_seq = max_seq
        self.h = lib().or_model_create(vocab, d, H, F, L, max_seq)
        assert self.h
        assert lib().or_model_num_params(self.h) == len(params)
        for i, p in enumerate(params):
            r, c = C.c_int64(), C.c_int64()
            lib().or_model_param_shape(self.h, i, C.byref(r), C.byref(c))
            assert r.value * c.value == p.size, (i, p.shape)
            assert lib().or_model_set_param(self.h, i, fptr(p)) == 0
        if quantize:
            assert lib().or_model_quantize_bits(self.h, bits) == 0

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None

    def quantized(self, layer, which, n_in, n_out):
        codes = np.zeros((n_in, n_out), np.int8)
        scales = np.zeros(n_out, np.float32)
        assert lib().or_model_get_quantized(self.h, layer, which,
                                            i8ptr(codes), fptr(scales)) == 0
        return codes, scales

    def save_weights(self, path):
        if lib().or_model_save_weights(self.h, os.fsencode(path)) != 0:
            raise RuntimeError(f"or_model_save_weights failed: {path}")

    def load_weights(self, path):
        """0 on success, else the oracle's error code (see oracle.h)."""
        return lib().or_model_load_weights(self.h, os.fsencode(path))

    def forward(self, ids, cache=None):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((len(ids), self.vocab), np.float32)
        rc = lib().or_forward(self.h, cache.h if cache is not None else None,
                              iptr(ids),
                              len(ids), fptr(out))
        if rc != 0:
            raise RuntimeError(
                "Sequence length S plus past cached length exceeds max_seq_len")
        return out


class Cache:
    def __init__(self, model, quantized=False):
        self.h = lib().or_cache_create_q(model.h, 1 if quantized else 0)
        self.H = model.H
        self.D = model.d // model.H

    def read_q8(self, layer):
        """Codes and scales of one layer of an int8 cache:
        (kq [H][len][D], ks [H][len], vq, vs)."""
        n = len(self)
        kq = np.zeros((self.H, n, self.D), np.int8)
        vq = np.zeros_like(kq)
        ks = np.zeros((self.H, n), np.float32)
        vs = np.zeros_like(ks)
        rc = lib().or_cache_read_q8(self.h, layer, i8ptr(kq), fptr(ks),
                                    i8ptr(vq), fptr(vs))
        if rc != 0:
            raise RuntimeError("or_cache_read_q8 failed")
        return kq, ks, vq, vs

    def read_raw(self, layer):
        """The fp32 k / v rows [H][len][D] an int8 cache quantised."""
        n = len(self)
        kr = np.zeros((self.H, n, self.D), np.float32)
        vr = np.zeros_like(kr)
        if lib().or_cache_read_raw(self.h, layer, fptr(kr), fptr(vr)) != 0:
            raise RuntimeError("or_cache_read_raw failed")
        return kr, vr

    def write_q8(self, layer, kq, ks, vq, vs):
        """Codes [H][n][D] / scales [H][n] into positions [0, n)."""
        kq, vq = (np.ascontiguousarray(a, np.int8) for a in (kq, vq))
        ks, vs = (np.ascontiguousarray(a, np.float32) for a in (ks, vs))
        if lib().or_cache_write_q8(self.h, layer, kq.shape[1], i8ptr(kq),
                                   fptr(ks), i8ptr(vq), fptr(vs)) != 0:
            raise RuntimeError("or_cache_write_q8 failed")

    def set_len(self, n):
        lib().or_cache_set_len(self.h, n)

    def freeze(self, frozen=True):
        lib().or_cache_freeze(self.h, 1 if frozen else 0)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_cache_free(self.h)
            self.h = None

    def __len__(self):
        return lib().or_cache_len(self.h)

    def truncate(self, n):
        lib().or_cache_truncate(self.h, n)


def get_probs(logits, T, top_k=0, top_p=1.0):
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.zeros_like(logits)
    lib().or_get_probs(fptr(logits), logits.size, T, top_k, top_p, fptr(out))
    return out


def sample(probs, u):
    probs = np.ascontiguousarray(probs, np.float32)
    return lib().or_sample(fptr(probs), probs.size, float(u))


def decision_margin(reset=True):
    """Smallest decision margin of the oracle's random decisions since the
    last reset (or_decision_margin)."""
    return lib().or_decision_margin(1 if reset else 0)


def accept_step(p, q, cand, greedy, has_bonus, u_accept, u_final):
    """or_accept_step: p [M(+1)][V], q [M][V] probability rows."""
    p = np.ascontiguousarray(p, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    cand = np.ascontiguousarray(cand, np.int32)
    ua = np.ascontiguousarray(u_accept, np.float32)
    tok, ties = C.c_int(), C.c_int64()
    n = lib().or_accept_step(fptr(p), fptr(q), iptr(cand), len(cand),
                             q.shape[-1], int(greedy), int(has_bonus),
                             fptr(ua), float(u_final), C.byref(tok),
                             C.byref(ties))
    return n, tok.value, ties.value


def generate_speculative(target, draft, prompt, max_new, k, T, seed, seq=0,
                         top_k=0, top_p=1.0, quantized_cache=False):
    prompt = np.ascontiguousarray(prompt, np.int32)
    # the first token is always appended (layer.cpp:1508-1510)
    out = np.zeros(len(prompt) + max(max_new, 1), np.int32)
    st = SpecStats()
    rc = lib().or_generate_speculative(target.h, draft.h, iptr(prompt),
                                       len(prompt), max_new, k, T, top_k,
                                       top_p, seed,
                                       1 if quantized_cache else 0, seq,
                                       iptr(out), C.byref(st))
    if rc != 0:
        raise RuntimeError(f"or_generate_speculative failed: {rc}")
    return out, st


class MT19937:
    """The oracle's std::mt19937 (or_mt): next() raw outputs, f() the
    uniform_real_distribution<float>(0, 1) draw, d() the
    generate_canonical<double, 53> draw."""

    def __init__(self, seed):
        self._buf = C.create_string_buffer(624 * 4 + 8)
        lib().or_mt_seed(self._buf, seed & 0xffffffff)

    def next(self):
        return int(lib().or_mt_next(self._buf))

    def f(self):
        return float(lib().or_mt_float(self._buf))

    def d(self):
        return float(lib().or_mt_double(self._buf))


def set_rng(mode):
    """0: Philox slots; 1: the reference's std::mt19937 stream (or_set_rng)."""
    lib().or_set_rng(int(mode))


def set_threads(n):
    """Threads of the oracle's Dense products and attention heads."""
    lib().or_set_threads(int(n))


def generate_speculative_traced(target, draft, prompt, max_new, k, T, seed,
                                seq=0, max_cycles=None, **kw):
    """generate_speculative with the oracle's per-cycle record (or_spec_trace):
    returns (out, stats, cycles, first_margin), cycles a list of dicts with
    the draft logits [M][V] of each drafting step, the candidates, M,
    accepted count, resampled / bonus token, the draft / target cache
    lengths at the start of the cycle and the cycle's smallest decision
    margin; first_margin that of the first token's draw."""
    V = target.vocab
    if max_cycles is None:
        max_cycles = max(max_new, 1)
    arrs = dict(dlogits=np.zeros((max_cycles, k, V), np.float32),
                cand=np.zeros((max_cycles, k), np.int32),
                M=np.zeros(max_cycles, np.int32),
                acc=np.zeros(max_cycles, np.int32),
                tok=np.zeros(max_cycles, np.int32),
                dstart=np.zeros(max_cycles, np.int32),
                tstart=np.zeros(max_cycles, np.int32),
                margin=np.zeros(max_cycles, np.float64))
    tr = SpecTrace(max_cycles, k, V, 0, fptr(arrs["dlogits"]),
                   *(iptr(arrs[n]) for n in ("cand", "M", "acc", "tok",
                                             "dstart", "tstart")),
                   arrs["margin"].ctypes.data_as(C.POINTER(C.c_double)), 1.0)
    lib().or_set_spec_trace(C.byref(tr))
    try:
        out, st = generate_speculative(target, draft, prompt, max_new, k, T,
                                       seed, seq=seq, **kw)
    finally:
        lib().or_set_spec_trace(None)
    cycles = []
    for c in range(tr.n):
        M = int(arrs["M"][c])
        cycles.append(dict(dlogits=arrs["dlogits"][c, :M].copy(),
                           cand=arrs["cand"][c, :M].copy(), M=M,
                           acc=int(arrs["acc"][c]), tok=int(arrs["tok"][c]),
                           dstart=int(arrs["dstart"][c]),
                           tstart=int(arrs["tstart"][c]),
                           margin=float(arrs["margin"][c])))
    return out, st, cycles, tr.first_margin


def generate_advanced(model, prompt, max_new, T, seed, seq=0, use_cache=True,
                      top_k=0, top_p=1.0):
    prompt = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(len(prompt) + max_new, np.int32)
    rc = lib().or_generate_advanced(model.h, iptr(prompt), len(prompt),
                                    max_new, T, top_k, top_p, seed, seq,
                                    1 if use_cache else 0, iptr(out))
    if rc != 0:
        raise RuntimeError(f"or_generate_advanced failed: {rc}")
    return out


def quantize_kv(x):
    """quantize_kv of MultiHeadAttention::forward over the rows of x [..., D]:
    (codes int8 [..., D], scales fp32 [...])."""
    x = np.ascontiguousarray(x, np.float32)
    D = x.shape[-1]
    rows = x.size // D
    codes = np.zeros(x.shape, np.int8)
    scales = np.zeros(x.shape[:-1], np.float32)
    lib().or_quantize_kv(fptr(x), rows, D, i8ptr(codes), fptr(scales))
    return codes, scales


def attention_q8(q, kq, ks, vq, vs, causal=True):
    """Fused attention of one sequence over an int8 cache: q [H][S][D],
    kq / vq [Hkv][St][D], ks / vs [Hkv][St]; returns [S][H][D]."""
    q = np.ascontiguousarray(q, np.float32)
    kq = np.ascontiguousarray(kq, np.int8)
    vq = np.ascontiguousarray(vq, np.int8)
    ks = np.ascontiguousarray(ks, np.float32)
    vs = np.ascontiguousarray(vs, np.float32)
    H, S, D = q.shape
    Hkv, St = kq.shape[0], kq.shape[1]
    out = np.zeros((S, H, D), np.float32)
    lib().or_attention_q8(fptr(q), i8ptr(kq), fptr(ks), i8ptr(vq), fptr(vs),
                          H, Hkv, S, St, D, 1 if causal else 0, fptr(out))
    return out


def assert_same_stream(got, want, cycles, first_margin, P, tol=1e-5,
                       what=""):
    """A sampled device stream equals the oracle's, or first differs inside
    a cycle (or the first token) whose random decisions the oracle made
    within `tol` of their boundary (|r - p/q| or |u - cdf edge|): there the
    fp32 rounding of the two implementations may legitimately decide
    differently.  Everything before the divergence must be equal.  Returns
    the first differing index, or None."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, what
    diff = np.nonzero(got != want)[0]
    if len(diff) == 0:
        return None
    i = int(diff[0])
    assert i >= P, f"{what}: prompt differs at {i}"
    if i == P:
        assert first_margin < tol, (what, i, first_margin)
        return i
    pos = P + 1
    for c in cycles:
        n = c["acc"] + (1 if c["tok"] >= 0 else 0)
        if pos <= i < pos + n:
            assert c["margin"] < tol, (
                f"{what}: streams differ at {i} in a cycle whose closest "
                f"decision is {c['margin']:.3g} from its boundary")
            return i
        pos += n
    raise AssertionError(f"{what}: divergence at {i} beyond the record")


def quantize_w(w, bits):
    """QuantizedDense ctor on w [in][out]: (codes int8 [in][out], scales)."""
    w = np.ascontiguousarray(w, np.float32)
    codes = np.zeros(w.shape, np.int8)
    scales = np.zeros(w.shape[1], np.float32)
    lib().or_quantize_w(fptr(w), w.shape[0], w.shape[1], bits, i8ptr(codes),
                        fptr(scales))
    return codes, scales


def pack_int4(codes):
    c = np.ascontiguousarray(codes, np.int8).ravel()
    out = np.zeros((c.size + 1) // 2, np.uint8)
    lib().or_pack_int4(i8ptr(c), c.size,
                       out.ctypes.data_as(C.POINTER(C.c_uint8)))
    return out


def unpack_int4(packed, n):
    p = np.ascontiguousarray(packed, np.uint8)
    out = np.zeros(n, np.int8)
    lib().or_unpack_int4(p.ctypes.data_as(C.POINTER(C.c_uint8)), n,
                         i8ptr(out))
    return out

"""ctypes binding of libnnhip.so (the C ABI in include/nnhip.h).

Used by the tests, bench.py and __graft_entry__.py.  Loading fails loudly when
the library has not been built: there is no CPU fallback.
"""
import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "libnnhip.so")

OK, EARG, ECAPACITY, EHIP, EUNSUPPORTED, EIO = 0, -1, -2, -3, -4, -5


class NNHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class SpecStats(C.Structure):
    _fields_ = [("cycles", C.c_int64), ("drafted", C.c_int64),
                ("accepted", C.c_int64), ("ties", C.c_int64),
                ("resampled", C.c_int64), ("bonus", C.c_int64)]


class SpecTiming(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double),
                ("cycles_launched", C.c_int64)]


MAX_RANK = 8
OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3
(OP_RELU_BACKWARD, OP_SIGMOID_BACKWARD, OP_TANH_BACKWARD, OP_SQRT_BACKWARD,
 OP_LOG_BACKWARD) = 4, 5, 6, 7, 8
OP_RELU, OP_SIGMOID, OP_TANH, OP_SQRT, OP_LOG = 16, 17, 18, 19, 20


class View(C.Structure):
    """nnhip_view: a dev buffer, an element offset, shape and strides."""
    _fields_ = [("data", C.c_void_p), ("offset", C.c_int64),
                ("rank", C.c_int32), ("shape", C.c_int64 * MAX_RANK),
                ("strides", C.c_int64 * MAX_RANK)]


def view(arr, shape=None, strides=None, offset=0):
    """A View of DeviceArray `arr`: its own shape and row-major strides, or
    the given ones (elements).  The view keeps `arr` alive."""
    shape = tuple(arr.shape if shape is None else shape)
    if strides is None:
        strides, acc = [], 1
        for n in reversed(shape):
            strides.insert(0, acc)
            acc *= n
    v = View()
    # the view holds its array: a view alone must not outlive the memory
    v._arr = arr
    v.data = arr.p
    v.offset = offset
    v.rank = len(shape)
    for i, (n, st) in enumerate(zip(shape, strides)):
        v.shape[i] = n
        v.strides[i] = st
    return v


# name -> argument types (all functions return int status unless listed)
_vp, _i, _i64, _u32, _u64, _f, _sz = (C.c_void_p, C.c_int, C.c_int64,
                                      C.c_uint32, C.c_uint64, C.c_float,
                                      C.c_size_t)
_pp = C.POINTER(C.c_void_p)
SIGNATURES = {
    "nnhip_init": [_i, _pp],
    "nnhip_destroy": [_vp],
    "nnhip_set_option": [_vp, C.c_char_p, _i],
    "nnhip_sync": [_vp],
    "nnhip_malloc": [_vp, _sz, _pp],
    "nnhip_free": [_vp, _vp],
    "nnhip_h2d": [_vp, _vp, _vp, _sz],
    "nnhip_d2h": [_vp, _vp, _vp, _sz],
    "nnhip_timer_begin": [_vp],
    "nnhip_timer_end": [_vp, C.POINTER(C.c_float)],
    "nnhip_decoder_create": [_vp, _i, _i, _i, _i, _i, _i, _pp],
    "nnhip_decoder_free": [_vp],
    "nnhip_decoder_num_params": [_vp, C.POINTER(C.c_int)],
    "nnhip_decoder_param_shape": [_vp, _i, C.POINTER(_i64), C.POINTER(_i64)],
    "nnhip_decoder_set_param": [_vp, _i, _vp],
    "nnhip_decoder_get_param": [_vp, _i, _vp],
    "nnhip_decoder_init_normal": [_vp, _u64, _f],
    "nnhip_decoder_quantize": [_vp, _i],
    "nnhip_decoder_get_quantized": [_vp, _i, _i, _vp, _vp],
    "nnhip_decoder_save_weights": [_vp, C.c_char_p],
    "nnhip_decoder_load_weights": [_vp, C.c_char_p],
    "nnhip_decoder_forward": [_vp, _vp, _vp, _i, _i, _vp],
    "nnhip_kvcache_create": [_vp, _i, _i, _pp],
    "nnhip_kvcache_read_q8": [_vp, _i, _i, _vp, _vp, _vp, _vp],
    "nnhip_kvcache_read": [_vp, _i, _i, _vp, _vp],
    "nnhip_kvcache_free": [_vp],
    "nnhip_kvcache_length": [_vp, _i, C.POINTER(C.c_int)],
    "nnhip_kvcache_truncate": [_vp, _i, _i],
    "nnhip_generate_speculative": [_vp, _vp, _vp, _i, _i, _i, _f, _i, _f,
                                   _u64, _i, _vp, _vp],
    "nnhip_generate_speculative_batch": [_vp, _vp, _i, _vp, _i, _i, _i, _f,
                                         _i, _f, _u64, _u32, _i, _vp, _vp,
                                         _vp],
    "nnhip_generate_advanced": [_vp, _vp, _i, _i, _f, _i, _f, _u64, _i, _vp],
    "nnhip_generate_advanced_batch": [_vp, _i, _vp, _i, _i, _f, _i, _f, _u64,
                                      _u32, _i, _vp],
    "nnhip_quantize_w8": [_vp, _vp, _i, _i, _vp, _vp],
    "nnhip_quantize_w4": [_vp, _vp, _i, _i, _vp, _vp],
    "nnhip_linear_w8a32": [_vp, _vp, _i, _i, _vp, _vp, _vp, _i, _vp, _i],
    "nnhip_linear_w8a32_noalloc": [_vp, _vp, _i, _i, _vp, _vp, _vp, _i, _vp,
                                   _i],
    "nnhip_layernorm_linear_w8a32": [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _i, _vp],
    "nnhip_linear_f32": [_vp, _vp, _i, _i, _vp, _vp, _i, _vp],
    "nnhip_linear_limb_totals": [_vp, _vp, _i, _i, _vp, _i, _vp, _vp, _vp],
    "nnhip_rope_kv_append": [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                             _i],
    "nnhip_rope_kv_append_gqa": [_vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp,
                                 _vp, _i],
    "nnhip_attention_kq": [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i,
                           _vp],
    "nnhip_rope_kv_append_q8": [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                                _vp, _vp, _i],
    "nnhip_attention_kq_q8": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i,
                              _i, _i, _i, _vp],
    "nnhip_layernorm": [_vp, _vp, _i, _i, _vp, _vp, _vp],
    "nnhip_sample_rows": [_vp, _vp, _i, _i, _f, _i, _f, _vp, _vp, _vp],
    "nnhip_spec_accept": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp,
                          _vp],
    "nnhip_binary_f32": [_vp, _i, C.POINTER(View), C.POINTER(View),
                         C.POINTER(View)],
    "nnhip_unary_f32": [_vp, _i, C.POINTER(View), C.POINTER(View)],
    "nnhip_matmul_f32": [_vp, C.POINTER(View), C.POINTER(View),
                         C.POINTER(View)],
    "nnhip_sum_f32": [_vp, C.POINTER(View), C.POINTER(View),
                      C.POINTER(C.c_int64), _i],
    "nnhip_softmax_f32": [_vp, C.POINTER(View), C.POINTER(View), _i],
    "nnhip_softmax_backward_f32": [_vp, C.POINTER(View), C.POINTER(View),
                                   C.POINTER(View), _i],
    "nnhip_embedding_f32": [_vp, C.POINTER(View), C.POINTER(View),
                            C.POINTER(View)],
    "nnhip_slice_backward_f32": [_vp, C.POINTER(View), C.POINTER(View), _i,
                                 _i64],
    "nnhip_fill_f32": [_vp, _vp, _sz, _f],
    "nnhip_bench_attention": [_vp, _i, _i, _i, _i, _i, _i, _i, _i,
                              C.POINTER(C.c_float)],
    "nnhip_bench_spec_accept": [_vp, _i, _i, _i, _f, _i, _i,
                                C.POINTER(C.c_float), _vp],
    "nnhip_bench_linear": [_vp, _i, _i, _i, _i, _i, _i, C.POINTER(C.c_float)],
    "nnhip_bench_forward": [_vp, _i, _i, _i, _i, _i, C.POINTER(C.c_float)],
}

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.nnhip_last_error.restype = C.c_char_p
        L.nnhip_last_error.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int
        _lib = L
    return _lib


def call(name, *args):
    L = load()
    rc = getattr(L, name)(*args)
    if rc != 0:
        raise NNHipError(rc, L.nnhip_last_error().decode())
    return rc


def ptr(a):
    """Host pointer of a C-contiguous numpy array."""
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


class Context:
    def __init__(self, device=0):
        h = C.c_void_p()
        call("nnhip_init", device, C.byref(h))
        self.h = h

    def close(self):
        if self.h:
            call("nnhip_destroy", self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def set_option(self, key, value):
        call("nnhip_set_option", self.h, key.encode(), int(value))

    def sync(self):
        call("nnhip_sync", self.h)

    def array(self, host=None, shape=None, dtype=np.float32):
        return DeviceArray(self, host, shape, dtype)

    def timer_begin(self):
        call("nnhip_timer_begin", self.h)

    def timer_end(self):
        ms = C.c_float()
        call("nnhip_timer_end", self.h, C.byref(ms))
        return ms.value


class DeviceArray:
    def __init__(self, ctx, host=None, shape=None, dtype=np.float32):
        self.ctx = ctx
        if host is not None:
            host = np.ascontiguousarray(host)
            self.shape, self.dtype = host.shape, host.dtype
        else:
            self.shape, self.dtype = tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * np.dtype(self.dtype).itemsize
        p = C.c_void_p()
        call("nnhip_malloc", ctx.h, max(self.nbytes, 1), C.byref(p))
        self.p = p
        if host is not None and self.nbytes:
            call("nnhip_h2d", ctx.h, self.p, ptr(host), self.nbytes)

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("nnhip_d2h", self.ctx.h, ptr(out), self.p, self.nbytes)
        return out

    def upload(self, host):
        host = np.ascontiguousarray(host, self.dtype)
        assert host.nbytes == self.nbytes
        call("nnhip_h2d", self.ctx.h, self.p, ptr(host), self.nbytes)

    def free(self):
        if self.p:
            call("nnhip_free", self.ctx.h, self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def bench_attention(ctx, B, S, H, D, n_cached, iters=100, nbuf=3,
                    quantized=False):
    ms = C.c_float()
    call("nnhip_bench_attention", ctx.h, B, S, H, D, n_cached, iters, nbuf,
         int(quantized), C.byref(ms))
    return ms.value


def bench_spec_accept(ctx, B, k, V, T, iters=100, nbuf=3):
    ms = C.c_float()
    n = np.zeros(B, np.int32)
    call("nnhip_bench_spec_accept", ctx.h, B, k, V, T, iters, nbuf,
         C.byref(ms), ptr(n))
    return ms.value, n


def bench_linear(ctx, rows, K, N, path, iters=100, nbuf=3):
    ms = C.c_float()
    call("nnhip_bench_linear", ctx.h, rows, K, N, path, iters, nbuf,
         C.byref(ms))
    return ms.value


def bench_forward(model, B, S, n_cached, quantized=False, iters=50):
    """Milliseconds per graph-replayed forward of `model` (a Decoder) over
    B x S new tokens after n_cached cached positions."""
    ms = C.c_float()
    call("nnhip_bench_forward", model.h, B, S, n_cached, int(quantized),
         iters, C.byref(ms))
    return ms.value


class Decoder:
    """TransformerDecoder(vocab, d_model, heads, d_ff, layers, max_seq)."""

    def __init__(self, ctx, vocab, d, H, F, L, max_seq):
        self.ctx = ctx
        self.vocab, self.d, self.H, self.F, self.L = vocab, d, H, F, L
        self.max_seq = max_seq
        h = C.c_void_p()
        call("nnhip_decoder_create", ctx.h, vocab, d, H, F, L, max_seq,
             C.byref(h))
        self.h = h

    def free(self):
        if self.h:
            call("nnhip_decoder_free", self.h)
            self.h = None

    def num_params(self):
        n = C.c_int()
        call("nnhip_decoder_num_params", self.h, C.byref(n))
        return n.value

    def param_shape(self, idx):
        r, c = C.c_int64(), C.c_int64()
        call("nnhip_decoder_param_shape", self.h, idx, C.byref(r), C.byref(c))
        return r.value, c.value

    def set_params(self, params):
        assert len(params) == self.num_params()
        for i, p in enumerate(params):
            p = np.ascontiguousarray(p, np.float32)
            r, c = self.param_shape(i)
            assert p.size == r * c, (i, p.shape, r, c)
            call("nnhip_decoder_set_param", self.h, i, ptr(p))

    def get_param(self, idx):
        r, c = self.param_shape(idx)
        out = np.empty((r, c), np.float32)
        call("nnhip_decoder_get_param", self.h, idx, ptr(out))
        return out

    def init_normal(self, seed, std):
        call("nnhip_decoder_init_normal", self.h, seed, std)

    def quantize(self, bits=8):
        call("nnhip_decoder_quantize", self.h, bits)

    def get_quantized(self, layer, which, n_in, n_out):
        codes = np.empty((n_in, n_out), np.int8)
        scales = np.empty(n_out, np.float32)
        call("nnhip_decoder_get_quantized", self.h, layer, which, ptr(codes),
             ptr(scales))
        return codes, scales

    def save_weights(self, path):
        call("nnhip_decoder_save_weights", self.h, os.fsencode(path))

    def load_weights(self, path):
        call("nnhip_decoder_load_weights", self.h, os.fsencode(path))

    def forward(self, ids, cache=None):
        ids = np.ascontiguousarray(np.atleast_2d(ids), np.int32)
        B, S = ids.shape
        out = np.empty((B, S, self.vocab), np.float32)
        call("nnhip_decoder_forward", self.h, cache.h if cache is not None
             else None, ptr(ids), B, S, ptr(out))
        return out

    def generate_speculative(self, draft, prompt, max_new, lookahead, T,
                             top_k=0, top_p=1.0, seed=42,
                             quantized_cache=False):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(len(prompt) + max(max_new, 1), np.int32)
        st = SpecStats()
        call("nnhip_generate_speculative", self.h, draft.h, ptr(prompt),
             len(prompt), max_new, lookahead, T, top_k, top_p, seed,
             int(quantized_cache), ptr(out), C.byref(st))
        # the reference always appends the first token (layer.cpp:1508-1510)
        return out, st

    def generate_speculative_batch(self, draft, prompts, max_new, lookahead,
                                   T, seed, seq0=0, top_k=0, top_p=1.0,
                                   quantized_cache=False):
        prompts = np.ascontiguousarray(prompts, np.int32)
        B, P = prompts.shape
        out = np.zeros((B, P + max(max_new, 1)), np.int32)
        stats = (SpecStats * B)()
        tm = SpecTiming()
        call("nnhip_generate_speculative_batch", self.h, draft.h, B,
             ptr(prompts), P, max_new, lookahead, T, top_k, top_p, seed,
             seq0, int(quantized_cache), ptr(out), stats, C.byref(tm))
        return out, list(stats), tm

    def generate_advanced(self, prompt, max_new, T, seed=42,
                          use_kv_cache=True, top_k=0, top_p=1.0):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(len(prompt) + max_new, np.int32)
        call("nnhip_generate_advanced", self.h, ptr(prompt), len(prompt),
             max_new, T, top_k, top_p, seed, int(use_kv_cache), ptr(out))
        return out

    def generate_advanced_batch(self, prompts, max_new, T, seed, seq0=0,
                                use_kv_cache=True, top_k=0, top_p=1.0):
        prompts = np.ascontiguousarray(prompts, np.int32)
        B, P = prompts.shape
        out = np.zeros((B, P + max_new), np.int32)
        call("nnhip_generate_advanced_batch", self.h, B, ptr(prompts), P,
             max_new, T, top_k, top_p, seed, seq0, int(use_kv_cache),
             ptr(out))
        return out


class KVCache:
    def __init__(self, model, batch=1, quantized=False):
        h = C.c_void_p()
        call("nnhip_kvcache_create", model.h, batch, int(quantized),
             C.byref(h))
        self.h = h
        self.batch = batch

    def free(self):
        if self.h:
            call("nnhip_kvcache_free", self.h)
            self.h = None

    def length(self, b=0):
        n = C.c_int()
        call("nnhip_kvcache_length", self.h, b, C.byref(n))
        return n.value

    def truncate(self, n, b=0):
        call("nnhip_kvcache_truncate", self.h, b, n)

    def read(self, layer, b=0, heads=None, head_dim=None):
        """k and v of one layer and sequence of an fp32 cache: [H][len][D]
        each (k after RoPE)."""
        n = self.length(b)
        k = np.zeros((heads, n, head_dim), np.float32)
        v = np.zeros_like(k)
        call("nnhip_kvcache_read", self.h, layer, b, ptr(k), ptr(v))
        return k, v

    def read_q8(self, layer, b=0, heads=None, head_dim=None):
        """Codes and scales of one layer and sequence of an int8 cache:
        (kq [H][len][D], ks [H][len], vq, vs)."""
        n = self.length(b)
        kq = np.zeros((heads, n, head_dim), np.int8)
        vq = np.zeros_like(kq)
        ks = np.zeros((heads, n), np.float32)
        vs = np.zeros_like(ks)
        call("nnhip_kvcache_read_q8", self.h, layer, b, ptr(kq), ptr(ks),
             ptr(vq), ptr(vs))
        return kq, ks, vq, vs

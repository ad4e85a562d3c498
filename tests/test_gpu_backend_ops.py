"""ExecutionBackend ops on the device (GPU): the strided fp32 ops a
HipBackend serves to the reference's Tensor (include/backend/backend.hpp:
35-220), against CpuBackend's semantics (src/backend/cpu_backend.cpp).

Bit-exact where the reference's arithmetic fixes every rounding: add / sub /
mul / div and the element-wise backward formulas (one IEEE operation per
step), relu, sum (the reference adds each output's inputs in ascending
input index, serially), matmul against the oracle's Dense product (ascending
k, separately rounded products and sums; the sgemm the reference calls for
row-major operands fixes no order, its naive loop does), embedding, slice
backward.  Within 1e-6 relative where a libm function enters (exp, tanh,
sqrt, log) or a reduction order is free (softmax's sum).
"""
import numpy as np
import pytest

import oracle_py as O
from gpu_util import nnhip

pytestmark = pytest.mark.gpu


def dev(ctx, a):
    return ctx.array(np.ascontiguousarray(a, np.float32))


def strided(ctx, host, perm):
    """A device copy of host transposed by perm, viewed back in host's
    logical order through permuted strides (a non-contiguous operand)."""
    t = np.ascontiguousarray(np.transpose(host, perm))
    d = dev(ctx, t)
    st_t = [int(np.prod(t.shape[i + 1:])) for i in range(t.ndim)]
    inv = np.argsort(perm)
    return d, nnhip.view(d, host.shape, [st_t[i] for i in inv])


def run_binary(ctx, op, a, b, a_view=None, b_view=None, out_shape=None):
    da, db = dev(ctx, a), dev(ctx, b)
    shape = out_shape or np.broadcast_shapes(a.shape, b.shape)
    do = ctx.array(shape=shape)
    nnhip.call("nnhip_binary_f32", ctx.h, op, a_view or nnhip.view(da),
               b_view or nnhip.view(db), nnhip.view(do))
    return do.numpy()


NP_BINARY = {nnhip.OP_ADD: np.add, nnhip.OP_SUB: np.subtract,
             nnhip.OP_MUL: np.multiply, nnhip.OP_DIV: np.divide}


@pytest.mark.parametrize("op", sorted(NP_BINARY))
@pytest.mark.parametrize("sa,sb", [((4, 5, 6), (4, 5, 6)), ((4, 5, 6), (6,)),
                                   ((4, 5, 6), (5, 1)), ((1, 5, 6), (4, 1, 6)),
                                   ((3000,), (3000,)), ((7,), (1,))])
def test_binary_broadcast_bit_exact(ctx, op, sa, sb):
    rng = np.random.default_rng(op)
    a = rng.standard_normal(sa).astype(np.float32)
    b = (rng.standard_normal(sb).astype(np.float32) + np.float32(3.0))
    got = run_binary(ctx, op, a, b)
    np.testing.assert_array_equal(got, NP_BINARY[op](a, b))


def test_binary_strided_and_offset(ctx):
    """Transposed operands, a view at an element offset, and a strided
    output (every second column of a wider buffer)."""
    rng = np.random.default_rng(1)
    a = rng.standard_normal((6, 9)).astype(np.float32)
    b = rng.standard_normal((6, 9)).astype(np.float32)
    da, va = strided(ctx, a, (1, 0))
    pad = np.concatenate([np.zeros(5, np.float32), b.ravel()])
    db = dev(ctx, pad)
    vb = nnhip.view(db, (6, 9), (9, 1), offset=5)
    do = ctx.array(shape=(6, 18))
    nnhip.call("nnhip_fill_f32", ctx.h, do.p, 6 * 18, -7.0)
    vo = nnhip.view(do, (6, 9), (18, 2))
    nnhip.call("nnhip_binary_f32", ctx.h, nnhip.OP_MUL, va, vb, vo)
    out = do.numpy()
    np.testing.assert_array_equal(out[:, 0::2], a * b)
    assert (out[:, 1::2] == -7.0).all()


def test_backward_elementwise_bit_exact(ctx):
    """relu / sigmoid / tanh / sqrt / log backward (cpu_backend.cpp:473-481,
    492-502, 513-521, 659-669, 680-690), each step one IEEE operation."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((37, 41)).astype(np.float32)
    y = np.abs(x) + np.float32(0.1)
    go = rng.standard_normal((37, 41)).astype(np.float32)
    one, eps = np.float32(1.0), np.float32(1e-8)
    cases = {nnhip.OP_RELU_BACKWARD: (x, np.where(x > 0, go, np.float32(0))),
             nnhip.OP_SIGMOID_BACKWARD: (y, (go * y) * (one - y)),
             nnhip.OP_TANH_BACKWARD: (y, go * (one - y * y)),
             nnhip.OP_SQRT_BACKWARD: (y, go * (np.float32(0.5) / (y + eps))),
             nnhip.OP_LOG_BACKWARD: (y, go / (y + eps))}
    for op, (a, want) in cases.items():
        np.testing.assert_array_equal(run_binary(ctx, op, a, go), want,
                                      err_msg=str(op))


def test_unary_ops(ctx):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 300)).astype(np.float32) * np.float32(3)
    pos = np.abs(x) + np.float32(1e-3)
    x64 = x.astype(np.float64)
    cases = {nnhip.OP_RELU: (x, np.maximum(x64, 0)),
             nnhip.OP_SIGMOID: (x, 1 / (1 + np.exp(-x64))),
             nnhip.OP_TANH: (x, np.tanh(x64)),
             nnhip.OP_SQRT: (pos, np.sqrt(pos.astype(np.float64))),
             nnhip.OP_LOG: (pos, np.log(pos.astype(np.float64) + 1e-8))}
    for op, (a, want) in cases.items():
        da, do = dev(ctx, a), ctx.array(shape=a.shape)
        nnhip.call("nnhip_unary_f32", ctx.h, op, nnhip.view(da), nnhip.view(do))
        got = do.numpy().astype(np.float64)
        # relative to max(|value|, 1): log crosses zero at x = 1, where a
        # correctly rounded fp32 result still differs from float64 by ~1e-8
        err = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
        assert err.max() <= 1e-6, (op, err.max())
    # a transposed input into a contiguous output
    da, va = strided(ctx, x, (1, 0))
    do = ctx.array(shape=x.shape)
    nnhip.call("nnhip_unary_f32", ctx.h, nnhip.OP_RELU, va, nnhip.view(do))
    np.testing.assert_array_equal(do.numpy(), np.maximum(x, 0))


@pytest.mark.parametrize("M,K,N", [(1, 64, 192), (7, 33, 5), (64, 128, 64),
                                   (130, 257, 70)])
def test_matmul_matches_oracle_dense(ctx, M, K, N):
    """Tensor::matmul -> ExecutionBackend::matmul (tensor.cpp:392-428): the
    oracle's Dense product without bias (or_dense: ascending k, separately
    rounded) bit for bit; against float64 within fp32 rounding."""
    rng = np.random.default_rng(M * 1000 + K)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    da, db, do = dev(ctx, a), dev(ctx, b), ctx.array(shape=(M, N))
    nnhip.call("nnhip_matmul_f32", ctx.h, nnhip.view(da), nnhip.view(db),
               nnhip.view(do))
    got = do.numpy()
    want = np.zeros((M, N), np.float32)
    O.lib().or_dense(O.fptr(a), M, K, N, O.fptr(b), None, None, None,
                     O.fptr(want))
    np.testing.assert_array_equal(got, want)
    ex = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(got - ex).max() <= 1e-5 * np.abs(a).max() * np.abs(b).max() * K
    # transposed operands (the reference's sgemm Trans cases) and a strided
    # output give the same values
    ta, va = strided(ctx, a, (1, 0))
    tb, vb = strided(ctx, b, (1, 0))
    do2 = ctx.array(shape=(M, 2 * N))
    nnhip.call("nnhip_matmul_f32", ctx.h, va, vb,
               nnhip.view(do2, (M, N), (2 * N, 2)))
    np.testing.assert_array_equal(do2.numpy()[:, 0::2], want)


def test_matmul_known_answer_and_errors(ctx):
    """TensorTest.MatmulContiguous (tensor_test.cpp:82-94): [[1,2,3],[4,5,6]]
    . [[7,8],[9,10],[11,12]] = [[58,64],[139,154]]; shape errors carry the
    reference's messages (cpu_backend.cpp:332-342)."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    da, db, do = dev(ctx, a), dev(ctx, b), ctx.array(shape=(2, 2))
    nnhip.call("nnhip_matmul_f32", ctx.h, nnhip.view(da), nnhip.view(db),
               nnhip.view(do))
    np.testing.assert_array_equal(do.numpy(), [[58, 64], [139, 154]])
    with pytest.raises(nnhip.NNHipError, match="Incompatible shapes"):
        nnhip.call("nnhip_matmul_f32", ctx.h, nnhip.view(da), nnhip.view(da),
                   nnhip.view(do))
    with pytest.raises(nnhip.NNHipError, match="only supports 2D"):
        nnhip.call("nnhip_matmul_f32", ctx.h, nnhip.view(da, (6,)),
                   nnhip.view(db), nnhip.view(do))


def serial_sum(x, axes, keep):
    """Sum over `axes` adding each output's inputs in ascending input index
    (float32 running sum: np.cumsum is sequential)."""
    kept = [d for d in range(x.ndim) if d not in axes]
    t = np.transpose(x, kept + sorted(axes))
    flat = t.reshape([x.shape[d] for d in kept] + [-1])
    s = np.cumsum(flat, axis=-1, dtype=np.float32)[..., -1]
    if keep:
        s = s.reshape([1 if d in axes else x.shape[d] for d in range(x.ndim)])
    return s


@pytest.mark.parametrize("axes,keep", [((0,), True), ((1,), False),
                                       ((0, 2), True), ((0, 1, 2), False),
                                       ((2,), False)])
def test_sum_bit_exact(ctx, axes, keep):
    rng = np.random.default_rng(len(axes))
    x = rng.standard_normal((6, 700, 9)).astype(np.float32)
    want = serial_sum(x, axes, keep)
    dx = dev(ctx, x)
    do = ctx.array(shape=want.shape if want.ndim else (1,))
    vo = nnhip.view(do, want.shape)
    ax = (np.ctypeslib.ctypes.c_int64 * len(axes))(*axes)
    nnhip.call("nnhip_sum_f32", ctx.h, nnhip.view(dx), vo, ax, len(axes))
    np.testing.assert_array_equal(do.numpy().reshape(want.shape), want)


def test_reference_tensor_known_answers(ctx):
    """The reference's Tensor KATs through the backend ops: BroadcastingAdd
    (tensor_test.cpp:53-67, [2,3] + [1,3]), ElementwiseSubAndMul (:69-80),
    SumReduction (:97-118: all axes -> rank 0 = 21, axis 0 -> [5,7,9],
    axis 1 keepdims -> [2,1] = [6,15]); and axis 0 of a transposed input."""
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    got = run_binary(ctx, nnhip.OP_ADD, x, np.array([[10, 20, 30]], np.float32))
    np.testing.assert_array_equal(got, [[11, 22, 33], [14, 25, 36]])
    a, b = np.array([10, 20], np.float32), np.array([2, 5], np.float32)
    np.testing.assert_array_equal(run_binary(ctx, nnhip.OP_SUB, a, b), [8, 15])
    np.testing.assert_array_equal(run_binary(ctx, nnhip.OP_MUL, a, b), [20, 100])
    for axes, shape, want in (((0, 1), (), [21]), ((0,), (3,), [5, 7, 9]),
                              ((1,), (2, 1), [6, 15])):
        dx = dev(ctx, x)
        do = ctx.array(shape=(len(want),))
        ax = (np.ctypeslib.ctypes.c_int64 * len(axes))(*axes)
        nnhip.call("nnhip_sum_f32", ctx.h, nnhip.view(dx),
                   nnhip.view(do, shape), ax, len(axes))
        np.testing.assert_array_equal(do.numpy(), want)
    _, vt = strided(ctx, x, (1, 0))
    do = ctx.array(shape=(3,))
    ax = (np.ctypeslib.ctypes.c_int64 * 1)(0)
    nnhip.call("nnhip_sum_f32", ctx.h, vt, nnhip.view(do), ax, 1)
    np.testing.assert_array_equal(do.numpy(), [5, 7, 9])


@pytest.mark.parametrize("shape,axis", [((4, 32000), 1), ((37, 5), 0),
                                        ((3, 7, 11), 1), ((2, 1, 9), 2)])
def test_softmax_and_backward(ctx, shape, axis):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    dx = dev(ctx, x)
    do = ctx.array(shape=shape)
    nnhip.call("nnhip_softmax_f32", ctx.h, nnhip.view(dx), nnhip.view(do), axis)
    y = do.numpy()
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=axis, keepdims=True))
    want = e / e.sum(axis=axis, keepdims=True)
    assert (np.abs(y - want) / want).max() <= 2e-6
    # softmax_backward: dx = y * (dy - sum(dy * y))
    g = rng.standard_normal(shape).astype(np.float32)
    dg, dgi = dev(ctx, g), ctx.array(shape=shape)
    nnhip.call("nnhip_softmax_backward_f32", ctx.h, nnhip.view(do),
               nnhip.view(dg), nnhip.view(dgi), axis)
    y64 = y.astype(np.float64)
    wb = y64 * (g - (g * y64).sum(axis=axis, keepdims=True))
    scale = np.abs(wb).max()
    assert np.abs(dgi.numpy() - wb).max() <= 1e-5 * scale
    # along a transposed (non-contiguous) input
    if len(shape) == 2:
        _, vt = strided(ctx, x, (1, 0))
        do2 = ctx.array(shape=shape)
        nnhip.call("nnhip_softmax_f32", ctx.h, vt, nnhip.view(do2), axis)
        np.testing.assert_allclose(do2.numpy(), y, rtol=2e-6)


def test_embedding_gather(ctx):
    """Tensor::embedding (tensor.cpp:915-967 -> cpu_backend.cpp:998-1033):
    rows of the weight by fp32 id; ids outside [0, V) take row 0;
    a transposed index tensor."""
    rng = np.random.default_rng(4)
    V, D = 50, 24
    w = rng.standard_normal((V, D)).astype(np.float32)
    ids = rng.integers(0, V, (3, 7)).astype(np.float32)
    ids[0, 0], ids[1, 3], ids[2, 6] = 50, 1e6, -3
    ids[2, 2] = 7.6                                  # truncates to 7
    dw, di = dev(ctx, w), dev(ctx, ids)
    do = ctx.array(shape=(3, 7, D))
    nnhip.call("nnhip_embedding_f32", ctx.h, nnhip.view(dw), nnhip.view(di),
               nnhip.view(do))
    idx = ids.astype(np.int64)
    idx[(ids < 0) | (ids >= V)] = 0
    np.testing.assert_array_equal(do.numpy(), w[idx])
    _, vt = strided(ctx, ids, (1, 0))
    do2 = ctx.array(shape=(3, 7, D))
    nnhip.call("nnhip_embedding_f32", ctx.h, nnhip.view(dw), vt,
               nnhip.view(do2))
    np.testing.assert_array_equal(do2.numpy(), w[idx])


def test_slice_backward_and_fill(ctx):
    rng = np.random.default_rng(5)
    gp = rng.standard_normal((4, 6, 5)).astype(np.float32)
    gs = rng.standard_normal((4, 5)).astype(np.float32)
    dgp, dgs = dev(ctx, gp), dev(ctx, gs)
    nnhip.call("nnhip_slice_backward_f32", ctx.h, nnhip.view(dgs),
               nnhip.view(dgp), 1, 3)
    want = gp.copy()
    want[:, 3, :] += gs
    np.testing.assert_array_equal(dgp.numpy(), want)
    nnhip.call("nnhip_fill_f32", ctx.h, dgp.p, gp.size, 2.5)
    assert (dgp.numpy() == 2.5).all()


def test_non_broadcastable_operands_are_refused(ctx):
    """An operand whose right-aligned dims are neither the output's nor 1
    ([3] against [4, 5]; [2, 5] against [4, 5]) is refused with NNHIP_EARG
    on the host, before any launch: the output keeps its contents."""
    da = dev(ctx, np.ones(3, np.float32))
    db = dev(ctx, np.ones((2, 5), np.float32))
    dc = dev(ctx, np.ones((4, 5), np.float32))
    do = ctx.array(shape=(4, 5))
    nnhip.call("nnhip_fill_f32", ctx.h, do.p, 20, -3.0)
    for bad in (da, db):
        with pytest.raises(nnhip.NNHipError) as e:
            nnhip.call("nnhip_binary_f32", ctx.h, nnhip.OP_ADD, nnhip.view(bad),
                       nnhip.view(dc), nnhip.view(do))
        assert e.value.code == nnhip.EARG
        with pytest.raises(nnhip.NNHipError) as e:
            nnhip.call("nnhip_unary_f32", ctx.h, nnhip.OP_RELU,
                       nnhip.view(bad), nnhip.view(do))
        assert e.value.code == nnhip.EARG
    assert (do.numpy() == -3.0).all()


def test_softmax_backward_broadcast_grad(ctx):
    """CpuBackend::softmax_backward reads grad_out through its broadcast
    offset against the output's shape (cpu_backend.cpp:585-640): a [1, L]
    gradient against [R, L] outputs gives y * (g - sum(g * y)) per row."""
    rng = np.random.default_rng(12)
    R, L = 5, 33
    y = rng.random((R, L)).astype(np.float32)
    y /= y.sum(1, keepdims=True)
    g = rng.standard_normal((1, L)).astype(np.float32)
    dy_, dg, dx = dev(ctx, y), dev(ctx, g), ctx.array(shape=(R, L))
    nnhip.call("nnhip_softmax_backward_f32", ctx.h, nnhip.view(dy_),
               nnhip.view(dg), nnhip.view(dx), 1)
    y64 = y.astype(np.float64)
    want = y64 * (g - (g * y64).sum(1, keepdims=True))
    assert np.abs(dx.numpy() - want).max() <= 1e-5 * np.abs(want).max()

"""nnhip_linear_w8a32_noalloc against nnhip_linear_w8a32 (GPU).

The no-allocation variant keeps its scratch in one fixed device array per
GPU; it runs the same kernels on the same inputs, so its outputs must equal
the allocating entry point's bit for bit -- on two calls in a row, the
second smaller than the first (the array keeps the first call's contents),
for every path, and for the GEMV path that needs no scratch.  Inputs too
large for the array are refused with NNHIP_EARG.
"""
import numpy as np
import pytest

from gpu_util import nnhip

pytestmark = pytest.mark.gpu


def linear_pair(ctx, rows, K, N, path, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    codes = rng.integers(-127, 128, (N, K)).astype(np.int8)
    scales = (rng.random(N).astype(np.float32) * np.float32(0.01) +
              np.float32(1e-3))
    bias = rng.standard_normal(N).astype(np.float32)
    dx, dc = ctx.array(x), ctx.array(codes)
    ds, db = ctx.array(scales), ctx.array(bias)
    y1 = ctx.array(shape=(rows, N))
    y2 = ctx.array(shape=(rows, N))
    nnhip.call("nnhip_linear_w8a32", ctx.h, dx.p, rows, K, dc.p, ds.p, db.p,
               N, y1.p, path)
    nnhip.call("nnhip_linear_w8a32_noalloc", ctx.h, dx.p, rows, K, dc.p, ds.p,
               db.p, N, y2.p, path)
    ctx.sync()
    a, b = y1.numpy(), y2.numpy()
    for arr in (dx, dc, ds, db, y1, y2):
        arr.free()
    return a, b


@pytest.mark.parametrize("path", [0, 2, 3, 4])
def test_noalloc_matches_allocating_linear(ctx, path):
    for rows, K, N in ((96, 1024, 1536), (20, 256, 512)):
        want, got = linear_pair(ctx, rows, K, N, path, seed=rows + path)
        np.testing.assert_array_equal(got, want, err_msg=f"{rows}x{K}x{N}")


def test_noalloc_gemv_and_limit(ctx):
    want, got = linear_pair(ctx, 5, 512, 640, 0, seed=3)
    np.testing.assert_array_equal(got, want)
    # just under the limit: 32512 x 1024 codes + 3 x 64 x 1024 digits + 64
    # exponents = 33,489,152 of 33,554,432 bytes
    want, got = linear_pair(ctx, 64, 1024, 32512, 2, seed=4)
    np.testing.assert_array_equal(got, want)
    # 32768 x 1024 codes alone fill the 32 MiB array; with the digit planes
    # and exponents the call exceeds it
    rows, K, N = 64, 1024, 32768
    dx = ctx.array(shape=(rows, K))
    dc = ctx.array(shape=(N, K), dtype=np.int8)
    ds, db = ctx.array(shape=(N,)), ctx.array(shape=(N,))
    y = ctx.array(shape=(rows, N))
    with pytest.raises(nnhip.NNHipError) as e:
        nnhip.call("nnhip_linear_w8a32_noalloc", ctx.h, dx.p, rows, K, dc.p,
                   ds.p, db.p, N, y.p, 2)
    assert e.value.code == nnhip.EARG
    for arr in (dx, dc, ds, db, y):
        arr.free()


def test_noalloc_refuses_a_second_context(ctx):
    """The first context that called the entry point owns this GPU's array;
    another context's call would run on another stream, unordered against
    the owner's, and is refused with NNHIP_EARG (no launch)."""
    want, got = linear_pair(ctx, 20, 256, 512, 2, seed=5)
    np.testing.assert_array_equal(got, want)
    other = nnhip.Context(0)
    try:
        rows, K, N = 20, 256, 512
        dx = other.array(shape=(rows, K))
        dc = other.array(shape=(N, K), dtype=np.int8)
        ds, db = other.array(shape=(N,)), other.array(shape=(N,))
        y = other.array(shape=(rows, N))
        with pytest.raises(nnhip.NNHipError) as e:
            nnhip.call("nnhip_linear_w8a32_noalloc", other.h, dx.p, rows, K,
                       dc.p, ds.p, db.p, N, y.p, 2)
        assert e.value.code == nnhip.EARG
        for arr in (dx, dc, ds, db, y):
            arr.free()
    finally:
        other.close()
    # the owner keeps working
    want, got = linear_pair(ctx, 20, 256, 512, 2, seed=6)
    np.testing.assert_array_equal(got, want)

"""spq4k_mul_mat_noalloc (include/spq4k.h): spq4k_mul_mat with its
intermediates in the library's fixed device array instead of the context's
scratch. Called through the C ABI and checked against spq4k_mul_mat on the
same inputs, to the parity bar of the other matmul tests (close_enough, 1e-4
relative or 1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48) and
against the CPU oracle; two calls in a row, the second with a smaller input,
so the second runs on what the first left in the array. Sizes beyond the
array are refused with -EINVAL."""
import ctypes as C
import errno

import numpy as np
import pytest

from _oracle import close_enough

pytestmark = pytest.mark.gpu


def _noalloc(ctx, W, x_ptr, y_ptr, T):
    lib = ctx.lib
    f = lib.spq4k_mul_mat_noalloc
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]
    return f(ctx.handle, W.handle, x_ptr, y_ptr, T)


def _case(ctx, oracle, qtype, M, K, T, seed):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    W = oracle.quantize_q8_0(w, ref_encoder=True) if qtype == 8 else oracle.quantize(qtype, w)
    X = rng.standard_normal((T, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K, type=qtype)
    xd = DeviceArray.from_host(X)
    ya, yb = DeviceArray((T, M)), DeviceArray((T, M))
    ctx.mul_mat_dev(Wd, xd.ptr, ya.ptr, T)
    rc = _noalloc(ctx, Wd, xd.ptr, yb.ptr, T)
    assert rc == 0, ctx.lib.spq4k_last_error(ctx.handle)
    ctx.synchronize()
    a, b = ya.to_host(), yb.to_host()
    ok = close_enough(b, a)
    assert ok.all(), f"type {qtype} M={M} K={K} T={T}: {int((~ok).sum())}/{ok.size} outside tolerance of spq4k_mul_mat"
    idx = np.r_[0:min(T, 4), max(0, T - 4):T]
    Xs = np.ascontiguousarray(X[idx])
    exp = oracle.mul_mat_q8_0(W, M, K, Xs) if qtype == 8 else oracle.mul_mat_type(qtype, W, M, K, Xs)
    ok = close_enough(b[idx], exp)
    assert ok.all(), f"type {qtype} M={M} K={K} T={T}: {int((~ok).sum())}/{ok.size} outside tolerance of the oracle"
    Wd.free()


@pytest.mark.parametrize("qtype", [12, 14, 8])
def test_noalloc_matches_mul_mat(ctx, oracle, qtype):
    # first call large (K split on the matrix cores), second smaller
    _case(ctx, oracle, qtype, 512, 4096, 300, 1 + qtype)
    _case(ctx, oracle, qtype, 192, 2048, 40, 2 + qtype)
    _case(ctx, oracle, qtype, 256, 4096, 3, 3 + qtype)


def test_noalloc_rejects_oversize(ctx, oracle):
    from spq4k.hip import DeviceArray
    M, K = 64, 4096
    rng = np.random.default_rng(5)
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    Wd = ctx.upload(W, M, K)
    T = 8192   # 8192 rows of 16 blocks: 44.6 MB of Q8_K planes, above the 24 MiB limit
    xd, yd = DeviceArray((T, K)), DeviceArray((T, M))
    assert _noalloc(ctx, Wd, xd.ptr, yd.ptr, T) == -errno.EINVAL
    assert b"no-allocation" in ctx.lib.spq4k_last_error(ctx.handle)
    Wd.free()

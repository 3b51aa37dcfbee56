"""spq4k_mul_mat_noalloc (include/spq4k.h): spq4k_mul_mat with its
intermediates in the library's fixed device array instead of the context's
scratch. Called through the C ABI and checked bit for bit against
spq4k_mul_mat on the same inputs (the same kernels and, with the K split's
fixed partial budget, the same split) and against the CPU oracle to the
parity bar of the other matmul tests (close_enough, 1e-4 relative or 1e-5
absolute, tests/desktop/test_sp_kernels.cpp:34-48); two calls in a row, the
second with a smaller input, so the second runs on what the first left in the
array. Also: captured into a HIP graph on a context whose own scratch is too
small for the call and replayed; device memory unchanged by a burst of calls;
sizes beyond the array refused with -EINVAL; a failed address lookup leaves
the context usable and the entry point reporting -EIO."""
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
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
        f"type {qtype} M={M} K={K} T={T}: {int((a.view(np.uint32) != b.view(np.uint32)).sum())}/{a.size} differ " \
        "from spq4k_mul_mat"
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


def test_noalloc_graph_capture_and_no_device_allocation(oracle):
    """captured into a graph on a fresh context whose own scratch (16 MiB) is
    too small for the call's activation planes (spq4k_mul_mat there would
    have to grow it, which a capture refuses), replayed twice with eager work
    between, each replay bit-equal to an eager spq4k_mul_mat; free device
    memory is unchanged by a burst of calls"""
    import spq4k
    from spq4k.hip import DeviceArray, Graph, mem_info
    ctx = spq4k.Context(0)
    M, K, T = 256, 4096, 3500   # 16 blocks a row: 19 MB of Q8_K planes, above 16 MiB and below 24 MiB
    rng = np.random.default_rng(21)
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    Wd = ctx.upload(W, M, K)
    xd = DeviceArray.from_host(rng.standard_normal((T, K)).astype(np.float32))
    yg = DeviceArray((T, M))
    yg.fill_byte(0)
    with Graph.capture(ctx.stream) as g:
        rc = _noalloc(ctx, Wd, xd.ptr, yg.ptr, T)
    assert rc == 0, ctx.lib.spq4k_last_error(ctx.handle)
    # the eager reference (this call grows the context's scratch: outside the capture)
    ye = DeviceArray((T, M))
    ctx.mul_mat_dev(Wd, xd.ptr, ye.ptr, T)
    ctx.synchronize()
    ref = ye.to_host()
    for rep in range(2):
        yg.fill_byte(0)
        g.launch()
        ctx.synchronize()
        got = yg.to_host()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep} differs from spq4k_mul_mat"
        ctx.mul_mat_dev(Wd, xd.ptr, ye.ptr, 7)   # eager work between the replays
        ctx.synchronize()
    # a burst of calls allocates nothing
    assert _noalloc(ctx, Wd, xd.ptr, yg.ptr, T) == 0
    ctx.synchronize()
    free0, _ = mem_info()
    for t in (T, 1, 64, 2000, T):
        assert _noalloc(ctx, Wd, xd.ptr, yg.ptr, t) == 0
    ctx.synchronize()
    free1, _ = mem_info()
    assert free1 == free0, f"free device memory {free0} -> {free1}"
    Wd.free()
    ctx.close()


def test_noalloc_lookup_failure_leaves_context_usable():
    """with the array's address lookup made to fail (SPQ4K_TEST_NOALLOC_LOOKUP_FAIL),
    in a process of its own (a successful lookup is kept for the process):
    spq4k_init succeeds, spq4k_mul_mat works, spq4k_mul_mat_noalloc reports -EIO"""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = r"""
import ctypes as C, errno, sys
import numpy as np
sys.path.insert(0, %r); sys.path.insert(0, %r)
import spq4k
from spq4k.hip import DeviceArray
ctx = spq4k.Context(0)
M, K = 64, 4096
W = ctx.alloc_weights(M, K)
x, y = DeviceArray((1, K)), DeviceArray((1, M))
x.fill_byte(0)
ctx.mul_mat_dev(W, x.ptr, y.ptr, 1)
ctx.synchronize()
f = ctx.lib.spq4k_mul_mat_noalloc
f.restype = C.c_int
f.argtypes = [C.c_void_p] * 4 + [C.c_int64]
rc = f(ctx.handle, W.handle, x.ptr, y.ptr, 1)
print("RC", rc, ctx.lib.spq4k_last_error(ctx.handle).decode())
sys.exit(0 if rc == -errno.EIO else 1)
""" % (os.path.join(os.path.dirname(here), "shannon-prime-burnhard_amd"), here)
    env = dict(os.environ, SPQ4K_TEST_NOALLOC_LOOKUP_FAIL="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "no-allocation" in r.stdout

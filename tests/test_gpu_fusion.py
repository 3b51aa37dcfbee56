"""GPU parity of the operations fused around the matvec (spq4k_rms_norm,
spq4k_mul_mat_rms_norm, spq4k_mul_mat_swiglu; include/spq4k.h).

Against the oracle (oracle/fusion_oracle.c and the matmul restatements, pinned
to the reference's ggml graphs in test_oracle_fusion.py):
  - the normalised rows: bit-exact;
  - y_i = W_i . rms_norm(x) * w and silu(Wg . xb) * (Wu . xb): every element
    within close_enough (1e-4 relative or 1e-5 absolute,
    tests/desktop/test_sp_kernels.cpp:34-48) of the oracle, for Q4_K, Q5_K,
    Q6_K and Q8_0, decode (T = 1, one fused launch where the decode kernel
    runs the type and K) and batches (the norm pass, then the matmul; gate and
    up, then the element-wise pass);
  - the fused T = 1 launch equals the unfused steps bit for bit (the same
    normalised rows feed the same lane arithmetic)."""
import numpy as np
import pytest

from _oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, close_enough

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _enc(oracle, qtype, M, K, rng, scale=0.02):
    x = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    return oracle.quantize_q8_0(x, ref_encoder=True) if qtype == TYPE_Q8_0 else oracle.quantize(qtype, x)


def _mm(oracle, qtype, W, M, K, X):
    return oracle.mul_mat_q8_0(W, M, K, X) if qtype == TYPE_Q8_0 else oracle.mul_mat_type(qtype, W, M, K, X)


def _check(got, exp, what):
    ok = close_enough(got, exp)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; first {tuple(i)} "
                             f"got {got[tuple(i)]!r} exp {exp[tuple(i)]!r}")


def _inputs(rng, T, K):
    X = rng.standard_normal((T, K)).astype(np.float32)
    X[:, ::11] *= 0.01
    w = (1.0 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    return X, w


@pytest.mark.parametrize("K,T", [(4096, 1), (12288, 1), (27648, 1), (5120, 3), (768, 17), (96, 2)])
def test_rms_norm_bitexact(ctx, oracle, K, T):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(K + T)
    X, w = _inputs(rng, T, K)
    X[0, :3] = [1e30, -1e-30, 0.0]
    xd, wd, yd = DeviceArray.from_host(X), DeviceArray.from_host(w), DeviceArray((T, K))
    ctx.rms_norm_dev(xd.ptr, wd.ptr, EPS, yd.ptr, K, T)
    ctx.synchronize()
    np.testing.assert_array_equal(yd.to_host().view(np.uint32), oracle.rms_norm(X, w, EPS).view(np.uint32))


@pytest.mark.parametrize("qtype", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("T", [1, 3, 9])
def test_mul_mat_rms_norm(ctx, oracle, qtype, T):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(100 * qtype + T)
    K = 4096
    shapes = (1024, 256, 256)            # q, k, v of one input
    Ws = [_enc(oracle, qtype, M, K, rng) for M in shapes]
    X, w = _inputs(rng, T, K)
    wd = [ctx.upload(W, M, K, type=qtype) for W, M in zip(Ws, shapes)]
    xd, nd = DeviceArray.from_host(X), DeviceArray.from_host(w)
    yd = [DeviceArray((T, M)) for M in shapes]
    ctx.mul_mat_rms_norm_dev(wd, xd.ptr, nd.ptr, EPS, [y.ptr for y in yd], T)
    ctx.synchronize()
    xb = oracle.rms_norm(X, w, EPS)
    for W, M, y in zip(Ws, shapes, yd):
        _check(y.to_host(), _mm(oracle, qtype, W, M, K, xb), f"type {qtype} T={T} M={M}")
    # the same through the unfused steps: bit for bit
    xn = DeviceArray((T, K))
    ctx.rms_norm_dev(xd.ptr, nd.ptr, EPS, xn.ptr, K, T)
    y2 = [DeviceArray((T, M)) for M in shapes]
    if T <= 8:
        ctx.gemv_multi_dev(wd, xn.ptr, [y.ptr for y in y2], T)
    else:
        ctx.gemm_multi_dev(wd, xn.ptr, [y.ptr for y in y2], T)
    ctx.synchronize()
    for a, b in zip(yd, y2):
        np.testing.assert_array_equal(a.to_host().view(np.uint32), b.to_host().view(np.uint32))


@pytest.mark.parametrize("qtype", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("T,norm", [(1, True), (1, False), (4, True), (12, False)])
def test_mul_mat_swiglu(ctx, oracle, qtype, T, norm):
    """silu(g) * u multiplies the rounding of u by silu(g): an output near
    zero carries an absolute error of its factors' size, so the product is
    not held element-wise to close_enough. Instead the device's gate and up
    (the unfused matmuls, the same lane arithmetic as the fused launch) are
    held to close_enough of the oracle, and the fused output to silu(g) * u of
    exactly those values (to the last bits of silu: device and host expf)."""
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(200 * qtype + T + norm)
    for M, K in ((1536, 4096), (384, 12288)):
        Wg = _enc(oracle, qtype, M, K, rng)
        Wu = _enc(oracle, qtype, M, K, rng)
        X, w = _inputs(rng, T, K)
        gd, ud = ctx.upload(Wg, M, K, type=qtype), ctx.upload(Wu, M, K, type=qtype)
        xd, nd, yd = DeviceArray.from_host(X), DeviceArray.from_host(w), DeviceArray((T, M))
        ctx.mul_mat_swiglu_dev(gd, ud, xd.ptr, nd.ptr if norm else None, EPS, yd.ptr, T)
        # the unfused steps on the device
        xin = xd
        if norm:
            xin = DeviceArray((T, K))
            ctx.rms_norm_dev(xd.ptr, nd.ptr, EPS, xin.ptr, K, T)
        g2, u2 = DeviceArray((T, M)), DeviceArray((T, M))
        if T <= 8:
            ctx.gemv_multi_dev([gd, ud], xin.ptr, [g2.ptr, u2.ptr], T)
        else:
            ctx.gemm_multi_dev([gd, ud], xin.ptr, [g2.ptr, u2.ptr], T)
        ctx.synchronize()
        g, u, got = g2.to_host(), u2.to_host(), yd.to_host()
        xb = oracle.rms_norm(X, w, EPS) if norm else X
        what = f"type {qtype} T={T} norm={norm} M={M} K={K}"
        _check(g, _mm(oracle, qtype, Wg, M, K, xb), "gate " + what)
        _check(u, _mm(oracle, qtype, Wu, M, K, xb), "up " + what)
        np.testing.assert_allclose(got, oracle.swiglu(g, u), rtol=4e-7, atol=1e-30, err_msg=what)


def test_fusion_errors(ctx, oracle):
    from spq4k import Spq4kError
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(5)
    a = ctx.upload(_enc(oracle, TYPE_Q4_K, 64, 256, rng), 64, 256)
    b = ctx.upload(_enc(oracle, TYPE_Q4_K, 32, 256, rng), 32, 256)
    c = ctx.upload(_enc(oracle, TYPE_Q6_K, 64, 256, rng), 64, 256, type=TYPE_Q6_K)
    x, y = DeviceArray(256), DeviceArray(64)
    with pytest.raises(Spq4kError):   # gate and up rows differ
        ctx.mul_mat_swiglu_dev(a, b, x.ptr, None, EPS, y.ptr, 1)
    with pytest.raises(Spq4kError):   # types differ
        ctx.mul_mat_swiglu_dev(a, c, x.ptr, None, EPS, y.ptr, 1)
    with pytest.raises(Spq4kError):   # a norm needs its weights
        ctx.mul_mat_rms_norm_dev([a], x.ptr, None, EPS, [y.ptr], 1)
    with pytest.raises(Spq4kError):   # eps < 0
        ctx.rms_norm_dev(x.ptr, x.ptr, -1.0, y.ptr, 64, 1)


@pytest.mark.parametrize("K", [2048, 3072, 8192, 14336])
def test_fused_any_k(ctx, oracle, K):
    """The fused decode forms at row lengths served by the runtime-length
    decode instances (norm prologue; SwiGLU epilogue where two rows in flight
    fit the register file, the unfused steps beyond): bit for bit against the
    unfused steps, and the parity bar against the oracle."""
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(K)
    shapes = (512, 128, 128)
    Ws = [_enc(oracle, TYPE_Q4_K, M, K, rng) for M in shapes]
    X, w = _inputs(rng, 1, K)
    wd = [ctx.upload(W, M, K) for W, M in zip(Ws, shapes)]
    xd, nd = DeviceArray.from_host(X), DeviceArray.from_host(w)
    yd = [DeviceArray((1, M)) for M in shapes]
    ctx.mul_mat_rms_norm_dev(wd, xd.ptr, nd.ptr, EPS, [y.ptr for y in yd], 1)
    xn = DeviceArray((1, K))
    ctx.rms_norm_dev(xd.ptr, nd.ptr, EPS, xn.ptr, K, 1)
    y2 = [DeviceArray((1, M)) for M in shapes]
    ctx.gemv_multi_dev(wd, xn.ptr, [y.ptr for y in y2], 1)
    ctx.synchronize()
    xb = oracle.rms_norm(X, w, EPS)
    for W, M, a, b in zip(Ws, shapes, yd, y2):
        np.testing.assert_array_equal(a.to_host().view(np.uint32), b.to_host().view(np.uint32))
        _check(a.to_host(), _mm(oracle, TYPE_Q4_K, W, M, K, xb), f"norm K={K} M={M}")
    # gate / up with the SwiGLU epilogue
    M = 640
    Wg, Wu = _enc(oracle, TYPE_Q4_K, M, K, rng), _enc(oracle, TYPE_Q4_K, M, K, rng)
    gd, ud = ctx.upload(Wg, M, K), ctx.upload(Wu, M, K)
    yg = DeviceArray((1, M))
    ctx.mul_mat_swiglu_dev(gd, ud, xd.ptr, nd.ptr, EPS, yg.ptr, 1)
    g2, u2 = DeviceArray((1, M)), DeviceArray((1, M))
    ctx.gemv_multi_dev([gd, ud], xn.ptr, [g2.ptr, u2.ptr], 1)
    ctx.synchronize()
    g, u = g2.to_host(), u2.to_host()
    _check(g, _mm(oracle, TYPE_Q4_K, Wg, M, K, xb), f"gate K={K}")
    _check(u, _mm(oracle, TYPE_Q4_K, Wu, M, K, xb), f"up K={K}")
    np.testing.assert_allclose(yg.to_host(), oracle.swiglu(g, u), rtol=4e-7, atol=1e-30, err_msg=f"swiglu K={K}")

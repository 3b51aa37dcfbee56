"""GPU parity of the matrix-core prefill matmul (spq4k_gemm / mul_mat, T > 8).

Against the reference's own GGML_OP_MUL_MAT outputs (golden vectors) and the
CPU oracle (ggml's x86 order, pinned bit-exact to the reference) on Q8_K
activations. Tolerance: close_enough, 1e-4 relative or 1e-5 absolute
(tests/desktop/test_sp_kernels.cpp:34-48)."""
import os

import numpy as np
import pytest

from _oracle import close_enough, parity_ok

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def _check(got, exp, what, exact=None):
    """close_enough of the oracle (ggml's x86 order); with `exact`, the parity
    bar's either-or: of the oracle or of the dequant-then-dot value"""
    ok = close_enough(got, exp) if exact is None else parity_ok(got, exp, exact)
    assert ok.all(), (f"{what}: {int((~ok).sum())}/{ok.size} outside tolerance; first {np.argwhere(~ok)[0]} "
                      f"got {got[tuple(np.argwhere(~ok)[0])]} exp {exp[tuple(np.argwhere(~ok)[0])]}")


def test_gemm_golden(ctx):
    G = np.load(os.path.join(HERE, "golden", "q4k_golden.npz"))
    M, K = (int(v) for v in G["mm_MK"])
    W = ctx.upload(G["mm_W"], M, K)
    _check(ctx.mul_mat(W, G["mm_X17"]), G["mm_Y17"], "golden T=17")


@pytest.mark.parametrize("M,K,T", [(256, 4096, 9), (256, 4096, 16), (192, 4096, 33), (256, 4096, 128),
                                   (128, 12288, 64), (100, 768, 40), (64, 27648, 20)])
def test_gemm_vs_oracle(ctx, oracle, M, K, T):
    rng = np.random.default_rng(M + K + T)
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K)
    _check(ctx.mul_mat(Wd, X), oracle.mul_mat(W, M, K, X), f"gemm M={M} K={K} T={T}",
           oracle.mul_mat_dq_f64(12, W, M, K, X))


@pytest.mark.parametrize("T", [1, 3, 8])
def test_gemm_small_t_matches_gemv(ctx, oracle, T):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(40 + T)
    M, K = 320, 2048
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K)
    xd = DeviceArray.from_host(X)
    yd = DeviceArray((T, M), np.float32)
    ctx.gemm_dev(Wd, xd.ptr, yd.ptr, T)
    ctx.synchronize()
    _check(yd.to_host(), oracle.mul_mat(W, M, K, X), f"gemm T={T}")


@pytest.mark.parametrize("mode", [1, 2])
def test_gemm_both_kernels(oracle, mode):
    """The skinny kernel (SPQ4K_GEMM_MODE=1: K split across the workgroup's
    waves, operands from the Q8_K planes) and the tiled kernel (=2: activations
    staged in LDS, shape chosen by size) at token counts on both sides of their default
    ranges, with ragged row and token tails."""
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMM_MODE": mode})
    try:
        for M, K, T in ((70, 4096, 9), (130, 2048, 17), (64, 12288, 31), (50, 768, 47), (96, 4096, 65),
                        (33, 5120, 130)):
            rng = np.random.default_rng(M * 3 + T)
            W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
            X = rng.standard_normal((T, K)).astype(np.float32)
            Wd = c.upload(W, M, K)
            _check(c.mul_mat(Wd, X), oracle.mul_mat(W, M, K, X), f"mode={mode} M={M} K={K} T={T}")
            Wd.free()
    finally:
        c.close()


def test_gemm_repeatable(ctx, oracle):
    """Fixed reduction order across the workgroup's waves: bit-identical reruns."""
    rng = np.random.default_rng(4)
    M, K, T = 200, 12288, 24
    Wd = ctx.upload(oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32)), M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    a = ctx.mul_mat(Wd, X)
    for _ in range(3):
        np.testing.assert_array_equal(ctx.mul_mat(Wd, X), a)


@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("K,shapes,T", [(4096, (256, 64, 64), 16), (2048, (300, 300), 40), (768, (17, 100, 5, 33), 100)])
def test_gemm_multi(oracle, mode, K, shapes, T):
    """q/k/v and gate/up of a prefill batch in one call: X quantised once,
    every matrix within tolerance of the oracle (both kernels take the
    matrices as segments of one launch)."""
    from spq4k.hip import DeviceArray
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMM_MODE": mode})
    try:
        rng = np.random.default_rng(K + T)
        Ws = [oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32)) for M in shapes]
        X = rng.standard_normal((T, K)).astype(np.float32)
        wd = [c.upload(w, M, K) for w, M in zip(Ws, shapes)]
        xd = DeviceArray.from_host(X)
        ys = [DeviceArray.from_host(np.full((T, M), np.nan, np.float32)) for M in shapes]
        c.gemm_multi_dev(wd, xd.ptr, [y.ptr for y in ys], T)
        c.synchronize()
        for w, M, y in zip(Ws, shapes, ys):
            _check(y.to_host(), oracle.mul_mat(w, M, K, X), f"multi mode={mode} K={K} M={M} T={T}")
    finally:
        c.close()


def _extreme_weights(oracle, rng, M, K):
    """Random Q4_K rows with every fourth super-block replaced by the largest
    one (d = dmin = 2^-6, all scales and mins 63, all nibbles 15)."""
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32)).reshape(M, K // 256, 144)
    ext = np.full(144, 0xFF, np.uint8)
    ext[0:2] = ext[2:4] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    W[:, ::4] = ext
    return W.reshape(-1)


def _one_sign_tokens(rng, T, K):
    X = np.abs(rng.standard_normal((T, K))).astype(np.float32) * np.where(np.arange(T) % 2, -1, 1)[:, None]
    X[0] = 1.0
    X[-1] = -1.0
    X[T // 2, : K // 2] = 3.0 * np.sign(X[T // 2, -1])
    return X.astype(np.float32)


@pytest.mark.parametrize("cfg", list(range(14)) + [32])
def test_gemm_tiled_shapes(oracle, cfg):
    """Every launch shape of the tiled kernel (SPQ4K_GEMM_CFG) with ragged row,
    token and super-block tails (K = 768 leaves a K-split wave idle), the
    largest Q4_K blocks against constant +-1 activations (|BS_j| = 4064, the
    edge of the exact fp16 min-term split), and four matrices in one launch.
    Each token has one sign: the largest blocks dequantise to 13.78 everywhere,
    and against mixed-sign tokens their sums would cancel to far below the fp32
    rounding of the terms, which no summation order can meet at 1e-4."""
    from spq4k.hip import DeviceArray
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMM_MODE": 2, "SPQ4K_GEMM_CFG": cfg})
    try:
        rng = np.random.default_rng(500 + cfg)
        for M, K, T in ((150, 4096, 70), (33, 768, 17), (200, 5120, 100), (64, 12288, 65)):
            W = _extreme_weights(oracle, rng, M, K)
            X = _one_sign_tokens(rng, T, K)
            Wd = c.upload(W, M, K)
            _check(c.mul_mat(Wd, X), oracle.mul_mat(W, M, K, X), f"cfg={cfg} M={M} K={K} T={T}")
            Wd.free()
        K, T, shapes = 2048, 50, (300, 17, 129, 64)
        Ws = [_extreme_weights(oracle, rng, M, K) for M in shapes]
        X = _one_sign_tokens(rng, T, K)
        wd = [c.upload(w, M, K) for w, M in zip(Ws, shapes)]
        xd = DeviceArray.from_host(X)
        ys = [DeviceArray.from_host(np.full((T, M), np.nan, np.float32)) for M in shapes]
        c.gemm_multi_dev(wd, xd.ptr, [y.ptr for y in ys], T)
        c.synchronize()
        for w, M, y in zip(Ws, shapes, ys):
            _check(y.to_host(), oracle.mul_mat(w, M, K, X), f"cfg={cfg} multi M={M}")
    finally:
        c.close()


@pytest.mark.parametrize("M,K,T,qtype", [(4096, 12288, 16, 12), (1000, 4096, 24, 12), (4096, 12288, 16, 14),
                                         (700, 8192, 40, 13), (2048, 4096, 16, 8)])
def test_gemm_k_split_fixup(ctx, oracle, M, K, T, qtype):
    """Matmuls the planner splits over K ranges (few output tiles: the ring
    kernel's partial planes, then gemm_reduce_kernel's sum in range order),
    Q4_K, Q6_K, Q5_K and Q8_0. The result matches the oracle; a graph of the
    call replayed three times, with eager calls of another split shape between
    the replays, gives the eager result bit for bit every time."""
    from spq4k.hip import DeviceArray, Graph
    rng = np.random.default_rng(M + K + T + qtype)
    Wf = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    X = rng.standard_normal((T, K)).astype(np.float32)
    W = oracle.quantize_q8_0(Wf, ref_encoder=True) if qtype == 8 else oracle.quantize(qtype, Wf)
    Wd = ctx.upload(W, M, K, type=qtype)
    xd = DeviceArray.from_host(X)
    yd = DeviceArray((T, M), np.float32)
    ctx.mul_mat_dev(Wd, xd.ptr, yd.ptr, T)
    ctx.synchronize()
    eager = yd.to_host()
    if qtype == 8:
        exp = oracle.mul_mat_q8_0(W, M, K, X)
        _check(eager, exp, f"Q8_0 M={M} K={K} T={T}")
    else:
        _check(eager, oracle.mul_mat_type(qtype, W, M, K, X), f"type {qtype} M={M} K={K} T={T}",
               oracle.mul_mat_dq_f64(qtype, W, M, K, X))
    # another split shape between the replays
    M2, K2, T2 = 512, 12288, 20
    W2 = oracle.quantize_q4K((rng.standard_normal((M2, K2)) * 0.02).astype(np.float32))
    W2d = ctx.upload(W2, M2, K2)
    X2 = rng.standard_normal((T2, K2)).astype(np.float32)
    exp2 = ctx.mul_mat(W2d, X2)
    yd.fill_byte(0)
    with Graph.capture(ctx.stream) as g:
        ctx.mul_mat_dev(Wd, xd.ptr, yd.ptr, T)
    for rep in range(3):
        yd.fill_byte(0)
        g.launch()
        ctx.synchronize()
        got = yd.to_host()
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep} differs from the eager call"
        assert np.array_equal(ctx.mul_mat(W2d, X2).view(np.uint32), exp2.view(np.uint32)), f"eager call after replay {rep}"
    del g
    for a in (Wd, W2d, xd, yd):
        a.free()

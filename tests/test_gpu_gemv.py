"""GPU parity of the fused Q4_K GEMV (T <= 8) against the CPU oracle.

Integer sub-block sums: bit-exact against the oracle's brute force.
Outputs: every element within the reference tolerance (close_enough, 1e-4
relative or 1e-5 absolute; tests/desktop/test_sp_kernels.cpp:34-48) of the
oracle's restatement of ggml's x86 path, which is bit-identical to the
reference's own ggml_vec_dot_q4_K_q8_K (pinned in test_oracle_golden.py)."""
import numpy as np
import pytest

from _oracle import close_enough, parity_ok

pytestmark = pytest.mark.gpu


def _weights(oracle, rng, M, K, scale=0.02):
    return oracle.quantize_q4K((rng.standard_normal((M, K)) * scale).astype(np.float32))


def _check(got, exp, what, exact=None):
    """close_enough of the oracle (ggml's x86 order); with `exact`, the parity
    bar's either-or: of the oracle or of the dequant-then-dot value"""
    ok = close_enough(got, exp) if exact is None else parity_ok(got, exp, exact)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; first {tuple(i)} "
                             f"got {got[tuple(i)]!r} exp {exp[tuple(i)]!r}")


def test_subblock_sums_exact(ctx, oracle):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(11)
    for M, K in ((64, 4096), (37, 768), (16, 27648)):
        W = _weights(oracle, rng, M, K)
        x = rng.standard_normal(K).astype(np.float32)
        q8 = oracle.quantize_q8K(x)
        Wd = DeviceArray.from_host(W)
        xd = DeviceArray.from_host(x)
        Sd = DeviceArray(M * (K // 256) * 8, np.int32)
        ctx.subblock_sums(Wd.ptr, M, K, xd.ptr, Sd.ptr)
        ctx.synchronize()
        got = Sd.to_host().reshape(M, -1)
        rb = K // 256 * 144
        for r in range(M):
            exp = oracle.subblock_sums(K, W[r * rb:(r + 1) * rb], q8)
            np.testing.assert_array_equal(got[r], exp, err_msg=f"row {r} M={M} K={K}")


@pytest.mark.parametrize("M,K", [(4096, 4096), (1024, 4096), (100, 768), (64, 2048), (1024, 12288), (512, 27648)])
def test_gemv_t1(ctx, oracle, M, K):
    rng = np.random.default_rng(M * 31 + K)
    W = _weights(oracle, rng, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K)
    got = ctx.mul_mat(Wd, x)
    exp = oracle.mul_mat(W, M, K, x)
    _check(got, exp, f"gemv M={M} K={K}", oracle.mul_mat_dq_f64(12, W, M, K, x))


@pytest.mark.parametrize("sdot4", [False, True])
@pytest.mark.parametrize("T", [2, 3, 4, 5, 8])
def test_gemv_batched(ctx, oracle, T, sdot4):
    """T <= 8 through spq4k_gemv: the sdot4 kernel below 4 tokens and the
    matrix-core kernel from 4 (sdot4=True keeps the sdot4 kernel for every T,
    SPQ4K_GEMV_MFMA_MIN_T=9)."""
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMV_MFMA_MIN_T": 9}) if sdot4 else ctx
    try:
        rng = np.random.default_rng(100 + T)
        for M, K in ((768, 2048), (100, 5120)):
            W = _weights(oracle, rng, M, K)
            x = rng.standard_normal((T, K)).astype(np.float32)
            Wd = c.upload(W, M, K)
            _check(c.mul_mat(Wd, x), oracle.mul_mat(W, M, K, x), f"gemv T={T} M={M} K={K} sdot4={sdot4}")
            Wd.free()
    finally:
        if sdot4:
            c.close()


@pytest.mark.parametrize("sdot4", [False, True])
def test_gemv_large_k_batched(ctx, oracle, sdot4):
    # K = 27648 with T = 8: several LDS chunks per K split (sdot4 kernel) or
    # sixteen waves splitting K (matrix cores)
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMV_MFMA_MIN_T": 9}) if sdot4 else ctx
    try:
        rng = np.random.default_rng(7)
        M, K, T = 128, 27648, 8
        W = _weights(oracle, rng, M, K)
        x = rng.standard_normal((T, K)).astype(np.float32)
        Wd = c.upload(W, M, K)
        _check(c.mul_mat(Wd, x), oracle.mul_mat(W, M, K, x), f"gemv K=27648 T=8 sdot4={sdot4}")
        Wd.free()
    finally:
        if sdot4:
            c.close()


def test_gemv_multi_matches_single(ctx, oracle):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(5)
    K = 4096
    shapes = (512, 128, 128)
    Ws = [_weights(oracle, rng, M, K) for M in shapes]
    x = rng.standard_normal(K).astype(np.float32)
    wd = [ctx.upload(w, M, K) for w, M in zip(Ws, shapes)]
    xd = DeviceArray.from_host(x)
    ys = [DeviceArray.from_host(np.full(M, np.nan, np.float32)) for M in shapes]
    ctx.gemv_multi_dev(wd, xd.ptr, [y.ptr for y in ys], 1)
    ctx.synchronize()
    for w, M, y in zip(Ws, shapes, ys):
        _check(y.to_host()[None], oracle.mul_mat(w, M, K, x[None]), f"multi M={M}")


def test_gemv_repeatable(ctx, oracle):
    # split-K partial sums are combined in a fixed order: bit-identical reruns
    rng = np.random.default_rng(9)
    M, K = 256, 4096
    W = _weights(oracle, rng, M, K)
    Wd = ctx.upload(W, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    a = ctx.mul_mat(Wd, x)
    for _ in range(5):
        np.testing.assert_array_equal(ctx.mul_mat(Wd, x), a)

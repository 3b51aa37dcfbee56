"""GPU parity of the matrix-core prefill matmul (spq4k_gemm / mul_mat, T > 8).

Against the reference's own GGML_OP_MUL_MAT outputs (golden vectors) and the
CPU oracle (ggml's x86 order, pinned bit-exact to the reference) on Q8_K
activations. Tolerance: close_enough, 1e-4 relative or 1e-5 absolute
(tests/desktop/test_sp_kernels.cpp:34-48)."""
import os

import numpy as np
import pytest

from _oracle import close_enough

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def _check(got, exp, what):
    ok = close_enough(got, exp)
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
    _check(ctx.mul_mat(Wd, X), oracle.mul_mat(W, M, K, X), f"gemm M={M} K={K} T={T}")


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

"""The oracle's restatement of the operations either side of the matvec
(oracle/fusion_oracle.c) pinned against the reference's own ggml graphs
(oracle/_ref): ggml_rms_norm + ggml_mul bit for bit; the dense SwiGLU front
half (two mul_mats, ggml_silu, ggml_mul) within the silu's last bits (the x86
kernels evaluate exp with their own vector code); and the mathematics of silu."""
import numpy as np
import pytest

from _oracle import TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0


@pytest.mark.parametrize("K,T,scale,eps", [(4096, 3, 1.0, 1e-6), (5120, 2, 1e-3, 1e-5), (768, 5, 30.0, 1e-6),
                                           (12288, 1, 1.0, 0.0), (96, 4, 1e4, 1e-6)])
def test_rms_norm_bits(oracle, ref, K, T, scale, eps):
    rng = np.random.default_rng(K + T)
    X = (rng.standard_normal((T, K)) * scale).astype(np.float32)
    X[0, ::7] = 0.0
    if T > 1:
        X[1, :5] *= 1000.0     # outliers
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    got = oracle.rms_norm(X, w, eps)
    exp = ref.rms_norm(X, w, eps)
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_rms_norm_math(oracle):
    """Closed forms: a constant row c normalises to sign(c) (eps = 0); the
    output's mean square is 1 / (1 + eps / mean(x^2)); w multiplies."""
    K = 1024
    for c in (3.0, -0.5, 1e-3):
        y = oracle.rms_norm(np.full((1, K), c, np.float32), np.ones(K, np.float32), 0.0)
        np.testing.assert_allclose(y, np.sign(c), rtol=2e-7)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, K)).astype(np.float32)
    for eps in (0.0, 1e-2, 1.0):
        y = oracle.rms_norm(x, None, eps).astype(np.float64)
        ms = (x.astype(np.float64) ** 2).mean(1)
        np.testing.assert_allclose((y ** 2).mean(1), ms / (ms + eps), rtol=1e-5)
    w = rng.standard_normal(K).astype(np.float32)
    np.testing.assert_array_equal(oracle.rms_norm(x, w, 1e-6), (oracle.rms_norm(x, None, 1e-6) * w).astype(np.float32))


def test_silu_math(oracle):
    g = np.array([0.0, 1e-20, -1e-20, 30.0, -30.0, 100.0, -100.0, 1.0, -1.0, 88.0, -88.0], np.float32)
    y = oracle.swiglu(g, np.ones_like(g))
    exp = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(y, exp, rtol=2e-7, atol=1e-37)
    assert y[0] == 0.0 and y[3] == pytest.approx(30.0, rel=1e-12) and abs(y[4]) < 3e-12
    u = np.linspace(-3, 3, g.size).astype(np.float32)
    np.testing.assert_array_equal(oracle.swiglu(g, u), (y * u).astype(np.float32))


@pytest.mark.parametrize("qtype,norm", [(TYPE_Q4_K, True), (TYPE_Q4_K, False), (TYPE_Q6_K, True), (TYPE_Q8_0, True)])
def test_swiglu_ffn_against_ggml_graph(oracle, ref, qtype, norm):
    rng = np.random.default_rng(11 + qtype)
    M, K, T = 96, 512, 3
    enc = (lambda x: oracle.quantize_q8_0(x, ref_encoder=True)) if qtype == TYPE_Q8_0 else \
        (lambda x: oracle.quantize(qtype, x))
    Wg = enc((rng.standard_normal((M, K)) * 0.05).astype(np.float32))
    Wu = enc((rng.standard_normal((M, K)) * 0.05).astype(np.float32))
    X = rng.standard_normal((T, K)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32) if norm else None
    xb = oracle.rms_norm(X, w, 1e-6) if norm else X
    mm = (lambda W: oracle.mul_mat_q8_0(W, M, K, xb)) if qtype == TYPE_Q8_0 else \
        (lambda W: oracle.mul_mat_type(qtype, W, M, K, xb))
    got = oracle.swiglu(mm(Wg), mm(Wu))
    exp = ref.swiglu_ffn(qtype, Wg, Wu, M, K, X, w, 1e-6)
    np.testing.assert_allclose(got, exp, rtol=3e-6, atol=1e-30)

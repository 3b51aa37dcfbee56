"""Pins the oracle's dequant-then-dot functions (CPU only).

- or_dequantize_row_q8K: bit for bit against the reference's own
  dequantize_row_q8_K (ggml-quants.c:2731-2740) through golden vectors, and
  live when oracle/_ref is built.
- or_mul_mat_dq_f64_type, the second form of the parity bar (sum of
  dequant(W) * dequant(Q(x)) in double): against an exact rational sum of the
  reference's own dequantised operands on small inputs (a wrong index, sign
  or dropped term changes the sum), and against the reference's
  ggml_vec_dot_q4_K_q8_K, which computes the same quantity with integer
  sub-block sums and an fp32 combine.
- or_mul_mat_dequant_f64_type (fp32 activations as given): the same exact
  rational check.
- or_beast_matvec_type: bit for bit against the reference's beast_matvec
  (desktop/beast_canyon/sp_beast_canyon.c:1122-1134) compiled from its source
  (golden vectors; live when oracle/_ref/beast is built), plus closed forms.
  For Q5_K and Q6_K rows it runs beast_matvec's loop over the format's own
  dequantiser (the reference's beast_dequant_q5_K / _q6_K read other bits,
  which test_reference_q5k_q6k_dequant_is_not_the_format records): one-hot
  inputs give the pinned dequantisers' weights bit for bit, and the loop is
  the one the Q4_K / Q8_0 goldens pin.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

from _oracle import BEAST_SO, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, BeastRef, ref_library_path

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "dq_golden.npz"))


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_dequant_q8K_golden(oracle):
    q, y = G["dq8_q"], G["dq8_y"]
    assert np.array_equal(_bits(oracle.dequant_q8K(q, y.size)), _bits(y))


def test_dequant_q8K_live(oracle, ref):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096), rng.standard_normal(256) * 1e-30,
                        np.zeros(256)]).astype(np.float32)
    q = oracle.quantize_q8K(x)
    assert np.array_equal(_bits(oracle.dequant_q8K(q, x.size)), _bits(ref.dequant_q8K(q, x.size)))


def _exact_dot(a, b):
    return float(sum((Fraction(float(u)) * Fraction(float(v)) for u, v in zip(a, b)), Fraction(0)))


def _weights(oracle, qtype, M, K, rng):
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    if qtype == TYPE_Q8_0:
        return oracle.quantize_q8_0(w, ref_encoder=True)
    return oracle.quantize(qtype, w)


def _dequant(oracle, qtype, W, K):
    return oracle.dequant_q8_0(W, K) if qtype == TYPE_Q8_0 else oracle.to_float(qtype, W, K)


def _act(oracle, qtype, x):
    """dequant(Q(x)): the activation the CPU backend dots for this weight type"""
    if qtype == TYPE_Q8_0:
        return oracle.dequant_q8_0(oracle.quantize_q8_0(x), x.size)
    return oracle.dequant_q8K(oracle.quantize_q8K(x), x.size)


@pytest.mark.parametrize("qtype", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
def test_dq_f64_exact_on_small_inputs(oracle, qtype):
    rng = np.random.default_rng(qtype)
    M, K, T = 3, 512, 2
    W = _weights(oracle, qtype, M, K, rng)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = oracle.mul_mat_dq_f64(qtype, W, M, K, X)
    raw = oracle.mul_mat_dequant_f64(qtype, W, M, K, X)
    rb = W.size // M
    for r in range(M):
        w = _dequant(oracle, qtype, W[r * rb:(r + 1) * rb], K)
        for t in range(T):
            # a double sum of K terms: within K * 2^-53 of the sum of |terms|
            for val, xs in ((got[t, r], _act(oracle, qtype, X[t])), (raw[t, r], X[t])):
                exact = _exact_dot(w, xs)
                bound = K * 2.0 ** -53 * float(np.sum(np.abs(w.astype(np.float64) * xs)))
                assert abs(val - exact) <= bound, (qtype, r, t, val, exact)


def test_dq_f64_uses_the_reference_operands(oracle, ref):
    """The reference's own dequantize_row_q4_K and quantize_row_q8_K /
    dequantize_row_q8_K give the same exact sum."""
    rng = np.random.default_rng(17)
    M, K = 2, 768
    W = ref.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32), M, K)
    x = rng.standard_normal(K).astype(np.float32)
    got = oracle.mul_mat_dq_f64(TYPE_Q4_K, W, M, K, x)[0]
    xs = ref.dequant_q8K(ref.quantize_q8K(x), K)
    for r in range(M):
        w = ref.dequant(W[r * (K // 256 * 144):(r + 1) * (K // 256 * 144)], K)
        exact = _exact_dot(w, xs)
        assert abs(got[r] - exact) <= K * 2.0 ** -53 * float(np.sum(np.abs(w.astype(np.float64) * xs)))


@pytest.mark.parametrize("K", [256, 4096, 12288])
def test_dq_f64_agrees_with_vec_dot(oracle, K):
    """ggml_vec_dot_q4_K_q8_K (x86 order, pinned to the reference) sums the same
    products with exact integer parts and an fp32 combine: on data without
    heavy cancellation the two agree to a few fp32 ulps."""
    rng = np.random.default_rng(K)
    M = 64
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((2, K)).astype(np.float32)
    vd = oracle.mul_mat(W, M, K, X).astype(np.float64)
    dq = oracle.mul_mat_dq_f64(TYPE_Q4_K, W, M, K, X)
    assert np.linalg.norm(vd - dq) <= 1e-6 * np.linalg.norm(dq)
    assert np.quantile(np.abs(vd - dq) / np.abs(dq), 0.9) < 1e-5


@pytest.mark.parametrize("tag,qtype", [("q4k", TYPE_Q4_K), ("q8_0", TYPE_Q8_0)])
@pytest.mark.parametrize("K", [256, 4096, 12288])
def test_beast_golden(oracle, tag, qtype, K):
    W, x, y = G[f"beast_{tag}_{K}_W"], G[f"beast_{tag}_{K}_x"], G[f"beast_{tag}_{K}_y"]
    assert np.array_equal(_bits(oracle.beast_matvec(qtype, W, y.size, K, x)), _bits(y))


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference's beast_matvec) not built")
@pytest.mark.parametrize("qtype", [TYPE_Q4_K, TYPE_Q8_0])
def test_beast_live(oracle, qtype):
    b = BeastRef()
    rng = np.random.default_rng(qtype + 100)
    for M, K, dist in ((32, 4096, "n"), (8, 27648, "t"), (16, 768, "big")):
        w = rng.standard_t(4, (M, K)) * 0.02 if dist == "t" else rng.standard_normal((M, K)) * (5.0 if dist == "big" else 0.02)
        W = oracle.quantize_q8_0(w.astype(np.float32), ref_encoder=True) if qtype == TYPE_Q8_0 else \
            oracle.quantize_q4K(w.astype(np.float32))
        x = rng.standard_normal(K).astype(np.float32)
        assert np.array_equal(_bits(oracle.beast_matvec(qtype, W, M, K, x)), _bits(b.matvec(qtype, W, M, K, x)))


def test_beast_closed_forms(oracle):
    rng = np.random.default_rng(9)
    M, K = 4, 1024
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    rb = K // 256 * 144
    wd = np.stack([oracle.dequant(W[r * rb:(r + 1) * rb], K) for r in range(M)])
    # one nonzero input: one rounded product
    x = np.zeros(K, np.float32)
    x[700] = np.float32(1.7)
    assert np.array_equal(_bits(oracle.beast_matvec(TYPE_Q4_K, W, M, K, x)), _bits(wd[:, 700] * np.float32(1.7)))
    # all-zero input
    assert not oracle.beast_matvec(TYPE_Q4_K, W, M, K, np.zeros(K, np.float32)).any()
    # the sum is taken in index order: an fp32 loop over the dequantised row
    x = rng.standard_normal(K).astype(np.float32)
    for r in range(M):
        s = np.float32(0)
        for c in range(K):
            s = np.float32(s + np.float32(wd[r, c] * x[c]))
        assert _bits(oracle.beast_matvec(TYPE_Q4_K, W, M, K, x))[r] == _bits(np.array([s]))[0]


@pytest.mark.parametrize("qtype", [TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_Q4_K])
def test_beast_one_hot_is_the_format_dequant(oracle, qtype):
    """a one-hot input picks one weight of each row, times 1.0 plus zeros:
    the format's dequantised weights (or_dequantize_row_*, pinned to the
    reference's ggml by the golden vectors) bit for bit, at every position
    class of the block (sub-block and nibble boundaries)"""
    rng = np.random.default_rng(qtype)
    M, K = 6, 512
    W = oracle.quantize(qtype, (rng.standard_normal((M, K)) * 0.05).astype(np.float32))
    wd = oracle.to_float(qtype, W, M * K).reshape(M, K)
    for c in (0, 15, 16, 31, 32, 63, 64, 100, 127, 128, 191, 200, 255, 256, 300, 511):
        x = np.zeros(K, np.float32)
        x[c] = 1.0
        # + 0.0: a weight of -0 (a negative scale times q = 0) sums to +0 from 0.0
        assert np.array_equal(_bits(oracle.beast_matvec(qtype, W, M, K, x)), _bits(wd[:, c] + np.float32(0))), \
            f"column {c}"
    # and the sum is within fp32 reassociation of the exact dequant-then-dot
    x = rng.standard_normal(K).astype(np.float32)
    exact = oracle.mul_mat_dequant_f64(qtype, W, M, K, x[None, :])[0]
    got = oracle.beast_matvec(qtype, W, M, K, x).astype(np.float64)
    bound = 2 * K * np.finfo(np.float32).eps * (np.abs(wd.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    assert (np.abs(got - exact) <= bound).all()


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference's beast_matvec) not built")
def test_reference_q5k_q6k_dequant_is_not_the_format(oracle):
    """why the format's dequantiser is followed for Q5_K / Q6_K rows: the
    reference's beast_matvec on those rows (beast_dequant_q5_K / _q6_K,
    sp_beast_canyon.c:1025-1085) does not return the format's weights for
    one-hot inputs, where for Q4_K and Q8_0 it does"""
    b = BeastRef()
    rng = np.random.default_rng(3)
    M, K = 4, 256
    differs = {}
    for qtype in (TYPE_Q4_K, TYPE_Q8_0, TYPE_Q5_K, TYPE_Q6_K):
        W = oracle.quantize(qtype, (rng.standard_normal((M, K)) * 0.05).astype(np.float32))
        wd = oracle.to_float(qtype, W, M * K).reshape(M, K)
        n = 0
        for c in range(K):
            x = np.zeros(K, np.float32)
            x[c] = 1.0
            n += int(not np.array_equal(b.matvec(qtype, W, M, K, x), wd[:, c]))
        differs[qtype] = n
    assert differs[TYPE_Q4_K] == 0 and differs[TYPE_Q8_0] == 0
    assert differs[TYPE_Q5_K] > K // 4 and differs[TYPE_Q6_K] > K // 4, differs

"""The Q8_0 oracle (oracle/q8_0_oracle.c) pinned two ways.

1. Golden vectors written by the reference's own ggml CPU code
   (tests/golden/q8_0_golden.npz): the model-file encoder (quantize_q8_0),
   dequantize_row_q8_0, the CPU backend's activation quantiser
   (quantize_row_q8_0, x86), ggml_vec_dot_q8_0_q8_0 (x86 and _generic),
   GGML_OP_MUL_MAT and GGML_OP_MUL_MAT_ID, each reproduced bit for bit.
2. The mathematics: the block layout decoded by numpy, brute-force integer
   block sums, the exact combine against both float orders, and the two
   roundings (the encoder's half away from zero, the activation quantiser's
   half to even) on exact ties."""
import os

import numpy as np
import pytest

from _oracle import Q8_0, TYPE_Q8_0

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q8_0_golden.npz"))


def _fields(q):
    b = q.reshape(-1, Q8_0)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    qs = b[:, 2:34].view(np.int8).astype(np.int64)
    return d, qs


def test_numpy_layout_matches_reference_dequant():
    d, qs = _fields(GOLD["deq_q"])
    y = (qs.astype(np.float32) * d[:, None]).astype(np.float32).ravel()
    np.testing.assert_array_equal(y.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_encoder_bytes(oracle):
    got = oracle.quantize_q8_0(GOLD["enc_x"], ref_encoder=True)
    np.testing.assert_array_equal(got, GOLD["enc_q"])


def test_dequant_bits(oracle):
    got = oracle.dequant_q8_0(GOLD["deq_q"], GOLD["deq_y"].size)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_activation_quantiser_bits(oracle):
    np.testing.assert_array_equal(oracle.quantize_q8_0(GOLD["act_x"]), GOLD["act_q"])


@pytest.mark.parametrize("order,key", [("avx2", "vd_avx2"), ("generic", "vd_generic")])
def test_vec_dot_bits(oracle, order, key):
    ow = oa = 0
    for i, K in enumerate(GOLD["vd_K"]):
        n = K // 32 * Q8_0
        w, a = GOLD["vd_w"][ow:ow + n], GOLD["vd_a"][oa:oa + n]
        ow += n
        oa += n
        got = np.float32(oracle.vec_dot_q8_0(int(K), w, a, order))
        assert got.view(np.uint32) == GOLD[key][i].view(np.uint32), (i, K, got, GOLD[key][i])


@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_bits(oracle, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = oracle.mul_mat_q8_0(GOLD["mm_W"], M, K, GOLD[f"mm_X{T}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mm_Y{T}"].view(np.uint32))


@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_bits(oracle, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    got = oracle.mul_mat_id_q8_0(GOLD["mmid_bank"], M, K, E, GOLD[f"mmid_X_{tag}"], GOLD[f"mmid_ids_{tag}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mmid_Y_{tag}"].view(np.uint32))


# ---- mathematics ------------------------------------------------------------------------
def test_rounding_of_exact_ties(oracle):
    """A block whose largest |x| is 127 has scale 1 in both quantisers, so
    x = n + 0.5 is an exact tie: the activation quantiser (x86 round, half to
    even) and the model-file encoder (roundf, half away from zero) differ."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, -126.5]
    _, act = _fields(oracle.quantize_q8_0(x))
    _, enc = _fields(oracle.quantize_q8_0(x, ref_encoder=True))
    np.testing.assert_array_equal(act[0, 1:9], [2, -2, 0, 0, 2, -2, 4, -126])
    np.testing.assert_array_equal(enc[0, 1:9], [3, -3, 1, -1, 2, -2, 4, -127])
    assert act[0, 0] == enc[0, 0] == 127


def test_quantiser_invariants(oracle):
    rng = np.random.default_rng(81)
    x = (rng.standard_normal(32 * 500) * np.repeat(10.0 ** rng.integers(-3, 3, 500), 32)).astype(np.float32)
    for ref_encoder in (False, True):
        d, qs = _fields(oracle.quantize_q8_0(x, ref_encoder))
        xb = x.reshape(-1, 32)
        amax = np.abs(xb).max(1)
        np.testing.assert_array_equal(d, (amax / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32))
        assert (np.abs(qs) <= 127).all()
        assert (np.abs(qs).max(1) == 127).all()                     # the largest value maps to +-127
        err = np.abs(xb - qs * (amax / 127)[:, None])
        assert (err <= (amax / 127)[:, None] * 0.5 * (1 + 1e-5)).all()


def test_block_sums_and_exact_combine(oracle):
    rng = np.random.default_rng(82)
    for K in (32, 4096, 27648):
        w = oracle.quantize_q8_0((rng.standard_normal(K) * 0.02).astype(np.float32), ref_encoder=True)
        a = oracle.quantize_q8_0(rng.standard_normal(K).astype(np.float32))
        dw, qw = _fields(w)
        da, qa = _fields(a)
        S = (qw * qa).sum(1)
        np.testing.assert_array_equal(oracle.block_sums_q8_0(K, w, a), S)
        terms = dw.astype(np.float64) * da * S
        exact = float(terms.sum())
        assert oracle.vec_dot_q8_0_exact(K, w, a) == pytest.approx(exact, rel=1e-12, abs=1e-12)
        for order in ("avx2", "generic"):
            assert abs(oracle.vec_dot_q8_0(K, w, a, order) - exact) <= 1e-6 * float(np.abs(terms).sum())


def test_live_reference_random(oracle, ref):
    rng = np.random.default_rng(2027)
    M, K = 24, 2048
    x = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    q = oracle.quantize_q8_0(x, ref_encoder=True)
    np.testing.assert_array_equal(q, ref.quantize_type(TYPE_Q8_0, x, M, K))
    a = rng.standard_normal((3, K)).astype(np.float32)
    np.testing.assert_array_equal(oracle.quantize_q8_0(a), ref.quantize_q8_0_act(a))
    np.testing.assert_array_equal(oracle.mul_mat_q8_0(q, M, K, a).view(np.uint32),
                                  ref.mul_mat(q, M, K, a, qtype=TYPE_Q8_0).view(np.uint32))

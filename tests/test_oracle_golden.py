"""The CPU oracle against golden vectors written by the reference itself.

tests/golden/q4k_golden.npz holds outputs of the reference's own ggml CPU code
(compiled from /root/reference by oracle/Makefile; see gen_golden.py). Every
oracle function must reproduce them bit for bit. Where oracle/_ref is built
(the development container) the oracle is also checked against the live
reference on fresh random inputs."""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q4k_golden.npz"))


def test_encoder_bytes(oracle):
    x = GOLD["enc_x"]
    got = oracle.quantize_q4K(x)
    exp = GOLD["enc_q"]
    bad = np.nonzero((got.reshape(-1, 144) != exp.reshape(-1, 144)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} Q4_K blocks differ from quantize_q4_K, first {bad[:5]}"


def test_dequant_bits(oracle):
    q = GOLD["deq_q"]
    got = oracle.dequant(q, GOLD["deq_y"].size)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_q8k_blocks(oracle):
    got = oracle.quantize_q8K(GOLD["q8_x"]).reshape(-1, 292)
    np.testing.assert_array_equal(got, GOLD["q8_y"].reshape(-1, 292))


@pytest.mark.parametrize("order,key", [("avx2", "vd_avx2"), ("generic", "vd_generic")])
def test_vec_dot_bits(oracle, order, key):
    Ks = GOLD["vd_K"]
    o4 = o8 = 0
    for i, K in enumerate(Ks):
        n4, n8 = K // 256 * 144, K // 256 * 292
        w = GOLD["vd_q4"][o4:o4 + n4]
        a = GOLD["vd_q8"][o8:o8 + n8]
        o4 += n4
        o8 += n8
        got = np.float32(oracle.vec_dot(int(K), w, a, order))
        assert got.view(np.uint32) == GOLD[key][i].view(np.uint32), (i, K, got, GOLD[key][i])


@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_bits(oracle, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = oracle.mul_mat(GOLD["mm_W"], M, K, GOLD[f"mm_X{T}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mm_Y{T}"].view(np.uint32))


@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_bits(oracle, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    got = oracle.mul_mat_id(GOLD["mmid_bank"], M, K, E, GOLD[f"mmid_X_{tag}"], GOLD[f"mmid_ids_{tag}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mmid_Y_{tag}"].view(np.uint32))


# ---- live reference (only where oracle/_ref is built) -----------------------
def test_live_reference_random(oracle, ref):
    rng = np.random.default_rng(2024)
    M, K = 24, 2048
    x = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    q_o = oracle.quantize_q4K(x)
    q_r = ref.quantize_q4K(x, M, K)
    np.testing.assert_array_equal(q_o, q_r)
    np.testing.assert_array_equal(oracle.dequant(q_o, M * K).view(np.uint32), ref.dequant(q_o, M * K).view(np.uint32))
    a = rng.standard_normal((3, K)).astype(np.float32)
    np.testing.assert_array_equal(oracle.quantize_q8K(a), ref.quantize_q8K(a))
    np.testing.assert_array_equal(oracle.mul_mat(q_o, M, K, a).view(np.uint32), ref.mul_mat(q_o, M, K, a).view(np.uint32))

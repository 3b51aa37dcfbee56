"""The Q5_K oracle (oracle/q5k_oracle.c) pinned two ways.

1. Golden vectors written by the reference's own ggml CPU code
   (tests/golden/q5k_golden.npz, from gen_golden.py): quantize_q5_K bytes,
   dequantize_row_q5_K, ggml_vec_dot_q5_K_q8_K (x86 kernel and _generic),
   GGML_OP_MUL_MAT and GGML_OP_MUL_MAT_ID through ggml_graph_compute, each
   reproduced bit for bit.
2. What the mathematics fixes, independently of the C code: a numpy decoder of
   the block layout (itself pinned against the reference's dequantisation)
   gives brute-force integer sub-block sums and the exact dot product;
   closed-form blocks; encoder invariants."""
import os

import numpy as np
import pytest

from _oracle import Q5K, TYPE_Q5_K
from test_oracle_math import _pack_scales

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q5k_golden.npz"))
QK = 256


# ---- numpy statement of the block layout (ggml-common.h:334-346) ------------------
def _q5_values(w):
    """(nblocks, 256) 5-bit values in element order: element 64 g + 32 h + l is
    nibble h of qs[32 g + l] plus 16 times bit 2 g + h of qh[l]."""
    b = w.reshape(-1, Q5K).astype(np.int64)
    qh = b[:, 16:48]
    qs = b[:, 48:176].reshape(-1, 4, 32)
    out = np.zeros((b.shape[0], 4, 2, 32), np.int64)
    for g in range(4):
        out[:, g, 0, :] = (qs[:, g] & 15) + 16 * ((qh >> (2 * g)) & 1)
        out[:, g, 1, :] = (qs[:, g] >> 4) + 16 * ((qh >> (2 * g + 1)) & 1)
    return out.reshape(-1, QK)


def _scales(w):
    b = w.reshape(-1, Q5K)[:, 4:16].astype(np.int64)
    sc = np.zeros((b.shape[0], 8), np.int64)
    m = np.zeros((b.shape[0], 8), np.int64)
    sc[:, :4] = b[:, 0:4] & 63
    m[:, :4] = b[:, 4:8] & 63
    sc[:, 4:] = (b[:, 8:12] & 15) | ((b[:, 0:4] >> 6) << 4)
    m[:, 4:] = (b[:, 8:12] >> 4) | ((b[:, 4:8] >> 6) << 4)
    return sc, m


def _dmin(w):
    h = w.reshape(-1, Q5K)[:, 0:4].copy().view(np.float16).astype(np.float32)
    return h[:, 0], h[:, 1]


def _q8_fields(a):
    b = a.reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8).astype(np.int64)
    bs = b[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, qs, bs


def _block(d16, dmin16, sc, m, q):
    """One 176-byte block from 8 scales, 8 mins (6-bit) and 256 five-bit values."""
    q = np.asarray(q, np.int64).reshape(4, 2, 32)
    blk = np.zeros(Q5K, np.uint8)
    blk[0:2] = np.array([d16], np.uint16).view(np.uint8)
    blk[2:4] = np.array([dmin16], np.uint16).view(np.uint8)
    blk[4:16] = _pack_scales(np.asarray(sc, np.uint8), np.asarray(m, np.uint8))
    for g in range(4):
        blk[48 + 32 * g:48 + 32 * g + 32] = ((q[g, 0] & 15) | ((q[g, 1] & 15) << 4)).astype(np.uint8)
        blk[16:48] |= (((q[g, 0] >> 4) << (2 * g)) | ((q[g, 1] >> 4) << (2 * g + 1))).astype(np.uint8)
    return blk


def test_numpy_layout_matches_reference_dequant():
    q = GOLD["deq_q"]
    sc, m = _scales(q)
    d, dmin = _dmin(q)
    d1 = (d[:, None] * np.repeat(sc, 32, axis=1).astype(np.float32)).astype(np.float32)
    m1 = (dmin[:, None] * np.repeat(m, 32, axis=1).astype(np.float32)).astype(np.float32)
    y = ((d1 * _q5_values(q).astype(np.float32)).astype(np.float32) - m1).astype(np.float32).ravel()
    np.testing.assert_array_equal(y.view(np.uint32), GOLD["deq_y"].view(np.uint32))


# ---- golden vectors ------------------------------------------------------------------
def test_encoder_bytes(oracle):
    got = oracle.quantize_q5K(GOLD["enc_x"]).reshape(-1, Q5K)
    exp = GOLD["enc_q"].reshape(-1, Q5K)
    bad = np.nonzero((got != exp).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} Q5_K blocks differ from quantize_q5_K, first {bad[:5]}"


def test_dequant_bits(oracle):
    got = oracle.dequant_q5K(GOLD["deq_q"], GOLD["deq_y"].size)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


@pytest.mark.parametrize("order,key", [("avx2", "vd_avx2"), ("generic", "vd_generic")])
def test_vec_dot_bits(oracle, order, key):
    o5 = o8 = 0
    for i, K in enumerate(GOLD["vd_K"]):
        n5, n8 = K // QK * Q5K, K // QK * 292
        w, a = GOLD["vd_w"][o5:o5 + n5], GOLD["vd_q8"][o8:o8 + n8]
        o5 += n5
        o8 += n8
        got = np.float32(oracle.vec_dot_q5K(int(K), w, a, order))
        assert got.view(np.uint32) == GOLD[key][i].view(np.uint32), (i, K, got, GOLD[key][i])


@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_bits(oracle, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = oracle.mul_mat_type(TYPE_Q5_K, GOLD["mm_W"], M, K, GOLD[f"mm_X{T}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mm_Y{T}"].view(np.uint32))


@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_bits(oracle, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    got = oracle.mul_mat_id_type(TYPE_Q5_K, GOLD["mmid_bank"], M, K, E, GOLD[f"mmid_X_{tag}"],
                                 GOLD[f"mmid_ids_{tag}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mmid_Y_{tag}"].view(np.uint32))


# ---- closed forms and brute force ---------------------------------------------------
def test_dequant_closed_forms(oracle):
    rng = np.random.default_rng(51)
    q = (np.arange(QK) * 13 + 7) % 32               # distinct pattern: catches element order slips
    ones = np.ones(8, np.uint8)
    # d = 1, dmin = 0, scales 1: y = q (every high bit position reached)
    y = oracle.dequant_q5K(_block(0x3C00, 0, ones, np.zeros(8, np.uint8), q), QK)
    np.testing.assert_array_equal(y, q.astype(np.float32))
    # d = 1, dmin = 0: y = sc_j * q
    sc = np.arange(1, 9, dtype=np.uint8) * 7
    y = oracle.dequant_q5K(_block(0x3C00, 0, sc, np.zeros(8, np.uint8), q), QK)
    np.testing.assert_array_equal(y, (np.repeat(sc, 32) * q).astype(np.float32))
    # d = 0, dmin = 0.5: y = -0.5 * m_j
    m = np.arange(8, dtype=np.uint8) * 9
    y = oracle.dequant_q5K(_block(0, 0x3800, np.zeros(8, np.uint8), m, q), QK)
    np.testing.assert_array_equal(y, -(0.5 * np.repeat(m, 32)).astype(np.float32))
    # general: (d * sc) * q - (dmin * m), each step rounded once
    for _ in range(20):
        d16, dm16 = (int(v) for v in rng.integers(0x0400, 0x6000, 2))
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        qq = rng.integers(0, 32, QK)
        d = np.array([d16], np.uint16).view(np.float16).astype(np.float32)[0]
        dm = np.array([dm16], np.uint16).view(np.float16).astype(np.float32)[0]
        d1 = (d * np.repeat(sc, 32).astype(np.float32)).astype(np.float32)
        m1 = (dm * np.repeat(m, 32).astype(np.float32)).astype(np.float32)
        exp = ((d1 * qq.astype(np.float32)).astype(np.float32) - m1).astype(np.float32)
        y = oracle.dequant_q5K(_block(d16, dm16, sc, m, qq), QK)
        np.testing.assert_array_equal(y.view(np.uint32), exp.view(np.uint32))


def _weights(oracle, rng, K, kind):
    if kind == "enc":
        return oracle.quantize_q5K((rng.standard_normal(K) * 0.02).astype(np.float32))
    b = rng.integers(0, 256, size=(K // QK, Q5K), dtype=np.uint8)
    b[:, 1] &= 0x3B
    b[:, 3] &= 0x3B
    return b.ravel()


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_subblock_sums_brute_force(oracle, kind):
    rng = np.random.default_rng(52)
    for K in (256, 768, 4096):
        w = _weights(oracle, rng, K, kind)
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        _, qs, _ = _q8_fields(a)
        exp = (_q5_values(w) * qs).reshape(-1, 8, 32).sum(-1).ravel()
        np.testing.assert_array_equal(oracle.subblock_sums_q5K(K, w, a), exp)


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_exact_combine_and_float_orders(oracle, kind):
    rng = np.random.default_rng(53)
    for K in (256, 4096, 27648):
        w = _weights(oracle, rng, K, kind)
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        d8, qs, bs = _q8_fields(a)
        sc, m = _scales(w)
        d, dmin = _dmin(w)
        S = (_q5_values(w) * qs).reshape(-1, 8, 32).sum(-1)
        I = (sc * S).sum(1)
        Mt = (m * (bs[:, 0::2] + bs[:, 1::2])).sum(1)
        terms = d.astype(np.float64) * d8 * I - dmin.astype(np.float64) * d8 * Mt
        exact = float(terms.sum())
        assert oracle.vec_dot_q5K_exact(K, w, a) == pytest.approx(exact, rel=1e-12, abs=1e-12)
        scale = float((np.abs(d.astype(np.float64) * d8 * I) + np.abs(dmin.astype(np.float64) * d8 * Mt)).sum())
        for order in ("avx2", "generic"):
            assert abs(oracle.vec_dot_q5K(K, w, a, order) - exact) <= 1e-6 * scale


def test_mul_mat_id_is_gathered_mul_mat(oracle):
    rng = np.random.default_rng(54)
    E, M, K, T, k = 6, 40, 512, 4, 3
    bank = oracle.quantize_q5K((rng.standard_normal((E * M, K)) * 0.02).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    eb = M * K // QK * Q5K
    for ne11 in (1, k):
        X = rng.standard_normal((T, ne11, K)).astype(np.float32)
        Y = oracle.mul_mat_id_type(TYPE_Q5_K, bank, M, K, E, X, ids)
        for t in range(T):
            for s in range(k):
                e = ids[t, s]
                exp = oracle.mul_mat_type(TYPE_Q5_K, bank[e * eb:(e + 1) * eb], M, K, X[t, s % ne11][None])
                np.testing.assert_array_equal(Y[t, s], exp[0])


def test_encoder_reconstruction(oracle):
    rng = np.random.default_rng(55)
    x = (rng.standard_normal(QK * 256) * 0.02).astype(np.float32)
    q = oracle.quantize_q5K(x)
    y = oracle.dequant_q5K(q, x.size)
    # 5-bit affine per 32 values: RMS error well below the data's spread and
    # below the 4-bit encoder's
    e5 = np.sqrt(np.mean((y - x) ** 2))
    y4 = oracle.dequant(oracle.quantize_q4K(x), x.size)
    assert e5 < 0.05 * 0.02 and e5 < 0.6 * np.sqrt(np.mean((y4 - x) ** 2))


# ---- live reference (only where oracle/_ref is built) -----------------------
def test_live_reference_random(oracle, ref):
    rng = np.random.default_rng(2026)
    M, K = 24, 2048
    x = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    q_o = oracle.quantize_q5K(x)
    np.testing.assert_array_equal(q_o, ref.quantize_type(TYPE_Q5_K, x, M, K))
    np.testing.assert_array_equal(oracle.dequant_q5K(q_o, M * K).view(np.uint32),
                                  ref.dequant_type(TYPE_Q5_K, q_o, M * K).view(np.uint32))
    a = rng.standard_normal((3, K)).astype(np.float32)
    np.testing.assert_array_equal(oracle.mul_mat_type(TYPE_Q5_K, q_o, M, K, a).view(np.uint32),
                                  ref.mul_mat(q_o, M, K, a, qtype=TYPE_Q5_K).view(np.uint32))

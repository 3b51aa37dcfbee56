"""The Q6_K oracle (oracle/q6k_oracle.c) pinned two ways.

1. Golden vectors written by the reference's own ggml CPU code
   (tests/golden/q6k_golden.npz, from gen_golden.py): quantize_q6_K bytes,
   dequantize_row_q6_K, ggml_vec_dot_q6_K_q8_K (x86 kernel and _generic),
   GGML_OP_MUL_MAT and GGML_OP_MUL_MAT_ID through ggml_graph_compute. Each must
   be reproduced bit for bit.
2. What the mathematics fixes, independently of the C code: a numpy decoder of
   the block layout (itself pinned against the golden dequantisation) gives
   brute-force integer sub-block sums and the exact dot product; closed-form
   blocks; encoder invariants."""
import os

import numpy as np
import pytest

from _oracle import Q6K, TYPE_Q6_K

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q6k_golden.npz"))
QK = 256


# ---- numpy statement of the block layout (ggml-common.h:348-357) ------------------
def _q6_values(w):
    """(nblocks, 256) unsigned 6-bit values in element order. Element
    128 n + 32 h + l takes nibble h >> 1 of ql[64 n + 32 (h & 1) + l] and bits
    2h, 2h+1 of qh[32 n + l] as its top two bits."""
    b = w.reshape(-1, Q6K).astype(np.int64)
    ql = b[:, 0:128].reshape(-1, 2, 2, 32)          # [n][h & 1][l]
    qh = b[:, 128:192].reshape(-1, 2, 32)           # [n][l]
    out = np.zeros((b.shape[0], 2, 4, 32), np.int64)
    for h in range(4):
        nib = ql[:, :, h & 1, :]
        nib = (nib >> 4) if h >> 1 else (nib & 15)
        out[:, :, h, :] = nib | (((qh >> (2 * h)) & 3) << 4)
    return out.reshape(-1, QK)


def _fields(w):
    b = w.reshape(-1, Q6K)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32).ravel()
    return sc, d


def _q8_fields(a):
    b = a.reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8).astype(np.int64)
    bs = b[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, qs, bs


def _block(d16, sc, q):
    """One 210-byte block from 16 int8 scales and 256 six-bit values."""
    q = np.asarray(q, np.int64).reshape(2, 4, 32)
    blk = np.zeros(Q6K, np.uint8)
    for n in range(2):
        for h in range(4):
            idx = 64 * n + 32 * (h & 1) + np.arange(32)
            blk[idx] |= ((q[n, h] & 15) << (4 * (h >> 1))).astype(np.uint8)
            blk[128 + 32 * n + np.arange(32)] |= ((q[n, h] >> 4) << (2 * h)).astype(np.uint8)
    blk[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    blk[208:210] = np.array([d16], np.uint16).view(np.uint8)
    return blk


def test_numpy_layout_matches_reference_dequant():
    q = GOLD["deq_q"]
    sc, d = _fields(q)
    v = _q6_values(q)
    ds = (d[:, None] * np.repeat(sc, 16, axis=1).astype(np.float32)).astype(np.float32)
    y = (ds * (v - 32).astype(np.float32)).astype(np.float32).ravel()
    np.testing.assert_array_equal(y.view(np.uint32), GOLD["deq_y"].view(np.uint32))


# ---- golden vectors ------------------------------------------------------------------
def test_encoder_bytes(oracle):
    got = oracle.quantize_q6K(GOLD["enc_x"]).reshape(-1, Q6K)
    exp = GOLD["enc_q"].reshape(-1, Q6K)
    bad = np.nonzero((got != exp).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} Q6_K blocks differ from quantize_q6_K, first {bad[:5]}"


def test_dequant_bits(oracle):
    got = oracle.dequant_q6K(GOLD["deq_q"], GOLD["deq_y"].size)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


@pytest.mark.parametrize("order,key", [("avx2", "vd_avx2"), ("generic", "vd_generic")])
def test_vec_dot_bits(oracle, order, key):
    o6 = o8 = 0
    for i, K in enumerate(GOLD["vd_K"]):
        n6, n8 = K // QK * Q6K, K // QK * 292
        w, a = GOLD["vd_q6"][o6:o6 + n6], GOLD["vd_q8"][o8:o8 + n8]
        o6 += n6
        o8 += n8
        got = np.float32(oracle.vec_dot_q6K(int(K), w, a, order))
        assert got.view(np.uint32) == GOLD[key][i].view(np.uint32), (i, K, got, GOLD[key][i])


@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_bits(oracle, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = oracle.mul_mat_type(TYPE_Q6_K, GOLD["mm_W"], M, K, GOLD[f"mm_X{T}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mm_Y{T}"].view(np.uint32))


@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_bits(oracle, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    got = oracle.mul_mat_id_type(TYPE_Q6_K, GOLD["mmid_bank"], M, K, E, GOLD[f"mmid_X_{tag}"],
                                 GOLD[f"mmid_ids_{tag}"], order=1)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD[f"mmid_Y_{tag}"].view(np.uint32))


# ---- closed forms and brute force ---------------------------------------------------
def test_dequant_closed_forms(oracle):
    rng = np.random.default_rng(61)
    q = (np.arange(QK) * 11 + 5) % 64                # distinct pattern: catches element order slips
    # d = 1, every scale 1: y = q - 32
    y = oracle.dequant_q6K(_block(0x3C00, np.ones(16), q), QK)
    np.testing.assert_array_equal(y, (q - 32).astype(np.float32))
    # d = 1, scale j = j - 8 (signed): y = (j - 8) * (q - 32) on sub-block j
    sc = np.arange(16) - 8
    y = oracle.dequant_q6K(_block(0x3C00, sc, q), QK)
    np.testing.assert_array_equal(y, (np.repeat(sc, 16) * (q - 32)).astype(np.float32))
    # extremes: scale -128 and 127, q = 0 and 63
    for s, qq in ((-128, 0), (-128, 63), (127, 0), (127, 63)):
        y = oracle.dequant_q6K(_block(0x3C00, np.full(16, s), np.full(QK, qq)), QK)
        assert (y == np.float32(s * (qq - 32))).all()
    # general: (d * scale) * (q - 32), each product rounded once
    for _ in range(20):
        d16 = int(rng.integers(0x0400, 0x6000))
        sc = rng.integers(-128, 128, 16)
        qq = rng.integers(0, 64, QK)
        d = np.array([d16], np.uint16).view(np.float16).astype(np.float32)[0]
        ds = (d * np.repeat(sc, 16).astype(np.float32)).astype(np.float32)
        exp = (ds * (qq - 32).astype(np.float32)).astype(np.float32)
        y = oracle.dequant_q6K(_block(d16, sc, qq), QK)
        np.testing.assert_array_equal(y.view(np.uint32), exp.view(np.uint32))


def _random_pair(rng, K, kind):
    if kind == "rand":
        w = rng.integers(0, 256, size=(K // QK, Q6K), dtype=np.uint8)
        w[:, 209] &= 0x3B
        w = w.ravel()
    else:
        from _oracle import Oracle
        w = Oracle().quantize_q6K((rng.standard_normal(K) * 0.02).astype(np.float32))
    return w


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_subblock_sums_brute_force(oracle, kind):
    rng = np.random.default_rng(62)
    for K in (256, 768, 4096):
        w = _random_pair(rng, K, kind)
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        _, qs, _ = _q8_fields(a)
        exp = ((_q6_values(w) - 32) * qs).reshape(-1, 16, 16).sum(-1).ravel()
        np.testing.assert_array_equal(oracle.subblock_sums_q6K(K, w, a), exp)


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_exact_combine_and_float_orders(oracle, kind):
    rng = np.random.default_rng(63)
    for K in (256, 4096, 27648):
        w = _random_pair(rng, K, kind)
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        d8, qs, bs = _q8_fields(a)
        sc, d = _fields(w)
        S = ((_q6_values(w) - 32) * qs).reshape(-1, 16, 16).sum(-1)
        I = (sc * S).sum(1)
        # the offset form the x86 kernel uses: sum q*q8 - 32 * bsums
        S_u = (_q6_values(w) * qs).reshape(-1, 16, 16).sum(-1)
        np.testing.assert_array_equal(I, (sc * (S_u - 32 * bs)).sum(1))
        terms = d.astype(np.float64) * d8 * I
        exact = float(terms.sum())
        assert oracle.vec_dot_q6K_exact(K, w, a) == pytest.approx(exact, rel=1e-12, abs=1e-12)
        scale = float(np.abs(terms).sum())
        for order in ("avx2", "generic"):
            assert abs(oracle.vec_dot_q6K(K, w, a, order) - exact) <= 1e-6 * scale


def test_mul_mat_id_is_gathered_mul_mat(oracle):
    rng = np.random.default_rng(64)
    E, M, K, T, k = 6, 40, 512, 4, 3
    bank = oracle.quantize_q6K((rng.standard_normal((E * M, K)) * 0.02).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    eb = M * K // QK * Q6K
    for ne11 in (1, k):
        X = rng.standard_normal((T, ne11, K)).astype(np.float32)
        Y = oracle.mul_mat_id_type(TYPE_Q6_K, bank, M, K, E, X, ids)
        for t in range(T):
            for s in range(k):
                e = ids[t, s]
                exp = oracle.mul_mat_type(TYPE_Q6_K, bank[e * eb:(e + 1) * eb], M, K, X[t, s % ne11][None])
                np.testing.assert_array_equal(Y[t, s], exp[0])


def test_encoder_invariants(oracle):
    rng = np.random.default_rng(65)
    x = (rng.standard_normal(QK * 256) * 0.02).astype(np.float32)
    q = oracle.quantize_q6K(x)
    sc, d = _fields(q)
    # the sub-block of largest fitted scale is stored as -128 (iscale = -128 / max_scale)
    assert (sc.min(axis=1) == -128).all()
    y = oracle.dequant_q6K(q, x.size)
    # 6-bit symmetric per 16 values: RMS error well below the data's own spread
    assert np.sqrt(np.mean((y - x) ** 2)) < 0.03 * 0.02
    # an all-zero (or below 1e-15) block is all-zero bytes
    z = oracle.quantize_q6K(np.concatenate([np.zeros(QK, np.float32), np.full(QK, 1e-16, np.float32)]))
    assert (z == 0).all()


# ---- live reference (only where oracle/_ref is built) -----------------------
def test_live_reference_random(oracle, ref):
    rng = np.random.default_rng(2025)
    M, K = 24, 2048
    x = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    q_o = oracle.quantize_q6K(x)
    np.testing.assert_array_equal(q_o, ref.quantize_type(TYPE_Q6_K, x, M, K))
    np.testing.assert_array_equal(oracle.dequant_q6K(q_o, M * K).view(np.uint32),
                                  ref.dequant_type(TYPE_Q6_K, q_o, M * K).view(np.uint32))
    a = rng.standard_normal((3, K)).astype(np.float32)
    np.testing.assert_array_equal(oracle.mul_mat_type(TYPE_Q6_K, q_o, M, K, a).view(np.uint32),
                                  ref.mul_mat(q_o, M, K, a, qtype=TYPE_Q6_K).view(np.uint32))

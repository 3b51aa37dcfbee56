"""Pins each oracle function by what the mathematics fixes, independently of
the reference build: IEEE half conversions against numpy, round-half-even,
an exhaustive scale/min packing round trip, closed-form dequantised blocks,
Q8_K invariants, brute-force integer sub-block sums and an exact dot-product
combine evaluated by a separate numpy implementation of the block layout."""
import ctypes as C

import numpy as np
import pytest

QK = 256


# ---- scalar conversions ------------------------------------------------------
def test_fp16_to_fp32_all_halves(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.L.or_fp16_to_fp32(int(v)) for v in h], np.float32)
    finite = np.isfinite(exp) | np.isinf(exp)
    np.testing.assert_array_equal(got[finite].view(np.uint32), exp[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()


def test_fp32_to_fp16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 4000),
        (rng.random(2000) * 6.2e-5).astype(np.float32),            # subnormal half range
        np.array([65504, 65519, 65520, 70000, 1e-8, 5.96e-8, 2.98e-8, 0.0, -0.0], np.float32),
    ])
    # exact ties: halfway between two halves
    base = rng.integers(0x0400, 0x7B00, 1000).astype(np.uint16).view(np.float16).astype(np.float32)
    ulp = np.spacing(base.astype(np.float16)).astype(np.float32)
    vals = np.concatenate([vals, base + ulp / 2, -(base + ulp / 2)]).astype(np.float32)
    got = np.array([oracle.L.or_fp32_to_fp16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        exp = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, exp)


def test_nearest_int_is_round_half_even(oracle):
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.uniform(-4e6, 4e6, 5000), np.arange(-300, 300) + 0.5,
                        rng.uniform(-130, 130, 5000)]).astype(np.float32)
    got = np.array([oracle.L.or_nearest_int(float(x)) for x in v])
    np.testing.assert_array_equal(got, np.rint(v).astype(np.int64))


# ---- the 12-byte scale/min packing ---------------------------------------------
def _pack_scales(sc, m):
    """Packs 8 six-bit scales and mins as the Q4_K format stores them
    (ggml-common.h:317-328): bytes 0-3 and 4-7 carry the low 6 bits of
    scale/min 0-3 with the top 2 bits of scale/min 4-7 in bits 6-7; bytes 8-11
    carry the low nibbles of scale 4-7 (bits 0-3) and min 4-7 (bits 4-7)."""
    b = np.zeros(12, np.uint8)
    for j in range(4):
        b[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return b


def test_scale_min_unpack_exhaustive(oracle):
    sc_out, m_out = C.c_uint8(), C.c_uint8()
    rng = np.random.default_rng(3)
    for v in range(64):
        for j in range(8):
            sc = rng.integers(0, 64, 8).astype(np.uint8)
            m = rng.integers(0, 64, 8).astype(np.uint8)
            sc[j] = v
            m[(j + 3) % 8] = 63 - v
            b = _pack_scales(sc, m)
            for jj in range(8):
                oracle.L.or_scale_min_k4(jj, b.ctypes.data, C.addressof(sc_out), C.addressof(m_out))
                assert (sc_out.value, m_out.value) == (sc[jj], m[jj]), (v, j, jj)


# ---- dequantisation in closed form --------------------------------------------
def _block(d16, dmin16, sc, m, q):
    """q: 256 values 0..15 in element order -> one 144-byte Q4_K block
    (element 64g + 32h + l is nibble h of qs[32g + l])."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d16], np.uint16).view(np.uint8)
    blk[2:4] = np.array([dmin16], np.uint16).view(np.uint8)
    blk[4:16] = _pack_scales(sc, m)
    for g in range(4):
        for l in range(32):
            blk[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return blk


def test_dequant_closed_forms(oracle):
    rng = np.random.default_rng(4)
    q = (np.arange(QK) * 7 + 3) % 16              # distinct pattern: catches element order slips
    # d = 1, dmin = 0: y = sc_j * q
    sc = np.arange(1, 9, dtype=np.uint8) * 7
    m = np.zeros(8, np.uint8)
    y = oracle.dequant(_block(0x3C00, 0, sc, m, q.astype(np.uint8)), QK)
    np.testing.assert_array_equal(y, (np.repeat(sc, 32) * q).astype(np.float32))
    # d = 0, dmin = 0.5: y = -0.5 * m_j
    m = np.arange(8, dtype=np.uint8) * 9
    y = oracle.dequant(_block(0, 0x3800, np.zeros(8, np.uint8), m, q.astype(np.uint8)), QK)
    np.testing.assert_array_equal(y, -(0.5 * np.repeat(m, 32)).astype(np.float32))
    # general: y = (d*sc)*q - (dmin*m), each product rounded to fp32 once
    for _ in range(20):
        d16, dm16 = (int(v) for v in rng.integers(0x0400, 0x6000, 2))
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        qq = rng.integers(0, 16, QK).astype(np.uint8)
        d = np.array([d16], np.uint16).view(np.float16).astype(np.float32)[0]
        dm = np.array([dm16], np.uint16).view(np.float16).astype(np.float32)[0]
        d1 = (d * np.repeat(sc, 32).astype(np.float32)).astype(np.float32)
        m1 = (dm * np.repeat(m, 32).astype(np.float32)).astype(np.float32)
        exp = ((d1 * qq.astype(np.float32)).astype(np.float32) - m1).astype(np.float32)
        y = oracle.dequant(_block(d16, dm16, sc, m, qq), QK)
        np.testing.assert_array_equal(y.view(np.uint32), exp.view(np.uint32))


# ---- Q8_K invariants ----------------------------------------------------------
def _q8_fields(b):
    b = b.reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8)
    bs = b[:, 260:292].copy().view(np.int16)
    return d, qs, bs


def test_q8k_invariants(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(QK * 64).astype(np.float32) * np.repeat(10.0 ** rng.integers(-3, 3, 64), QK).astype(np.float32)
    d, qs, bs = _q8_fields(oracle.quantize_q8K(x))
    xb = x.reshape(-1, QK)
    assert (np.abs(qs.astype(np.int32)) <= 127).all()
    np.testing.assert_array_equal(bs, qs.reshape(-1, 16, 16).astype(np.int32).sum(-1))
    first = np.argmax(np.abs(xb), axis=1)          # numpy argmax returns the first maximum
    assert (qs[np.arange(len(first)), first] == -127).all()
    vmax = xb[np.arange(len(first)), first]
    iscale = (np.float32(-127.0) / vmax).astype(np.float32)
    np.testing.assert_array_equal(d, (np.float32(1.0) / iscale).astype(np.float32))
    err = np.abs(xb - d[:, None] * qs)
    assert (err <= np.abs(d)[:, None] * 0.5 * (1 + 1e-5) + 1e-30).all()


def test_q8k_tie_break_and_zero(oracle):
    x = np.zeros(3 * QK, np.float32)
    x[10], x[200] = -4.0, 4.0                      # block 0: first max is negative
    x[QK + 10], x[QK + 200] = 4.0, -4.0            # block 1: first max is positive
    d, qs, bs = _q8_fields(oracle.quantize_q8K(x))
    assert d[0] > 0 and d[1] < 0 and d[2] == 0     # block 2: all zero -> d = 0
    assert qs[0, 10] == -127 and qs[0, 200] == 127
    assert qs[1, 10] == -127 and qs[1, 200] == 127
    assert (qs[2] == 0).all() and (bs[2] == 0).all()


# ---- integer sub-block sums and the dot-product combine ------------------------
def _nibbles(q4):
    """(nblocks, 256) 4-bit values in element order from 144-byte blocks."""
    qs = q4.reshape(-1, 144)[:, 16:144].reshape(-1, 4, 32)
    lo, hi = qs & 15, qs >> 4
    return np.concatenate([lo[:, :, None, :], hi[:, :, None, :]], axis=2).reshape(-1, QK).astype(np.int64)


def _scales(q4):
    b = q4.reshape(-1, 144)[:, 4:16].astype(np.int64)
    sc = np.zeros((b.shape[0], 8), np.int64)
    m = np.zeros((b.shape[0], 8), np.int64)
    sc[:, :4] = b[:, 0:4] & 63
    m[:, :4] = b[:, 4:8] & 63
    sc[:, 4:] = (b[:, 8:12] & 15) | ((b[:, 0:4] >> 6) << 4)
    m[:, 4:] = (b[:, 8:12] >> 4) | ((b[:, 4:8] >> 6) << 4)
    return sc, m


def test_subblock_sums_brute_force(oracle):
    rng = np.random.default_rng(6)
    for K in (256, 768, 4096):
        w = oracle.quantize_q4K((rng.standard_normal(K) * 0.02).astype(np.float32))
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        _, qs, _ = _q8_fields(a)
        exp = (_nibbles(w) * qs.astype(np.int64)).reshape(-1, 8, 32).sum(-1).ravel()
        np.testing.assert_array_equal(oracle.subblock_sums(K, w, a), exp)


def test_exact_combine_and_float_orders(oracle):
    rng = np.random.default_rng(7)
    for K in (256, 4096, 27648):
        w = oracle.quantize_q4K((rng.standard_normal(K) * 0.02).astype(np.float32))
        a = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        d8, qs, bs = _q8_fields(a)
        S = (_nibbles(w) * qs.astype(np.int64)).reshape(-1, 8, 32).sum(-1)
        sc, m = _scales(w)
        I = (sc * S).sum(1)
        Mt = (m * (bs[:, 0::2].astype(np.int64) + bs[:, 1::2])).sum(1)
        hdr = w.reshape(-1, 144)[:, 0:4].copy().view(np.float16).astype(np.float64)
        exact = float((hdr[:, 0] * d8 * I - hdr[:, 1] * d8 * Mt).sum())
        assert oracle.vec_dot_exact(K, w, a) == pytest.approx(exact, rel=1e-12, abs=1e-12)
        scale = float((np.abs(hdr[:, 0] * d8 * I) + np.abs(hdr[:, 1] * d8 * Mt)).sum())
        for order in ("avx2", "generic"):
            assert abs(oracle.vec_dot(K, w, a, order) - exact) <= 1e-6 * scale


def test_mul_mat_id_is_gathered_mul_mat(oracle):
    rng = np.random.default_rng(8)
    E, M, K, T, k = 6, 40, 512, 4, 3
    bank = oracle.quantize_q4K((rng.standard_normal((E * M, K)) * 0.02).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    eb = M * K // 256 * 144
    for ne11 in (1, k):
        X = rng.standard_normal((T, ne11, K)).astype(np.float32)
        Y = oracle.mul_mat_id(bank, M, K, E, X, ids)
        for t in range(T):
            for s in range(k):
                e = ids[t, s]
                exp = oracle.mul_mat(bank[e * eb:(e + 1) * eb], M, K, X[t, s % ne11][None])
                np.testing.assert_array_equal(Y[t, s], exp[0])


# ---- encoder properties ------------------------------------------------------------
def test_encoder_reconstruction(oracle):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(QK * 256) * 0.02).astype(np.float32)
    q = oracle.quantize_q4K(x)
    y = oracle.dequant(q, x.size)
    # 4-bit affine per 32 values: RMS error well below the data's own spread
    assert np.sqrt(np.mean((y - x) ** 2)) < 0.1 * 0.02
    hdr = q.reshape(-1, 144)[:, 0:4].copy().view(np.float16)
    assert (hdr >= 0).all()


# ---- synthetic data ----------------------------------------------------------------
def test_synth_deterministic_and_distributed(oracle):
    a = oracle.synth(100_000, 42)
    b = oracle.synth(90_000, 42, offset=10_000)
    np.testing.assert_array_equal(a[10_000:], b)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1.0) < 0.02
    t = oracle.synth(400_000, 43, dist=1, cols=1000, std=1.0, mult=1.0)
    assert abs(t.var() - 2.0) < 0.2                   # var of Student-t(4) = 4/(4-2)
    o = oracle.synth(200_000, 44, dist=0, cols=1000, std=1.0, mult=8.0).reshape(-1, 1000)
    col_sd = o.std(axis=0)
    frac = (col_sd > 4).mean()
    assert 0.002 < frac < 0.03                         # about 1% outlier columns

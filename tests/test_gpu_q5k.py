"""GPU parity of the Q5_K kernels (GGML_TYPE_Q5_K weights, Q8_K activations).

Against the reference's own golden vectors (tests/golden/q5k_golden.npz) and
the CPU oracle (oracle/q5k_oracle.c, pinned bit for bit to the reference in
test_oracle_q5k.py):
  - dequantisation (dequantize_row_q5_K) and the encoder (quantize_q5_K):
    bit-exact;
  - integer sub-block sums: bit-exact against the oracle's brute force;
  - vec_dot, GEMV (T = 1 decode kernel and the sdot4 kernel), batches (the
    matrix-core ring for T >= 4, every launch shape; the sdot4 GEMV over
    8-token slices under SPQ4K_GEMM_MODE=1) and the expert-gathered matvec
    (decode mapping, single-launch and grouped sdot4 kernels, the matrix-core
    expert kernel): every element within close_enough (1e-4 relative or 1e-5
    absolute, tests/desktop/test_sp_kernels.cpp:34-48) of ggml's x86 order.
Weights are encoder output (N(0, 0.02)) or arbitrary block bytes; outputs of
arbitrary bytes are held to the fp32 summation bound around the exact result
(their scale/min terms cancel)."""
import os

import numpy as np
import pytest

from _envctx import context_with
from _oracle import Q5K, TYPE_Q5_K, close_enough

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q5k_golden.npz"))
QK = 256


def _rand_blocks(rng, nblk, dmax=1e-3):
    """Arbitrary Q5_K blocks; fp16 d and dmin uniform in (0, dmax]."""
    b = rng.integers(0, 256, size=(nblk, Q5K), dtype=np.uint8)
    for off in (0, 2):
        v = (rng.uniform(0.05, 1.0, nblk) * dmax).astype(np.float16)
        b[:, off:off + 2] = v.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def _enc(oracle, rng, M, K, scale=0.02):
    return oracle.quantize_q5K((rng.standard_normal((M, K)) * scale).astype(np.float32))


def _gpu_enc(ctx, rng, M, K, scale=0.02):
    """N(0, scale) weights from the GPU encoder (bit-exact with quantize_q5_K:
    test_encoder_*_bitexact), for shapes the CPU encoder would take long on."""
    return ctx.quantize_chunk((rng.standard_normal((M, K)) * scale).astype(np.float32), M, K, type=TYPE_Q5_K)


def _scales(W, M, nb):
    b = W.reshape(M, nb, Q5K)[:, :, 4:16].astype(np.int64)
    sc = np.zeros((M, nb, 8), np.int64)
    m = np.zeros((M, nb, 8), np.int64)
    sc[..., :4] = b[..., 0:4] & 63
    m[..., :4] = b[..., 4:8] & 63
    sc[..., 4:] = (b[..., 8:12] & 15) | ((b[..., 0:4] >> 6) << 4)
    m[..., 4:] = (b[..., 8:12] >> 4) | ((b[..., 4:8] >> 6) << 4)
    return sc, m


def _exact_rows(oracle, W, M, K, X):
    """Per output: the exact dot product and the magnitude of its terms."""
    nb = K // QK
    sc, m = _scales(W, M, nb)
    hd = W.reshape(M, nb, Q5K)[:, :, 0:4].copy().view(np.float16).astype(np.float64)
    d, dmin = hd[..., 0], hd[..., 1]
    exact = np.zeros((X.shape[0], M))
    mag = np.zeros((X.shape[0], M))
    rb = nb * Q5K
    for t in range(X.shape[0]):
        q8 = oracle.quantize_q8K(X[t])
        blk = q8.reshape(nb, 292)
        d8 = blk[:, 0:4].copy().view(np.float32).astype(np.float64).ravel()
        bs = blk[:, 260:292].copy().view(np.int16).astype(np.int64)
        bsp = bs[:, 0::2] + bs[:, 1::2]
        for r in range(M):
            S = oracle.subblock_sums_q5K(K, W[r * rb:(r + 1) * rb], q8).reshape(nb, 8).astype(np.int64)
            ti = d[r] * d8 * (sc[r] * S).sum(1)
            tm = dmin[r] * d8 * (m[r] * bsp).sum(1)
            exact[t, r] = (ti - tm).sum()
            mag[t, r] = (np.abs(ti) + np.abs(tm)).sum()
    return exact, mag


def _check_bounded(got, exact, mag, nb, what):
    tol = (2 * nb + 8) * 2.0 ** -23 * mag + 1e-30
    bad = np.abs(got.astype(np.float64) - exact) > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} beyond the summation bound; first "
                           f"{tuple(np.argwhere(bad)[0])}")


def _check(got, exp, what):
    ok = close_enough(got, exp)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; first {tuple(i)} "
                             f"got {got[tuple(i)]!r} exp {exp[tuple(i)]!r}")


# ---- conversions --------------------------------------------------------------------
def test_dequant_golden_bitexact(ctx):
    got = ctx.to_float(GOLD["deq_q"], GOLD["deq_y"].size, type=TYPE_Q5_K)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_dequant_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(501)
    for nblk in (1, 3, 4097):
        q = _rand_blocks(rng, nblk, dmax=60000.0)
        got = ctx.to_float(q, nblk * QK, type=TYPE_Q5_K)
        np.testing.assert_array_equal(got.view(np.uint32), oracle.dequant_q5K(q, nblk * QK).view(np.uint32))


def test_encoder_golden_bitexact(ctx):
    x = GOLD["enc_x"]
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q5_K).reshape(-1, Q5K)
    bad = np.nonzero((got != GOLD["enc_q"].reshape(-1, Q5K)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ from quantize_q5_K, first {bad[:8]}"


def test_encoder_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(502)
    x = np.concatenate([(rng.standard_normal((33, 768)) * 0.02).astype(np.float32).ravel(),
                        (rng.standard_t(4, size=(8, 4096)) * 0.05).astype(np.float32).ravel(),
                        (rng.standard_normal(QK * 5) * 1e3).astype(np.float32)])
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q5_K).reshape(-1, Q5K)
    bad = np.nonzero((got != oracle.quantize_q5K(x).reshape(-1, Q5K)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:8]}"


def test_vec_dot_golden(ctx):
    o5 = o8 = 0
    for i, K in enumerate(GOLD["vd_K"]):
        K = int(K)
        n5, n8 = K // QK * Q5K, K // QK * 292
        w, a = GOLD["vd_w"][o5:o5 + n5], GOLD["vd_q8"][o8:o8 + n8]
        o5 += n5
        o8 += n8
        got = ctx.vec_dot(K, w, a, type=TYPE_Q5_K)
        assert close_enough(got, GOLD["vd_avx2"][i]), (i, K, got, GOLD["vd_avx2"][i])


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_subblock_sums_exact(ctx, oracle, kind):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(503)
    for M, K in ((64, 4096), (37, 768), (16, 27648), (9, 5120)):
        W = _enc(oracle, rng, M, K) if kind == "enc" else _rand_blocks(rng, M * K // QK)
        x = rng.standard_normal(K).astype(np.float32)
        q8 = oracle.quantize_q8K(x)
        Wd, xd = DeviceArray.from_host(W), DeviceArray.from_host(x)
        Sd = DeviceArray(M * (K // QK) * 8, np.int32)
        ctx.subblock_sums(Wd.ptr, M, K, xd.ptr, Sd.ptr, type=TYPE_Q5_K)
        ctx.synchronize()
        got = Sd.to_host().reshape(M, -1)
        rb = K // QK * Q5K
        for r in range(M):
            np.testing.assert_array_equal(got[r], oracle.subblock_sums_q5K(K, W[r * rb:(r + 1) * rb], q8),
                                          err_msg=f"row {r} M={M} K={K}")


# ---- matvec ---------------------------------------------------------------------------------
@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_golden(ctx, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = ctx.mul_mat(ctx.upload(GOLD["mm_W"], M, K, type=TYPE_Q5_K), GOLD[f"mm_X{T}"])
    _check(got, GOLD[f"mm_Y{T}"], f"golden mul_mat T={T}")


@pytest.mark.parametrize("M,K,kind", [(4096, 4096, "enc"), (1024, 12288, "enc"), (300, 768, "enc"),
                                      (512, 5120, "enc"), (256, 27648, "enc"), (33000, 4096, "gpu_enc"),
                                      (64, 2048, "rand"), (64, 27648, "rand"), (160, 4096, "rand")])
def test_gemv_t1(ctx, oracle, M, K, kind):
    rng = np.random.default_rng(M * 5 + K)
    if kind == "enc":
        W = _enc(oracle, rng, M, K)
    elif kind == "gpu_enc":
        W = _gpu_enc(ctx, rng, M, K)
    else:
        W = _rand_blocks(rng, M * K // QK)
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q5_K), x)
    if kind == "rand":
        exact, mag = _exact_rows(oracle, W, M, K, x)
        _check_bounded(got, exact, mag, K // QK, f"q5k gemv M={M} K={K}")
        _check_bounded(oracle.mul_mat_type(TYPE_Q5_K, W, M, K, x), exact, mag, K // QK, "oracle")
    else:
        _check(got, oracle.mul_mat_type(TYPE_Q5_K, W, M, K, x), f"q5k gemv M={M} K={K}")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_GEMV_GENERIC": 1}, {"SPQ4K_DEC_WAVES": 8, "SPQ4K_DEC_DEPTH": 2},
                                 {"SPQ4K_DEC_WAVES": 16, "SPQ4K_DEC_XFIRST": 0}])
def test_gemv_t1_launch_shapes(oracle, env):
    rng = np.random.default_rng(504)
    c = context_with(env)
    try:
        for M, K in ((2048, 4096), (512, 12288)):
            W = _enc(oracle, rng, M, K)
            x = rng.standard_normal((1, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q5_K), x)
            _check(got, oracle.mul_mat_type(TYPE_Q5_K, W, M, K, x), f"{env} M={M} K={K}")
    finally:
        c.close()


@pytest.mark.parametrize("T", [2, 3, 5, 8, 9, 16, 40])
def test_mul_mat_batched(ctx, oracle, T):
    rng = np.random.default_rng(505 + T)
    for M, K in ((512, 4096), (200, 768)):
        W = _enc(oracle, rng, M, K)
        X = rng.standard_normal((T, K)).astype(np.float32)
        got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q5_K), X)
        _check(got, oracle.mul_mat_type(TYPE_Q5_K, W, M, K, X), f"q5k mul_mat T={T} M={M} K={K}")


@pytest.mark.parametrize("cfg", [19, 20, 21, 22, 23, 30])
def test_ring_launch_shapes(oracle, cfg):
    """Every Q5_K matrix-core launch shape, on ragged rows and tokens."""
    rng = np.random.default_rng(510 + cfg)
    c = context_with({"SPQ4K_GEMM_CFG": cfg})
    try:
        for M, K, T in ((300, 768, 5), (200, 4096, 33), (1000, 2048, 100)):
            W = _enc(oracle, rng, M, K)
            X = rng.standard_normal((T, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q5_K), X)
            _check(got, oracle.mul_mat_type(TYPE_Q5_K, W, M, K, X), f"cfg={cfg} M={M} K={K} T={T}")
    finally:
        c.close()


@pytest.mark.parametrize("M,K,T", [(64, 27648, 64), (4096, 4096, 128), (512, 12288, 256), (96, 5120, 7)])
def test_ring_planned(ctx, oracle, M, K, T):
    """The planner's choice, including K splits (few rows, long K) and the
    reduction of their partial sums."""
    rng = np.random.default_rng(M + K + T + 5)
    W = _gpu_enc(ctx, rng, M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q5_K), X)
    _check(got, oracle.mul_mat_type(TYPE_Q5_K, W, M, K, X), f"planned M={M} K={K} T={T}")


def _const_block(sc, mn, q5, d, dmin):
    """One Q5_K block whose 8 sub-blocks all hold scale sc, min mn (6-bit)
    and value q5 (5-bit), packed as get_scale_min_k4 and dequantize_row_q5_K
    unpack them (ggml-quants.c)."""
    b = np.zeros(Q5K, np.uint8)
    b[0:4] = np.array([d, dmin], np.float16).view(np.uint8)
    b[4:8] = (sc & 63) | ((sc >> 4) << 6)
    b[8:12] = (mn & 63) | ((mn >> 4) << 6)
    b[12:16] = (sc & 15) | ((mn & 15) << 4)
    b[16:48] = 0xFF if q5 >> 4 else 0
    b[48:176] = (q5 & 15) | ((q5 & 15) << 4)
    return b


def test_ring_extreme_operands(ctx, oracle):
    """Blocks at the ends of the split operand range: scale 63 (every part of
    sc = 16a + 4b + c at 3, operands a q5 up to 93) and the single-part
    scales 48, 12, 3, with value 0 or 31 and min 0 or 63, one combination a
    row; dmin < 0 so that with one-sign activations the scale and min terms
    add (every Q8_K block holds -128 at its largest magnitude). Then
    arbitrary blocks, held to the summation bound."""
    rng = np.random.default_rng(520)
    M, K, T = 64, 1024, 48
    nb = K // QK
    blk = np.zeros((M, nb, Q5K), np.uint8)
    for r in range(M):
        v = r % 16
        sc, q5, mn = (63, 48, 12, 3)[v % 4], (0, 31)[(v >> 2) & 1], (0, 63)[(v >> 3) & 1]
        for b in range(nb):
            blk[r, b] = _const_block(sc, mn, q5, 2.0 ** -12 * (1 + r % 5), -2.0 ** -13 * (1 + r % 3))
    W = blk.ravel()
    for X in (np.abs(rng.standard_normal((T, K))), -np.abs(rng.standard_normal((T, K)))):
        X = X.astype(np.float32)
        _check(ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q5_K), X),
               oracle.mul_mat_type(TYPE_Q5_K, W, M, K, X), "extreme one-sign")
    W2 = _rand_blocks(rng, M * nb)
    X2 = rng.standard_normal((T, K)).astype(np.float32)
    exact, mag = _exact_rows(oracle, W2, M, K, X2)
    _check_bounded(ctx.mul_mat(ctx.upload(W2, M, K, type=TYPE_Q5_K), X2), exact, mag, nb, "arbitrary blocks")


@pytest.mark.parametrize("T", [4, 40])
def test_ring_matches_sdot4_slices(oracle, T):
    """SPQ4K_GEMM_MODE=1 keeps Q5_K batches on the sdot4 kernels: both paths
    within tolerance of the oracle on the same inputs."""
    rng = np.random.default_rng(530 + T)
    M, K = 384, 4096
    W = _enc(oracle, rng, M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    exp = oracle.mul_mat_type(TYPE_Q5_K, W, M, K, X)
    for env in ({}, {"SPQ4K_GEMM_MODE": 1}):
        c = context_with(env)
        try:
            _check(c.mul_mat(c.upload(W, M, K, type=TYPE_Q5_K), X), exp, f"{env} T={T}")
        finally:
            c.close()


@pytest.mark.parametrize("T", [1, 4, 12])
def test_gemv_multi_device(ctx, oracle, T):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(506 + T)
    K, shapes = 4096, (1024, 256)
    Ws = [_enc(oracle, rng, M, K) for M in shapes]
    X = rng.standard_normal((T, K)).astype(np.float32)
    wd = [ctx.upload(w, M, K, type=TYPE_Q5_K) for w, M in zip(Ws, shapes)]
    xd = DeviceArray.from_host(X)
    yd = [DeviceArray(T * M, np.float32) for M in shapes]
    if T <= 8:
        ctx.gemv_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    else:
        ctx.gemm_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    ctx.synchronize()
    for w, M, y in zip(Ws, shapes, yd):
        _check(y.to_host().reshape(T, M), oracle.mul_mat_type(TYPE_Q5_K, w, M, K, X), f"multi M={M} T={T}")


# ---- expert-gathered matvec -------------------------------------------------------------------
@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_golden(ctx, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    bank = ctx.upload(GOLD["mmid_bank"], M, K, E, type=TYPE_Q5_K)
    got = ctx.mul_mat_id(bank, GOLD[f"mmid_X_{tag}"], GOLD[f"mmid_ids_{tag}"])
    _check(got, GOLD[f"mmid_Y_{tag}"], f"golden mul_mat_id {tag}")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_MODE": 3}, {"SPQ4K_MOE_UNFUSED": 1}, {"SPQ4K_MOE_MODE": 2}, {"SPQ4K_MOE_RING_WAVES": 8}])
@pytest.mark.parametrize("T,ne11", [(1, 1), (3, 8), (12, 1), (32, 8)])
def test_moe(oracle, env, T, ne11):
    rng = np.random.default_rng(508 + T)
    E, n_used = 32, 8
    c = context_with(env)
    try:
        for M, K in ((256, 768), (128, 2048)):
            bank = _enc(oracle, rng, E * M, K)
            ids = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            X = rng.standard_normal((T, ne11, K)).astype(np.float32)
            got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q5_K), X, ids)
            _check(got, oracle.mul_mat_id_type(TYPE_Q5_K, bank, M, K, E, X, ids),
                   f"q5k moe {env} T={T} ne11={ne11} M={M} K={K}")
    finally:
        c.close()


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_UNFUSED": 1}])
def test_moe_ring_ragged(oracle, env):
    """The matrix-core expert kernel on a bank whose rows are not a multiple
    of its 128-row tile, with one expert chosen by every token (pairs over
    several 16-token tiles, the last one partial) and the rest spread; the
    sdot4 grouped kernels on the same inputs."""
    rng = np.random.default_rng(540)
    E, n_used, M, K, T = 16, 4, 200, 1024, 70
    bank = _enc(oracle, rng, E * M, K)
    ids = np.stack([np.concatenate([[0], rng.choice(np.arange(1, E), n_used - 1, replace=False)])
                    for _ in range(T)]).astype(np.int32)
    X = rng.standard_normal((T, 1, K)).astype(np.float32)
    c = context_with(env)
    try:
        got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q5_K), X, ids)
        _check(got, oracle.mul_mat_id_type(TYPE_Q5_K, bank, M, K, E, X, ids), f"q5k moe ring {env}")
    finally:
        c.close()

"""GPU parity of the Q8_0 kernels (GGML_TYPE_Q8_0 weights, Q8_0 activations).

Against the reference's own golden vectors (tests/golden/q8_0_golden.npz)
and the CPU oracle (oracle/q8_0_oracle.c, pinned bit for bit to the
reference in test_oracle_q8_0.py):
  - dequantisation (dequantize_row_q8_0), the model-file encoder
    (quantize_q8_0) and the activation quantiser (the CPU backend's
    quantize_row_q8_0, which rounds ties to even where the encoder rounds
    them away from zero): bit-exact;
  - integer block sums: bit-exact against the oracle's brute force;
  - vec_dot, the matvec at every lanes-per-row shape (K from 32 to 147456,
    the last too long for LDS) and its weight-staging form (K a multiple of
    256: contiguous loads into per-wave LDS buffers), batches (over 8 tokens and K a multiple of
    256: the matrix-core ring, every launch shape, K splits, the int8 ends;
    otherwise the matvec over token slices), several matrices in one launch
    and the expert-gathered matvec (one sweep for small batches, grouped by
    expert otherwise): every element within close_enough
    (1e-4 relative or 1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48)
    of ggml's x86 order.
Weights are encoder output (N(0, 0.02)) or arbitrary block bytes; outputs of
arbitrary bytes are held to the fp32 summation bound around the exact result
(their terms cancel)."""
import os

import numpy as np
import pytest

from _envctx import context_with
from _oracle import Q8_0, TYPE_Q8_0, close_enough

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q8_0_golden.npz"))
QK = 32


def _rand_blocks(rng, nblk, dmax=1e-3):
    """Arbitrary Q8_0 blocks: random int8 values, fp16 d of either sign with
    |d| in (0.05, 1] * dmax."""
    b = rng.integers(0, 256, size=(nblk, Q8_0), dtype=np.uint8)
    d = (rng.uniform(0.05, 1.0, nblk) * dmax * rng.choice([-1.0, 1.0], nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def _enc(oracle, rng, M, K, scale=0.02):
    return oracle.quantize_q8_0((rng.standard_normal((M, K)) * scale).astype(np.float32), ref_encoder=True)


def _fields(q, nblk):
    b = q.reshape(nblk, Q8_0)
    return b[:, 0:2].copy().view(np.float16).astype(np.float64).ravel(), b[:, 2:].view(np.int8).astype(np.int64)


def _exact_rows(oracle, W, M, K, X):
    """Per output: the exact dot product and the magnitude of its terms."""
    nb = K // QK
    exact = np.zeros((X.shape[0], M))
    mag = np.zeros((X.shape[0], M))
    acts = [_fields(oracle.quantize_q8_0(X[t]), nb) for t in range(X.shape[0])]
    rows = max(1, (1 << 22) // K)
    for r0 in range(0, M, rows):
        r1 = min(M, r0 + rows)
        dw, qw = _fields(W[r0 * nb * Q8_0:r1 * nb * Q8_0], (r1 - r0) * nb)
        dw, qw = dw.reshape(r1 - r0, nb), qw.reshape(r1 - r0, nb, QK)
        for t, (da, qa) in enumerate(acts):
            terms = dw * da[None, :] * (qw * qa[None, :, :]).sum(2)
            exact[t, r0:r1] = terms.sum(1)
            mag[t, r0:r1] = np.abs(terms).sum(1)
    return exact, mag


def _check_bounded(got, exact, mag, nb, what):
    tol = (nb + 8) * 2.0 ** -23 * mag + 1e-30
    bad = np.abs(got.astype(np.float64) - exact) > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} beyond the summation bound; first "
                           f"{tuple(np.argwhere(bad)[0])}")


def _check(got, exp, what):
    ok = close_enough(got, exp)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; first {tuple(i)} "
                             f"got {got[tuple(i)]!r} exp {exp[tuple(i)]!r}")


def _ties(rng, nblk):
    """Blocks whose largest |x| is 127 (scale 1 in both quantisers), the other
    values random halves: every one an exact rounding tie."""
    x = (rng.integers(-253, 254, size=(nblk, QK)) / 2.0).astype(np.float32)
    x[:, 0] = rng.choice([-127.0, 127.0], nblk)
    return x.ravel()


# ---- conversions --------------------------------------------------------------------
def test_dequant_golden_bitexact(ctx):
    got = ctx.to_float(GOLD["deq_q"], GOLD["deq_y"].size, type=TYPE_Q8_0)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_dequant_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(801)
    for nblk in (1, 3, 8193):
        q = _rand_blocks(rng, nblk, dmax=60000.0)
        got = ctx.to_float(q, nblk * QK, type=TYPE_Q8_0)
        np.testing.assert_array_equal(got.view(np.uint32), oracle.dequant_q8_0(q, nblk * QK).view(np.uint32))


def test_encoder_golden_bitexact(ctx):
    x = GOLD["enc_x"]
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q8_0)
    np.testing.assert_array_equal(got, GOLD["enc_q"])


def test_encoder_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(802)
    x = np.concatenate([(rng.standard_normal((33, 768)) * 0.02).astype(np.float32).ravel(),
                        (rng.standard_t(4, size=(8, 4096)) * 0.05).astype(np.float32).ravel(),
                        (rng.standard_normal(QK * 5) * 1e3).astype(np.float32), np.zeros(QK, np.float32),
                        _ties(rng, 64)])
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q8_0)
    np.testing.assert_array_equal(got, oracle.quantize_q8_0(x, ref_encoder=True))


def test_activation_quantiser_golden_bitexact(ctx):
    np.testing.assert_array_equal(ctx.from_float(GOLD["act_x"], type=TYPE_Q8_0), GOLD["act_q"])


def test_activation_quantiser_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(803)
    x = np.concatenate([rng.standard_normal(4096 * 3).astype(np.float32),
                        (rng.standard_normal(QK * 40) * np.repeat(10.0 ** rng.integers(-6, 6, 40), QK)).astype(
                            np.float32), np.zeros(QK, np.float32), _ties(rng, 64)])
    got = ctx.from_float(x, type=TYPE_Q8_0)
    np.testing.assert_array_equal(got, oracle.quantize_q8_0(x))
    # the two quantisers differ on the ties, as the reference's do
    t = _ties(rng, 8)
    assert (ctx.from_float(t, type=TYPE_Q8_0) != ctx.quantize_chunk(t, 1, t.size, type=TYPE_Q8_0)).any()


def test_vec_dot_golden(ctx):
    o = 0
    for i, K in enumerate(GOLD["vd_K"]):
        K = int(K)
        n = K // QK * Q8_0
        w, a = GOLD["vd_w"][o:o + n], GOLD["vd_a"][o:o + n]
        o += n
        got = ctx.vec_dot(K, w, a, type=TYPE_Q8_0)
        assert close_enough(got, GOLD["vd_avx2"][i]), (i, K, got, GOLD["vd_avx2"][i])


@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_block_sums_exact(ctx, oracle, kind):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(804)
    for M, K in ((64, 4096), (37, 768), (16, 27648), (9, 96)):
        W = _enc(oracle, rng, M, K) if kind == "enc" else _rand_blocks(rng, M * K // QK)
        x = rng.standard_normal(K).astype(np.float32)
        a = oracle.quantize_q8_0(x)
        Wd, xd = DeviceArray.from_host(W), DeviceArray.from_host(x)
        Sd = DeviceArray(M * (K // QK), np.int32)
        ctx.subblock_sums(Wd.ptr, M, K, xd.ptr, Sd.ptr, type=TYPE_Q8_0)
        ctx.synchronize()
        got = Sd.to_host().reshape(M, -1)
        rb = K // QK * Q8_0
        for r in range(M):
            np.testing.assert_array_equal(got[r], oracle.block_sums_q8_0(K, W[r * rb:(r + 1) * rb], a),
                                          err_msg=f"row {r} M={M} K={K}")


# ---- matvec ---------------------------------------------------------------------------------
@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_golden(ctx, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    got = ctx.mul_mat(ctx.upload(GOLD["mm_W"], M, K, type=TYPE_Q8_0), GOLD[f"mm_X{T}"])
    _check(got, GOLD[f"mm_Y{T}"], f"golden mul_mat T={T}")


# K covers every (lanes per row, blocks a lane holds) shape: 32 and 96 (one
# and three blocks, 8 lanes), 768 (24), 1536 (48, 16 lanes), 2048 (64, 32
# lanes), 4096 / 5120 (64 lanes, 4 blocks), 12288 / 27648 (64 lanes, 8 blocks
# and two passes), 147456 (too long for LDS: activations read from planes)
@pytest.mark.parametrize("M,K,kind", [(4096, 4096, "enc"), (1024, 12288, "enc"), (300, 768, "enc"),
                                      (512, 5120, "enc"), (256, 27648, "enc"), (77, 1536, "enc"),
                                      (130, 2048, "enc"), (33, 32, "enc"), (65, 96, "enc"),
                                      (40, 147456, "enc"), (64, 2048, "rand"), (64, 27648, "rand"),
                                      (160, 4096, "rand"), (50, 96, "rand")])
def test_gemv_t1(ctx, oracle, M, K, kind):
    rng = np.random.default_rng(M * 5 + K)
    W = _enc(oracle, rng, M, K) if kind == "enc" else _rand_blocks(rng, M * K // QK)
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q8_0), x)
    if kind == "rand":
        exact, mag = _exact_rows(oracle, W, M, K, x)
        _check_bounded(got, exact, mag, K // QK, f"q8_0 gemv M={M} K={K}")
        _check_bounded(oracle.mul_mat_q8_0(W, M, K, x), exact, mag, K // QK, "oracle")
    else:
        _check(got, oracle.mul_mat_q8_0(W, M, K, x), f"q8_0 gemv M={M} K={K}")


def test_gemv_large_m(ctx, oracle):
    """151936 x 4096 (an output projection) from the GPU encoder, checked
    against the summation bound around the exact result."""
    rng = np.random.default_rng(805)
    M, K = 151936, 4096
    W = ctx.quantize_chunk(rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02), M, K, type=TYPE_Q8_0)
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q8_0), x)
    exact, mag = _exact_rows(oracle, W, M, K, x)
    _check_bounded(got, exact, mag, K // QK, "q8_0 gemv 151936 x 4096")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_Q80_STAGED": 0}, {"SPQ4K_Q80_STAGED": 2}, {"SPQ4K_Q80_GRID": 1},
                                 {"SPQ4K_Q80_GRID": 7},
                                 {"SPQ4K_Q80_STAGED": 0, "SPQ4K_Q80_PREQ": 1}, {"SPQ4K_Q80_PREQ": 1},
                                 {"SPQ4K_Q80_PREQ": 2}])
def test_launch_shapes(oracle, env):
    rng = np.random.default_rng(806)
    c = context_with(env)
    try:
        for M, K, T in ((2048, 4096, 1), (512, 12288, 1), (300, 768, 3), (257, 2048, 8), (100, 27648, 6)):
            W = _enc(oracle, rng, M, K)
            X = rng.standard_normal((T, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q8_0), X)
            _check(got, oracle.mul_mat_q8_0(W, M, K, X), f"{env} M={M} K={K} T={T}")
    finally:
        c.close()


@pytest.mark.parametrize("T", [2, 3, 5, 8, 9, 16, 40])
def test_mul_mat_batched(ctx, oracle, T):
    rng = np.random.default_rng(807 + T)
    # 27648: five tokens fill LDS, so 8-token slices run as 5 + 3
    for M, K in ((512, 4096), (200, 768), (48, 27648)):
        W = _enc(oracle, rng, M, K)
        X = rng.standard_normal((T, K)).astype(np.float32)
        got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q8_0), X)
        _check(got, oracle.mul_mat_q8_0(W, M, K, X), f"q8_0 mul_mat T={T} M={M} K={K}")


@pytest.mark.parametrize("cfg", [24, 25, 26, 27, 28, 31])
def test_ring_launch_shapes(oracle, cfg):
    """Every Q8_0 matrix-core launch shape (K a multiple of 256), on ragged
    rows and tokens."""
    rng = np.random.default_rng(820 + cfg)
    c = context_with({"SPQ4K_GEMM_CFG": cfg})
    try:
        for M, K, T in ((300, 768, 17), (200, 4096, 33), (1000, 2048, 100)):
            W = _enc(oracle, rng, M, K)
            X = rng.standard_normal((T, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q8_0), X)
            _check(got, oracle.mul_mat_q8_0(W, M, K, X), f"cfg={cfg} M={M} K={K} T={T}")
    finally:
        c.close()


@pytest.mark.parametrize("M,K,T", [(64, 27648, 64), (4096, 4096, 128), (512, 12288, 256), (96, 5120, 9)])
def test_ring_planned(ctx, oracle, M, K, T):
    """The planner's choice, including K splits (few rows, long K) and the
    reduction of their partial sums."""
    rng = np.random.default_rng(M + K + T + 8)
    W = ctx.quantize_chunk((rng.standard_normal((M, K)) * 0.02).astype(np.float32), M, K, type=TYPE_Q8_0)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q8_0), X)
    _check(got, oracle.mul_mat_q8_0(W, M, K, X), f"planned M={M} K={K} T={T}")


def test_ring_extreme_operands(ctx, oracle):
    """Blocks of values -128 or 127 throughout (the int8 ends, every block of
    a row alike; d of either sign, one sign a row), one-sign activations so
    that a row's blocks add up without cancellation; then arbitrary blocks,
    held to the summation bound."""
    rng = np.random.default_rng(830)
    M, K, T = 64, 1024, 40
    nb = K // QK
    blk = np.zeros((M, nb, Q8_0), np.uint8)
    for r in range(M):
        v = -128 if r % 2 == 0 else 127
        d = (2.0 ** -12) * (1 + r % 5) * (1 if (r >> 1) % 2 == 0 else -1)
        blk[r, :, 0:2] = np.array([d], np.float16).view(np.uint8)
        blk[r, :, 2:] = np.array([v], np.int8).view(np.uint8)
    W = blk.ravel()
    Wd = ctx.upload(W, M, K, type=TYPE_Q8_0)
    for X in (np.abs(rng.standard_normal((T, K))), -np.abs(rng.standard_normal((T, K)))):
        X = X.astype(np.float32)
        _check(ctx.mul_mat(Wd, X), oracle.mul_mat_q8_0(W, M, K, X), "extreme one-sign")
    W2 = _rand_blocks(rng, M * nb)
    X2 = rng.standard_normal((T, K)).astype(np.float32)
    exact, mag = _exact_rows(oracle, W2, M, K, X2)
    _check_bounded(ctx.mul_mat(ctx.upload(W2, M, K, type=TYPE_Q8_0), X2), exact, mag, nb, "arbitrary blocks")


@pytest.mark.parametrize("T", [9, 40])
def test_ring_matches_matvec_slices(oracle, T):
    """SPQ4K_GEMM_MODE=1 keeps Q8_0 batches on the matvec over token slices;
    K = 800 (not a multiple of 256) always does. Both paths within tolerance
    of the oracle on the same inputs."""
    rng = np.random.default_rng(840 + T)
    for M, K in ((384, 4096), (256, 800)):
        W = _enc(oracle, rng, M, K)
        X = rng.standard_normal((T, K)).astype(np.float32)
        exp = oracle.mul_mat_q8_0(W, M, K, X)
        for env in ({}, {"SPQ4K_GEMM_MODE": 1}):
            c = context_with(env)
            try:
                _check(c.mul_mat(c.upload(W, M, K, type=TYPE_Q8_0), X), exp, f"{env} M={M} K={K} T={T}")
            finally:
                c.close()


@pytest.mark.parametrize("T", [1, 3])
def test_rows_longer_than_lds(ctx, oracle, T):
    """K = 147456: one token's Q8_0 activations (166 KB) exceed LDS; every
    token reads its planes from global memory."""
    rng = np.random.default_rng(808 + T)
    M, K = 24, 147456
    W = _enc(oracle, rng, M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q8_0), X)
    _check(got, oracle.mul_mat_q8_0(W, M, K, X), f"q8_0 K={K} T={T}")


@pytest.mark.parametrize("T", [1, 4, 12])
def test_gemv_multi_device(ctx, oracle, T):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(809 + T)
    K, shapes = 4096, (1024, 256, 33)
    Ws = [_enc(oracle, rng, M, K) for M in shapes]
    X = rng.standard_normal((T, K)).astype(np.float32)
    wd = [ctx.upload(w, M, K, type=TYPE_Q8_0) for w, M in zip(Ws, shapes)]
    xd = DeviceArray.from_host(X)
    yd = [DeviceArray(T * M, np.float32) for M in shapes]
    if T <= 8:
        ctx.gemv_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    else:
        ctx.gemm_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    ctx.synchronize()
    for w, M, y in zip(Ws, shapes, yd):
        _check(y.to_host().reshape(T, M), oracle.mul_mat_q8_0(w, M, K, X), f"multi M={M} T={T}")


def test_shape_and_type_errors(ctx, oracle):
    from spq4k import Spq4kError, TYPE_Q4_K
    rng = np.random.default_rng(810)
    with pytest.raises(Spq4kError):   # K not a multiple of 32
        ctx.upload(np.zeros(Q8_0 * 2, np.uint8), 1, 48, type=TYPE_Q8_0)
    w8 = ctx.upload(_enc(oracle, rng, 16, 256), 16, 256, type=TYPE_Q8_0)
    w4 = ctx.upload(np.zeros(16 * 144, np.uint8), 16, 256, type=TYPE_Q4_K)
    from spq4k.hip import DeviceArray
    xd, y0, y1 = DeviceArray(256, np.float32), DeviceArray(16, np.float32), DeviceArray(16, np.float32)
    with pytest.raises(Spq4kError):   # matrices of one call share the type
        ctx.gemv_multi_dev([w8, w4], xd.ptr, [y0.ptr, y1.ptr], 1)
    with pytest.raises(Spq4kError):   # the Q8_K dot does not take Q8_0 weights
        ctx.vec_dot_q8K_dev(TYPE_Q8_0, 256, y0.ptr, xd.ptr, xd.ptr)


# ---- expert-gathered matvec -------------------------------------------------------------------
@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_golden(ctx, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    bank = ctx.upload(GOLD["mmid_bank"], M, K, E, type=TYPE_Q8_0)
    got = ctx.mul_mat_id(bank, GOLD[f"mmid_X_{tag}"], GOLD[f"mmid_ids_{tag}"])
    _check(got, GOLD[f"mmid_Y_{tag}"], f"golden mul_mat_id {tag}")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_MODE": 2}, {"SPQ4K_MOE_UNFUSED": 1}, {"SPQ4K_MOE_RING_WAVES": 4}])
@pytest.mark.parametrize("T,ne11", [(1, 1), (3, 8), (12, 1), (32, 8), (200, 1)])
def test_moe(oracle, env, T, ne11):
    """Every MoE path: the one-launch sweep (small batches), the matrix-core
    expert kernel (two pairs an expert on average, K a multiple of 256) and
    the grouped matvec (K = 96, or SPQ4K_MOE_UNFUSED)."""
    rng = np.random.default_rng(811 + T)
    E, n_used = 32, 8
    c = context_with(env)
    try:
        for M, K in ((256, 768), (128, 2048), (40, 96)):
            bank = _enc(oracle, rng, E * M, K)
            ids = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            X = rng.standard_normal((T, ne11, K)).astype(np.float32)
            got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q8_0), X, ids)
            _check(got, oracle.mul_mat_id_q8_0(bank, M, K, E, X, ids),
                   f"q8_0 moe {env} T={T} ne11={ne11} M={M} K={K}")
    finally:
        c.close()


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_UNFUSED": 1}])
def test_moe_rand_blocks(oracle, env):
    """Arbitrary expert bytes, matrix-core expert kernel and grouped matvec:
    the summation bound per pair."""
    rng = np.random.default_rng(812)
    E, n_used, T, M, K = 16, 4, 24, 96, 2048
    bank = _rand_blocks(rng, E * M * K // QK)
    ids = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
    X = rng.standard_normal((T, 1, K)).astype(np.float32)
    c = context_with(env)
    try:
        got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q8_0), X, ids)
    finally:
        c.close()
    rb = M * K // QK * Q8_0
    for t in range(T):
        for s in range(n_used):
            e = ids[t, s]
            exact, mag = _exact_rows(oracle, bank[e * rb:(e + 1) * rb], M, K, X[t])
            _check_bounded(got[t, s][None], exact, mag, K // QK, f"pair ({t}, {s})")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_UNFUSED": 1}])
def test_moe_ring_ragged(oracle, env):
    """The matrix-core expert kernel on a bank whose rows are not a multiple
    of its 128-row tile, one expert chosen by every token (pairs over several
    16-token tiles, the last partial) and the rest spread; the grouped matvec
    on the same inputs."""
    rng = np.random.default_rng(850)
    E, n_used, M, K, T = 16, 4, 200, 1024, 70
    bank = _enc(oracle, rng, E * M, K)
    ids = np.stack([np.concatenate([[0], rng.choice(np.arange(1, E), n_used - 1, replace=False)])
                    for _ in range(T)]).astype(np.int32)
    X = rng.standard_normal((T, 1, K)).astype(np.float32)
    c = context_with(env)
    try:
        got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q8_0), X, ids)
        _check(got, oracle.mul_mat_id_q8_0(bank, M, K, E, X, ids), f"q8_0 moe ring {env}")
    finally:
        c.close()

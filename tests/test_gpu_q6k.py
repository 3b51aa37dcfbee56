"""GPU parity of the Q6_K kernels (GGML_TYPE_Q6_K weights, Q8_K activations).

Against the reference's own golden vectors (tests/golden/q6k_golden.npz) and
the CPU oracle (oracle/q6k_oracle.c, pinned bit for bit to the reference in
test_oracle_q6k.py):
  - dequantisation (dequantize_row_q6_K) and the encoder (quantize_q6_K):
    bit-exact;
  - integer sub-block sums: bit-exact against the oracle's brute force;
  - vec_dot, GEMV (T = 1 decode kernel and the sdot4 kernel), batches on the
    matrix-core ring (every Q6_K launch shape, K split, ragged edges) and on
    the sdot4 slices, expert-gathered matvec (every MoE path): every element within
    close_enough (1e-4 relative or 1e-5 absolute,
    tests/desktop/test_sp_kernels.cpp:34-48) of ggml's x86 order.
Weights are encoder output (N(0, 0.02)) or arbitrary block bytes, which reach
every scale (-128..127) and 6-bit value; outputs of arbitrary bytes are held
to the fp32 summation bound around the exact result instead (their
random-sign scales cancel). Rows of an odd number of 210-byte blocks put
block starts at 2-byte-aligned addresses."""
import os

import numpy as np
import pytest

from _envctx import context_with
from _oracle import Q6K, TYPE_Q6_K, close_enough

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "q6k_golden.npz"))
QK = 256


def _rand_blocks(rng, nblk, dmax=1e-3):
    """Arbitrary Q6_K blocks; fp16 d uniform in (0, dmax] with either sign."""
    b = rng.integers(0, 256, size=(nblk, Q6K), dtype=np.uint8)
    d = (rng.uniform(0.05, 1.0, nblk) * dmax * rng.choice([-1, 1], nblk)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def _enc(oracle, rng, M, K, scale=0.02):
    return oracle.quantize_q6K((rng.standard_normal((M, K)) * scale).astype(np.float32))


def _gpu_enc(ctx, rng, M, K, scale=0.02):
    """N(0, scale) weights encoded by the GPU encoder (bit-exact with
    quantize_q6_K: test_encoder_*_bitexact), for shapes the CPU encoder would
    take too long on."""
    return ctx.quantize_chunk((rng.standard_normal((M, K)) * scale).astype(np.float32), M, K, type=TYPE_Q6_K)


def _exact_rows(oracle, W, M, K, X):
    """Per output: the exact dot product (integer sub-block sums, combine in
    double) and the sum of the magnitudes of its per-block terms, the scale
    against which fp32 summation-order differences are bounded."""
    nb = K // QK
    sc = W.reshape(M, nb, Q6K)[:, :, 192:208].view(np.int8).astype(np.int64)
    d = W.reshape(M, nb, Q6K)[:, :, 208:210].copy().view(np.float16).astype(np.float64)[..., 0]
    exact = np.zeros((X.shape[0], M))
    mag = np.zeros((X.shape[0], M))
    rb = nb * Q6K
    for t in range(X.shape[0]):
        q8 = oracle.quantize_q8K(X[t])
        d8 = q8.reshape(nb, 292)[:, 0:4].copy().view(np.float32).astype(np.float64).ravel()
        for r in range(M):
            S = oracle.subblock_sums_q6K(K, W[r * rb:(r + 1) * rb], q8).reshape(nb, 16).astype(np.int64)
            terms = d[r] * d8 * (sc[r] * S).sum(1)
            exact[t, r] = terms.sum()
            mag[t, r] = np.abs(terms).sum()
    return exact, mag


def _check_bounded(got, exact, mag, nb, what):
    """|got - exact| within (nb + 8) fp32 roundings of the terms' magnitude:
    arbitrary block bytes (random-sign scales) make outputs that cancel far
    below their terms, where an element-wise relative bound says nothing
    about the kernel."""
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


# ---- conversions --------------------------------------------------------------------
def test_dequant_golden_bitexact(ctx):
    q = GOLD["deq_q"]
    got = ctx.to_float(q, GOLD["deq_y"].size, type=TYPE_Q6_K)
    np.testing.assert_array_equal(got.view(np.uint32), GOLD["deq_y"].view(np.uint32))


def test_dequant_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(601)
    for nblk in (1, 3, 4097):
        q = _rand_blocks(rng, nblk, dmax=60000.0)
        got = ctx.to_float(q, nblk * QK, type=TYPE_Q6_K)
        exp = oracle.dequant_q6K(q, nblk * QK)
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32), err_msg=f"nblk={nblk}")


def test_encoder_golden_bitexact(ctx):
    x = GOLD["enc_x"]
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q6_K).reshape(-1, Q6K)
    exp = GOLD["enc_q"].reshape(-1, Q6K)
    bad = np.nonzero((got != exp).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ from quantize_q6_K, first {bad[:8]}"


def test_encoder_random_bitexact(ctx, oracle):
    rng = np.random.default_rng(602)
    x = np.concatenate([(rng.standard_normal((33, 768)) * 0.02).astype(np.float32).ravel(),
                        (rng.standard_t(4, size=(8, 4096)) * 0.05).astype(np.float32).ravel(),
                        (rng.standard_normal(QK * 5) * 1e3).astype(np.float32)])
    got = ctx.quantize_chunk(x, 1, x.size, type=TYPE_Q6_K).reshape(-1, Q6K)
    exp = oracle.quantize_q6K(x).reshape(-1, Q6K)
    bad = np.nonzero((got != exp).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:8]}"


def test_vec_dot_golden(ctx):
    o6 = o8 = 0
    for i, K in enumerate(GOLD["vd_K"]):
        K = int(K)
        n6, n8 = K // QK * Q6K, K // QK * 292
        w, a = GOLD["vd_q6"][o6:o6 + n6], GOLD["vd_q8"][o8:o8 + n8]
        o6 += n6
        o8 += n8
        got = ctx.vec_dot(K, w, a, type=TYPE_Q6_K)
        assert close_enough(got, GOLD["vd_avx2"][i]), (i, K, got, GOLD["vd_avx2"][i])


# ---- exact integer core -------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["enc", "rand"])
def test_subblock_sums_exact(ctx, oracle, kind):
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(603)
    for M, K in ((64, 4096), (37, 768), (16, 27648), (9, 5120)):
        W = _enc(oracle, rng, M, K) if kind == "enc" else _rand_blocks(rng, M * K // QK)
        x = rng.standard_normal(K).astype(np.float32)
        q8 = oracle.quantize_q8K(x)
        Wd = DeviceArray.from_host(W)
        xd = DeviceArray.from_host(x)
        Sd = DeviceArray(M * (K // QK) * 16, np.int32)
        ctx.subblock_sums(Wd.ptr, M, K, xd.ptr, Sd.ptr, type=TYPE_Q6_K)
        ctx.synchronize()
        got = Sd.to_host().reshape(M, -1)
        rb = K // QK * Q6K
        for r in range(M):
            exp = oracle.subblock_sums_q6K(K, W[r * rb:(r + 1) * rb], q8)
            np.testing.assert_array_equal(got[r], exp, err_msg=f"row {r} M={M} K={K}")


# ---- matvec ---------------------------------------------------------------------------------
@pytest.mark.parametrize("T", [1, 3, 8, 17])
def test_mul_mat_golden(ctx, T):
    M, K = (int(v) for v in GOLD["mm_MK"])
    W = ctx.upload(GOLD["mm_W"], M, K, type=TYPE_Q6_K)
    got = ctx.mul_mat(W, GOLD[f"mm_X{T}"])
    _check(got, GOLD[f"mm_Y{T}"], f"golden mul_mat T={T}")


@pytest.mark.parametrize("M,K,kind", [(4096, 4096, "enc"), (1024, 12288, "enc"), (300, 768, "enc"),
                                      (512, 5120, "enc"), (256, 27648, "enc"), (33000, 4096, "gpu_enc"),
                                      (64, 2048, "rand"), (96, 5120, "rand"), (64, 27648, "rand"),
                                      (160, 4096, "rand")])
def test_gemv_t1(ctx, oracle, M, K, kind):
    rng = np.random.default_rng(M * 7 + K)
    if kind == "enc":
        W = _enc(oracle, rng, M, K)
    elif kind == "gpu_enc":
        W = _gpu_enc(ctx, rng, M, K)
    else:
        W = _rand_blocks(rng, M * K // QK)
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q6_K), x)
    if kind == "rand":
        exact, mag = _exact_rows(oracle, W, M, K, x)
        _check_bounded(got, exact, mag, K // QK, f"q6k gemv M={M} K={K}")
        # the oracle (ggml's x86 order) obeys the same bound
        _check_bounded(oracle.mul_mat_type(TYPE_Q6_K, W, M, K, x), exact, mag, K // QK, "oracle")
    else:
        _check(got, oracle.mul_mat_type(TYPE_Q6_K, W, M, K, x), f"q6k gemv M={M} K={K}")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_GEMV_GENERIC": 1}, {"SPQ4K_DEC_WAVES": 8, "SPQ4K_DEC_DEPTH": 2},
                                 {"SPQ4K_DEC_WAVES": 16, "SPQ4K_DEC_XFIRST": 0}])
def test_gemv_t1_launch_shapes(oracle, env):
    rng = np.random.default_rng(604)
    c = context_with(env)
    try:
        for M, K in ((2048, 4096), (512, 12288)):
            W = _enc(oracle, rng, M, K)
            x = rng.standard_normal((1, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q6_K), x)
            _check(got, oracle.mul_mat_type(TYPE_Q6_K, W, M, K, x), f"{env} M={M} K={K}")
    finally:
        c.close()


@pytest.mark.parametrize("T", [2, 3, 5, 8, 9, 16, 40])
def test_mul_mat_batched(ctx, oracle, T):
    rng = np.random.default_rng(605 + T)
    for M, K in ((512, 4096), (200, 768)):
        W = _enc(oracle, rng, M, K)
        X = rng.standard_normal((T, K)).astype(np.float32)
        got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q6_K), X)
        _check(got, oracle.mul_mat_type(TYPE_Q6_K, W, M, K, X), f"q6k mul_mat T={T} M={M} K={K}")


@pytest.mark.parametrize("cfg", [14, 15, 16, 17, 18, 29])
def test_ring_launch_shapes(oracle, cfg):
    """Every Q6_K matrix-core launch shape, on ragged rows and tokens and on
    rows of an odd number of blocks (2-byte-aligned block starts)."""
    rng = np.random.default_rng(610 + cfg)
    c = context_with({"SPQ4K_GEMM_CFG": cfg})
    try:
        for M, K, T in ((300, 768, 5), (200, 4096, 33), (1000, 2048, 100)):
            W = _enc(oracle, rng, M, K)
            X = rng.standard_normal((T, K)).astype(np.float32)
            got = c.mul_mat(c.upload(W, M, K, type=TYPE_Q6_K), X)
            _check(got, oracle.mul_mat_type(TYPE_Q6_K, W, M, K, X), f"cfg={cfg} M={M} K={K} T={T}")
    finally:
        c.close()


@pytest.mark.parametrize("M,K,T", [(64, 27648, 64), (4096, 4096, 128), (512, 12288, 256), (96, 5120, 7)])
def test_ring_planned(ctx, oracle, M, K, T):
    """The planner's choice, including K splits (few rows, long K) and the
    reduction of their partial sums."""
    rng = np.random.default_rng(M + K + T)
    W = _gpu_enc(ctx, rng, M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=TYPE_Q6_K), X)
    _check(got, oracle.mul_mat_type(TYPE_Q6_K, W, M, K, X), f"planned M={M} K={K} T={T}")


def test_ring_extreme_operands(ctx, oracle):
    """Blocks at the ends of the folded operand range: scale -128 or 127 with
    6-bit values 0 or 63 (w = scale (q - 32) from -4064 to 4096), every
    combination, one combination a row so that with one-sign activations a
    row's blocks add up without cancellation; and arbitrary blocks held to the
    summation bound."""
    rng = np.random.default_rng(620)
    M, K, T = 64, 1024, 48
    nb = K // QK
    blk = np.zeros((M, nb, Q6K), np.uint8)
    for r in range(M):
        for b in range(nb):
            v = r % 4
            s = -128 if v < 2 else 127
            qv = 0 if v % 2 == 0 else 63
            blk[r, b, 0:128] = (qv & 15) | ((qv & 15) << 4)
            hb = qv >> 4
            blk[r, b, 128:192] = hb | (hb << 2) | (hb << 4) | (hb << 6)
            blk[r, b, 192:208] = np.array([s] * 16, np.int8).view(np.uint8)
            blk[r, b, 208:210] = np.array([2.0 ** -12 * (1 + r % 5)], np.float16).view(np.uint8)
    W = blk.ravel()
    X = np.abs(rng.standard_normal((T, K))).astype(np.float32)
    Wd = ctx.upload(W, M, K, type=TYPE_Q6_K)
    _check(ctx.mul_mat(Wd, X), oracle.mul_mat_type(TYPE_Q6_K, W, M, K, X), "extreme one-sign")
    W2 = _rand_blocks(rng, M * nb)
    X2 = rng.standard_normal((T, K)).astype(np.float32)
    exact, mag = _exact_rows(oracle, W2, M, K, X2)
    _check_bounded(ctx.mul_mat(ctx.upload(W2, M, K, type=TYPE_Q6_K), X2), exact, mag, nb, "arbitrary blocks")


@pytest.mark.parametrize("T", [4, 40])
def test_ring_matches_sdot4_slices(oracle, T):
    """SPQ4K_GEMM_MODE=1 keeps Q6_K batches on the sdot4 kernels: both paths
    within tolerance of the oracle on the same inputs."""
    rng = np.random.default_rng(630 + T)
    M, K = 384, 4096
    W = _enc(oracle, rng, M, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    exp = oracle.mul_mat_type(TYPE_Q6_K, W, M, K, X)
    for env in ({}, {"SPQ4K_GEMM_MODE": 1}):
        c = context_with(env)
        try:
            _check(c.mul_mat(c.upload(W, M, K, type=TYPE_Q6_K), X), exp, f"{env} T={T}")
        finally:
            c.close()


@pytest.mark.parametrize("T", [1, 4, 12])
def test_gemv_multi_device(ctx, oracle, T):
    """Two Q6_K matrices sharing one input in one launch (the device-pointer
    *_multi forms), each within tolerance of its own dense product."""
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(606 + T)
    K, shapes = 4096, (1024, 256)
    Ws = [_enc(oracle, rng, M, K) for M in shapes]
    X = rng.standard_normal((T, K)).astype(np.float32)
    wd = [ctx.upload(w, M, K, type=TYPE_Q6_K) for w, M in zip(Ws, shapes)]
    xd = DeviceArray.from_host(X)
    yd = [DeviceArray(T * M, np.float32) for M in shapes]
    if T <= 8:
        ctx.gemv_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    else:
        ctx.gemm_multi_dev(wd, xd.ptr, [y.ptr for y in yd], T)
    ctx.synchronize()
    for w, M, y in zip(Ws, shapes, yd):
        _check(y.to_host().reshape(T, M), oracle.mul_mat_type(TYPE_Q6_K, w, M, K, X), f"multi M={M} T={T}")


def test_mixed_types_rejected(ctx, oracle):
    import spq4k
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(607)
    K = 1024
    w4 = ctx.upload(oracle.quantize_q4K((rng.standard_normal((64, K)) * 0.02).astype(np.float32)), 64, K)
    w6 = ctx.upload(_enc(oracle, rng, 64, K), 64, K, type=TYPE_Q6_K)
    xd = DeviceArray.from_host(rng.standard_normal(K).astype(np.float32))
    y = [DeviceArray(64, np.float32), DeviceArray(64, np.float32)]
    with pytest.raises(spq4k.Spq4kError, match="EINVAL"):
        ctx.gemv_multi_dev([w4, w6], xd.ptr, [v.ptr for v in y], 1)
    with pytest.raises(spq4k.Spq4kError, match="EINVAL"):       # GGML_TYPE_Q3_K: not a type the library runs
        ctx.upload(np.zeros(210, np.uint8), 1, 256, type=11)


# ---- expert-gathered matvec -------------------------------------------------------------------
@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_mul_mat_id_golden(ctx, tag):
    E, M, K = (int(v) for v in GOLD["mmid_EMK"])
    bank = ctx.upload(GOLD["mmid_bank"], M, K, E, type=TYPE_Q6_K)
    got = ctx.mul_mat_id(bank, GOLD[f"mmid_X_{tag}"], GOLD[f"mmid_ids_{tag}"])
    _check(got, GOLD[f"mmid_Y_{tag}"], f"golden mul_mat_id {tag}")


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_MODE": 3}, {"SPQ4K_MOE_UNFUSED": 1}, {"SPQ4K_MOE_MODE": 2}, {"SPQ4K_MOE_RING_WAVES": 8}])
@pytest.mark.parametrize("T,ne11", [(1, 1), (3, 8), (12, 1), (32, 8)])
def test_moe(oracle, env, T, ne11):
    """A Q6_K expert bank of the MoE shape (down projection K = 768, and
    K = 2048) through every MoE path: the decode mapping (T <= 8), the
    single-launch kernel, and routing + Q8_K planes + grouped matvec."""
    rng = np.random.default_rng(608 + T)
    E, n_used = 32, 8
    c = context_with(env)
    try:
        for M, K in ((256, 768), (128, 2048)):
            bank = _enc(oracle, rng, E * M, K)
            ids = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            X = rng.standard_normal((T, ne11, K)).astype(np.float32)
            got = c.mul_mat_id(c.upload(bank, M, K, E, type=TYPE_Q6_K), X, ids)
            exp = oracle.mul_mat_id_type(TYPE_Q6_K, bank, M, K, E, X, ids)
            _check(got, exp, f"q6k moe {env} T={T} ne11={ne11} M={M} K={K}")
    finally:
        c.close()

"""GPU parity of the format conversions against the CPU oracle (bit-exact).

dequant (dequantize_row_q4_K), Q8_K (quantize_row_q8_K), the Q4_K encoder
(quantize_row_q4_K_ref) and the synthetic-data generator must be identical
bit for bit; the one-row vec_dot must be within the reference tolerance."""
import numpy as np
import pytest

from _oracle import close_enough

pytestmark = pytest.mark.gpu

SEED = 0xDEADBEEF


def _random_blocks(rng, nblk):
    """Arbitrary Q4_K blocks with finite fp16 d/dmin (any scale/qs bytes)."""
    b = rng.integers(0, 256, size=(nblk, 144), dtype=np.uint8)
    # d, dmin: clear the top exponent bit so they are finite (exp <= 15)
    b[:, 1] &= 0xBF
    b[:, 3] &= 0xBF
    return b.ravel()


def test_synth_matches_host(ctx, oracle):
    from spq4k.hip import DeviceArray
    n = 200_003
    for dist, cols, mult in ((0, 0, 1.0), (1, 5120, 8.0)):
        dev = DeviceArray(n, np.float32)
        ctx.synth_fill_dev(dev.ptr, n, 1234, dist, cols, 0.0, 0.02, mult, 777)
        ctx.synchronize()
        host = oracle.synth(n, 1234, dist, cols, 0.0, 0.02, mult, 777)
        np.testing.assert_array_equal(dev.to_host().view(np.uint32), host.view(np.uint32))


def test_dequant_bitexact(ctx, oracle):
    rng = np.random.default_rng(SEED)
    q = _random_blocks(rng, 4096)
    k = 4096 * 256
    got = ctx.to_float(q, k)
    exp = oracle.dequant(q, k)
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def _q8k_cases(rng):
    cases = [rng.standard_normal(256 * 64).astype(np.float32)]
    z = np.zeros(256, np.float32)
    cases.append(z)                                     # d = 0 branch
    t = np.zeros(256, np.float32); t[7] = 3.0; t[200] = -3.0; cases.append(t)    # tie: first wins (+)
    t = np.zeros(256, np.float32); t[7] = -3.0; t[200] = 3.0; cases.append(t)    # tie: first wins (-)
    cases.append(np.full(256, -0.5, np.float32))
    t = np.zeros(256, np.float32); t[255] = 1e-42; cases.append(t)               # subnormal max
    cases.append((rng.standard_normal(256) * 1e30).astype(np.float32))
    h = (np.arange(256, dtype=np.float32) - 128.0) / 2.0; cases.append(h)        # many .5 roundings
    t = rng.standard_normal(256).astype(np.float32); t[3] = np.nan; cases.append(t)
    t = np.zeros(256, np.float32); t[3] = -2.0; t[10] = 2.0; cases.append(t)      # tie inside one 16-lane share
    t = np.zeros(256, np.float32); t[9] = 2.0; t[2] = -2.0; cases.append(t)
    t = rng.standard_normal(256).astype(np.float32); t[40] = np.inf; cases.append(t)
    t = rng.standard_normal(256).astype(np.float32); t[41] = -np.inf; cases.append(t)
    t = rng.standard_normal(256).astype(np.float32); t[50] = -np.inf; t[60] = np.inf; cases.append(t)
    cases.append(np.full(256, np.nan, np.float32))                                # all NaN: d = 0
    cases.append(np.full(256, -0.0, np.float32))
    t = np.zeros(256, np.float32); t[255] = -7.0; cases.append(t)                 # max at the last index
    t = np.zeros(256, np.float32); t[0] = 7.0; t[255] = -7.0; cases.append(t)
    t = (rng.standard_normal(256) * 0.1).astype(np.float32); t[128] = 3.0; t[129] = -3.0; cases.append(t)
    return np.concatenate(cases)


def test_q8k_bitexact(ctx, oracle):
    rng = np.random.default_rng(SEED + 1)
    x = _q8k_cases(rng)
    got = ctx.from_float(x).reshape(-1, 292)
    exp = oracle.quantize_q8K(x).reshape(-1, 292)
    np.testing.assert_array_equal(got, exp)


def _encoder_cases(rng):
    rows = [(rng.standard_normal((32, 4096)) * 0.02).astype(np.float32).ravel()]
    t = rng.standard_t(4, size=(16, 5120)).astype(np.float32) * 0.02
    t[:, ::97] *= 8.0
    rows.append(t.ravel())
    rows.append(np.zeros(256, np.float32))
    rows.append(np.full(256, 0.3, np.float32))
    rows.append(np.full(256, -0.3, np.float32))
    s = np.zeros(256, np.float32); s[17] = 5.0; rows.append(s)
    rows.append(np.abs(rng.standard_normal(256)).astype(np.float32))
    rows.append(-np.abs(rng.standard_normal(256)).astype(np.float32))
    rows.append((rng.standard_normal(256) * 1e-30).astype(np.float32))
    rows.append((rng.standard_normal(256) * 1e4).astype(np.float32))
    return np.concatenate(rows)


def test_q4k_encoder_bitexact(ctx, oracle):
    rng = np.random.default_rng(SEED + 2)
    x = _encoder_cases(rng)
    got = ctx.quantize_chunk(x, 1, x.size)
    exp = oracle.quantize_q4K(x)
    bad = np.nonzero((got.reshape(-1, 144) != exp.reshape(-1, 144)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:8]}"


def test_vec_dot_one_row(ctx, oracle):
    rng = np.random.default_rng(SEED + 3)
    for K in (256, 768, 4096, 27648):
        w = oracle.quantize_q4K((rng.standard_normal(K) * 0.02).astype(np.float32))
        y = oracle.quantize_q8K(rng.standard_normal(K).astype(np.float32))
        got = ctx.vec_dot(K, w, y)
        exp = oracle.vec_dot(K, w, y, "avx2")
        assert close_enough(got, exp), (K, got, exp)

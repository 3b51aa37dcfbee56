"""GPU parity of the T = 1 decode GEMV (gemv_decode_kernel) and of every launch
shape the planner can pick, against the CPU oracle.

The decode kernel serves K = 4096, 5120, 12288 and 27648 (the 8B and large-K
shapes) from instances compiled for that row length, and every other K up to
28672 (Q6_K and Q5_K: up to 8192) from instances that read the row length at
run time, one per multiple of 16 blocks; the generic kernel serves longer
rows at T = 1, and T = 2, 3. Launch shapes are forced through the
context's environment overrides (read when a context is created), so each
(waves, depth, x-first) instantiation and each lanes-per-row choice of the
generic kernel is checked, not only the ones the planner picks for the sizes
below. Tolerance: the reference's close_enough (1e-4 relative or 1e-5
absolute, tests/desktop/test_sp_kernels.cpp:34-48) against the oracle's
restatement of ggml's x86 path (bit-identical to the reference's own
ggml_vec_dot_q4_K_q8_K, pinned in test_oracle_golden.py)."""
import numpy as np
import pytest

from _envctx import context_with as _context_with
from _oracle import close_enough, parity_ok

pytestmark = pytest.mark.gpu


def _weights(oracle, rng, M, K, scale=0.02):
    return oracle.quantize_q4K((rng.standard_normal((M, K)) * scale).astype(np.float32))


def _check(got, exp, what, exact=None):
    """close_enough of the oracle (ggml's x86 order); with `exact`, the parity
    bar's either-or: of the oracle or of the dequant-then-dot value"""
    ok = close_enough(got, exp) if exact is None else parity_ok(got, exp, exact)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; first {tuple(i)} "
                             f"got {got[tuple(i)]!r} exp {exp[tuple(i)]!r}")


@pytest.mark.parametrize("M,K", [(1, 4096), (100, 4096), (4096, 4096), (37, 12288), (4096, 12288), (300, 5120),
                                 (3000, 5120), (5, 27648), (700, 27648)])
def test_decode_single(ctx, oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    W = _weights(oracle, rng, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K)
    _check(ctx.mul_mat(Wd, x), oracle.mul_mat(W, M, K, x), f"decode M={M} K={K}", oracle.mul_mat_dq_f64(12, W, M, K, x))


@pytest.mark.parametrize("K,shapes", [(4096, (4096, 1024, 1024)), (4096, (12288, 12288)), (12288, (4096,)),
                                      (4096, (5, 300, 77, 1))])
def test_decode_grouped(ctx, oracle, K, shapes):
    """q/k/v and gate/up as one launch: rows of all matrices in one sweep."""
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(sum(shapes) + K)
    Ws = [_weights(oracle, rng, M, K) for M in shapes]
    x = rng.standard_normal(K).astype(np.float32)
    wd = [ctx.upload(w, M, K) for w, M in zip(Ws, shapes)]
    xd = DeviceArray.from_host(x)
    ys = [DeviceArray.from_host(np.full(M, np.nan, np.float32)) for M in shapes]
    ctx.gemv_multi_dev(wd, xd.ptr, [y.ptr for y in ys], 1)
    ctx.synchronize()
    for w, M, y in zip(Ws, shapes, ys):
        _check(y.to_host()[None], oracle.mul_mat(w, M, K, x[None]), f"grouped K={K} M={M}")


_CFGS = [(w, d, xf) for w in (8, 12, 16) for d in (1, 2) for xf in (0, 1)]


@pytest.mark.parametrize("waves,depth,xfirst", _CFGS)
def test_decode_launch_shapes(oracle, waves, depth, xfirst):
    """Every compiled instantiation, with a small grid so that each wave walks
    several rows (the depth pipeline and its ragged tail; 2000 rows over 24
    waves: 84 rows a wave, past the 64 results one register collects) and a
    full grid (K = 27648 runs 8 waves and one row in flight whatever is
    asked)."""
    rng = np.random.default_rng(1000 + waves * 10 + depth * 2 + xfirst)
    cases = [(1000, 4096), (2000, 4096), (333, 12288), (210, 5120), (77, 27648), (130, 2048), (90, 8192), (61, 14336),
             (40, 20480), (33, 24576), (29, 28416)]
    data = [(M, K, _weights(oracle, rng, M, K), rng.standard_normal((1, K)).astype(np.float32)) for M, K in cases]
    for grid in (3, 0):
        env = {"SPQ4K_DEC_WAVES": waves, "SPQ4K_DEC_DEPTH": depth, "SPQ4K_DEC_XFIRST": xfirst}
        if grid:
            env["SPQ4K_DEC_GRID"] = grid
        c = _context_with(env)
        try:
            for M, K, W, x in data:
                Wd = c.upload(W, M, K)
                _check(c.mul_mat(Wd, x), oracle.mul_mat(W, M, K, x),
                       f"decode waves={waves} depth={depth} xfirst={xfirst} grid={grid} M={M} K={K}")
                Wd.free()
        finally:
            c.close()


@pytest.mark.parametrize("bpr", [1, 2, 4, 8])
def test_generic_lanes_per_row(oracle, bpr):
    """The generic kernel at each lanes-per-row choice (T = 1 and T = 3)."""
    c = _context_with({"SPQ4K_GEMV_GENERIC": 1, "SPQ4K_GEMV_BPR": bpr})
    rng = np.random.default_rng(77 + bpr)
    try:
        for M, K, T in ((300, 4096, 1), (129, 12288, 1), (64, 5120, 3)):
            W = _weights(oracle, rng, M, K)
            x = rng.standard_normal((T, K)).astype(np.float32)
            Wd = c.upload(W, M, K)
            _check(c.mul_mat(Wd, x), oracle.mul_mat(W, M, K, x), f"generic bpr={bpr} M={M} K={K} T={T}")
            Wd.free()
    finally:
        c.close()


def test_decode_matches_generic(ctx, oracle):
    """Same bytes through the decode and the generic kernels: both within the
    tolerance of the oracle and of each other."""
    rng = np.random.default_rng(31)
    M, K = 2048, 4096
    W = _weights(oracle, rng, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    a = ctx.mul_mat(ctx.upload(W, M, K), x)
    g = _context_with({"SPQ4K_GEMV_GENERIC": 1})
    try:
        b = g.mul_mat(g.upload(W, M, K), x)
    finally:
        g.close()
    exp = oracle.mul_mat(W, M, K, x)
    _check(a, exp, "decode")
    _check(b, exp, "generic")
    _check(a, b, "decode vs generic")


def test_decode_repeatable(ctx, oracle):
    """Fixed combination order: bit-identical reruns."""
    rng = np.random.default_rng(9)
    M, K = 1536, 12288
    Wd = ctx.upload(_weights(oracle, rng, M, K), M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    a = ctx.mul_mat(Wd, x)
    for _ in range(3):
        np.testing.assert_array_equal(ctx.mul_mat(Wd, x), a)


@pytest.mark.parametrize("K", [256, 512, 2048, 3072, 4352, 6144, 8192, 11264, 14336, 16384, 18432, 20480, 24576,
                               28672])
def test_decode_any_k(ctx, oracle, K):
    """Row lengths without an exact instance: the runtime-length instance of
    the next multiple of 16 blocks (a partial last pass of 16 blocks where K
    is not a multiple of 4096), against the oracle and the generic kernel."""
    rng = np.random.default_rng(K)
    M = 2048 if K <= 8192 else 384
    W = _weights(oracle, rng, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    a = ctx.mul_mat(ctx.upload(W, M, K), x)
    exp = oracle.mul_mat(W, M, K, x)
    _check(a, exp, f"decode any-K M={M} K={K}", oracle.mul_mat_dq_f64(12, W, M, K, x))
    g = _context_with({"SPQ4K_GEMV_GENERIC": 1})
    try:
        b = g.mul_mat(g.upload(W, M, K), x)
    finally:
        g.close()
    _check(a, b, f"decode vs generic K={K}")


@pytest.mark.parametrize("qtype", [13, 14])
@pytest.mark.parametrize("K", [512, 2048, 5120, 8192])
def test_decode_any_k_q5k_q6k(ctx, oracle, qtype, K):
    """Q5_K / Q6_K rows of up to 32 blocks in the runtime-length instances"""
    rng = np.random.default_rng(K + qtype)
    M = 1024
    W = oracle.quantize(qtype, (rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = ctx.mul_mat(ctx.upload(W, M, K, type=qtype), x)
    _check(got, oracle.mul_mat_type(qtype, W, M, K, x), f"decode type={qtype} K={K}",
           oracle.mul_mat_dq_f64(qtype, W, M, K, x))


@pytest.mark.parametrize("M,K,shape", [(4096, 4096, (16, 1)), (6144, 4096, (16, 1)), (33000, 4096, (8, 2)),
                                       (4096, 12288, (8, 2)), (300, 12288, (8, 2))])
def test_decode_stamps(ctx, oracle, M, K, shape):
    """The timestamped decode instances (spq4k_set_decode_stamps,
    include/spq4k_diag.h): the same outputs bit for bit as the plain
    instances, one stamp set per wave of the launch, each wave's stamps in
    order (start <= barrier <= first row <= last row), and -EINVAL for a
    buffer too small or a shape without a timestamped instance."""
    from spq4k import Spq4kError
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(M + K)
    W = _weights(oracle, rng, M, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    Wd = ctx.upload(W, M, K)
    plain = ctx.mul_mat(Wd, x)
    n = 256 * 16 * 4
    buf = DeviceArray(n, np.uint64)
    buf.fill_byte(0)
    try:
        ctx.set_decode_stamps(buf.ptr, n)
        stamped = ctx.mul_mat(Wd, x)
        ctx.set_decode_stamps(None)
        np.testing.assert_array_equal(stamped.view(np.uint32), plain.view(np.uint32))
        _check(stamped, oracle.mul_mat(W, M, K, x), f"stamped decode M={M} K={K}")
        s = buf.to_host().reshape(-1, 4).astype(np.int64)
        live = s[:, 0] != 0
        waves, _ = shape
        grid = min(256, (M + waves - 1) // waves)
        assert live.sum() == grid * waves and live[:grid * waves].all(), (int(live.sum()), grid * waves)
        s = s[live]
        rows = s[:, 2] != 0
        assert rows.sum() == min(M, grid * waves)
        assert (s[:, 0] <= s[:, 1]).all() and (s[:, 1] <= s[:, 3]).all()
        assert (s[rows, 1] <= s[rows, 2]).all() and (s[rows, 2] <= s[rows, 3]).all()
        assert (s[:, 3] - s[:, 0]).max() < 100_000_000   # under a second of the 100 MHz clock
        # errors while stamps are set: a buffer smaller than grid * waves * 4,
        # and a row length without a timestamped instance
        ctx.set_decode_stamps(buf.ptr, 4 * grid * waves - 1)
        with pytest.raises(Spq4kError):
            ctx.mul_mat(Wd, x)
        ctx.set_decode_stamps(buf.ptr, n)
        W2 = _weights(oracle, rng, 64, 8192)
        W2d = ctx.upload(W2, 64, 8192)
        x2 = rng.standard_normal((1, 8192)).astype(np.float32)
        with pytest.raises(Spq4kError):
            ctx.mul_mat(W2d, x2)
        ctx.set_decode_stamps(None)
        _check(ctx.mul_mat(W2d, x2), oracle.mul_mat(W2, 64, 8192, x2), "after stamps off")
        W2d.free()
    finally:
        ctx.set_decode_stamps(None)
        buf.free()
        Wd.free()

"""GPU parity at the full shapes of two BASELINE configurations that the
kernel-level tests reach only at reduced sizes:

- configs[2], prefill at T = 512 on the 8B matrices (6144 x 4096 q/k/v,
  12288 x 4096 gate/up, 4096 x 12288 down): the planner's own launch shape
  for those sizes (32 x 32 matrix-core tiles over eight 64-token tiles), and
  that shape forced on smaller matrices;
- configs[4], large-K matvecs (5120 x 27648 and 27648 x 5120, T = 1, 4, 8)
  on its skewed weights: seeded Student-t(nu = 4) * 0.02 with 1% of the input
  columns scaled by 8, synthesised and Q4_K-encoded on the GPU exactly as the
  bench makes them, then compared on the same bytes.

The GPU computes every row of the full matrix; the CPU oracle (ggml's x86
order, pinned to the reference) recomputes a sample of rows spread over the
matrix (rows of a matmul are independent). Tolerance: the north star's bar,
each output within close_enough (1e-4 relative or 1e-5 absolute,
tests/desktop/test_sp_kernels.cpp:34-48) of ggml_vec_dot_q4_K_q8_K's value or
of the dequant-then-dot value (sum of dequant(W) * dequant(Q8_K(x)) in
double). The skewed weights need the second: where a row's products cancel
(sums of |terms| 4000 times the result), ggml's own x86 order lands more than
1e-4 of the result away from the exact sum."""
import numpy as np
import pytest

from _oracle import parity_ok

pytestmark = pytest.mark.gpu
Q4K = 144


def _sample_rows(M, n=96):
    """first, middle and last rows, plus a spread"""
    rows = set(range(0, min(M, 24))) | set(range(M // 2 - 12, M // 2 + 12)) | set(range(M - 24, M))
    rows |= set(np.linspace(0, M - 1, n - len(rows) if n > len(rows) else 8).astype(int).tolist())
    return np.array(sorted(r for r in rows if 0 <= r < M))


def _rows_of(Wbytes, K, rows):
    rb = K // 256 * Q4K
    return np.ascontiguousarray(Wbytes.reshape(-1, rb)[rows]).ravel()


def _check(got, exp, exact, what):
    ok = parity_ok(got, exp, exact)
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        raise AssertionError(f"{what}: {int((~ok).sum())}/{ok.size} outside tolerance; first {i} got {got[i]} "
                             f"exp {exp[i]}")


def _device_weights(ctx, M, K, seed, dist, outlier, oracle=None, check_rows=()):
    """Q4_K weights synthesised and encoded on the device (as bench.py makes
    them); returns the device weights and their bytes. With `oracle`, the
    fp32 values of `check_rows` must equal the oracle's synthesis and their
    blocks the oracle's encoding of them, bit for bit."""
    import spq4k
    from spq4k.hip import DeviceArray, download
    tmp = DeviceArray(M * K, np.float32)
    W = ctx.alloc_weights(M, K)
    ctx.synth_fill_dev(tmp.ptr, M * K, seed, dist, K, 0.0, 0.02, outlier, 0)
    ctx.quantize_chunk_dev(spq4k.TYPE_Q4_K, tmp.ptr, W.data_ptr, M, K)
    ctx.synchronize()
    wb = download(W.data_ptr, W.nbytes)
    for r in check_rows:
        dev = download(tmp.ptr + 4 * r * K, 4 * K).view(np.float32)
        exp = oracle.synth(K, seed, dist, K, 0.0, 0.02, outlier, r * K)
        assert np.array_equal(dev.view(np.uint32), exp.view(np.uint32)), f"synthesis of row {r}"
        assert np.array_equal(_rows_of(wb, K, [r]), oracle.quantize_q4K(exp)), f"encoding of row {r}"
    tmp.free()
    return W, wb


def _run(ctx, Ws, X, T):
    from spq4k.hip import DeviceArray
    xd = DeviceArray.from_host(X)
    ys = [DeviceArray((T, w.M)) for w in Ws]
    if len(Ws) == 1:
        ctx.mul_mat_dev(Ws[0], xd.ptr, ys[0].ptr, T)
    else:
        ctx.gemm_multi_dev(Ws, xd.ptr, [y.ptr for y in ys], T)
    ctx.synchronize()
    return [y.to_host() for y in ys]


@pytest.mark.parametrize("shapes", [[(6144, 4096)], [(12288, 4096), (12288, 4096)], [(4096, 12288)]],
                         ids=["qkv", "gate_up", "down"])
def test_prefill_t512_planner(ctx, oracle, shapes):
    import spq4k
    T = 512
    K = shapes[0][1]
    rng = np.random.default_rng(512 + K + len(shapes))
    X = rng.standard_normal((T, K)).astype(np.float32)
    made = [_device_weights(ctx, M, K, 900 + i, spq4k.DIST_NORMAL, 1.0) for i, (M, _) in enumerate(shapes)]
    outs = _run(ctx, [w for w, _ in made], X, T)
    for (w, wb), Y in zip(made, outs):
        rows = _sample_rows(w.M)
        Wr = _rows_of(wb, K, rows)
        exp = oracle.mul_mat(Wr, len(rows), K, X)
        _check(Y[:, rows], exp, oracle.mul_mat_dq_f64(12, Wr, len(rows), K, X), f"prefill T={T} {w.M}x{K}")
        w.free()


@pytest.mark.parametrize("cfg", [11, 32])
@pytest.mark.parametrize("M,K,T", [(512, 4096, 512), (256, 12288, 512), (300, 4096, 500)])
def test_prefill_t512_forced_32x32(oracle, M, K, T, cfg):
    """The 32 x 32-tile launch shapes -- 11 (256 rows x 64 tokens, 8 waves)
    and 32 (128 rows x 64 tokens, 4 waves, two workgroups a CU: the planner's
    choice from T = 256 on 12288 rows or more) -- on matrices the oracle
    covers whole, with a ragged token tile at T = 500."""
    from _envctx import context_with
    c = context_with({"SPQ4K_GEMM_CFG": cfg})
    try:
        rng = np.random.default_rng(M + T)
        W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
        X = rng.standard_normal((T, K)).astype(np.float32)
        Wd = c.upload(W, M, K)
        _check(c.mul_mat(Wd, X), oracle.mul_mat(W, M, K, X), oracle.mul_mat_dq_f64(12, W, M, K, X),
               f"cfg {cfg} {M}x{K} T={T}")
        Wd.free()
    finally:
        c.close()


@pytest.mark.parametrize("M,K", [(5120, 27648), (27648, 5120)])
@pytest.mark.parametrize("T", [1, 4, 8])
def test_largek_skewed(ctx, oracle, M, K, T):
    import spq4k
    w, wb = _device_weights(ctx, M, K, 4242 + T, spq4k.DIST_STUDENT_T4, 8.0, oracle, (0, M // 2, M - 1))
    rng = np.random.default_rng(M + 7 * T)
    X = rng.standard_normal((T, K)).astype(np.float32)
    (Y,) = _run(ctx, [w], X, T)
    rows = _sample_rows(M, 160)
    Wr = _rows_of(wb, K, rows)
    exp = oracle.mul_mat(Wr, len(rows), K, X)
    _check(Y[:, rows], exp, oracle.mul_mat_dq_f64(12, Wr, len(rows), K, X), f"large-K skewed {M}x{K} T={T}")
    w.free()

"""GPU parity of the fp32-activation dequant-then-dot (spq4k_dequant_matvec,
include/spq4k.h): the arithmetic of the reference's scalar BurnHard matvec
beast_matvec (desktop/beast_canyon/sp_beast_canyon.c:1122-1134), which
dequantises each Q4_K row and dots it with the activations as given (no Q8_K).

Checks:
  - one-hot activations: y[r] is then one dequantised weight exactly (a
    single non-zero product, times 1.0, plus zeros), so the kernel's
    dequantisation is compared bit for bit with the oracle's
    dequantize_row_q4_K (itself pinned to the reference);
  - random activations, against the oracle's restatement of beast_matvec
    (pinned bit for bit to the reference's own beast_matvec, compiled from its
    source) within close_enough (1e-4 relative or 1e-5 absolute,
    tests/desktop/test_sp_kernels.cpp:34-48), or of the double-precision
    dequant-then-dot sum where the fp32 orders part (products that cancel);
  - shapes: the 8B shapes, the large-K skewed weights of BASELINE configs[4],
    the MoE expert shapes, several tokens, ragged K (a partial pass of 16
    blocks)."""
import numpy as np
import pytest

from _oracle import TYPE_Q4_K, close_enough

pytestmark = pytest.mark.gpu


def _weights(ctx, M, K, seed, dist=0, mult=1.0):
    from spq4k.hip import DeviceArray, download
    w = ctx.alloc_weights(M, K)
    tmp = DeviceArray(M * K, np.float32)
    ctx.synth_fill_dev(tmp.ptr, M * K, seed, dist, K, 0.0, 0.02, mult, 0)
    ctx.quantize_chunk_dev(TYPE_Q4_K, tmp.ptr, w.data_ptr, M, K)
    ctx.synchronize()
    tmp.free()
    return w, download(w.data_ptr, w.nbytes)


def _rows(wb, K, rows):
    rb = K // 256 * 144
    return np.ascontiguousarray(wb.reshape(-1, rb)[rows]).ravel()


def test_dequant_matvec_one_hot_is_dequant(ctx, oracle):
    M, K = 64, 4096
    w, wb = _weights(ctx, M, K, 5)
    cols = np.array([0, 1, 31, 32, 63, 64, 255, 256, 1000, 2047, 2048, 4095])
    X = np.zeros((cols.size, K), np.float32)
    X[np.arange(cols.size), cols] = 1.0
    got = ctx.dequant_matvec(w, X)
    deq = oracle.dequant(wb, M * K).reshape(M, K)
    exp = deq[:, cols].T
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(exp, np.float32).view(np.uint32))
    w.free()


@pytest.mark.parametrize("K", [256, 512, 1024, 3072, 4096])
def test_dequant_matvec_one_hot_one_token(ctx, oracle, K):
    """one token with rows of at most 16 blocks (the one-token kernel, every
    lane count): one-hot activations give the dequantised weights bit for bit"""
    M = 333
    w, wb = _weights(ctx, M, K, 11 + K)
    deq = oracle.dequant(wb, M * K).reshape(M, K)
    for c in (0, 33, K // 2 + 5, K - 1):
        x = np.zeros((1, K), np.float32)
        x[0, c] = 1.0
        got = ctx.dequant_matvec(w, x)
        assert np.array_equal(got[0].view(np.uint32), np.ascontiguousarray(deq[:, c]).view(np.uint32)), f"K={K} col {c}"
    w.free()


@pytest.mark.parametrize("M,K,T,dist", [(4096, 4096, 1, 0), (256, 12288, 1, 0), (300, 2048, 3, 0), (768, 2048, 1, 0),
                                        (2048, 768, 8, 0), (96, 27648, 1, 1), (512, 5120, 4, 1), (40, 4352, 11, 0),
                                        (12288, 4096, 1, 1), (1001, 256, 1, 0), (37, 1024, 1, 0), (5000, 3072, 1, 0),
                                        (130, 512, 1, 1), (1, 4096, 1, 0), (3, 256, 1, 0)])
def test_dequant_matvec_vs_beast(ctx, oracle, M, K, T, dist):
    rng = np.random.default_rng(M + K + T)
    w, wb = _weights(ctx, M, K, 7 + T, dist, 8.0 if dist else 1.0)
    X = rng.standard_normal((T, K)).astype(np.float32)
    got = ctx.dequant_matvec(w, X)
    rows = np.unique(np.concatenate([np.arange(min(M, 24)), np.linspace(0, M - 1, 96).astype(int),
                                     np.arange(max(0, M - 8), M)]))
    Wr = _rows(wb, K, rows)
    exact = oracle.mul_mat_dequant_f64(TYPE_Q4_K, Wr, rows.size, K, X)
    for t in range(T):
        beast = oracle.beast_matvec(TYPE_Q4_K, Wr, rows.size, K, X[t])
        ok = close_enough(got[t, rows], beast) | close_enough(got[t, rows], exact[t])
        assert ok.all(), (f"M={M} K={K} T={T} t={t}: {int((~ok).sum())}/{ok.size} outside tolerance; "
                          f"first row {rows[np.argmax(~ok)]}")
    w.free()


def test_dequant_matvec_rejects(ctx):
    import spq4k
    from spq4k.hip import DeviceArray
    w, _ = _weights(ctx, 8, 256, 1)
    x = DeviceArray(256, np.float32)
    y = DeviceArray(8, np.float32)
    with pytest.raises(spq4k.Spq4kError):
        ctx.dequant_matvec_dev(w, x.ptr + 4, y.ptr, 1)   # misaligned activations
    with pytest.raises(spq4k.Spq4kError):
        ctx.dequant_matvec_dev(w, x.ptr, y.ptr, 0)
    big = ctx.alloc_weights(1, 33 * 1024)
    with pytest.raises(spq4k.Spq4kError):
        ctx.dequant_matvec(big, np.zeros((1, 33 * 1024), np.float32))

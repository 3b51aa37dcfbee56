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
    blocks).
The same for Q5_K, Q6_K and Q8_0 rows (the rows beast_dequant_row dispatches,
sp_beast_canyon.c:1087-1106): one-hot inputs against the format's own
dequantiser (the oracle's, pinned to ggml's to_float), random inputs against
the oracle's beast_matvec loop over it (for Q8_0 pinned to the reference's own
beast_matvec) or the double sum; Q8_0 rows whose K is not a multiple of 256
(partial groups of eight blocks)."""
import numpy as np
import pytest

from _oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, close_enough

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


def _typed(ctx, oracle, qtype, M, K, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    W = oracle.quantize(qtype, (rng.standard_normal((M, K)) * scale).astype(np.float32))
    return ctx.upload(W, M, K, type=qtype), W


@pytest.mark.parametrize("qtype", [TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("K", [256, 1024, 4096, 5120, 12288])
def test_dequant_matvec_types_one_hot(ctx, oracle, qtype, K):
    """one-hot inputs: the format's dequantised weights bit for bit (+0 for a
    weight of -0, which a sum from 0.0 returns as +0), one token and three"""
    M = 70
    w, W = _typed(ctx, oracle, qtype, M, K, qtype * 100 + K)
    wd = oracle.to_float(qtype, W, M * K).reshape(M, K) + np.float32(0)
    cols = np.array([0, 15, 16, 31, 32, 127, 128, 191, K // 2 + 3, K - 1])
    X = np.zeros((cols.size, K), np.float32)
    X[np.arange(cols.size), cols] = 1.0
    got1 = np.stack([ctx.dequant_matvec(w, X[i:i + 1])[0] for i in range(cols.size)])
    got3 = ctx.dequant_matvec(w, X)
    exp = np.ascontiguousarray(wd[:, cols].T)
    assert np.array_equal(got1.view(np.uint32), exp.view(np.uint32)), f"type {qtype} K={K} one token"
    assert np.array_equal(got3.view(np.uint32), exp.view(np.uint32)), f"type {qtype} K={K} {cols.size} tokens"
    w.free()


@pytest.mark.parametrize("K", [32, 96, 2880, 4128])
def test_dequant_matvec_q8_0_ragged_groups(ctx, oracle, K):
    """Q8_0 rows of K a multiple of 32 but not of 256 (the last group of eight
    blocks partial): one-hot bit for bit at the row's last values, random
    inputs against the reference-pinned beast_matvec"""
    M = 45
    w, W = _typed(ctx, oracle, TYPE_Q8_0, M, K, K)
    wd = oracle.to_float(TYPE_Q8_0, W, M * K).reshape(M, K) + np.float32(0)
    for c in sorted({0, K - 33, K - 32, K - 1}):
        if c < 0:
            continue
        x = np.zeros((1, K), np.float32)
        x[0, c] = 1.0
        assert np.array_equal(ctx.dequant_matvec(w, x)[0].view(np.uint32), wd[:, c].view(np.uint32)), f"K={K} col {c}"
    x = np.random.default_rng(K + 1).standard_normal(K).astype(np.float32)
    got = ctx.dequant_matvec(w, x[None, :])[0]
    beast = oracle.beast_matvec(TYPE_Q8_0, W, M, K, x)
    exact = oracle.mul_mat_dequant_f64(TYPE_Q8_0, W, M, K, x[None, :])[0]
    ok = close_enough(got, beast) | close_enough(got, exact)
    assert ok.all(), f"K={K}: {int((~ok).sum())} of {ok.size}"
    w.free()


@pytest.mark.parametrize("qtype", [TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("M,K,T", [(4096, 4096, 1), (300, 2048, 3), (768, 2048, 1), (2048, 768, 5), (96, 14336, 1),
                                   (40, 4352, 11), (1001, 256, 2), (5, 27648, 1), (257, 512, 8)])
def test_dequant_matvec_types_vs_beast(ctx, oracle, qtype, M, K, T):
    """random inputs against beast_matvec's loop over the format's dequantiser
    (the oracle's; for Q8_0 pinned to the reference's own) within
    close_enough, or of the double-precision dequant-then-dot where the fp32
    orders part"""
    w, W = _typed(ctx, oracle, qtype, M, K, M + K + T + qtype)
    X = np.random.default_rng(M * T + K).standard_normal((T, K)).astype(np.float32)
    got = ctx.dequant_matvec(w, X)
    rb = W.size // M
    rows = np.unique(np.concatenate([np.arange(min(M, 16)), np.linspace(0, M - 1, 48).astype(int),
                                     np.arange(max(0, M - 4), M)]))
    Wr = np.ascontiguousarray(W.reshape(M, rb)[rows]).ravel()
    exact = oracle.mul_mat_dequant_f64(qtype, Wr, rows.size, K, X)
    for t in range(T):
        beast = oracle.beast_matvec(qtype, Wr, rows.size, K, X[t])
        ok = close_enough(got[t, rows], beast) | close_enough(got[t, rows], exact[t])
        assert ok.all(), (f"type {qtype} M={M} K={K} T={T} t={t}: {int((~ok).sum())}/{ok.size} outside tolerance; "
                          f"first row {rows[np.argmax(~ok)]}")
    w.free()


def test_dequant_matvec_types_reject(ctx, oracle):
    """an expert bank (E > 1) and rows longer than the staging area are refused"""
    import spq4k
    bank, _ = _typed(ctx, oracle, TYPE_Q8_0, 8, 256, 1)
    rng = np.random.default_rng(2)
    E2 = ctx.upload(oracle.quantize(TYPE_Q6_K, (rng.standard_normal((16, 256)) * 0.05).astype(np.float32)), 8, 256,
                    E=2, type=TYPE_Q6_K)
    with pytest.raises(spq4k.Spq4kError):
        ctx.dequant_matvec(E2, np.zeros((1, 256), np.float32))
    long_ = ctx.alloc_weights(1, 33 * 1024, type=TYPE_Q8_0)
    with pytest.raises(spq4k.Spq4kError):
        ctx.dequant_matvec(long_, np.zeros((1, 33 * 1024), np.float32))
    long_.free()
    bank.free()
    E2.free()

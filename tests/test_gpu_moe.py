"""GPU parity of the expert-gathered Q4_K matvec (GGML_OP_MUL_MAT_ID).

Against the reference's own outputs (golden vectors) and against the CPU
oracle's ggml_compute_forward_mul_mat_id restatement at the 30B-A3B-like
shapes of BASELINE configs[3] (128 experts, top-8 routing, gate/up 768x2048,
down 2048x768, T = 1..32). Tolerance: the reference's close_enough
(1e-4 relative or 1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48)."""
import os

import numpy as np
import pytest

from _oracle import close_enough

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _check(got, exp, what):
    ok = close_enough(got, exp)
    assert ok.all(), f"{what}: {int((~ok).sum())}/{ok.size} outside tolerance, first {np.argwhere(~ok)[0]}"


def _gpu_bank(ctx, E, M, K, seed):
    """Q4_K expert bank synthesised on the GPU (encoder pinned bit-exact in
    test_gpu_convert); returns the device weights and a host copy."""
    from spq4k.hip import DeviceArray, _lib, check
    w = ctx.alloc_weights(M, K, E)
    tmp = DeviceArray(E * M * K, np.float32)
    ctx.synth_fill_dev(tmp.ptr, E * M * K, seed, 0, K, 0.0, 0.02, 1.0, 0)
    ctx.quantize_q4K_dev(tmp.ptr, w.data_ptr, E * M, K)
    ctx.synchronize()
    tmp.free()
    host = np.empty(w.nbytes, np.uint8)
    check(_lib().hipMemcpy(host.ctypes.data, w.data_ptr, w.nbytes, 2), "D2H")
    return w, host


def _topk_ids(rng, T, E, k):
    logits = rng.standard_normal((T, E)).astype(np.float32)
    return np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)


@pytest.mark.parametrize("tag", ["2_1", "4_4"])
def test_moe_golden(ctx, tag):
    G = np.load(os.path.join(HERE, "golden", "q4k_golden.npz"))
    E, M, K = (int(v) for v in G["mmid_EMK"])
    bank = ctx.upload(G["mmid_bank"], M, K, E)
    got = ctx.mul_mat_id(bank, G[f"mmid_X_{tag}"], G[f"mmid_ids_{tag}"])
    _check(got, G[f"mmid_Y_{tag}"], f"golden mul_mat_id {tag}")


@pytest.mark.parametrize("M,K", [(768, 2048), (2048, 768)])
@pytest.mark.parametrize("T,ne11", [(1, 1), (4, 8), (32, 1), (32, 8)])
def test_moe_30b_shapes(ctx, oracle, M, K, T, ne11):
    E, k = 128, 8
    rng = np.random.default_rng(M + K + T * 7 + ne11)
    bank, host = _gpu_bank(ctx, E, M, K, seed=M * 3 + K)
    ids = _topk_ids(rng, T, E, k)
    X = rng.standard_normal((T, ne11, K)).astype(np.float32)
    got = ctx.mul_mat_id(bank, X, ids)
    exp = oracle.mul_mat_id(host, M, K, E, X, ids)
    _check(got, exp, f"moe M={M} K={K} T={T} ne11={ne11}")


def test_moe_many_tokens_per_expert(ctx, oracle):
    # every token picks the same 8 experts: 32 pairs per expert, several TC chunks
    E, M, K, T, k = 16, 256, 1024, 32, 8
    rng = np.random.default_rng(77)
    bank, host = _gpu_bank(ctx, E, M, K, seed=5)
    ids = np.tile(np.array([3, 1, 4, 15, 9, 2, 6, 5], np.int32), (T, 1))
    X = rng.standard_normal((T, k, K)).astype(np.float32)
    _check(ctx.mul_mat_id(bank, X, ids), oracle.mul_mat_id(host, M, K, E, X, ids), "moe shared experts")


def test_moe_rejects_bad_ids(ctx):
    import spq4k
    rng = np.random.default_rng(1)
    bank, _ = _gpu_bank(ctx, 4, 64, 256, seed=1)
    X = rng.standard_normal((2, 1, 256)).astype(np.float32)
    with pytest.raises(spq4k.Spq4kError):
        ctx.mul_mat_id(bank, X, np.array([[0, 4], [1, 2]], np.int32))

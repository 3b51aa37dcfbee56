"""GPU parity of the expert-gathered Q4_K matvec (GGML_OP_MUL_MAT_ID).

Against the reference's own outputs (golden vectors) and against the CPU
oracle's ggml_compute_forward_mul_mat_id restatement at the 30B-A3B-like
shapes of BASELINE configs[3] (128 experts, top-8 routing, gate/up 768x2048,
down 2048x768, T = 1..32). Tolerance: the reference's close_enough
(1e-4 relative or 1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48)."""
import os

import numpy as np
import pytest

from _oracle import close_enough, parity_ok

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _check(got, exp, what, exact=None):
    """close_enough of the oracle (ggml's x86 order); with `exact`, the parity
    bar's either-or: of the oracle or of the dequant-then-dot value"""
    ok = close_enough(got, exp) if exact is None else parity_ok(got, exp, exact)
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
    _check(got, exp, f"moe M={M} K={K} T={T} ne11={ne11}", oracle.mul_mat_id_dq_f64(12, host, M, K, E, X, ids))


@pytest.mark.parametrize("env", [{}, {"SPQ4K_MOE_MODE": 3}])
def test_moe_many_tokens_per_expert(oracle, env):
    # every token picks the same 8 experts: 32 pairs per expert, two 16-pair
    # tiles of the ring kernel (several TC chunks of the sdot4 kernel)
    from _envctx import context_with
    ctx = context_with(env)
    E, M, K, T, k = 16, 256, 1024, 32, 8
    rng = np.random.default_rng(77)
    bank, host = _gpu_bank(ctx, E, M, K, seed=5)
    ids = np.tile(np.array([3, 1, 4, 15, 9, 2, 6, 5], np.int32), (T, 1))
    X = rng.standard_normal((T, k, K)).astype(np.float32)
    try:
        _check(ctx.mul_mat_id(bank, X, ids), oracle.mul_mat_id(host, M, K, E, X, ids), f"moe shared experts {env}")
    finally:
        bank.free()
        ctx.close()


def test_moe_rejects_bad_ids(ctx):
    import spq4k
    rng = np.random.default_rng(1)
    bank, _ = _gpu_bank(ctx, 4, 64, 256, seed=1)
    X = rng.standard_normal((2, 1, 256)).astype(np.float32)
    with pytest.raises(spq4k.Spq4kError):
        ctx.mul_mat_id(bank, X, np.array([[0, 4], [1, 2]], np.int32))


@pytest.mark.parametrize("T,ne11,M,K", [(1, 1, 768, 2048), (1, 8, 2048, 768), (3, 8, 2048, 768), (4, 1, 512, 4096),
                                        (5, 8, 2048, 768), (32, 1, 768, 2048), (33, 8, 200, 1280)])
def test_moe_paths_agree(oracle, T, ne11, M, K):
    """Every MoE path against the oracle: the planner's choice, the matrix-core
    path at any batch (SPQ4K_MOE_MODE=2: routing pass, Q8_K planes, ring
    kernel of 8 waves, and of 4 with SPQ4K_MOE_RING_WAVES=4), the single-launch sdot4 kernel (=3) and the three-launch sdot4
    path (SPQ4K_MOE_UNFUSED)."""
    from _envctx import context_with
    E, k = 128, 8
    ids = _topk_ids(np.random.default_rng(T), T, E, k)
    X = np.random.default_rng(T + 1).standard_normal((T, ne11, K)).astype(np.float32)
    outs, host = [], None
    for env in ({}, {"SPQ4K_MOE_MODE": 2}, {"SPQ4K_MOE_MODE": 2, "SPQ4K_MOE_RING_WAVES": 4}, {"SPQ4K_MOE_MODE": 3},
                {"SPQ4K_MOE_UNFUSED": 1}):
        c = context_with(env)
        try:
            bank, host = _gpu_bank(c, E, M, K, 71)
            outs.append((env, c.mul_mat_id(bank, X, ids)))
            bank.free()
        finally:
            c.close()
    exp = oracle.mul_mat_id(host, M, K, E, X, ids)
    for env, got in outs:
        _check(got, exp, f"{env} T={T} ne11={ne11} M={M} K={K}")


@pytest.mark.parametrize("mode", [0, 2, 3])
def test_moe_device_ids_out_of_range_leave_outputs(oracle, mode):
    """Device-pointer entry point: an id outside [0, E) is not routed, so its
    output rows keep their previous contents (the host entry point rejects it)."""
    from spq4k.hip import DeviceArray
    from _envctx import context_with
    ctx = context_with({"SPQ4K_MOE_MODE": mode})
    E, M, K, T, k = 16, 256, 2048, 2, 4
    bank, host = _gpu_bank(ctx, E, M, K, 5)
    ids = np.array([[3, 99, 7, -1], [1, 2, 3, 4]], np.int32)
    X = np.random.default_rng(2).standard_normal((T, 1, K)).astype(np.float32)
    idd, Xd = DeviceArray.from_host(ids), DeviceArray.from_host(X)
    Yd = DeviceArray.from_host(np.full((T, k, M), 7.0, np.float32))
    ctx.moe_dev(bank, idd.ptr, k, 1, T, Xd.ptr, Yd.ptr)
    ctx.synchronize()
    Y = Yd.to_host().reshape(T, k, M)
    assert (Y[0, 1] == 7.0).all() and (Y[0, 3] == 7.0).all()
    ok_ids = ids.copy(); ok_ids[0, 1] = 0; ok_ids[0, 3] = 0
    exp = oracle.mul_mat_id(host, M, K, E, X, ok_ids)
    for t, s in ((0, 0), (0, 2), (1, 0), (1, 1), (1, 2), (1, 3)):
        _check(Y[t, s], exp[t, s], f"slot {t},{s}")
    bank.free()
    ctx.close()


@pytest.mark.parametrize("qtype", [12, 13, 14, 8])
@pytest.mark.parametrize("T,ne11", [(1, 1), (3, 8), (4, 1), (8, 1), (32, 8)])
@pytest.mark.parametrize("shapes", [(768, 768), (768, 512)])
def test_moe_multi(ctx, oracle, qtype, T, ne11, shapes):
    """spq4k_moe_multi: two banks sharing ids and input (gate and up of 768
    rows; a second bank of 512 rows) in one call, each output bit for bit the
    one spq4k_moe gives that bank alone (both the two-bank sweep and the
    two-bank expert ring run every row with the same arithmetic), and within
    tolerance of the oracle. K-quant banks: T <= 8 sweeps both banks in one
    launch; larger batches of banks of equal rows share one prep and one
    ring launch; the rest run the banks one after the other."""
    from spq4k.hip import DeviceArray
    E, k, K = 32, 8, 2048
    rng = np.random.default_rng(900 + 10 * T + ne11 + qtype + shapes[1])
    hosts, banks = [], []
    for M in shapes:
        # the GPU encoder (bit-exact with ggml's, pinned in the per-type tests)
        x = (rng.standard_normal((E * M, K)) * 0.02).astype(np.float32)
        h = ctx.quantize_chunk(x, E * M, K, type=qtype)
        hosts.append(h)
        banks.append(ctx.upload(h, M, K, E, type=qtype))
    ids = _topk_ids(rng, T, E, k)
    X = rng.standard_normal((T, ne11, K)).astype(np.float32)
    idd, xd = DeviceArray.from_host(ids), DeviceArray.from_host(X)
    ym = [DeviceArray((T, k, M)) for M in shapes]
    ys = [DeviceArray((T, k, M)) for M in shapes]
    ctx.moe_multi_dev(banks, idd.ptr, k, ne11, T, xd.ptr, [y.ptr for y in ym])
    for b, y in zip(banks, ys):
        ctx.moe_dev(b, idd.ptr, k, ne11, T, xd.ptr, y.ptr)
    ctx.synchronize()
    for i, (M, h) in enumerate(zip(shapes, hosts)):
        got, alone = ym[i].to_host(), ys[i].to_host()
        np.testing.assert_array_equal(got.view(np.uint32), alone.view(np.uint32), err_msg=f"bank {i} M={M}")
        if i == 0:
            exp = (oracle.mul_mat_id_q8_0(h, M, K, E, X, ids) if qtype == 8
                   else oracle.mul_mat_id_type(qtype, h, M, K, E, X, ids))
            _check(got, exp, f"type {qtype} T={T} ne11={ne11} bank {i}")


def test_moe_multi_errors(ctx, oracle):
    from spq4k import Spq4kError
    from spq4k.hip import DeviceArray
    rng = np.random.default_rng(7)
    E, M, K = 4, 64, 256
    a = ctx.upload(oracle.quantize(12, (rng.standard_normal((E * M, K)) * 0.02).astype(np.float32)), M, K, E)
    b = ctx.upload(oracle.quantize(14, (rng.standard_normal((E * M, K)) * 0.02).astype(np.float32)), M, K, E,
                   type=14)
    ids, x, y = DeviceArray.from_host(np.zeros((1, 2), np.int32)), DeviceArray(K), DeviceArray(2 * M)
    with pytest.raises(Spq4kError):   # types differ
        ctx.moe_multi_dev([a, b], ids.ptr, 2, 1, 1, x.ptr, [y.ptr, y.ptr])
    with pytest.raises(Spq4kError):   # three banks
        ctx.moe_multi_dev([a, a, a], ids.ptr, 2, 1, 1, x.ptr, [y.ptr, y.ptr, y.ptr])

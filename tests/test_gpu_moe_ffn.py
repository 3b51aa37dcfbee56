"""GPU parity of the routed-expert FFN block (spq4k_moe_ffn, include/spq4k.h):
the unit the reference's BURN_MOE custom op replaces
(desktop/engine/src/burn_moe_op.cpp:202-372) with the arithmetic of the stock
ggml graph it stands for (forward.cpp:1098-1117) -- gate and up
MUL_MAT_ID, silu(gate) * up, down MUL_MAT_ID on each pair's own hidden row,
then the router-weighted sum over the slots.

Checks, at the 30B-A3B-like shapes of BASELINE configs[3] (128 experts, top-8,
gate/up 768x2048, down 2048x768) and ragged ones:
  - the fused call equals, bit for bit, the entry points it is made of run one
    after the other (spq4k_moe_multi, spq4k_swiglu, spq4k_moe) followed by the
    weighted sum as ggml computes it (fp32 products added in double in slot
    order, ggml_sum_rows' ggml_vec_sum_f32, ggml-cpu/vec.h:1513-1519);
  - each stage's GPU output is within the parity bar of the CPU oracle fed the
    same stage input (gate and up from X; down from the GPU's own hidden rows:
    close_enough of ggml_vec_dot's order or of the dequant-then-dot sum);
  - the whole block against the oracle's own chain, normwise: the down stage
    re-quantises hidden rows that already differ from the CPU's in the last
    fp32 bits, so an element that crosses a Q8_K rounding boundary moves by
    d8 * w, and element-wise agreement of a chain is not a property any
    reordering of the fp32 sums keeps (the reference ggml graph itself is the
    adapter test's target, tests/test_gpu_ggml_adapter.py)."""
import numpy as np
import pytest

from _oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, close_enough, parity_ok

pytestmark = pytest.mark.gpu
CHAIN_NORMWISE = 2e-3


def _bank(ctx, qtype, E, M, K, seed):
    """seeded N(0, 0.02) expert bank encoded on the GPU; device weights and host bytes"""
    from spq4k.hip import DeviceArray, download
    w = ctx.alloc_weights(M, K, E, type=qtype)
    tmp = DeviceArray(E * M * K, np.float32)
    ctx.synth_fill_dev(tmp.ptr, E * M * K, seed, 0, K, 0.0, 0.02, 1.0, 0)
    ctx.quantize_chunk_dev(qtype, tmp.ptr, w.data_ptr, E * M, K)
    ctx.synchronize()
    tmp.free()
    return w, download(w.data_ptr, w.nbytes)


def _routing(rng, T, E, k):
    """top-k of N(0, 1) router logits and their softmax weights renormalised over the k"""
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    top = np.take_along_axis(logits, ids, axis=1).astype(np.float64)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def _weighted_sum(D, w):
    """ggml_mul by the weights (fp32 products), then ggml_sum_rows over the slots (double, slot order)"""
    prod = (D * w[:, :, None]).astype(np.float32)
    acc = np.zeros((D.shape[0], D.shape[2]), np.float64)
    for s in range(D.shape[1]):
        acc += prod[:, s, :].astype(np.float64)
    return acc.astype(np.float32)


def _mmid(oracle, qtype, bank, M, K, E, X, ids):
    """the oracle's mul_mat_id for a bank of any of the types"""
    if qtype == TYPE_Q8_0:
        return oracle.mul_mat_id_q8_0(bank, M, K, E, X, ids)
    return oracle.mul_mat_id_type(qtype, bank, M, K, E, X, ids)


def _bits_equal(a, b, what):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    diff = a.view(np.uint32) != b.view(np.uint32)
    assert not diff.any(), f"{what}: {int(diff.sum())} of {a.size} differ, first {np.argwhere(diff)[0]}"


@pytest.mark.parametrize("down_type", [TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("T", [1, 4, 32])
def test_moe_ffn_30b(ctx, oracle, down_type, T):
    from spq4k.hip import DeviceArray
    E, k, D_, F = 128, 8, 2048, 768
    rng = np.random.default_rng(100 + T + down_type)
    gate, gh = _bank(ctx, TYPE_Q4_K, E, F, D_, 11)
    up, uh = _bank(ctx, TYPE_Q4_K, E, F, D_, 12)
    down, dh = _bank(ctx, down_type, E, D_, F, 13)
    ids, w = _routing(rng, T, E, k)
    X = rng.standard_normal((T, D_)).astype(np.float32)
    Y = ctx.moe_ffn(gate, up, down, ids, w, X)
    assert Y.shape == (T, D_) and np.isfinite(Y).all()

    # the same entry points one after the other
    ids_d, X_d = DeviceArray.from_host(ids), DeviceArray.from_host(X)
    G_d, U_d, H_d = (DeviceArray(T * k * F, np.float32) for _ in range(3))
    Dn_d = DeviceArray(T * k * D_, np.float32)
    ctx.moe_multi_dev([gate, up], ids_d.ptr, k, 1, T, X_d.ptr, [G_d.ptr, U_d.ptr])
    ctx.swiglu_dev(G_d.ptr, U_d.ptr, H_d.ptr, T * k * F)
    ctx.moe_dev(down, ids_d.ptr, k, k, T, H_d.ptr, Dn_d.ptr)
    ctx.synchronize()
    G, U = G_d.to_host().reshape(T, k, F), U_d.to_host().reshape(T, k, F)
    H, Dn = H_d.to_host().reshape(T, k, F), Dn_d.to_host().reshape(T, k, D_)
    _bits_equal(Y, _weighted_sum(Dn, w), f"T={T} fused vs composed")

    # each stage against the oracle on the same stage input
    X3 = X[:, None, :]
    for name, got, bank in (("gate", G, gh), ("up", U, uh)):
        exp = oracle.mul_mat_id(bank, F, D_, E, X3, ids)
        ok = parity_ok(got, exp, oracle.mul_mat_id_dq_f64(TYPE_Q4_K, bank, F, D_, E, X3, ids))
        assert ok.all(), f"{name} T={T}: {int((~ok).sum())}/{ok.size} outside tolerance"
    ok = close_enough(H, oracle.swiglu(G, U))
    assert ok.all(), f"swiglu T={T}: {int((~ok).sum())}/{ok.size}"
    exp = _mmid(oracle, down_type, dh, D_, F, E, H, ids)
    ok = parity_ok(Dn, exp, oracle.mul_mat_id_dq_f64(down_type, dh, D_, F, E, H, ids))
    assert ok.all(), f"down T={T} type={down_type}: {int((~ok).sum())}/{ok.size} outside tolerance"

    # the whole block through the oracle's own chain
    Go = oracle.mul_mat_id(gh, F, D_, E, X3, ids)
    Uo = oracle.mul_mat_id(uh, F, D_, E, X3, ids)
    Ho = oracle.swiglu(Go, Uo)
    Yo = _weighted_sum(_mmid(oracle, down_type, dh, D_, F, E, Ho, ids), w)
    err = np.linalg.norm(Y.astype(np.float64) - Yo) / np.linalg.norm(Yo.astype(np.float64))
    assert err < CHAIN_NORMWISE, f"block T={T} normwise {err:.3e}"
    for a in (gate, up, down):
        a.free()


@pytest.mark.parametrize("n_ff,n_used,T,down_type", [
    (768, 8, 8, TYPE_Q4_K),      # 64 pairs, the largest small batch
    (768, 8, 9, TYPE_Q4_K),      # 72 pairs: down on the matrix cores, then the combine
    (768, 1, 5, TYPE_Q4_K),
    (768, 3, 2, TYPE_Q6_K),
    (2048, 6, 3, TYPE_Q4_K),     # 8 super-blocks a down row, two lane groups a wave
    (2048, 8, 1, TYPE_Q5_K),
    (4096, 8, 2, TYPE_Q4_K),     # 16 super-blocks a down row, one lane group a wave
    (4096, 5, 1, TYPE_Q6_K),
])
def test_moe_ffn_down_sum_shapes(ctx, oracle, n_ff, n_used, T, down_type):
    """the down projection with the slot sum in its epilogue (small batches)
    equals the down launch followed by the combine, bit for bit, for every
    down row length the small-batch sweep serves and n_used up to 8; and the
    batch past it still runs the two launches"""
    from spq4k.hip import DeviceArray
    E, D_ = 16, 512
    rng = np.random.default_rng(7 * n_ff + n_used + T)
    gate, _ = _bank(ctx, TYPE_Q4_K, E, n_ff, D_, 31)
    up, _ = _bank(ctx, TYPE_Q4_K, E, n_ff, D_, 32)
    down, dh = _bank(ctx, down_type, E, D_, n_ff, 33)
    ids, w = _routing(rng, T, E, n_used)
    X = rng.standard_normal((T, D_)).astype(np.float32)
    Y = ctx.moe_ffn(gate, up, down, ids, w, X)
    ids_d, X_d = DeviceArray.from_host(ids), DeviceArray.from_host(X)
    G_d, U_d, H_d = (DeviceArray(T * n_used * n_ff, np.float32) for _ in range(3))
    Dn_d = DeviceArray(T * n_used * D_, np.float32)
    ctx.moe_multi_dev([gate, up], ids_d.ptr, n_used, 1, T, X_d.ptr, [G_d.ptr, U_d.ptr])
    ctx.swiglu_dev(G_d.ptr, U_d.ptr, H_d.ptr, T * n_used * n_ff)
    ctx.moe_dev(down, ids_d.ptr, n_used, n_used, T, H_d.ptr, Dn_d.ptr)
    ctx.synchronize()
    H = H_d.to_host().reshape(T, n_used, n_ff)
    Dn = Dn_d.to_host().reshape(T, n_used, D_)
    _bits_equal(Y, _weighted_sum(Dn, w), f"n_ff={n_ff} n_used={n_used} T={T} fused vs composed")
    exp = _mmid(oracle, down_type, dh, D_, n_ff, E, H, ids)
    ok = parity_ok(Dn, exp, oracle.mul_mat_id_dq_f64(down_type, dh, D_, n_ff, E, H, ids))
    assert ok.all(), f"down: {int((~ok).sum())}/{ok.size} outside tolerance"
    for a in (gate, up, down):
        a.free()
    for d in (ids_d, X_d, G_d, U_d, H_d, Dn_d):
        d.free()


def test_moe_ffn_device_ids_out_of_range(ctx):
    """Device ids are not validated on the host: through the small-batch down
    projection an id outside [0, E) contributes nothing to the slot sum (the
    weighted sum over the valid slots, in slot order), and the other tokens'
    outputs are untouched by it."""
    from spq4k.hip import DeviceArray
    E, k, D_, F, T = 8, 4, 512, 768, 2
    rng = np.random.default_rng(91)
    gate, _ = _bank(ctx, TYPE_Q4_K, E, F, D_, 41)
    up, _ = _bank(ctx, TYPE_Q4_K, E, F, D_, 42)
    down, _ = _bank(ctx, TYPE_Q4_K, E, D_, F, 43)
    ids = np.array([[1, 5, 2, 7], [3, 0, 6, 4]], np.int32)
    w = rng.random((T, k)).astype(np.float32)
    X = rng.standard_normal((T, D_)).astype(np.float32)
    ids_d, w_d, X_d = DeviceArray.from_host(ids), DeviceArray.from_host(w), DeviceArray.from_host(X)
    Y_d = DeviceArray(T * D_, np.float32)
    ctx.moe_ffn_dev(gate, up, down, ids_d.ptr, w_d.ptr, k, T, X_d.ptr, Y_d.ptr)
    ctx.synchronize()
    Y = Y_d.to_host().reshape(T, D_)
    bad = ids.copy()
    bad[0, 2] = E          # token 0, slot 2 out of range
    bad_d = DeviceArray.from_host(bad)
    ctx.moe_ffn_dev(gate, up, down, bad_d.ptr, w_d.ptr, k, T, X_d.ptr, Y_d.ptr)
    ctx.synchronize()
    Yb = Y_d.to_host().reshape(T, D_)
    _bits_equal(Yb[1], Y[1], "the other token")
    # token 0 without slot 2: the composed down rows of the valid slots
    H_d = DeviceArray(T * k * F, np.float32)
    G_d, U_d = DeviceArray(T * k * F, np.float32), DeviceArray(T * k * F, np.float32)
    Dn_d = DeviceArray(T * k * D_, np.float32)
    ctx.moe_multi_dev([gate, up], ids_d.ptr, k, 1, T, X_d.ptr, [G_d.ptr, U_d.ptr])
    ctx.swiglu_dev(G_d.ptr, U_d.ptr, H_d.ptr, T * k * F)
    ctx.moe_dev(down, ids_d.ptr, k, k, T, H_d.ptr, Dn_d.ptr)
    ctx.synchronize()
    Dn = Dn_d.to_host().reshape(T, k, D_)
    keep = [0, 1, 3]
    exp = _weighted_sum(Dn[:1, keep, :], w[:1, keep])[0]
    _bits_equal(Yb[0], exp, "token 0 with slot 2 out of range")
    for a in (gate, up, down):
        a.free()
    for d in (ids_d, w_d, X_d, Y_d, bad_d, H_d, G_d, U_d, Dn_d):
        d.free()


def test_moe_ffn_ragged(ctx, oracle):
    """n_used 2 of 16 experts, an expert picked by several tokens, n_ff 256"""
    E, k, D_, F, T = 16, 2, 512, 256, 5
    rng = np.random.default_rng(3)
    gate, gh = _bank(ctx, TYPE_Q4_K, E, F, D_, 21)
    up, uh = _bank(ctx, TYPE_Q4_K, E, F, D_, 22)
    down, dh = _bank(ctx, TYPE_Q4_K, E, D_, F, 23)
    ids = np.array([[3, 1], [3, 15], [0, 3], [15, 14], [7, 3]], np.int32)
    w = rng.random((T, k)).astype(np.float32)
    X = rng.standard_normal((T, D_)).astype(np.float32)
    Y = ctx.moe_ffn(gate, up, down, ids, w, X)
    X3 = X[:, None, :]
    Ho = oracle.swiglu(oracle.mul_mat_id(gh, F, D_, E, X3, ids), oracle.mul_mat_id(uh, F, D_, E, X3, ids))
    Yo = _weighted_sum(oracle.mul_mat_id(dh, D_, F, E, Ho, ids), w)
    err = np.linalg.norm(Y.astype(np.float64) - Yo) / np.linalg.norm(Yo.astype(np.float64))
    assert err < CHAIN_NORMWISE, f"ragged block normwise {err:.3e}"


def test_moe_ffn_rejects_bad_banks(ctx):
    import spq4k
    E, D_, F = 4, 256, 256
    gate, _ = _bank(ctx, TYPE_Q4_K, E, F, D_, 1)
    up6, _ = _bank(ctx, TYPE_Q6_K, E, F, D_, 2)
    down, _ = _bank(ctx, TYPE_Q4_K, E, D_, F, 3)
    down_bad, _ = _bank(ctx, TYPE_Q4_K, E, D_, 2 * F, 4)
    ids = np.array([[0, 1]], np.int32)
    w = np.ones((1, 2), np.float32)
    X = np.ones((1, D_), np.float32)
    with pytest.raises(spq4k.Spq4kError):
        ctx.moe_ffn(gate, up6, down, ids, w, X)
    with pytest.raises(spq4k.Spq4kError):
        ctx.moe_ffn(gate, gate, down_bad, ids, w, X)
    with pytest.raises(spq4k.Spq4kError):
        ctx.moe_ffn(gate, gate, down, np.array([[0, 4]], np.int32), w, X)

"""GPU parity of the BurnHard MoE forward (spq4k_beast_moe_forward,
include/spq4k.h) with the reference's own sp_beast_route_experts and
sp_beast_moe_forward loop (desktop/beast_canyon/sp_beast_canyon.c:385-443,
:455-562), built from its source into oracle/_ref/beast, and with the golden
vectors that build wrote (tests/golden/beast_moe_golden.npz).

The routing is the reference's: the same experts in the same order; scores
within 2e-6 (expf on the GPU and in libm may differ in the last place). The
output is the score-weighted sum of beast_matvec's dequant-then-dot (fp32
activations, no Q8_K), whose fp32 sums the GPU takes per lane and across the
wave where the reference adds serially: element-wise within close_enough
(1e-4 relative or 1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48) of
the reference's output or of the same forward in double (the parity bar's
either-or: where a long row's products cancel, the two fp32 orders can differ
by more than 1e-4 of the small result while both stay near the exact one)."""
import os

import numpy as np
import pytest

from _oracle import BEAST_SO, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, BeastRef, close_enough, parity_ok

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "beast_moe_golden.npz"))


def _check(got, exp, what, exact=None):
    ok = close_enough(got, exp) if exact is None else parity_ok(got, exp, exact)
    assert ok.all(), f"{what}: {int((~ok).sum())}/{ok.size} outside tolerance, first {np.argwhere(~ok)[0]}"


def _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids, scores, hidden, types=(TYPE_Q4_K,) * 3):
    """sp_beast_moe_forward's sum over the selected experts in double: each
    expert's dequantised banks (fp32 values, exact in double) against the fp32
    hidden state, silu(g) * u, down, score-weighted"""
    def deq(t, bank, e, rows, cols):
        eb = bank.size // E
        return oracle.to_float(t, bank[e * eb:(e + 1) * eb], rows * cols).reshape(rows, cols).astype(np.float64)
    x = hidden.astype(np.float64)
    y = np.zeros(n_embd)
    for e, sc in zip(ids, scores):
        g, u = deq(types[0], Wg, e, n_ff, n_embd) @ x, deq(types[1], Wu, e, n_ff, n_embd) @ x
        y += float(sc) * (deq(types[2], Wd, e, n_embd, n_ff) @ (g / (1.0 + np.exp(-g)) * u))
    return y


def test_beast_moe_golden(ctx):
    E, k, n_embd, n_ff = (int(v) for v in G["moe_shape"])
    gate = ctx.upload(G["moe_gate"], n_ff, n_embd, E=E)
    up = ctx.upload(G["moe_up"], n_ff, n_embd, E=E)
    down = ctx.upload(G["moe_down"], n_embd, n_ff, E=E)
    y, ids, sc = ctx.beast_moe_forward(gate, up, down, G["moe_logits"], k, G["moe_hidden"])
    assert np.array_equal(ids, G["moe_ids"])
    np.testing.assert_allclose(sc, G["moe_scores"], rtol=2e-6)
    _check(y, G["moe_y"], "golden forward")


@pytest.mark.parametrize("case", range(4))
def test_beast_route_golden(ctx, case):
    """the routing of the golden logits (ties, -inf, 128 experts) through a
    forward over small banks of as many experts"""
    l, k = G[f"route{case}_logits"], int(G[f"route{case}_k"])
    E, n = l.size, 256
    rng = np.random.default_rng(case)
    from _oracle import Oracle
    o = Oracle()
    banks = [ctx.upload(o.quantize_q4K((rng.standard_normal((E * n, n)) * 0.05).astype(np.float32)), n, n, E=E)
             for _ in range(3)]
    _, ids, sc = ctx.beast_moe_forward(*banks, l, k, rng.standard_normal(n).astype(np.float32))
    assert np.array_equal(ids, G[f"route{case}_ids"])
    np.testing.assert_allclose(sc, G[f"route{case}_scores"], rtol=2e-6)
    for b in banks:
        b.free()


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")
@pytest.mark.parametrize("E,k,n_embd", [(300, 16, 256), (1000, 9, 256), (4096, 16, 256), (257, 3, 256),
                                        (4096, 16, 2304)])
def test_beast_route_many_experts(ctx, E, k, n_embd):
    """routings of more than 256 experts against the reference's own
    sp_beast_route_experts: runs of equal logits, -inf logits, the largest
    logit at the last index; 4096 experts beside 2304-wide rows take more than
    64 KB of LDS in the routing launch"""
    rng = np.random.default_rng(E + k)
    logits = (rng.standard_normal(E) * 3.0).astype(np.float32)
    logits[rng.choice(E, E // 10, replace=False)] = -np.inf
    tie = rng.choice(E, 20, replace=False)
    logits[tie] = np.float32(logits.max() + 0.5)     # twenty equal top scores, the rank order by index
    logits[-1] = np.float32(logits.max() + 1.0)
    ids_ref, sc_ref = BeastRef().route(logits, k)
    zero = np.zeros(E * n_embd * 144, np.uint8)        # all-zero blocks: the outputs are not checked here
    banks = [ctx.upload(zero, 256, n_embd, E=E), ctx.upload(zero, 256, n_embd, E=E),
             ctx.upload(zero, n_embd, 256, E=E)]
    _, ids, sc = ctx.beast_moe_forward(*banks, logits, k, np.ones(n_embd, np.float32))
    assert np.array_equal(ids, ids_ref), f"experts {ids} against {ids_ref}"
    np.testing.assert_allclose(sc, sc_ref, rtol=2e-6)
    for b in banks:
        b.free()


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")
@pytest.mark.parametrize("E,k,n_embd,n_ff", [(32, 8, 2048, 768), (16, 2, 1024, 512), (8, 0, 512, 256),
                                             (6, 9, 256, 1024), (8, 4, 4096, 1536), (20, 16, 512, 768),
                                             (4, 2, 768, 4096), (4, 3, 4608, 512), (2, 2, 4352, 4352),
                                             (4, 2, 1024, 4352), (1, 1, 256, 256), (3, 1, 2048, 768),
                                             (2, 2, 256, 8448), (2, 2, 8448, 256), (2, 1, 256, 16640),
                                             (2, 1, 16640, 256)])
def test_beast_moe_vs_reference(ctx, oracle, E, k, n_embd, n_ff):
    """the forward against the reference's own build: the 30B-A3B widths
    (top-8, 2048 -> 768 -> 2048) over 32 experts, the default top-2 (k = 0),
    k above E (every expert), top-16, rows of 1 to 16 blocks (the one-wave
    kernels at every lane count) and of more than 16 (the row-a-wave kernels,
    rows of 2, 4 and 8 passes of 16 blocks), each side of the forward on
    either"""
    b = BeastRef()
    rng = np.random.default_rng(E * 7 + k + n_embd)

    def bank(rows, cols):
        return oracle.quantize_q4K(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.03))

    Wg, Wu, Wd = bank(E * n_ff, n_embd), bank(E * n_ff, n_embd), bank(E * n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2.0).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y_ref, ids_ref, sc_ref = b.moe(TYPE_Q4_K, Wg, Wu, Wd, E, n_embd, n_ff, logits, k, hidden)
    gate, up = ctx.upload(Wg, n_ff, n_embd, E=E), ctx.upload(Wu, n_ff, n_embd, E=E)
    down = ctx.upload(Wd, n_embd, n_ff, E=E)
    y, ids, sc = ctx.beast_moe_forward(gate, up, down, logits, k, hidden)
    assert np.array_equal(ids, ids_ref), f"experts {ids} against {ids_ref}"
    np.testing.assert_allclose(sc, sc_ref, rtol=2e-6)
    _check(y, y_ref, f"E={E} k={k} {n_embd}->{n_ff}",
           _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids_ref, sc_ref, hidden))
    for w in (gate, up, down):
        w.free()


def test_beast_moe_device_pointers_and_rejects(ctx):
    """the device entry point leaves ids / scores alone when not asked, and
    refuses banks of another type or shape"""
    import spq4k
    from spq4k.hip import DeviceArray
    E, n = 4, 256
    rng = np.random.default_rng(5)
    from _oracle import Oracle
    o = Oracle()
    W = [o.quantize_q4K((rng.standard_normal((E * n, n)) * 0.05).astype(np.float32)) for _ in range(3)]
    banks = [ctx.upload(w, n, n, E=E) for w in W]
    logits = np.array([0.1, 2.0, -1.0, 1.5], np.float32)
    hidden = rng.standard_normal(n).astype(np.float32)
    y_host, ids_host, _ = ctx.beast_moe_forward(*banks, logits, 2, hidden)
    ld, hd, od = DeviceArray.from_host(logits), DeviceArray.from_host(hidden), DeviceArray(n, np.float32)
    ctx.beast_moe_forward_dev(*banks, ld.ptr, 2, hd.ptr, od.ptr)
    ctx.synchronize()
    assert np.array_equal(od.to_host().view(np.uint32), y_host.view(np.uint32))
    assert ids_host.tolist() == [1, 3]
    wide = ctx.upload(o.quantize_q4K((rng.standard_normal((E * n, 2 * n)) * 0.05).astype(np.float32)), n, 2 * n,
                      E=E)
    with pytest.raises(spq4k.Spq4kError):
        ctx.beast_moe_forward(banks[0], banks[1], wide, logits, 2, hidden)
    q6 = ctx.upload(o.quantize_q6K((rng.standard_normal((E * 2 * n, n)) * 0.05).astype(np.float32)), 2 * n, n, E=E,
                    type=TYPE_Q6_K)
    with pytest.raises(spq4k.Spq4kError):       # a gate bank of another shape than up's, whatever its type
        ctx.beast_moe_forward(q6, banks[1], banks[2], logits, 2, hidden)
    for w in banks + [q6, wide]:
        w.free()
    for d in (ld, hd, od):
        d.free()


def _mixed_banks(oracle, rng, types, E, n_embd, n_ff):
    def bank(t, rows, cols):
        return oracle.quantize(t, rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.03))
    return bank(types[0], E * n_ff, n_embd), bank(types[1], E * n_ff, n_embd), bank(types[2], E * n_embd, n_ff)


def _upload3(ctx, types, Wg, Wu, Wd, E, n_embd, n_ff):
    return (ctx.upload(Wg, n_ff, n_embd, E=E, type=types[0]), ctx.upload(Wu, n_ff, n_embd, E=E, type=types[1]),
            ctx.upload(Wd, n_embd, n_ff, E=E, type=types[2]))


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")
@pytest.mark.parametrize("types", [(TYPE_Q8_0,) * 3, (TYPE_Q4_K, TYPE_Q4_K, TYPE_Q8_0), (TYPE_Q8_0, TYPE_Q8_0, TYPE_Q4_K),
                                   (TYPE_Q8_0, TYPE_Q4_K, TYPE_Q8_0)])
@pytest.mark.parametrize("E,k,n_embd,n_ff", [(32, 8, 2048, 768), (8, 2, 1024, 4352), (4, 3, 4608, 512),
                                             (6, 2, 256, 256)])
def test_beast_moe_q8_0_banks_vs_reference(ctx, oracle, types, E, k, n_embd, n_ff):
    """Q8_0 banks, alone and beside Q4_K ones, against the reference's own
    forward (its beast_dequant_q8_0 is the format's): the same experts and
    scores, the output within close_enough of the reference's or of the
    forward in double"""
    rng = np.random.default_rng(E + k + n_embd + sum(types))
    Wg, Wu, Wd = _mixed_banks(oracle, rng, types, E, n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2.0).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y_ref, ids_ref, sc_ref = BeastRef().moe(types, Wg, Wu, Wd, E, n_embd, n_ff, logits, k, hidden)
    banks = _upload3(ctx, types, Wg, Wu, Wd, E, n_embd, n_ff)
    y, ids, sc = ctx.beast_moe_forward(*banks, logits, k, hidden)
    assert np.array_equal(ids, ids_ref), f"experts {ids} against {ids_ref}"
    np.testing.assert_allclose(sc, sc_ref, rtol=2e-6)
    _check(y, y_ref, f"types {types} E={E} k={k} {n_embd}->{n_ff}",
           _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids_ref, sc_ref, hidden, types))
    for w in banks:
        w.free()


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")
@pytest.mark.parametrize("types", [(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K), (TYPE_Q6_K,) * 3, (TYPE_Q5_K, TYPE_Q5_K, TYPE_Q6_K),
                                   (TYPE_Q8_0, TYPE_Q8_0, TYPE_Q6_K)])
@pytest.mark.parametrize("E,k,n_embd,n_ff", [(32, 8, 2048, 768), (8, 2, 4096, 1536), (4, 2, 512, 8448)])
def test_beast_moe_q6k_down_vs_oracle(ctx, oracle, types, E, k, n_embd, n_ff):
    """a Q6_K down bank (the Q4_K_M files' usual one) and Q5_K / Q6_K gate /
    up banks: the reference's routing (its own build), and the output against
    the oracle's forward over that routing with the formats' dequantisers
    (the reference's beast_dequant_q5_K / _q6_K are not the formats') within
    close_enough, or of the forward in double"""
    rng = np.random.default_rng(3 * E + k + n_ff + sum(types))
    Wg, Wu, Wd = _mixed_banks(oracle, rng, types, E, n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2.0).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    ids_ref, sc_ref = BeastRef().route(logits, k)
    banks = _upload3(ctx, types, Wg, Wu, Wd, E, n_embd, n_ff)
    y, ids, sc = ctx.beast_moe_forward(*banks, logits, k, hidden)
    assert np.array_equal(ids, ids_ref), f"experts {ids} against {ids_ref}"
    np.testing.assert_allclose(sc, sc_ref, rtol=2e-6)
    y_or = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, ids_ref, sc_ref, hidden)
    _check(y, y_or, f"types {types} E={E} k={k} {n_embd}->{n_ff}",
           _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids_ref, sc_ref, hidden, types))
    for w in banks:
        w.free()


def test_beast_moe_q8_0_ragged_rows(ctx, oracle):
    """Q8_0 banks whose rows are not a multiple of 256 values (n_embd 2880,
    n_ff 1440: partial groups of eight blocks) against the oracle's forward"""
    types = (TYPE_Q8_0,) * 3
    E, k, n_embd, n_ff = 8, 4, 2880, 1440
    rng = np.random.default_rng(11)
    Wg, Wu, Wd = _mixed_banks(oracle, rng, types, E, n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2.0).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    banks = _upload3(ctx, types, Wg, Wu, Wd, E, n_embd, n_ff)
    y, ids, sc = ctx.beast_moe_forward(*banks, logits, k, hidden)
    y_or = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, ids, sc, hidden)
    _check(y, y_or, "ragged Q8_0", _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids, sc, hidden, types))
    for w in banks:
        w.free()


@pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")
def test_beast_moe_q8_0_long_hidden_rows_vs_reference(ctx, oracle):
    """hidden rows too long for every selected expert's row to be staged at
    once (3 x 16384 values): the down sum that stages one expert at a time,
    against the reference's own forward"""
    types = (TYPE_Q8_0,) * 3
    E, k, n_embd, n_ff = 4, 3, 256, 16384
    rng = np.random.default_rng(17)
    Wg, Wu, Wd = _mixed_banks(oracle, rng, types, E, n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2.0).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y_ref, ids_ref, sc_ref = BeastRef().moe(types, Wg, Wu, Wd, E, n_embd, n_ff, logits, k, hidden)
    banks = _upload3(ctx, types, Wg, Wu, Wd, E, n_embd, n_ff)
    y, ids, sc = ctx.beast_moe_forward(*banks, logits, k, hidden)
    assert np.array_equal(ids, ids_ref)
    _check(y, y_ref, "long hidden rows", _forward_f64(oracle, Wg, Wu, Wd, E, n_embd, n_ff, ids_ref, sc_ref, hidden,
                                                      types))
    for w in banks:
        w.free()

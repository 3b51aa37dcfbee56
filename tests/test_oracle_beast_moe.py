"""The BurnHard routing and MoE forward checkers (host only): the reference's
own sp_beast_route_experts and sp_beast_moe_forward loop
(desktop/beast_canyon/sp_beast_canyon.c:385-443, :455-562), built into
oracle/_ref/beast from its source, against the golden vectors it wrote
(tests/golden/beast_moe_golden.npz) and against what the mathematics fixes:
the top-k of a softmax is the top-k of the logits (the lowest index first
among equal ones), the renormalised scores are the softmax restricted to the
chosen experts, and the forward is the score-weighted sum of the reference's
own beast_matvec calls around silu(gate) * up."""
import os

import numpy as np
import pytest

from _oracle import BEAST_SO, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, BeastRef

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "beast_moe_golden.npz"))
live = pytest.mark.skipif(not os.path.exists(BEAST_SO), reason="oracle/_ref/beast (the reference) not built")


def _topk_closed_form(logits, k):
    """argsort by value, the lowest index first among ties; softmax in double over the chosen"""
    order = sorted(range(logits.size), key=lambda i: (-float(logits[i]), i))[:k]
    e = np.exp(logits.astype(np.float64) - float(np.max(logits)))
    p = e[order] / e.sum()
    return np.array(order, np.int32), p / p.sum()


@pytest.mark.parametrize("case", range(4))
def test_route_golden_closed_form(case):
    l, k = G[f"route{case}_logits"], int(G[f"route{case}_k"])
    ids, sc = G[f"route{case}_ids"], G[f"route{case}_scores"]
    exp_ids, exp_sc = _topk_closed_form(l, k)
    assert np.array_equal(ids, exp_ids)
    np.testing.assert_allclose(sc, exp_sc, rtol=2e-6)


@live
def test_route_live_matches_golden():
    b = BeastRef()
    for case in range(4):
        ids, sc = b.route(G[f"route{case}_logits"], int(G[f"route{case}_k"]))
        assert np.array_equal(ids, G[f"route{case}_ids"]) and np.array_equal(sc, G[f"route{case}_scores"])


@live
def test_route_defaults():
    """top_k <= 0 routes to 2 experts; more than E routes to all E"""
    b = BeastRef()
    l = np.array([0.3, -1.0, 2.0, 0.7, 0.1], np.float32)
    assert b.route(l, 0)[0].tolist() == [2, 3]
    assert sorted(b.route(l, 9)[0].tolist()) == [0, 1, 2, 3, 4]


@live
def test_moe_golden_and_decomposition(oracle):
    """the forward against its golden output, and against the reference's own
    beast_matvec calls composed by hand (score-weighted sum of down(silu(gate) * up))"""
    b = BeastRef()
    E, k, n_embd, n_ff = (int(v) for v in G["moe_shape"])
    y, ids, sc = b.moe(TYPE_Q4_K, G["moe_gate"], G["moe_up"], G["moe_down"], E, n_embd, n_ff, G["moe_logits"], k,
                       G["moe_hidden"])
    assert np.array_equal(y.view(np.uint32), G["moe_y"].view(np.uint32))
    assert np.array_equal(ids, G["moe_ids"]) and np.array_equal(sc, G["moe_scores"])
    gb, db = n_ff * (n_embd // 256) * 144, n_embd * (n_ff // 256) * 144
    acc = np.zeros(n_embd, np.float64)
    for e, s in zip(ids, sc):
        g = b.matvec(TYPE_Q4_K, G["moe_gate"][e * gb:(e + 1) * gb], n_ff, n_embd, G["moe_hidden"])
        u = b.matvec(TYPE_Q4_K, G["moe_up"][e * gb:(e + 1) * gb], n_ff, n_embd, G["moe_hidden"])
        h = (g / (np.float32(1) + np.exp(-g))) * u
        d = b.matvec(TYPE_Q4_K, G["moe_down"][e * db:(e + 1) * db], n_embd, n_ff, h.astype(np.float32))
        acc += float(s) * d.astype(np.float64)
    # the forward accumulates in fp32 (and numpy's float32 exp may differ from
    # expf in the last place): normwise against the double sum
    err = np.linalg.norm(acc - y) / np.linalg.norm(acc)
    assert err < 1e-6, f"normwise {err:.2e}"


def _banks(oracle, rng, types, E, n_embd, n_ff):
    def bank(t, rows, cols):
        return oracle.quantize(t, (rng.standard_normal((rows, cols)) * 0.03).astype(np.float32))
    return bank(types[0], E * n_ff, n_embd), bank(types[1], E * n_ff, n_embd), bank(types[2], E * n_embd, n_ff)


@live
@pytest.mark.parametrize("types", [(TYPE_Q4_K,) * 3, (TYPE_Q8_0,) * 3, (TYPE_Q4_K, TYPE_Q4_K, TYPE_Q8_0),
                                   (TYPE_Q8_0, TYPE_Q8_0, TYPE_Q4_K)])
def test_moe_routed_is_the_reference_forward(oracle, types):
    """or_beast_moe_routed (the per-expert loop over a given routing, a type
    per bank) on the reference's own routing reproduces the reference's
    forward bit for bit wherever the reference's dequantisers are the
    formats' (Q4_K, Q8_0), mixed banks included"""
    rng = np.random.default_rng(sum(types))
    E, k, n_embd, n_ff = 8, 3, 512, 768
    Wg, Wu, Wd = _banks(oracle, rng, types, E, n_embd, n_ff)
    logits = (rng.standard_normal(E) * 2).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y_ref, ids, sc = BeastRef().moe(types, Wg, Wu, Wd, E, n_embd, n_ff, logits, k, hidden)
    y = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, ids, sc, hidden)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


@pytest.mark.parametrize("types", [(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K), (TYPE_Q6_K,) * 3, (TYPE_Q5_K,) * 3])
def test_moe_routed_q5k_q6k_against_double(oracle, types):
    """banks of Q5_K / Q6_K, whose reference dequantisers are not the
    format's: the routed forward against the same forward in double over the
    format's dequantised weights (normwise, fp32 rounding of each stage)"""
    rng = np.random.default_rng(7 + sum(types))
    E, n_embd, n_ff = 6, 512, 512
    Wg, Wu, Wd = _banks(oracle, rng, types, E, n_embd, n_ff)
    ids = np.array([4, 1, 5], np.int32)
    sc = np.array([0.5, 0.3, 0.2], np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, ids, sc, hidden)

    def deq(t, bank, e, rows, cols):
        eb = bank.size // E
        return oracle.to_float(t, bank[e * eb:(e + 1) * eb], rows * cols).reshape(rows, cols).astype(np.float64)
    x = hidden.astype(np.float64)
    acc = np.zeros(n_embd)
    for e, s in zip(ids, sc):
        g, u = deq(types[0], Wg, e, n_ff, n_embd) @ x, deq(types[1], Wu, e, n_ff, n_embd) @ x
        acc += float(s) * (deq(types[2], Wd, e, n_embd, n_ff) @ (g / (1.0 + np.exp(-g)) * u))
    err = np.linalg.norm(acc - y) / np.linalg.norm(acc)
    assert err < 1e-5, f"normwise {err:.2e}"
    # an id outside the bank is skipped
    y2 = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, np.array([4, 99, 1], np.int32),
                                 np.array([0.5, 0.3, 0.2], np.float32), hidden)
    y3 = oracle.beast_moe_routed(types, Wg, Wu, Wd, E, n_embd, n_ff, np.array([4, 1], np.int32),
                                 np.array([0.5, 0.2], np.float32), hidden)
    assert np.array_equal(y2.view(np.uint32), y3.view(np.uint32))

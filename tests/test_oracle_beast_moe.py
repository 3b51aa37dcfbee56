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

from _oracle import BEAST_SO, TYPE_Q4_K, BeastRef

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

"""Pins of the MoE router / GLU references (oracle/moe.py) and the attention
reference (oracle/attention.py) by closed forms and identities, independent
of the formulas they restate."""
import math

import numpy as np
import pytest

from oracle import attention as oat
from oracle import moe as omoe


def test_router_softmax_closed_form():
    # logits ln(1), ln(2), ln(4), ln(8): softmax = (1, 2, 4, 8) / 15
    lg = np.log(np.array([[1.0, 2.0, 4.0, 8.0]]))
    inds, w = omoe.router_topk(lg, 2, norm_topk_prob=False, shared_gate=False)
    assert inds.tolist() == [[3, 2]]
    assert np.allclose(w, [[8 / 15, 4 / 15]], rtol=1e-15)
    inds, w = omoe.router_topk(lg, 2, norm_topk_prob=True, shared_gate=False)
    assert np.allclose(w, [[2 / 3, 1 / 3]], rtol=1e-15)


def test_router_shared_gate_appends_sigmoid_of_last_column():
    # [t, E + 1]: the last column is the shared expert's gate, never routed
    lg = np.array([[0.0, 3.0, 1.0, 100.0], [2.0, 0.0, 0.0, -math.log(3.0)]])
    inds, w = omoe.router_topk(lg, 1, norm_topk_prob=True, shared_gate=True)
    assert inds.tolist() == [[1], [0]]
    assert np.allclose(w[:, 0], 1.0)                       # one pick, renormalised
    assert np.allclose(w[:, 1], [1 / (1 + math.exp(-100.0)), 0.25])


def test_router_renormalised_softmax_equals_softmax_of_picked_logits():
    """The identity gemma4's fused router relies on (gmlx/modules.py:1031-
    1033): softmax over all logits renormalised over the picks equals the
    softmax of the picked logits alone."""
    rng = np.random.default_rng(0)
    lg = rng.normal(0, 2, size=(6, 40))
    inds, w = omoe.router_topk(lg, 5, norm_topk_prob=True, shared_gate=False)
    picked = np.take_along_axis(lg, inds, axis=-1)
    e = np.exp(picked - picked.max(-1, keepdims=True))
    assert np.allclose(w, e / e.sum(-1, keepdims=True), rtol=1e-12)
    # picks are the k largest logits, in descending order
    assert np.array_equal(inds, np.argsort(-lg, axis=-1)[:, :5])


def test_router_bias_selects_but_does_not_weight():
    # sqrt(softplus): x = 0 -> sqrt(ln 2); a selection bias promotes expert 0
    lg = np.array([[0.0, 1.0, 2.0]])
    sp = np.sqrt(np.log1p(np.exp(lg[0])))
    inds, w = omoe.router_topk(lg, 1, norm_topk_prob=False, shared_gate=False, scoring="sqrtsoftplus",
                               bias=np.array([10.0, 0.0, 0.0]))
    assert inds.tolist() == [[0]]
    assert np.allclose(w, [[sp[0]]], rtol=1e-15) and abs(sp[0] - math.sqrt(math.log(2.0))) < 1e-15
    # renormalised with the epsilon, then the routed scale
    inds, w = omoe.router_topk(lg, 2, norm_topk_prob=True, shared_gate=False, scoring="sqrtsoftplus", scale=2.5)
    assert inds.tolist() == [[2, 1]]
    assert np.allclose(w, 2.5 * sp[[2, 1]][None] / (sp[2] + sp[1] + 1e-20), rtol=1e-15)


def test_router_sigmoid_and_per_expert_scale():
    lg = np.array([[0.0, math.log(3.0)]])                  # sigmoid: 1/2, 3/4
    inds, w = omoe.router_topk(lg, 2, norm_topk_prob=False, shared_gate=False, scoring="sigmoid",
                               per_expert_scale=np.array([2.0, 10.0]))
    assert inds.tolist() == [[1, 0]]
    assert np.allclose(w, [[7.5, 1.0]], rtol=1e-15)


def test_router_ties_go_to_lower_id():
    inds, _ = omoe.router_topk(np.zeros((1, 6)), 3, shared_gate=False)
    assert inds.tolist() == [[0, 1, 2]]


@pytest.mark.parametrize("act", ["silu", "silu_limit", "swiglu_clamp", "gelu"])
def test_glu_closed_forms(act):
    if act == "silu":
        assert omoe.glu(0.0, 5.0, act) == 0.0
        assert abs(omoe.glu(1.0, 2.0, act) - 2.0 / (1.0 + math.exp(-1.0))) < 1e-15
    elif act == "silu_limit":
        # inside the limit it is silu(g) * u; outside, g and u saturate
        assert omoe.glu(1.0, 2.0, act, limit=7.0) == omoe.glu(1.0, 2.0, "silu")
        assert omoe.glu(50.0, -40.0, act, limit=7.0) == omoe.glu(7.0, -7.0, "silu")
    elif act == "swiglu_clamp":
        a = 1.702
        # u' = -1 zeroes the output; g' = 0 zeroes it
        assert omoe.glu(3.0, -1.0, act, limit=7.0, alpha=a) == 0.0
        assert omoe.glu(-2.0, 5.0, act, limit=7.0, alpha=a, gate_bias=2.0) == 0.0
        want = (2.0 + 1.0) * 1.0 / (1.0 + math.exp(-a))
        assert abs(omoe.glu(1.0, 2.0, act, limit=7.0, alpha=a) - want) < 1e-15
        # biases are added before the clamps
        assert omoe.glu(6.0, 6.5, act, limit=7.0, alpha=a, gate_bias=3.0, up_bias=3.0) == \
            omoe.glu(7.0, 7.0, act, limit=7.0, alpha=a)
    else:
        # gelu_tanh(0) = 0, odd part: gelu(x) - gelu(-x) = x
        assert omoe.glu(0.0, 1.0, act) == 0.0
        x = 0.8
        assert abs(omoe.glu(x, 1.0, act) - omoe.glu(-x, 1.0, act) - x) < 1e-15


def test_attention_reference_closed_forms():
    rng = np.random.default_rng(1)
    D, Hkv, G, L = 16, 2, 3, 9
    v = rng.normal(size=(Hkv, L, D))
    # equal keys: uniform weights, the mean of V for every head of the group
    k = np.ones((Hkv, L, D))
    q = rng.normal(size=(Hkv * G, D))
    out = oat.row_attention(q, k, v, 0.5)
    for hq in range(Hkv * G):
        assert np.allclose(out[hq], v[hq // G].mean(0), rtol=1e-12)
    # one key far above the others picks its value row
    k = np.zeros((Hkv, L, D))
    k[:, 4, 0] = 1e3
    q = np.zeros((Hkv * G, D))
    q[:, 0] = 1.0
    out = oat.row_attention(q, k, v, 1.0)
    for hq in range(Hkv * G):
        assert np.allclose(out[hq], v[hq // G, 4], rtol=1e-12)
    assert np.all(oat.row_attention(q, np.zeros((Hkv, 0, D)), np.zeros((Hkv, 0, D)), 1.0) == 0)

"""MoE routing and GLU epilogue references (TEST INFRASTRUCTURE ONLY).

fp64 numpy restatements of the reference's stock forms, which the fused
mlx-kquant ops replace:

  router_topk   gmlx/modules.py:754-763 (softmax -> top-k -> renormalise, the
                shared expert's sigmoid gate appended), gmlx/deepseek_v4_model.py:
                690-717 (_score_func / _expert_select: scoring functions,
                selection bias, renormalisation with +1e-20, routed scale),
                gmlx/modules.py:1029-1046 (gemma4 per-expert scale on the
                picked weights)
  glu           gmlx/modules.py:263-291 (act kinds), gmlx/deepseek_v4_model.py:
                740-744 (_limited_swiglu), gmlx/minimax_m3_model.py:134-138
                (clamped SwiGLU of gpt-oss)
  moe_layer     gate|up GLU per (token, slot), down projection, routing mix
                (gmlx/modules.py:540-605)
"""
from __future__ import annotations

import numpy as np


def score_func(logits, scoring):
    """_score_func (gmlx/deepseek_v4_model.py:690-697) in fp64."""
    x = np.asarray(logits, np.float64)
    if scoring == "softmax":
        e = np.exp(x - x.max(-1, keepdims=True))
        return e / e.sum(-1, keepdims=True)
    if scoring == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if scoring == "sqrtsoftplus":
        return np.sqrt(np.logaddexp(x, 0.0))
    raise ValueError(scoring)


def router_topk(logits, k, norm_topk_prob=True, shared_gate=True, per_expert_scale=None, bias=None,
                scoring="softmax", scale=1.0):
    """Returns (inds int (t, k) by descending biased score, weights float64
    (t, k + shared_gate)).  Ties go to the lower expert id (a stable sort of
    the negated scores)."""
    lg = np.asarray(logits, np.float64)
    lg = lg.reshape(-1, lg.shape[-1])
    if shared_gate:
        routed, gate = lg[:, :-1], lg[:, -1]
    else:
        routed, gate = lg, None
    sc = score_func(routed, scoring)
    sel = sc + (0.0 if bias is None else np.asarray(bias, np.float64)[None, :])
    inds = np.argsort(-sel, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(sc, inds, axis=-1)
    if norm_topk_prob:
        w = w / (w.sum(-1, keepdims=True) + 1e-20)
    if per_expert_scale is not None:
        w = w * np.asarray(per_expert_scale, np.float64)[inds]
    w = w * scale
    if shared_gate:
        w = np.concatenate([w, (1.0 / (1.0 + np.exp(-gate)))[:, None]], axis=-1)
    return inds, w


def silu(g):
    return g / (1.0 + np.exp(-g))


def glu(g, u, act="silu", limit=None, alpha=1.702, gate_bias=None, up_bias=None):
    """The fused GLU epilogue in fp64 over gate / up products g, u."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    if act == "silu":
        return silu(g) * u
    if act == "gelu":  # tanh approximation (mlx nn.gelu_approx)
        return 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
    if act == "silu_limit":
        return silu(np.minimum(g, limit)) * np.clip(u, -limit, limit)
    if act == "swiglu_clamp":
        if gate_bias is not None:
            g = g + gate_bias
        if up_bias is not None:
            u = u + up_bias
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
        return (u + 1.0) * g / (1.0 + np.exp(-alpha * g))
    raise ValueError(act)


def moe_layer(x, gate_deq, up_deq, down_deq, inds, weights, act="silu"):
    """fp64 MoE layer over dequantized expert stacks (only the rows of the
    touched experts are used): y[t] = sum_s w[t, s] * down[e] . glu(gate[e] .
    x[t], up[e] . x[t]), e = inds[t, s].  gate_deq / up_deq / down_deq map an
    expert id to its fp64 matrix ([I, D], [I, D], [D, I])."""
    x = np.asarray(x, np.float64)
    T, k = inds.shape
    out = np.zeros((T, down_deq(int(inds[0, 0])).shape[0]))
    h = np.zeros((T, k, gate_deq(int(inds[0, 0])).shape[0]))
    for t in range(T):
        for s in range(k):
            e = int(inds[t, s])
            h[t, s] = glu(gate_deq(e) @ x[t], up_deq(e) @ x[t], act)
            out[t] += weights[t, s] * (down_deq(e) @ h[t, s])
    return h, out

"""Ragged GQA decode attention reference (TEST INFRASTRUCTURE ONLY).

fp64 numpy restatement of the semantics of ragged_decode_attention
(gmlx/qwen35_attn.py:395-493): per (row, q head hq) softmax(scale * q . K^T) . V
over the row's visible keys, kv head h = hq // (Hq // Hkv)
(gmlx/qwen35_attn.py:71-73), as the reference's own test computes it
(tests/test_ragged_decode.py:48-58).
"""
from __future__ import annotations

import numpy as np


def row_attention(q, k_rows, v_rows, scale):
    """One row: q (Hq, D), k_rows / v_rows (Hkv, L, D) -> (Hq, D) float64.
    A row with no keys yields zeros."""
    q = np.asarray(q, np.float64)
    Hq, D = q.shape
    Hkv, L = k_rows.shape[0], k_rows.shape[1]
    G = Hq // Hkv
    out = np.zeros((Hq, v_rows.shape[-1]), np.float64)
    if L == 0:
        return out
    kf = np.asarray(k_rows, np.float64)
    vf = np.asarray(v_rows, np.float64)
    for h in range(Hkv):
        qh = q[h * G:(h + 1) * G]                  # (G, D)
        s = (qh @ kf[h].T) * scale                 # (G, L)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        out[h * G:(h + 1) * G] = (p @ vf[h]) / p.sum(-1, keepdims=True)
    return out


def slab_attention(q, k_flat, v_flat, offsets, lens, Hkv, D, scale, rows=None):
    """Rows of the per-row slab layout ([Hkv, len_b, D] at element offset
    offsets[b] of flat caches): returns {b: (Hq, D) float64} for `rows`
    (default all)."""
    out = {}
    for b in (range(len(lens)) if rows is None else rows):
        L = int(lens[b])
        o = int(offsets[b])
        kb = np.asarray(k_flat[o:o + Hkv * L * D]).reshape(Hkv, L, D)
        vb = np.asarray(v_flat[o:o + Hkv * L * D]).reshape(Hkv, L, D)
        out[b] = row_attention(q[b], kb, vb, scale)
    return out

"""Shared helpers for the test suite (seeded inputs, fp64 references)."""
import numpy as np

from oracle import kquant as okq

TOL = 2e-3          # north-star max-rel for matmul / attention outputs (fp16)
BF16_TOL = 8e-3     # reference's BF16_ULP (tests/test_ragged_decode.py:41)


def quantized_weights(rng, codec, n, k, std=0.02):
    w = rng.normal(0.0, std, size=(n, k)).astype(np.float32)
    return okq.quantize(w, codec)


def fp16_rows(rng, m, k):
    return rng.normal(0.0, 1.0, size=(m, k)).astype(np.float16)


def bf16_round(a):
    """fp32 -> bf16 (round to nearest even) -> fp32, in numpy."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def attention_ref(q, k_rows, v_rows, scale):
    """fp64 decode attention for one row: q (Hq, D), k_rows/v_rows (Hkv, L, D)."""
    Hq, D = q.shape
    Hkv = k_rows.shape[0]
    G = Hq // Hkv
    out = np.zeros((Hq, D), np.float64)
    for hq in range(Hq):
        h = hq // G
        L = k_rows.shape[1]
        if L == 0:
            continue
        s = (k_rows[h].astype(np.float64) @ q[hq].astype(np.float64)) * scale
        s = s - s.max()
        p = np.exp(s)
        out[hq] = (p @ v_rows[h].astype(np.float64)) / p.sum()
    return out

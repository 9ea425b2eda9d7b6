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


def q8_affine(x, dtype_name="float16", group=64):
    """8-bit affine group quantization of x (..., D) as mlx stores a
    quantized KV cache (bits 8, group 64): q = round((x - bias) / scale) in
    0..255 with scale = (max - min) / 255 and bias = min per group, scale and
    bias rounded to `dtype_name`.  Returns (words int32 (..., D/4) with four
    values per word lowest byte first, scales, biases as torch tensors of
    that dtype, and the dequantized values scale * q + bias rounded to the
    dtype, as float64 numpy)."""
    import torch
    tdt = getattr(torch, dtype_name)
    x = np.asarray(x, np.float32)
    *lead, D = x.shape
    g = x.reshape(*lead, D // group, group)
    lo, hi = g.min(-1), g.max(-1)
    sc = torch.from_numpy(np.maximum(hi - lo, 1e-6) / 255.0).to(tdt)
    bi = torch.from_numpy(lo).to(tdt)
    scf, bif = sc.float().numpy()[..., None], bi.float().numpy()[..., None]
    q = np.clip(np.rint((g - bif) / scf), 0, 255).astype(np.uint8)
    deq = torch.from_numpy((scf * q.astype(np.float32) + bif).reshape(*lead, D)).to(tdt).double().numpy()
    words = torch.from_numpy(q.reshape(*lead, D).copy()).view(torch.int32)
    return words, sc, bi, deq

"""K-quant codec oracle (TEST INFRASTRUCTURE ONLY -- never imported by gmlx_amd).

Three independent restatements of the public GGML block definitions
(ggml-common.h layouts, ggml-quants.c ``dequantize_row_*``), which is what
mlx-kquant (the un-vendored dependency gmlx binds through, pyproject.toml:26-34)
implements for ``kq.dequantize`` (gmlx/modules.py:1461):

1. ``value_*``: per-value scalar formulas in pure Python (index arithmetic
   straight from the block spec; for tiny brute-force cases);
2. ``dequant_*_np``: vectorized numpy, fp32 operations in GGML order;
3. ``dequantize`` via ``liboracle.so`` (kq_oracle.c), the C loops built with
   -ffp-contract=off -- the bit-exact target for the GPU kernels.

Quantizers (``quantize``) are the C restatements in kq_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from .iq2_tables import grid_from_c_header, ksigns

QK_K = 256
BLOCK_BYTES = {"q4_k": 144, "q6_k": 210, "iq2_xxs": 66}
GGML_TYPE = {"q4_k": 12, "q6_k": 14, "iq2_xxs": 16}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_GRID = None


def iq2xxs_grid():
    """The oracle's u64 grid, as transcribed in kq_oracle_tables.h."""
    global _GRID
    if _GRID is None:
        _GRID = grid_from_c_header(os.path.join(_HERE, "kq_oracle_tables.h"))
        assert len(_GRID) == 256
    return _GRID


def build(force=False):
    """Compile liboracle.so with the committed Makefile."""
    so = os.path.join(_HERE, "liboracle.so")
    if force or not os.path.exists(so):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return so


def lib():
    global _LIB
    if _LIB is None:
        so = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(so):
            build()
        L = ctypes.CDLL(so)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        f32p = ctypes.POINTER(ctypes.c_float)
        for name in ("kqo_dequant_q4_k", "kqo_dequant_q6_k", "kqo_dequant_iq2_xxs"):
            getattr(L, name).argtypes = [u8p, ctypes.c_int64, f32p]
            getattr(L, name).restype = None
        for name in ("kqo_quantize_q4_k", "kqo_quantize_q6_k", "kqo_quantize_iq2_xxs"):
            getattr(L, name).argtypes = [f32p, ctypes.c_int64, u8p]
            getattr(L, name).restype = None
        L.kqo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.kqo_f16_to_f32.restype = ctypes.c_float
        L.kqo_f32_to_f16.argtypes = [ctypes.c_float]
        L.kqo_f32_to_f16.restype = ctypes.c_uint16
        L.kqo_qmm_f32.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.kqo_qmm_f32.restype = ctypes.c_int
        L.kqo_ragged_attn_f32.argtypes = [ctypes.c_void_p] * 6 + \
            [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
        L.kqo_ragged_attn_f32.restype = None
        L.kqo_max_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ------------------------------------------------------------------ C oracle

def dequantize(wire, codec):
    """Wire bytes [..., nb*bpb] -> fp32 [..., nb*256] via the C oracle."""
    wire = np.ascontiguousarray(wire, dtype=np.uint8)
    bpb = BLOCK_BYTES[codec]
    assert wire.shape[-1] % bpb == 0
    nb_total = wire.size // bpb
    out = np.empty(nb_total * QK_K, np.float32)
    getattr(lib(), f"kqo_dequant_{codec}")(_ptr(wire, ctypes.c_uint8), nb_total,
                                            _ptr(out, ctypes.c_float))
    return out.reshape(*wire.shape[:-1], (wire.shape[-1] // bpb) * QK_K)


def quantize(w, codec):
    """fp32 weights [..., K] (K % 256 == 0) -> wire bytes [..., K/256*bpb]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    assert w.shape[-1] % QK_K == 0
    bpb = BLOCK_BYTES[codec]
    nb_total = w.size // QK_K
    out = np.empty(nb_total * bpb, np.uint8)
    getattr(lib(), f"kqo_quantize_{codec}")(_ptr(w, ctypes.c_float), nb_total,
                                             _ptr(out, ctypes.c_uint8))
    return out.reshape(*w.shape[:-1], (w.shape[-1] // QK_K) * bpb)


def f32_to_f16_bits(x):
    L = lib()
    return np.array([L.kqo_f32_to_f16(float(v)) for v in np.ravel(x)], np.uint16)


def qmm_f32_cpu(x16, wire, codec, nthreads=None):
    """CPU baseline: fused dequant GEMM in fp32 (OpenMP).  x16: fp16 [M, K]."""
    x16 = np.ascontiguousarray(x16, dtype=np.float16)
    wire = np.ascontiguousarray(wire, dtype=np.uint8)
    M, K = x16.shape
    N = wire.shape[0]
    y = np.empty((M, N), np.float32)
    nt = nthreads or lib().kqo_max_threads()
    rc = lib().kqo_qmm_f32(x16.ctypes.data, M, K, wire.ctypes.data, N, GGML_TYPE[codec],
                           y.ctypes.data, nt)
    assert rc == 0
    return y


# ------------------------------------------------------------ numpy restatement

def _f16(words):
    return np.asarray(words, np.uint16).view(np.float16).astype(np.float32)


def _blocks(wire, bpb):
    wire = np.ascontiguousarray(wire, dtype=np.uint8)
    lead = wire.shape[:-1]
    nb = wire.shape[-1] // bpb
    return wire.reshape(-1, nb, bpb), lead, nb


def dequant_q4_k_np(wire):
    blk, lead, nb = _blocks(wire, 144)
    d = _f16(blk[..., 0:2].copy().view(np.uint16)[..., 0])
    dmin = _f16(blk[..., 2:4].copy().view(np.uint16)[..., 0])
    s = blk[..., 4:16].astype(np.uint8)
    sc = np.empty(s.shape[:-1] + (8,), np.uint8)
    mn = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    dsc = d[..., None] * sc.astype(np.float32)          # [.., 8]
    dmn = dmin[..., None] * mn.astype(np.float32)
    qs = blk[..., 16:144].reshape(blk.shape[0], nb, 4, 32)
    q = np.stack([qs & 0xF, qs >> 4], axis=-2).reshape(blk.shape[0], nb, 8, 32)
    y = dsc[..., None] * q.astype(np.float32) - dmn[..., None]
    return y.astype(np.float32).reshape(*lead, nb * QK_K)


def dequant_q6_k_np(wire):
    blk, lead, nb = _blocks(wire, 210)
    R = blk.shape[0]
    d = _f16(blk[..., 208:210].copy().view(np.uint16)[..., 0])
    sc = blk[..., 192:208].copy().view(np.int8).astype(np.float32)   # [R, nb, 16]
    ql = blk[..., 0:128].reshape(R, nb, 2, 64).astype(np.int32)
    qh = blk[..., 128:192].reshape(R, nb, 2, 32).astype(np.int32)
    q = np.empty((R, nb, 2, 4, 32), np.int32)
    q[..., 0, :] = (ql[..., 0:32] & 0xF) | (((qh >> 0) & 3) << 4)
    q[..., 1, :] = (ql[..., 32:64] & 0xF) | (((qh >> 2) & 3) << 4)
    q[..., 2, :] = (ql[..., 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[..., 3, :] = (ql[..., 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    q = (q - 32).reshape(R, nb, 16, 16)      # value index = 16*sub + l
    y = (d[..., None, None] * sc[..., None]) * q.astype(np.float32)
    return y.astype(np.float32).reshape(*lead, nb * QK_K)


def dequant_iq2_xxs_np(wire):
    blk, lead, nb = _blocks(wire, 66)
    R = blk.shape[0]
    grid = np.array(iq2xxs_grid(), dtype=np.uint64)
    gbytes = grid.view(np.uint8).reshape(256, 8).astype(np.float32)
    signs = np.array([ksigns(i) for i in range(128)], np.uint8)
    d = _f16(blk[..., 0:2].copy().view(np.uint16)[..., 0])
    qs = blk[..., 2:66].copy().reshape(R, nb, 8, 8)
    idx = qs[..., 0:4].astype(np.int64)                              # [R,nb,8,4]
    aux1 = qs[..., 4:8].copy().view(np.uint32)[..., 0]               # [R,nb,8]
    db = (d[..., None] * (np.float32(0.5) + (aux1 >> 28).astype(np.float32))) * np.float32(0.25)
    sidx = np.stack([(aux1 >> (7 * l)) & 127 for l in range(4)], axis=-1)
    sbits = signs[sidx]                                              # [R,nb,8,4]
    neg = ((sbits[..., None] >> np.arange(8, dtype=np.uint8)) & 1).astype(bool)
    mag = gbytes[idx]                                                # [R,nb,8,4,8]
    y = (db[..., None, None] * mag) * np.where(neg, np.float32(-1), np.float32(1))
    return y.astype(np.float32).reshape(*lead, nb * QK_K)


DEQUANT_NP = {"q4_k": dequant_q4_k_np, "q6_k": dequant_q6_k_np, "iq2_xxs": dequant_iq2_xxs_np}


# -------------------------------------------------------- per-value spec form

def _f16s(b0, b1):
    return float(np.array([b0 | (b1 << 8)], np.uint16).view(np.float16)[0])


def value_q4_k(block, i):
    """Value i (0..255) of one Q4_K block, from the spec by index arithmetic."""
    block = bytes(block)
    d, dmin = np.float32(_f16s(block[0], block[1])), np.float32(_f16s(block[2], block[3]))
    s = block[4:16]
    j = i // 32                       # sub-block
    if j < 4:
        sc, mn = s[j] & 63, s[j + 4] & 63
    else:
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    byte = block[16 + 32 * (i // 64) + (i % 32)]
    q = (byte >> 4) if (j % 2) else (byte & 0xF)
    return np.float32(np.float32(d * np.float32(sc)) * np.float32(q)) - np.float32(dmin * np.float32(mn))


def value_q6_k(block, i):
    block = bytes(block)
    d = np.float32(_f16s(block[208], block[209]))
    h, r = divmod(i, 128)
    quarter, l = divmod(r, 32)
    ql = block[64 * h: 64 * h + 64]
    qh = block[128 + 32 * h: 128 + 32 * h + 32]
    lo = ql[l + (32 if quarter in (1, 3) else 0)]
    lo = (lo >> 4) if quarter >= 2 else (lo & 0xF)
    hi = (qh[l] >> (2 * quarter)) & 3
    q = (lo | (hi << 4)) - 32
    sc = np.int8(np.uint8(block[192 + i // 16]).view(np.int8))
    return np.float32(np.float32(d * np.float32(sc)) * np.float32(q))


def value_iq2_xxs(block, i):
    block = bytes(block)
    d = np.float32(_f16s(block[0], block[1]))
    g, r = divmod(i, 32)
    l, j = divmod(r, 8)
    grp = block[2 + 8 * g: 10 + 8 * g]
    idx = grp[l]
    aux1 = int.from_bytes(grp[4:8], "little")
    db = np.float32(np.float32(d * np.float32(0.5 + (aux1 >> 28))) * np.float32(0.25))
    mag = (iq2xxs_grid()[idx] >> (8 * j)) & 0xFF
    neg = (ksigns((aux1 >> (7 * l)) & 127) >> j) & 1
    v = np.float32(db * np.float32(mag))
    return -v if neg else v


VALUE_FN = {"q4_k": value_q4_k, "q6_k": value_q6_k, "iq2_xxs": value_iq2_xxs}


# --------------------------------------------------------------- references

def qmm_ref(x, wire, codec):
    """fp64 reference: x [M, K] . dequant(W [N, K])^T -> [M, N] float64."""
    w = dequantize(wire, codec).astype(np.float64)
    return np.asarray(x, np.float64) @ w.T


def max_rel(got, ref):
    """max|got - ref| / max|ref| -- the reference's _rel_err
    (tests/test_ragged_decode.py:78-81)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-6))


def rel_norm(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(float(np.linalg.norm(ref)), 1e-12))


def random_valid_blocks(rng, codec, nblocks):
    """Uniformly random block bytes with a finite, moderate fp16 d (and dmin):
    every bit pattern of the remaining fields is a valid encoding."""
    bpb = BLOCK_BYTES[codec]
    raw = rng.integers(0, 256, size=(nblocks, bpb), dtype=np.uint8)
    def put_f16(col, vals):
        raw[:, col:col + 2] = np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)
    scale = rng.uniform(1e-4, 2e-3, size=nblocks)
    if codec == "q4_k":
        put_f16(0, scale)
        put_f16(2, scale * rng.uniform(0.5, 2.0, size=nblocks))
    elif codec == "q6_k":
        put_f16(208, scale)
    else:
        put_f16(0, scale)
    return raw

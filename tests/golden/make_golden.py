"""Write the committed dequantization fixtures tests/golden/dequant_<codec>.npz.

Each fixture holds hand-built edge-case super-blocks (every 4-bit / 6-bit
code, every packed scale/min position, every IQ2_XXS grid index, sign index
and scale field, fp16 subnormal / zero / negative-zero / largest-finite
scales) and their fp32 dequantization.  The expectation is computed by the
oracle's C restatement and cross-checked here against the independent numpy
and per-value restatements before it is written; the reference repository
holds no K-quant vectors of its own (its numerics live in mlx-kquant).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import kquant as okq  # noqa: E402

F16 = {"one": 0x3C00, "half": 0x3800, "sub_min": 0x0001, "sub_max": 0x03FF, "max": 0x7BFF,
       "neg_zero": 0x8000, "neg_one": 0xBC00, "small": 0x1C00, "zero": 0x0000}


def _put16(blk, off, v):
    blk[off] = v & 0xFF
    blk[off + 1] = v >> 8


def q4k_blocks(rng):
    out = []
    for d, dmin in [("one", "half"), ("sub_min", "sub_max"), ("max", "small"), ("neg_zero", "neg_one"),
                    ("small", "zero"), ("half", "max")]:
        for variant in range(4):
            blk = np.zeros(144, np.uint8)
            _put16(blk, 0, F16[d])
            _put16(blk, 2, F16[dmin])
            if variant == 0:   # every scale byte value pattern incl. high bits
                blk[4:16] = np.arange(12, dtype=np.uint8) * 21 + 7
            elif variant == 1:
                blk[4:16] = 0xFF
            elif variant == 2:
                blk[4:16] = rng.integers(0, 256, 12, dtype=np.uint8)
            else:
                blk[4:16] = np.array([0xC0, 0x40, 0x80, 0x3F, 0xC1, 0x01, 0x7E, 0xBF, 0x0F, 0xF0, 0xA5, 0x5A],
                                     np.uint8)
            # every nibble value in both halves of every chunk
            blk[16:144] = (np.arange(128, dtype=np.uint32) * 37 + variant).astype(np.uint8)
            out.append(blk)
    return np.stack(out)


def q6k_blocks(rng):
    out = []
    for d in ["one", "sub_min", "max", "neg_zero", "small", "neg_one"]:
        for variant in range(3):
            blk = np.zeros(210, np.uint8)
            blk[0:192] = (np.arange(192, dtype=np.uint32) * 53 + 11 * variant).astype(np.uint8)
            if variant == 0:
                blk[192:208] = np.array([-128, 127, 0, 1, -1, 64, -64, 100, -100, 2, -2, 17, -17, 33, -33, 5],
                                        np.int8).view(np.uint8)
            else:
                blk[192:208] = rng.integers(0, 256, 16, dtype=np.uint8)
            _put16(blk, 208, F16[d])
            out.append(blk)
    return np.stack(out)


def iq2xxs_blocks(rng):
    out = []
    # 8 blocks x 8 groups x 4 = 256 grid indices, every one used once
    idx = np.arange(256)
    for b in range(8):
        blk = np.zeros(66, np.uint8)
        _put16(blk, 0, F16[["one", "half", "sub_max", "max", "neg_zero", "small", "neg_one", "one"][b]])
        for g in range(8):
            base = 2 + 8 * g
            for l in range(4):
                blk[base + l] = idx[(32 * b + 4 * g + l) % 256]
            signs = [(16 * b + 4 * g + l) % 128 for l in range(4)]   # 4 sign indices per group
            scale = (2 * b + g) % 16
            aux = scale << 28
            for l in range(4):
                aux |= signs[l] << (7 * l)
            blk[base + 4: base + 8] = np.array([aux], np.uint32).view(np.uint8)
        out.append(blk)
    # 4 more blocks: remaining sign indices (128 over 12 blocks) and random fields
    for b in range(4):
        blk = rng.integers(0, 256, 66, dtype=np.uint8)
        _put16(blk, 0, F16["one"])
        out.append(blk)
    return np.stack(out)


def main():
    rng = np.random.default_rng(2024)
    makers = {"q4_k": q4k_blocks, "q6_k": q6k_blocks, "iq2_xxs": iq2xxs_blocks}
    for codec, make in makers.items():
        wire = make(rng)
        exp = okq.dequantize(wire, codec)
        alt = okq.DEQUANT_NP[codec](wire)
        # NaN-free by construction; compare bit patterns
        assert np.array_equal(exp.view(np.uint32), alt.view(np.uint32)), codec
        for bi in range(wire.shape[0]):
            scal = np.array([okq.VALUE_FN[codec](wire[bi], i) for i in range(256)], np.float32)
            assert np.array_equal(scal.view(np.uint32), exp[bi].view(np.uint32)), (codec, bi)
        path = os.path.join(HERE, f"dequant_{codec}.npz")
        np.savez_compressed(path, wire=wire, expected=exp)
        print(path, wire.shape, exp.shape)


if __name__ == "__main__":
    main()

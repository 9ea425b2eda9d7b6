"""Pin the CPU oracle (no GPU): the IQ2_XXS table against its independent
2-bit form and the E8 invariants; the three dequant restatements against each
other, the committed golden fixtures and closed forms that a plausible
mistake (swapped nibble halves, wrong scale packing index, sign/parity error,
transposed operand) would break; quantizer round trips; fp64 references."""
import os

import numpy as np
import pytest

from oracle import iq2_tables, kquant as okq
from helpers import attention_ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- tables

def test_iq2_grid_matches_2bit_codes():
    assert okq.iq2xxs_grid() == iq2_tables.grid_from_kgrid()


def test_iq2_grid_invariants():
    g = okq.iq2xxs_grid()
    assert len(g) == 256 and len(set(g)) == 256
    assert all(a < b for a, b in zip(g, g[1:]))
    digit = {0x08: 0, 0x19: 1, 0x2B: 2}
    for v in g:
        bs = [(v >> (8 * j)) & 0xFF for j in range(8)]
        assert all(b in digit for b in bs)
        # E8 coset: magnitudes 2d+1 with sum(2d+1) = 8 + 2*sum(d) = 0 mod 4
        assert sum(digit[b] for b in bs) % 2 == 0


def test_ksigns_closed_form_even_parity():
    for i in range(128):
        s = iq2_tables.ksigns(i)
        assert s & 127 == i
        assert bin(s).count("1") % 2 == 0


def test_product_table_equals_oracle_table():
    """The product's C table (csrc/kq_tables.h) is the pinned grid."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    prod = iq2_tables.grid_from_c_header(os.path.join(root, "gmlx_amd", "csrc", "kq_tables.h"))
    assert prod == okq.iq2xxs_grid()


# ------------------------------------------------------- fp16 conversion

def test_f16_roundtrip_all_finite_patterns():
    L = okq.lib()
    bits = np.arange(0, 1 << 16, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    for b in range(0, 1 << 16, 97):
        if (b & 0x7C00) == 0x7C00:
            continue
        v = L.kqo_f16_to_f32(b)
        assert np.float32(v).view(np.uint32) == ref[b].view(np.uint32)
        assert L.kqo_f32_to_f16(v) == b


def test_f32_to_f16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.normal(0, 1e-5, 2000), rng.normal(0, 1, 2000), rng.normal(0, 3e4, 500),
                           [65519.9, 65520.0, 1e-8, 2.0 ** -25, 3 * 2.0 ** -26, -0.0]]).astype(np.float32)
    got = okq.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        exp = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


# ---------------------------------------------------------- dequant

@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
def test_three_restatements_agree_on_random_blocks(codec):
    rng = np.random.default_rng(1)
    wire = okq.random_valid_blocks(rng, codec, 200)
    c = okq.dequantize(wire, codec)
    n = okq.DEQUANT_NP[codec](wire)
    assert np.array_equal(c.view(np.uint32), n.view(np.uint32))
    for bi in (0, 7, 199):
        s = np.array([okq.VALUE_FN[codec](wire[bi], i) for i in range(256)], np.float32)
        assert np.array_equal(s.view(np.uint32), c[bi].view(np.uint32))


@pytest.mark.parametrize("codec", ["q4_k", "q6_k", "iq2_xxs"])
def test_golden_fixtures(codec):
    f = np.load(os.path.join(GOLDEN, f"dequant_{codec}.npz"))
    got = okq.dequantize(f["wire"], codec)
    assert np.array_equal(got.view(np.uint32), f["expected"].view(np.uint32))


def _q4k_block(d, dmin, sc, mn, q):
    """Build a Q4_K block from per-sub-block 6-bit (sc, mn) and 256 4-bit q
    with the GGML packing: bytes 0-3 low 6 bits of sc[0..3], 4-7 of mn[0..3];
    bytes 8-11 low nibbles sc[4..7] | mn[4..7] << 4; the top two bits of
    sc[4..7] / mn[4..7] sit in bits 6-7 of bytes 0-3 / 4-7."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    for j in range(4):
        b[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for c in range(4):
        for l in range(32):
            b[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return b


def test_q4k_closed_form_each_subblock_scale_and_min():
    """Only sub-block j carries a scale (or a min): exactly its 32 values move."""
    q = np.arange(256) % 16
    for j in range(8):
        for which in ("sc", "mn"):
            sc = [0] * 8
            mn = [0] * 8
            if which == "sc":
                sc[j] = 37 + j          # >= 16: exercises the 2 high bits
            else:
                mn[j] = 50 - j
            blk = _q4k_block(1.0, 0.5, sc, mn, q)
            y = okq.dequantize(blk[None], "q4_k")[0]
            exp = np.zeros(256, np.float32)
            sl = slice(32 * j, 32 * j + 32)
            exp[sl] = (np.float32(sc[j]) * q[sl].astype(np.float32)) - np.float32(0.5 * mn[j])
            assert np.array_equal(y, exp), (j, which)


def test_q4k_low_nibbles_feed_even_subblocks():
    sc = [1] * 8
    mn = [0] * 8
    q = np.zeros(256, np.int64)
    q[0:32] = 3      # sub-block 0 = low nibbles of bytes 0..31
    q[32:64] = 9     # sub-block 1 = high nibbles of the same bytes
    blk = _q4k_block(1.0, 0.0, sc, mn, q)
    assert blk[16] == 3 | (9 << 4)
    y = okq.dequantize(blk[None], "q4_k")[0]
    assert np.all(y[0:32] == 3) and np.all(y[32:64] == 9) and np.all(y[64:] == 0)


def test_q6k_closed_form_codes_and_signed_scales():
    # all 64 codes with scale +1 in the first half, -1 in the second
    L = np.concatenate([np.arange(64), np.arange(64)[::-1], np.arange(64), np.arange(64)[::-1]])
    b = np.zeros(210, np.uint8)
    for h in range(2):
        for l in range(32):
            a, bq, c, e = (L[128 * h + l + o] for o in (0, 32, 64, 96))
            b[64 * h + l] = (a & 15) | ((c & 15) << 4)
            b[64 * h + l + 32] = (bq & 15) | ((e & 15) << 4)
            b[128 + 32 * h + l] = (a >> 4) | ((bq >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6)
    b[192:208] = np.array([1] * 8 + [-1] * 8, np.int8).view(np.uint8)
    b[208:210] = np.array([0.25], np.float16).view(np.uint8)
    y = okq.dequantize(b[None], "q6_k")[0]
    sign = np.array([1] * 128 + [-1] * 128)
    assert np.array_equal(y, (0.25 * sign * (L - 32)).astype(np.float32))


def test_iq2xxs_closed_form_single_group():
    g = okq.iq2xxs_grid()
    b = np.zeros(66, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    idx = [5, 100, 200, 255]
    s7 = [0, 1, 0x55, 127]
    aux = (3 << 28) | sum(s << (7 * l) for l, s in enumerate(s7))
    b[2:6] = idx
    b[6:10] = np.array([aux], np.uint32).view(np.uint8)
    y = okq.dequantize(b[None], "iq2_xxs")[0]
    db = np.float32(np.float32(1.0 * 3.5) * np.float32(0.25))
    for l in range(4):
        sg = iq2_tables.ksigns(s7[l])
        for j in range(8):
            mag = (g[idx[l]] >> (8 * j)) & 0xFF
            exp = db * np.float32(mag)
            exp = -exp if (sg >> j) & 1 else exp
            assert y[8 * l + j] == exp
    # groups 1..7 are zero bytes: grid[0] (all 8s), no signs, scale field 0
    assert np.all(y[32:] == np.float32(np.float32(0.5) * np.float32(0.25)) * np.float32(8))


# ------------------------------------------------------------ quantizers

@pytest.mark.parametrize("codec,max_rel_rmse", [("q4_k", 0.09), ("q6_k", 0.025), ("iq2_xxs", 0.40)])
def test_quantizer_round_trip_quality(codec, max_rel_rmse):
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, size=(16, 1024)).astype(np.float32)
    wire = okq.quantize(w, codec)
    assert wire.shape == (16, 1024 // 256 * okq.BLOCK_BYTES[codec])
    back = okq.dequantize(wire, codec)
    rel = np.sqrt(np.mean((back - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert rel < max_rel_rmse


def test_quantizers_exact_on_representable_inputs():
    # Q6_K: values on a 6-bit grid come back to within the 8-bit sub-block
    # scale and fp16 block-scale rounding (<2% of the range)
    rng = np.random.default_rng(3)
    q = rng.integers(-32, 32, size=256).astype(np.float32)
    q[0] = -32
    wire = okq.quantize((q * 0.01).astype(np.float32)[None], "q6_k")
    back = okq.dequantize(wire, "q6_k")[0]
    assert np.max(np.abs(back - q * 0.01)) < 0.32 * 0.02
    # all-zero blocks stay zero
    for codec in ("q4_k", "q6_k", "iq2_xxs"):
        z = okq.quantize(np.zeros((1, 256), np.float32), codec)
        assert np.all(okq.dequantize(z, codec) == 0)


def test_quantize_deterministic():
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.02, size=(4, 512)).astype(np.float32)
    for codec in ("q4_k", "q6_k", "iq2_xxs"):
        assert np.array_equal(okq.quantize(w, codec), okq.quantize(w, codec))


# ------------------------------------------------------------ references

def test_qmm_ref_brute_force_tiny():
    rng = np.random.default_rng(5)
    wire = okq.random_valid_blocks(rng, "q4_k", 3).reshape(3, 144)
    x = rng.normal(0, 1, size=(2, 256)).astype(np.float16)
    ref = okq.qmm_ref(x, wire, "q4_k")
    for m in range(2):
        for n in range(3):
            acc = sum(float(x[m, i]) * float(okq.value_q4_k(wire[n], i)) for i in range(256))
            assert abs(acc - ref[m, n]) <= 1e-9 * max(1.0, abs(acc))


def test_cpu_baseline_qmm_matches_ref():
    rng = np.random.default_rng(6)
    wire = okq.quantize(rng.normal(0, 0.02, size=(64, 512)).astype(np.float32), "q6_k")
    x = rng.normal(0, 1, size=(3, 512)).astype(np.float16)
    got = okq.qmm_f32_cpu(x, wire, "q6_k", nthreads=2)
    assert okq.max_rel(got, okq.qmm_ref(x, wire, "q6_k")) < 1e-5


def test_attention_ref_closed_forms():
    rng = np.random.default_rng(7)
    D, L = 64, 50
    v = rng.normal(0, 1, size=(1, L, D))
    # identical keys -> uniform softmax -> mean of V
    k = np.ones((1, L, D))
    q = rng.normal(0, 1, size=(2, D))
    out = attention_ref(q, k, v, 0.125)
    assert np.allclose(out, v[0].mean(0)[None].repeat(2, 0))
    # a single key -> that value row, whatever q is
    out1 = attention_ref(q, k[:, :1], v[:, :1], 0.125)
    assert np.allclose(out1, v[0, 0][None].repeat(2, 0))
    # GQA map: q head hq reads kv head hq // G
    k2 = rng.normal(0, 1, size=(2, 7, D))
    v2 = rng.normal(0, 1, size=(2, 7, D))
    q4 = rng.normal(0, 1, size=(4, D))
    o = attention_ref(q4, k2, v2, 0.1)
    o_h1 = attention_ref(q4[2:], k2[1:], v2[1:], 0.1)
    assert np.allclose(o[2:], o_h1)


def test_cpu_baseline_attention_matches_ref():
    rng = np.random.default_rng(8)
    B, Hq, Hkv, D = 3, 8, 2, 64
    lens = [5, 40, 1]
    k = [rng.normal(0, 1, size=(Hkv, L, D)).astype(np.float16) for L in lens]
    v = [rng.normal(0, 1, size=(Hkv, L, D)).astype(np.float16) for L in lens]
    offs = np.cumsum([0] + [Hkv * L * D for L in lens])[:-1].astype(np.int64)
    kf = np.concatenate([a.reshape(-1) for a in k])
    vf = np.concatenate([a.reshape(-1) for a in v])
    q = rng.normal(0, 1, size=(B, Hq, D)).astype(np.float16)
    out = np.empty((B, Hq, D), np.float32)
    hs = np.array([L * D for L in lens], np.int64)
    ln = np.array(lens, np.int32)
    okq.lib().kqo_ragged_attn_f32(q.ctypes.data, kf.ctypes.data, vf.ctypes.data, offs.ctypes.data, hs.ctypes.data,
                                  ln.ctypes.data, B, Hq, Hkv, D, 0.125, out.ctypes.data, 2)
    ref = np.stack([attention_ref(q[b], k[b], v[b], 0.125) for b in range(B)])
    assert okq.max_rel(out, ref) < 1e-5

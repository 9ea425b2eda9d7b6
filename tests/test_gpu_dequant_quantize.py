"""GPU dequantization is bit-exact to the oracle's GGML-order definition, and
the GPU quantizers reproduce the oracle's bytes (through the C ABI)."""
import numpy as np
import pytest

from helpers import bf16_round, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu

CODECS = ["q4_k", "q6_k", "iq2_xxs"]


def _torch():
    import torch
    return torch


def _dev(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("codec", CODECS)
def test_dequant_f32_bit_exact(codec):
    from gmlx_amd import ops
    rng = np.random.default_rng(11)
    wire = np.concatenate([
        okq.random_valid_blocks(rng, codec, 257).reshape(-1),
        quantized_weights(rng, codec, 3, 512).reshape(-1),
    ]).reshape(-1, okq.BLOCK_BYTES[codec])
    ref = okq.dequantize(wire, codec)
    got = ops.dequantize(_dev(wire), None, codec).cpu().numpy()
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("codec", CODECS)
def test_dequant_f16_bf16_rounding(codec):
    torch = _torch()
    from gmlx_amd import ops
    rng = np.random.default_rng(12)
    wire = okq.random_valid_blocks(rng, codec, 64)
    ref = okq.dequantize(wire, codec)
    h = ops.dequantize(_dev(wire), None, codec, torch.float16).cpu().numpy()
    assert np.array_equal(h.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    b = ops.dequantize(_dev(wire), None, codec, torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(b.view(np.uint32), bf16_round(ref).view(np.uint32))


@pytest.mark.parametrize("codec", CODECS)
def test_dequant_golden_fixture(codec):
    """Committed edge-case blocks: GPU output equals the stored expectation."""
    import os
    from gmlx_amd import ops
    path = os.path.join(os.path.dirname(__file__), "golden", f"dequant_{codec}.npz")
    f = np.load(path)
    got = ops.dequantize(_dev(f["wire"]), None, codec).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), f["expected"].view(np.uint32))


@pytest.mark.parametrize("codec,rows,k", [("q4_k", 24, 1024), ("q6_k", 24, 768), ("iq2_xxs", 4, 512)])
def test_quantize_matches_oracle_bytes(codec, rows, k):
    from gmlx_amd import ops
    rng = np.random.default_rng(13)
    w = rng.normal(0.0, 0.02, size=(rows, k)).astype(np.float32)
    w[0, :256] = 0.0                      # an all-zero block
    w[1, :256] *= 1e-3                    # tiny scales
    ref = okq.quantize(w, codec)
    wire, scales = ops.quantize(_dev(w), codec)
    got = wire.cpu().numpy()
    assert got.shape == ref.shape and scales.numel() == 1
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} bytes differ"

"""Parity of the 17..64-row tile kernel (kq_mm.hip, reached through
kq_quantized_matmul_grouped with the mid-batch streaming kernel declined):
every tile-group size, both codecs and their mix, ragged super-block counts
per wave, bf16 activations, strided rows and every output dtype, against the
fp64 oracle (max-rel <= 2e-3; bf16 activations 8e-3), plus bitwise
determinism and grouped == separate."""
import numpy as np
import pytest

from helpers import BF16_TOL, TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu

ENV = ("GMLX_KQ_MM", "GMLX_KQ_MM_T")


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _clear(monkeypatch):
    for k in ENV:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("GMLX_KQ_MMS", "0")  # the tile kernel, not the mid-batch streaming one


@pytest.mark.parametrize("codec", ["q4_k", "q6_k"])
@pytest.mark.parametrize("M", [17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("K", [256, 1280, 4096])
def test_mid_batch_parity(codec, M, K, monkeypatch):
    """N = 200 (13 tiles, the last partial), K = 1 / 5 / 16 super-blocks
    (idle waves; waves with 2 and 1 blocks; 4 blocks each), every T."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(1000 * M + K)
    wire = quantized_weights(rng, codec, 200, K)
    x16 = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x16, wire, codec)
    x, w = _dev(x16), _dev(wire)
    for t in ("1", "2", "3", "4", "6"):
        monkeypatch.setenv("GMLX_KQ_MM_T", t)
        got = ops.quantized_matmul(x, w, None, codec).float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, (t, okq.max_rel(got, ref))


def test_mid_batch_long_k_q6k(monkeypatch):
    """Down-projection geometry: K = 12288 (48 super-blocks, 12 per wave)."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(5)
    wire = quantized_weights(rng, "q6_k", 96, 12288)
    for M in (20, 64):
        x16 = fp16_rows(rng, M, 12288)
        ref = okq.qmm_ref(x16, wire, "q6_k")
        got = ops.quantized_matmul(_dev(x16), _dev(wire), None, "q6_k").float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, M


@pytest.mark.parametrize("M", [17, 40, 64])
def test_mid_batch_mixed_group(M, monkeypatch):
    """q|k (Q4_K) with v (Q6_K) in one launch, tile groups across problem
    boundaries, against the fp64 reference and against the dense kernel."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(M)
    K = 2048
    mats = [(quantized_weights(rng, "q4_k", 300, K), "q4_k"), (quantized_weights(rng, "q4_k", 70, K), "q4_k"),
            (quantized_weights(rng, "q6_k", 90, K), "q6_k")]
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    refs = [okq.qmm_ref(x16, w, c) for w, c in mats]
    args = [(x, _dev(w), c) for w, c in mats]
    for t in ("1", "2"):
        monkeypatch.setenv("GMLX_KQ_MM_T", t)
        outs = ops.quantized_matmul_grouped(args)
        for o, ref in zip(outs, refs):
            assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL, t
    monkeypatch.setenv("GMLX_KQ_MM", "0")
    dense = ops.quantized_matmul_grouped(args)
    for o, ref in zip(dense, refs):
        assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("y_dtype", ["float16", "float32", "bfloat16"])
def test_mid_batch_bf16_and_out_dtypes(y_dtype, monkeypatch):
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(11)
    K, M = 1024, 36
    wire = quantized_weights(rng, "q4_k", 130, K)
    xf = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    xb = torch.from_numpy(xf).to(torch.bfloat16)
    ref = okq.qmm_ref(xb.float().numpy(), wire, "q4_k")
    got = ops.quantized_matmul(xb.cuda(), _dev(wire), None, "q4_k", out_dtype=getattr(torch, y_dtype))
    assert got.dtype == getattr(torch, y_dtype)
    tol = BF16_TOL if y_dtype == "bfloat16" else TOL
    assert okq.max_rel(got.float().cpu().numpy(), ref) <= max(tol, BF16_TOL)


def test_mid_batch_strided_rows_and_determinism(monkeypatch):
    """x rows at a stride of K + 64 (read in place) and of K + 3 (copied by
    the wrapper to an aligned stride) give the reference; repeated calls are
    bitwise equal; one grouped call equals separate calls bitwise."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(3)
    K, M = 1536, 29
    wa = quantized_weights(rng, "q4_k", 64, K)
    wb = quantized_weights(rng, "q4_k", 48, K)
    x16 = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x16, wa, "q4_k")
    for pad in (64, 3):
        big = torch.zeros(M, K + pad, dtype=torch.float16)
        big[:, :K] = torch.from_numpy(x16)
        xv = big.cuda()[:, :K]
        got = ops.quantized_matmul(xv, _dev(wa), None, "q4_k").float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, pad
    x = _dev(x16)
    a1 = ops.quantized_matmul(x, _dev(wa), None, "q4_k")
    a2 = ops.quantized_matmul(x, _dev(wa), None, "q4_k")
    assert torch.equal(a1, a2)
    ga, gb = ops.quantized_matmul_grouped([(x, _dev(wa), "q4_k"), (x, _dev(wb), "q4_k")])
    sb = ops.quantized_matmul(x, _dev(wb), None, "q4_k")
    assert torch.equal(ga, a1) and torch.equal(gb, sb)


@pytest.mark.parametrize("M", [8, 17, 64, 80])
def test_strided_rows_through_the_c_abi(M, monkeypatch):
    """kq_quantized_matmul_grouped with x rows at a stride of K + 64 and y rows
    at a stride of N + 40 (outputs written into a wider buffer), on every route
    (M = 8: LDS-staged small batch; 17, 64: mid-batch; 80: general kernel):
    the reference in the first N columns, the padding columns untouched."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(40 + M)
    K, N = 2048, 136
    wa = quantized_weights(rng, "q4_k", N, K)
    wb = quantized_weights(rng, "q6_k", N, K)
    x16 = fp16_rows(rng, M, K)
    xb = torch.zeros(M, K + 64, dtype=torch.float16)
    xb[:, :K] = torch.from_numpy(x16)
    xv = xb.cuda()[:, :K]
    ys = [torch.full((M, N + 40), 7.0, dtype=torch.float32, device="cuda") for _ in range(2)]
    wd = [_dev(wa), _dev(wb)]  # the problems hold raw pointers: keep the tensors alive
    probs = [ops._problem(xv, w, c, y[:, :N]) for w, c, y in zip(wd, ("q4_k", "q6_k"), ys)]
    ops._launch_grouped(probs, ops._dt(torch.float16), ops._dt(torch.float32), xv.device, ops._stream(xv))
    torch.cuda.synchronize()
    for w, c, y in zip((wa, wb), ("q4_k", "q6_k"), ys):
        ref = okq.qmm_ref(x16, w, c)
        assert okq.max_rel(y[:, :N].cpu().numpy(), ref) <= TOL, c
        assert bool((y[:, N:] == 7.0).all()), c

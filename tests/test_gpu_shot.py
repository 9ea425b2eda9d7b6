"""The one-shot kernel (kq_shot_kernel: a workgroup's one or two weight tiles
and the activations in LDS at once) against the fp64 oracle: the o and
q|k|v launches of a Qwen3-8B decode step at 1..32 rows, single and paired
tiles of each codec, partial last tiles,
K of 8 and 16 super-blocks, prepared bf16 / fp32 activations, strided rows
and outputs through the C ABI,
repeat determinism, and agreement with the paths it replaces."""
import ctypes

import numpy as np
import pytest

from helpers import BF16_TOL, TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu

KNOBS = ("GMLX_KQ_SHOT", "GMLX_KQ_STREAM", "GMLX_KQ_MV", "GMLX_KQ_SPLITK", "GMLX_KQ_STREAM_WGS", "GMLX_KQ_MV_WGS")


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _kernels(fn):
    """Names of the GPU kernels `fn` launched (torch profiler)."""
    import torch
    from torch.profiler import ProfilerActivity, profile
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        out = fn()
        torch.cuda.synchronize()
    names = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    return out, names


def _clean(monkeypatch):
    for k in KNOBS:
        monkeypatch.delenv(k, raising=False)


# (name, [(codec, N)], K, rows)
CASES = [
    ("o", [("q4_k", 4096)], 4096, [1, 3, 8, 9, 16, 20, 32]),
    ("qkv", [("q4_k", 4096), ("q4_k", 1024), ("q6_k", 1024)], 4096, [1, 5, 8, 12, 16, 17, 25, 32]),
    ("q4 pairs, partial tile, K 2048", [("q4_k", 300 * 16 + 5)], 2048, [2, 8]),
    ("q6 pairs, K 2048", [("q6_k", 400 * 16)], 2048, [4]),
    ("q4 with q6 pairs, K 2048", [("q6_k", 200 * 16 + 3), ("q4_k", 200 * 16)], 2048, [7, 13]),
    ("q6 singles", [("q6_k", 1000)], 4096, [6, 30]),
    ("q4 pairs", [("q4_k", 7000)], 4096, [8, 16, 24]),
    ("q4 with q6 singles, K 2048", [("q4_k", 100 * 16 + 7), ("q6_k", 30 * 16)], 2048, [3]),
]


@pytest.mark.parametrize("name,mats,K,rows", CASES, ids=[c[0] for c in CASES])
def test_shot_matches_oracle(name, mats, K, rows, monkeypatch):
    import torch
    from gmlx_amd import ops
    _clean(monkeypatch)
    rng = np.random.default_rng(sum(name.encode()))
    wires = [(quantized_weights(rng, c, n, K), c) for c, n in mats]
    dw = [(_dev(w), c) for w, c in wires]
    for M in rows:
        x16 = fp16_rows(rng, M, K)
        x = _dev(x16)
        items = [(x, w, c) for w, c in dw]
        outs, names = _kernels(lambda: ops.quantized_matmul_grouped(items, out_dtype=torch.float32))
        assert any("kq_shot_kernel" in n for n in names), names
        again = ops.quantized_matmul_grouped(items, out_dtype=torch.float32)
        for (w, c), o, o2 in zip(wires, outs, again):
            err = okq.max_rel(o.cpu().numpy(), okq.qmm_ref(x16, w, c))
            assert err <= TOL, (name, M, c, err)
            assert torch.equal(o, o2)          # deterministic
        # the path it replaces, within tolerance
        monkeypatch.setenv("GMLX_KQ_SHOT", "0")
        other = ops.quantized_matmul_grouped(items, out_dtype=torch.float32)
        monkeypatch.delenv("GMLX_KQ_SHOT")
        for o, o2 in zip(outs, other):
            assert okq.max_rel(o.cpu().numpy(), o2.cpu().numpy()) <= TOL


def test_shot_wide_range_and_one_signed_rows(monkeypatch):
    """bf16 / fp32 activations enter as prepared fp16 rows with per-row
    exponents (x_exp); rows of +-1e5 and of 1e-6 and one-signed rows (mean
    2e4, std 1.2e4) stay within tolerance."""
    import torch
    from gmlx_amd import ops
    _clean(monkeypatch)
    rng = np.random.default_rng(5)
    K = 4096
    wq = quantized_weights(rng, "q4_k", 1024, K)
    wv = quantized_weights(rng, "q6_k", 512, K)
    four = [rng.normal(0, 1e5, K), rng.normal(0, 1e-6, K), rng.normal(2e4, 1.2e4, K), rng.normal(0, 1, K)]
    # 12 rows: the 16-row form; 28 rows: the 32-row form
    for rows, dt, tol in ((np.stack(four * 3).astype(np.float32), torch.float32, TOL),
                          (np.stack(four * 3).astype(np.float32), torch.bfloat16, TOL),
                          (np.stack(four * 7).astype(np.float32), torch.bfloat16, TOL)):
        xt = torch.from_numpy(rows).to(dt)
        xr = xt.float().numpy()
        xd = xt.cuda()  # one activation tensor shared by both problems
        items = [(xd, _dev(wq), "q4_k"), (xd, _dev(wv), "q6_k")]
        outs, names = _kernels(lambda: ops.quantized_matmul_grouped(items, out_dtype=torch.float32))
        assert any("kq_shot_kernel" in n for n in names), names
        for o, (w, c) in zip(outs, [(wq, "q4_k"), (wv, "q6_k")]):
            ref = okq.qmm_ref(xr, w, c)
            for m in range(rows.shape[0]):
                assert okq.max_rel(o[m:m + 1].cpu().numpy(), ref[m:m + 1]) <= tol, (dt, c, m)
    # fp16 one-signed rows
    x16 = rng.normal(2e4, 1.2e4, size=(8, K)).clip(-6e4, 6e4).astype(np.float16)
    o = ops.quantized_matmul(_dev(x16), _dev(wq), None, "q4_k", out_dtype=torch.float32)
    assert okq.max_rel(o.cpu().numpy(), okq.qmm_ref(x16, wq, "q4_k")) <= TOL


def test_shot_strided_rows_and_outputs_through_the_c_abi(monkeypatch):
    """x rows at a stride past K and y rows at a stride past N, bf16 output,
    through kq_quantized_matmul_grouped directly (no workspace)."""
    import torch
    from gmlx_amd import _lib
    _clean(monkeypatch)
    lib = _lib.lib()
    rng = np.random.default_rng(6)
    K, N, M, xs, ys = 4096, 1000, 6, 4096 + 64, 1000 + 24
    w = quantized_weights(rng, "q4_k", N, K)
    x16 = fp16_rows(rng, M, K)
    xbuf = torch.zeros((M, xs), dtype=torch.float16)
    xbuf[:, :K] = torch.from_numpy(x16)
    xd, wd = xbuf.cuda(), _dev(w)
    y = torch.full((M, ys), 7.0, dtype=torch.bfloat16, device="cuda")

    p = _lib.MatmulProblem(wd.data_ptr(), w.shape[1], xd.data_ptr(), xs, y.data_ptr(), ys, M, N, K, 12)
    stream = torch.cuda.current_stream().cuda_stream
    _, names = _kernels(lambda: _lib.check("kq_quantized_matmul_grouped", lib.kq_quantized_matmul_grouped(
        ctypes.byref(p), 1, _lib.DTYPE_F16, _lib.DTYPE_BF16, None, 0, stream)))
    assert any("kq_shot_kernel" in n for n in names), names
    got = y.float().cpu().numpy()
    assert okq.max_rel(got[:, :N], okq.qmm_ref(x16, w, "q4_k")) <= BF16_TOL
    assert np.all(got[:, N:] == 7.0)   # nothing written past N


def test_shot_declines_past_its_shapes(monkeypatch):
    """33 rows, 17 rows at K = 2048, K of 12 or 48 super-blocks, more than
    two tiles per CU and paired Q6_K tiles at K = 4096 (past 160 KB of LDS)
    take the other kernels (and GMLX_KQ_SHOT=0 declines), with the same
    numerics."""
    import torch
    from gmlx_amd import ops
    _clean(monkeypatch)
    rng = np.random.default_rng(7)
    for M, N, K, c in ((33, 512, 4096, "q4_k"), (17, 512, 2048, "q4_k"), (8, 256, 12288, "q4_k"), (8, 16 * 600, 2048, "q4_k"),
                       (4, 512, 3072, "q4_k"), (8, 16 * 300, 4096, "q6_k")):
        w = quantized_weights(rng, c, N, K)
        x16 = fp16_rows(rng, M, K)
        out, names = _kernels(lambda: ops.quantized_matmul(_dev(x16), _dev(w), None, c, out_dtype=torch.float32))
        assert not any("kq_shot_kernel" in n for n in names), (M, N, K, c, names)
        assert okq.max_rel(out.cpu().numpy(), okq.qmm_ref(x16, w, c)) <= TOL
    monkeypatch.setenv("GMLX_KQ_SHOT", "0")
    w = quantized_weights(rng, "q4_k", 4096, 4096)
    x16 = fp16_rows(rng, 8, 4096)
    out, names = _kernels(lambda: ops.quantized_matmul(_dev(x16), _dev(w), None, "q4_k", out_dtype=torch.float32))
    assert not any("kq_shot_kernel" in n for n in names)
    assert okq.max_rel(out.cpu().numpy(), okq.qmm_ref(x16, w, "q4_k")) <= TOL

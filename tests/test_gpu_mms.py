"""Parity of the mid-batch streaming kernel (kq_stream.hip kq_mms_kernel,
17..64 rows of Q4_K, Q6_K or both, reached through
kq_quantized_matmul_grouped): row counts on both sides of the 32-row form
change, K of one to sixteen super-blocks, unsplit and in K slices (even and
uneven, forced with GMLX_KQ_MMS_S), partial tile groups, several problems
per launch (one codec and Q4_K with Q6_K), few workgroups (several units per
workgroup), bf16 activations, strided rows and every output dtype; a
gate|up-size group by default.  Against the fp64 oracle (max-rel <= 2e-3;
bf16 activations 8e-3), plus bitwise determinism over repeated split calls
(the arrival counters left zero)."""
import numpy as np
import pytest

from helpers import BF16_TOL, TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu

ENV = ("GMLX_KQ_MM", "GMLX_KQ_MM_T", "GMLX_KQ_MMS", "GMLX_KQ_MMS_S", "GMLX_KQ_STREAM_WGS")


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _clear(monkeypatch):
    """Every shape the kernel serves taken (these problems are far smaller
    than the ones it is routed at)."""
    for k in ENV:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("GMLX_KQ_MMS", "2")


@pytest.mark.parametrize("codec", ["q4_k", "q6_k"])
@pytest.mark.parametrize("M", [17, 32, 33, 64])
@pytest.mark.parametrize("K", [256, 2048, 4096])
def test_parity(codec, M, K, monkeypatch):
    """N = 200: 13 tiles in groups of 6, 6 and 1 (the last tile partial),
    unsplit and in the planned K slices (one per super-block here)."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(7000 + 10 * M + K // 256)
    wire = quantized_weights(rng, codec, 200, K)
    x16 = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x16, wire, codec)
    x, w = _dev(x16), _dev(wire)
    for s in ("1", None):
        if s:
            monkeypatch.setenv("GMLX_KQ_MMS_S", s)
        else:
            monkeypatch.delenv("GMLX_KQ_MMS_S", raising=False)
        got = ops.quantized_matmul(x, w, None, codec).float().cpu().numpy()
        assert okq.max_rel(got, ref) <= TOL, (s, okq.max_rel(got, ref))


@pytest.mark.parametrize("S", ["2", "3", "5"])
@pytest.mark.parametrize("M", [17, 40, 64])
def test_split_and_mixed_codecs(S, M, monkeypatch):
    """K = 5 super-blocks in S slices (2 + 3; 1 + 2 + 2; 1 each), groups of
    six tiles over three problems (19, 5 and 6 tiles), for Q4_K alone, Q6_K
    alone and q|k Q4_K with v Q6_K; a second call equals the first bitwise
    (the counters were left zero)."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    monkeypatch.setenv("GMLX_KQ_MMS_S", S)
    rng = np.random.default_rng(100 * M + 10 * int(S))
    K = 1280
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    for codecs in (("q4_k",) * 3, ("q6_k",) * 3, ("q4_k", "q4_k", "q6_k")):
        wires = [quantized_weights(rng, c, n, K) for c, n in zip(codecs, (300, 70, 90))]
        args = [(x, _dev(w), c) for w, c in zip(wires, codecs)]
        outs = ops.quantized_matmul_grouped(args)
        for o, w, c in zip(outs, wires, codecs):
            assert okq.max_rel(o.float().cpu().numpy(), okq.qmm_ref(x16, w, c)) <= TOL, codecs
        again = ops.quantized_matmul_grouped(args)
        assert all(torch.equal(a, b) for a, b in zip(outs, again)), codecs


@pytest.mark.parametrize("codec", ["q4_k", "q6_k"])
@pytest.mark.parametrize("wgs", ["", "1", "3"])
def test_groups_and_few_workgroups(codec, wgs, monkeypatch):
    """Three problems (19, 5 and 6 tiles: groups 6 6 6 1 | 5 | 6) in one
    launch, in the planned five K slices; with 1 or 3 workgroups each walks
    several units (groups, slices, problems and group sizes), the ring
    carrying stages across unit changes."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    if wgs:
        monkeypatch.setenv("GMLX_KQ_STREAM_WGS", wgs)
    rng = np.random.default_rng(71 + len(wgs) + (codec == "q6_k"))
    K, M = 1280, 40
    wires = [quantized_weights(rng, codec, n, K) for n in (300, 70, 96)]
    x16 = fp16_rows(rng, M, K)
    x = _dev(x16)
    outs = ops.quantized_matmul_grouped([(x, _dev(w), codec) for w in wires])
    for o, w in zip(outs, wires):
        ref = okq.qmm_ref(x16, w, codec)
        assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL, (codec, wgs)


@pytest.mark.parametrize("y_dtype", ["float16", "float32", "bfloat16"])
def test_bf16_activations_and_out_dtypes(y_dtype, monkeypatch):
    """bf16 rows reach the kernel as fp16 rows with a power of two per row."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(12)
    K, M = 1024, 50
    wire = quantized_weights(rng, "q4_k", 130, K)
    xf = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    xf[3] *= 300.0  # rows far apart in scale
    xb = torch.from_numpy(xf).to(torch.bfloat16)
    ref = okq.qmm_ref(xb.float().numpy(), wire, "q4_k")
    got = ops.quantized_matmul(xb.cuda(), _dev(wire), None, "q4_k", out_dtype=getattr(torch, y_dtype))
    assert got.dtype == getattr(torch, y_dtype)
    g = got.float().cpu().numpy()
    for row in range(M):  # each row against its own scale
        assert okq.max_rel(g[row], ref[row]) <= BF16_TOL, row


def test_strided_rows_and_determinism(monkeypatch):
    """x rows at a stride of K + 64 read in place; repeated calls bitwise
    equal; the result within the tolerance of the 17..64-row tile kernel's."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(13)
    K, M = 1536, 29
    wire = quantized_weights(rng, "q6_k", 150, K)
    x16 = fp16_rows(rng, M, K)
    ref = okq.qmm_ref(x16, wire, "q6_k")
    big = torch.zeros(M, K + 64, dtype=torch.float16)
    big[:, :K] = torch.from_numpy(x16)
    xv = big.cuda()[:, :K]
    w = _dev(wire)
    a1 = ops.quantized_matmul(xv, w, None, "q6_k")
    a2 = ops.quantized_matmul(xv, w, None, "q6_k")
    assert torch.equal(a1, a2)
    assert okq.max_rel(a1.float().cpu().numpy(), ref) <= TOL
    monkeypatch.setenv("GMLX_KQ_MMS", "0")
    tile = ops.quantized_matmul(xv, w, None, "q6_k").float().cpu().numpy()
    assert okq.max_rel(a1.float().cpu().numpy(), tile) <= TOL


@pytest.mark.parametrize("M", [24, 64])
def test_default_route_gate_up_size(M, monkeypatch):
    """A gate|up-size pair (2 x 12416 rows, K = 4096: 1552 tiles, six per CU
    and more) takes the kernel by default; the weights repeat a 1552-row
    block of distinct rows, so a tile read from the wrong group or problem
    shows (no group offset is a multiple of 1552 rows)."""
    from gmlx_amd import ops
    _clear(monkeypatch)
    monkeypatch.delenv("GMLX_KQ_MMS")
    rng = np.random.default_rng(500 + M)
    K = 4096
    base = quantized_weights(rng, "q4_k", 1552, K)
    gate, up = np.tile(base, (8, 1)), np.tile(base[::-1], (8, 1))
    x16 = fp16_rows(rng, M, K)
    r = okq.qmm_ref(x16, base, "q4_k")
    refs = [np.tile(r, (1, 8)), np.tile(r[:, ::-1], (1, 8))]
    x = _dev(x16)
    outs = ops.quantized_matmul_grouped([(x, _dev(gate), "q4_k"), (x, _dev(up), "q4_k")])
    for o, ref in zip(outs, refs):
        assert okq.max_rel(o.float().cpu().numpy(), ref) <= TOL, M


@pytest.mark.parametrize("M", [17, 64])
def test_strided_rows_through_the_c_abi_split(M, monkeypatch):
    """kq_quantized_matmul_grouped with x rows at a stride of K + 64 and y rows
    at a stride of N + 40, in the planned K slices (the workspace sized by
    kq_matmul_workspace_bytes): the reference in the first N columns, the
    padding columns untouched."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    rng = np.random.default_rng(60 + M)
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


def test_split_launch_graph_replays(monkeypatch):
    """A split launch (the down projection's shape at 40 rows: 5 K slices)
    captured in a HIP graph: three replays, with eager calls on other inputs
    between them, each equal bitwise to the eager result (the arrival
    counters return to zero every call, inside the graph too)."""
    import torch
    from gmlx_amd import ops
    _clear(monkeypatch)
    monkeypatch.delenv("GMLX_KQ_MMS")
    rng = np.random.default_rng(21)
    K, N, M = 12288, 4096, 40
    w = _dev(quantized_weights(rng, "q6_k", N, K))
    x = _dev(fp16_rows(rng, M, K))
    x2 = _dev(fp16_rows(rng, M, K))
    eager = ops.quantized_matmul(x, w, None, "q6_k")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.quantized_matmul(x, w, None, "q6_k")
    for _ in range(3):
        other = ops.quantized_matmul(x2, w, None, "q6_k")
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert not torch.equal(other, eager)

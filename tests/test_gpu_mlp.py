"""The fused dense MLP (kq_fused_mlp / ops.fused_mlp): gmlx's _FusedMLP
forward, down_proj(swiglu(gate(x), up(x))) (gmlx/occupancy_fuse.py:270-316),
in one launch, against fp64 over the same wire bytes by the reference's
metric (max |err| / max |ref|, tests/test_ragged_decode.py:78-81), against
the unfused composition of the same three steps, repeated calls, graph
replays, and the launch's give-up status."""
import numpy as np
import pytest

from helpers import BF16_TOL, TOL, fp16_rows, quantized_weights
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _ref(x, gw, uw, dw, dcodec, act):
    xf = np.asarray(x, np.float64)
    G = okq.dequantize(gw, "q4_k").astype(np.float64)
    U = okq.dequantize(uw, "q4_k").astype(np.float64)
    D = okq.dequantize(dw, dcodec).astype(np.float64)
    g, u = xf @ G.T, xf @ U.T
    if act == "silu":
        a = 0.5 * g * (1.0 + np.tanh(0.5 * g))  # g * sigmoid(g), no overflow for large |g|
    else:
        a = 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))
    return (a * u) @ D.T


@pytest.mark.parametrize("M,K,I,N,dcodec,act", [
    (8, 4096, 12288, 4096, "q6_k", "silu"),   # the Qwen3-8B MLP at B = 8
    (1, 4096, 12288, 4096, "q6_k", "silu"),
    (5, 2048, 6144, 1024, "q6_k", "gelu"),
    (3, 4096, 4096, 1000, "q4_k", "silu"),    # Q4_K down, a partial last tile
    (8, 2048, 2048, 512, "q6_k", "silu"),     # one slice: more workgroups per slice than down tiles
    (2, 4096, 16384, 2048, "q4_k", "gelu"),   # eight slices
])
def test_fused_mlp_matches_fp64(M, K, I, N, dcodec, act):
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(M * 7 + K + I + N)
    gw = quantized_weights(rng, "q4_k", I, K)
    uw = quantized_weights(rng, "q4_k", I, K)
    dw = quantized_weights(rng, dcodec, N, I)
    x = fp16_rows(rng, M, K)
    n0 = ops.counts()["fused_mlp_launches"]
    y = ops.fused_mlp(_dev(x), _dev(gw), _dev(uw), _dev(dw), "q4_k", dcodec, act=act, out_dtype=torch.float32)
    assert ops.counts()["fused_mlp_launches"] == n0 + 1  # the single launch ran
    ref = _ref(x, gw, uw, dw, dcodec, act)
    got = y.cpu().numpy()
    assert okq.max_rel(got, ref) <= TOL, okq.max_rel(got, ref)
    assert ops.fused_mlp_status() == 0


def test_fused_mlp_equals_composition_repeats_and_graph_replays():
    """One launch against the three separate steps (grouped gate|up, GLU,
    down) within tolerance; repeated calls bitwise equal (the slice and tile
    counters return to zero); a captured launch replayed between eager calls
    of another shape equals the eager result bitwise."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(5)
    M, K, I, N = 6, 4096, 8192, 3072
    gw, uw = _dev(quantized_weights(rng, "q4_k", I, K)), _dev(quantized_weights(rng, "q4_k", I, K))
    dw = _dev(quantized_weights(rng, "q6_k", N, I))
    x = _dev(fp16_rows(rng, M, K))
    x2 = _dev(fp16_rows(rng, 4, K))
    n0 = ops.counts()["fused_mlp_launches"]
    outs = [ops.fused_mlp(x, gw, uw, dw, "q4_k", "q6_k") for _ in range(4)]
    assert ops.counts()["fused_mlp_launches"] == n0 + 4
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    g, u = ops.quantized_matmul_grouped([(x, gw, "q4_k"), (x, uw, "q4_k")], out_dtype=torch.float32)
    h = (torch.nn.functional.silu(g) * u).half()
    comp = ops.quantized_matmul(h, dw, None, "q6_k")
    assert okq.max_rel(outs[0].float().cpu().numpy(), comp.float().cpu().numpy()) <= TOL
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out_g = ops.fused_mlp(x, gw, uw, dw, "q4_k", "q6_k")
    for _ in range(3):
        other = ops.fused_mlp(x2, gw, uw, dw, "q4_k", "q6_k")
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, outs[0])
        assert other.shape == (4, N)
    assert ops.fused_mlp_status() == 0


@pytest.mark.parametrize("dt", ["bfloat16", "float32"])
def test_fused_mlp_other_activation_dtypes(dt):
    """bf16 / fp32 activations (rows of very different magnitudes) take the
    three-step composition with h in the activation dtype, as the
    reference's swiglu keeps it: every row matches fp64 on its own scale."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(31)
    M, K, I, N = 4, 2048, 4096, 512
    gw, uw = quantized_weights(rng, "q4_k", I, K), quantized_weights(rng, "q4_k", I, K)
    dw = quantized_weights(rng, "q6_k", N, I)
    x = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    x[0] *= 300.0
    x[1] *= 1e-3
    xd = torch.from_numpy(x).to(getattr(torch, dt))
    y = ops.fused_mlp(xd.cuda(), _dev(gw), _dev(uw), _dev(dw), "q4_k", "q6_k", out_dtype=torch.float32)
    ref = _ref(xd.float().numpy(), gw, uw, dw, "q6_k", "silu")
    got = y.cpu().numpy()
    tol = BF16_TOL if dt == "bfloat16" else TOL
    for m in range(M):
        assert okq.max_rel(got[m], ref[m]) <= tol, (m, okq.max_rel(got[m], ref[m]))


def test_fused_mlp_declines_to_the_composition():
    """Shapes the single launch does not serve (9 rows; K = 1024) run as the
    three separate steps, with the same numerics contract."""
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(9)
    for M, K, I, N in ((9, 4096, 2048, 256), (2, 1024, 2048, 256)):
        gw, uw = quantized_weights(rng, "q4_k", I, K), quantized_weights(rng, "q4_k", I, K)
        dw = quantized_weights(rng, "q6_k", N, I)
        x = fp16_rows(rng, M, K)
        n0 = ops.counts()["fused_mlp_launches"]
        y = ops.fused_mlp(_dev(x), _dev(gw), _dev(uw), _dev(dw), "q4_k", "q6_k", out_dtype=torch.float32)
        assert ops.counts()["fused_mlp_launches"] == n0
        assert okq.max_rel(y.cpu().numpy(), _ref(x, gw, uw, dw, "q6_k", "silu")) <= TOL

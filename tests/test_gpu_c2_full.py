"""Workload C2 at full size: the four launches of a Qwen3-8B Q4_K_M
layer (q|k|v grouped, o, gate|up grouped, down), with the default routing
the benchmark uses, at every batch width the metric is quoted on
(B = 1, 2, 4, 8, 16, 32, 64), against fp64 over the same wire bytes.

Shapes and draws follow the benchmark (bench.py's Qwen3-8B stack; the
reference's occupancy-fused q|k|v and gate|up groups,
gmlx/occupancy_fuse.py:141-344):
N(0, 0.02) weights in the draw order q, k, v, o, gate, up, down, quantised on
the GPU (kq_quantize, byte-identical to the oracle quantiser), fp16 N(0, 1)
activations.  Two weight rows of every 16-row tile of every matrix are
checked (rows 7t mod 16 and 7t + 8 mod 16 of tile t: every tile, both lane
halves), over the whole K, by the reference's metric max |err| / max |ref|
(tests/test_ragged_decode.py:78-81)."""
import numpy as np
import pytest

from helpers import TOL
from oracle import kquant as okq

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 4096, 12288
LAYER = [("q", 4096, 4096, "q4_k"), ("k", 1024, 4096, "q4_k"), ("v", 1024, 4096, "q6_k"),
         ("o", 4096, 4096, "q4_k"), ("gate", INTER, 4096, "q4_k"), ("up", INTER, 4096, "q4_k"),
         ("down", 4096, INTER, "q6_k")]


def _sample_rows(N):
    t = np.arange((N + 15) // 16)
    rows = np.concatenate([16 * t + (7 * t) % 16, 16 * t + (7 * t + 8) % 16])
    return np.sort(rows[rows < N])


@pytest.fixture(scope="module")
def layer():
    import torch
    from gmlx_amd import ops
    rng = np.random.default_rng(0)
    wires, deq = {}, {}
    for name, N, K, codec in LAYER:
        w = torch.from_numpy(rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)).cuda()
        wires[name] = ops.quantize(w, codec)[0]
        del w
        rows = _sample_rows(N)
        sub = wires[name][torch.from_numpy(rows).cuda()].cpu().numpy()
        deq[name] = (rows, okq.dequantize(sub, codec).reshape(len(rows), K).astype(np.float64))
    torch.cuda.synchronize()
    yield wires, deq
    del wires
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 2, 4, 8, 16, 32, 64])
def test_c2_layer_every_batch_width(layer, B, monkeypatch):
    import torch
    from gmlx_amd import ops
    for k in ("GMLX_KQ_STREAM", "GMLX_KQ_MV", "GMLX_KQ_MMS", "GMLX_KQ_MM", "GMLX_KQ_SPLITK",
              "GMLX_KQ_STREAM_WGS", "GMLX_KQ_MV_WGS"):
        monkeypatch.delenv(k, raising=False)
    wires, deq = layer
    rng = np.random.default_rng(100 + B)
    x16 = rng.normal(0.0, 1.0, size=(B, HIDDEN)).astype(np.float16)
    xd16 = rng.normal(0.0, 1.0, size=(B, INTER)).astype(np.float16)
    x, xd = torch.from_numpy(x16).cuda(), torch.from_numpy(xd16).cuda()
    q, k, v = ops.quantized_matmul_grouped([(x, wires["q"], "q4_k"), (x, wires["k"], "q4_k"),
                                            (x, wires["v"], "q6_k")])
    o = ops.quantized_matmul(x, wires["o"], None, "q4_k")
    gate, up = ops.quantized_matmul_grouped([(x, wires["gate"], "q4_k"), (x, wires["up"], "q4_k")])
    down = ops.quantized_matmul(xd, wires["down"], None, "q6_k")
    outs = {"q": q, "k": k, "v": v, "o": o, "gate": gate, "up": up, "down": down}
    for name, N, K, codec in LAYER:
        rows, W = deq[name]
        xin = (xd16 if K == INTER else x16).astype(np.float64)
        ref = xin @ W.T
        got = outs[name].float().cpu().numpy()[:, rows]
        err = okq.max_rel(got, ref)
        assert err <= TOL, (name, B, err)

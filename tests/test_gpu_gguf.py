"""GGUF wire bytes feed the kernels unchanged: tensors written to a GGUF
file, loaded to the GPU through the native reader, multiplied by the
quantized matmul and dequantized, against the oracle on the same bytes."""
import numpy as np
import pytest

from gguf_writer import STRING, write_gguf
from helpers import TOL
from oracle import kquant as okq

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("codec,tid", [("q4_k", 12), ("q6_k", 14), ("iq2_xxs", 16)])
def test_gguf_tensor_to_kernel(tmp_path, codec, tid):
    import torch
    from gmlx_amd import gguf, ops
    rng = np.random.default_rng(tid)
    N, K = 48, 1024
    wire = okq.quantize(rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32), codec)
    p = write_gguf(tmp_path / "w.gguf", kv=[("general.architecture", STRING, "llama")],
                   tensors=[("blk.0.ffn_up.weight", (K, N), tid, wire.tobytes())])
    arrays, codecs, meta, shapes = gguf.load_gguf(p, device="cuda")
    w = arrays["blk.0.ffn_up.weight"]
    assert w.is_cuda and w.dtype == torch.uint8 and tuple(w.shape) == wire.shape
    assert codecs["blk.0.ffn_up.weight"] == codec
    x = rng.normal(0.0, 1.0, size=(3, K)).astype(np.float16)
    y = ops.quantized_matmul(torch.from_numpy(x).cuda(), w, arrays["blk.0.ffn_up.scales"], codec)
    assert okq.max_rel(y.float().cpu().numpy(), okq.qmm_ref(x, wire, codec)) <= TOL
    deq = ops.dequantize(w, None, codec).cpu().numpy()
    assert np.array_equal(deq.view(np.uint32), okq.dequantize(wire, codec).view(np.uint32))

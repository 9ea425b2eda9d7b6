"""Host-side checks that need no GPU: the C-ABI library loads and exports
every symbol include/kq_capi.h and include/kq_gguf.h declare, capability probes and error strings,
the ops' CPU-side validation and decline rails, fault injection, the wire-K
rule, and the leaf-module swap."""
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    names = set()
    for h in ("kq_capi.h", "kq_gguf.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(kq_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    from gmlx_amd import _lib
    L = _lib.lib()
    declared = _header_symbols()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(L, name), name
    assert set(declared) == set(_lib.EXPORTS)


def test_header_sizes_match_the_python_mirror():
    from gmlx_amd import _lib
    text = open(os.path.join(ROOT, "include", "kq_capi.h")).read()

    def define(name):
        m = re.search(r"#define\s+" + name + r"\s+(.+)", text)
        expr = re.sub(r"\(size_t\)", "", m.group(1))
        return eval(expr, {})

    assert define("KQ_MATMUL_COUNTER_BYTES") == _lib.MATMUL_COUNTER_BYTES
    assert define("KQ_SDPA_NOALLOC_SCRATCH_BYTES") == _lib.SDPA_NOALLOC_SCRATCH_BYTES
    assert define("KQ_MAX_GROUP") == _lib.MAX_GROUP


def test_version_strerror_and_capabilities():
    from gmlx_amd import _lib, ops
    assert "gfx950" in _lib.version()
    L = _lib.lib()
    assert L.kq_strerror(0) == b"ok"
    assert b"workspace" in L.kq_strerror(_lib.KQ_ERR_WORKSPACE_TOO_SMALL)
    assert L.kq_codec_block_bytes(12) == 144 and L.kq_codec_block_bytes(14) == 210
    assert L.kq_codec_block_bytes(16) == 66 and L.kq_codec_block_bytes(2) == 0
    assert ops.codecs() == ("q4_k", "q6_k", "iq2_xxs")
    assert all(ops.codec_has_matmul(c) and ops.codec_has_moe_glu(c) for c in ops.codecs())
    assert not ops.codec_has_matmul("q8_0")
    assert L.kq_supports(_lib.OP_SDPA, 0, _lib.DTYPE_F32) == 0
    # matmul / gather activations: fp16, bf16 and fp32 (prepared as scaled fp16)
    assert all(L.kq_supports(op, 12, dt) == 1 for op in (_lib.OP_MATMUL, _lib.OP_GATHER, _lib.OP_MOE_GLU)
               for dt in (_lib.DTYPE_F16, _lib.DTYPE_BF16, _lib.DTYPE_F32))


def test_library_grid_table_is_pinned():
    from gmlx_amd import _lib
    from oracle import kquant as okq
    ptr = _lib.lib().kq_iq2xxs_grid_host()
    assert [ptr[i] for i in range(256)] == okq.iq2xxs_grid()


def test_host_validation_rejects_before_launch():
    """Bad shapes / codecs / workspaces are refused by the C ABI with status
    codes and nothing is launched (null stream, no GPU needed)."""
    import ctypes
    from gmlx_amd import _lib
    L = _lib.lib()
    P = _lib.MatmulProblem
    good = dict(w=16, w_row_bytes=144 * 4, x=16, x_row_stride=1024, y=16, y_row_stride=64, M=2, N=64, K=1024,
                codec=12)

    def call(**over):
        d = dict(good, **over)
        arr = (P * 1)(P(**d))
        return L.kq_quantized_matmul_grouped(arr, 1, _lib.DTYPE_F16, _lib.DTYPE_F16, None, 0, None)

    assert call(K=1000) == _lib.KQ_ERR_BAD_SHAPE
    assert call(codec=3) == _lib.KQ_ERR_UNSUPPORTED_CODEC
    assert call(w_row_bytes=100) == _lib.KQ_ERR_BAD_SHAPE
    assert call(x=18) == _lib.KQ_ERR_BAD_ALIGN
    assert call(w=0) == _lib.KQ_ERR_NULL_POINTER
    arr = (P * 1)(P(**good))
    assert L.kq_quantized_matmul_grouped(arr, 1, 7, _lib.DTYPE_F16, None, 0, None) == _lib.KQ_ERR_UNSUPPORTED_DTYPE
    # fp32 / bf16 activations are prepared in the workspace first: none given, nothing launched
    assert L.kq_quantized_matmul_grouped(arr, 1, _lib.DTYPE_F32, _lib.DTYPE_F16, None, 0, None) == \
        _lib.KQ_ERR_WORKSPACE_TOO_SMALL
    assert L.kq_quantized_matmul_grouped(arr, 9, _lib.DTYPE_F16, _lib.DTYPE_F16, None, 0, None) == \
        _lib.KQ_ERR_TOO_MANY_PROBLEMS
    # fp16 activations at K <= 16 super-blocks need no workspace; bf16 / fp32
    # ones the counter region, then an fp16 copy of the rows (256-byte
    # aligned) and an int32 exponent per row
    ctr = _lib.MATMUL_COUNTER_BYTES
    small_n = dict(good, N=16, K=4096, w_row_bytes=144 * 16, x_row_stride=4096)
    arr = (P * 1)(P(**small_n))
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == 0
    M = small_n["M"]
    want = -(-M * 4096 * 2 // 256) * 256 + -(-M * 4 // 256) * 256
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_BF16) == ctr + want
    # gathers: pair p reads row p / x_pair_div + p / x_skip
    assert L.kq_gather_workspace_bytes(8, 2, 0, 512, _lib.DTYPE_F16) == 0
    assert L.kq_gather_workspace_bytes(8, 2, 0, 512, _lib.DTYPE_F32) == ctr + 4 * 512 * 2 + 256
    assert L.kq_gather_workspace_bytes(9, 1, 4, 256, _lib.DTYPE_BF16) == ctr + (9 + 2) * 256 * 2 + 256
    assert L.kq_sdpa_decode_ragged(16, 16, 16, 16, 16, 16, 2, 8, 3, 128, 100, 0.1, _lib.DTYPE_F16, 16, 16,
                                   1 << 20, None) == _lib.KQ_ERR_BAD_SHAPE
    assert L.kq_sdpa_decode_ragged(16, 16, 16, 16, 16, 16, 2, 8, 2, 80, 100, 0.1, _lib.DTYPE_F16, 16, 16,
                                   1 << 20, None) == _lib.KQ_ERR_BAD_SHAPE
    assert L.kq_sdpa_decode_ragged(16, 16, 16, 16, 16, 16, 2, 8, 2, 128, 100, 0.1, _lib.DTYPE_F16, 16, 16,
                                   16, None) == _lib.KQ_ERR_WORKSPACE_TOO_SMALL
    assert L.kq_moe_router_topk(16, 0, 2000, 4, 2000, 8, None, 16, 16, None) == _lib.KQ_ERR_BAD_SHAPE
    # the shared gate needs one more logit column than the routed experts
    opts = _lib.RouterOptions(1, 1, 0, 1.0, None, 0, None, 0)
    assert L.kq_moe_router_topk(16, 0, 64, 4, 64, 8, ctypes.byref(opts), 16, 16, None) == _lib.KQ_ERR_BAD_SHAPE
    opts = _lib.RouterOptions(1, 0, 7, 1.0, None, 0, None, 0)
    assert L.kq_moe_router_topk(16, 0, 64, 4, 64, 8, ctypes.byref(opts), 16, 16, None) == _lib.KQ_ERR_BAD_ARGUMENT
    # swiglu_clamp needs a positive limit; a plain gather takes no up bias
    ep = _lib.GatherEpilogue(3, 0.0, 1.702, None, None, 0)
    assert L.kq_moe_gather_rows(16, 1, 256, 1, 0, 16, 16, 144 * 16, 144, 16, 256, 12, ctypes.byref(ep), 16, 16,
                                4, 2, 16, 0, 16, 0, None, 0, None) == _lib.KQ_ERR_BAD_ARGUMENT
    ep = _lib.GatherEpilogue(0, 0.0, 0.0, 16, 16, 16)
    assert L.kq_moe_gather_rows(16, 1, 256, 1, 0, 16, None, 144 * 16, 144, 16, 256, 12, ctypes.byref(ep), 16, 16,
                                4, 2, 16, 1, 16, 0, None, 0, None) == _lib.KQ_ERR_BAD_ARGUMENT
    assert L.kq_dequantize(16, 4, 99, 16, 0, None) == _lib.KQ_ERR_UNSUPPORTED_CODEC
    assert L.kq_quantize(16, 2, 100, 100, 12, 16, None) == _lib.KQ_ERR_BAD_SHAPE
    _ = ctypes


def test_split_k_workspace(monkeypatch):
    """K past 16 super-blocks at <= 16 rows (a down projection) cuts K into
    slices of 8 super-blocks (12 past 8 rows): 512 (1024 past 8 rows) bytes of fp32 partials
    per (16-row weight tile, slice) after the counter region; with
    GMLX_KQ_SPLITK=1, none (17..64 rows: test_mid_batch_split_workspace)."""
    from gmlx_amd import _lib
    L = _lib.lib()
    P = _lib.MatmulProblem
    ctr = _lib.MATMUL_COUNTER_BYTES
    down = dict(w=1 << 20, w_row_bytes=210 * 48, x=1 << 21, x_row_stride=12288, y=1 << 22, y_row_stride=4096,
                M=8, N=4096, K=12288, codec=_lib.CODEC_ID["q6_k"])
    arr = (P * 1)(P(**down))
    tiles, slices = 4096 // 16, 48 // 8
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == ctr + tiles * slices * 512
    prepared = 8 * 12288 * 2 + 256
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_BF16) == ctr + prepared + tiles * slices * 512
    monkeypatch.setenv("GMLX_KQ_SPLITK", "3")
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == ctr + tiles * 3 * 512
    monkeypatch.setenv("GMLX_KQ_SPLITK", "1")
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == 0
    monkeypatch.delenv("GMLX_KQ_SPLITK")
    # 9..16 rows: 16-row partial tiles in slices of 12 super-blocks
    arr = (P * 1)(P(**dict(down, M=9)))
    assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == ctr + tiles * (48 // 12) * 1024
    # slices of 8 super-blocks first, then 12, 6, 4: K of 56 -> 7 slices, 36
    # -> 3 (of 12), 28 -> 7 (of 4); 43 (no width divides it): none
    for nb, slices in ((56, 7), (36, 3), (28, 7), (43, 0)):
        arr = (P * 1)(P(**dict(down, K=256 * nb, x_row_stride=256 * nb, w_row_bytes=210 * nb)))
        want = ctr + tiles * slices * 512 if slices else 0
        assert L.kq_matmul_workspace_bytes(arr, 1, _lib.DTYPE_F16) == want, nb


def test_mid_batch_split_workspace(monkeypatch):
    """17..64 rows (the mid-batch streaming kernel): groups of six 16-row
    tiles in K slices, the split leaving the fewest rounds of (stages + one)
    per CU on 256 CUs, with 2 KB (17..32 rows) or 4 KB (33..64) of partials per
    tile and slice: the down projection (43 groups, 48 super-blocks) in 5
    slices, q|k|v (65 groups) in 3, gate|up (256 groups) unsplit; o (43
    groups in 4 slices: 172 units, under three quarters of the CUs) is left
    to the tile kernel and needs none.  GMLX_KQ_MMS=2 takes it anyway;
    GMLX_KQ_MMS_S forces the count (1: none)."""
    from gmlx_amd import _lib
    L = _lib.lib()
    P = _lib.MatmulProblem
    ctr = _lib.MATMUL_COUNTER_BYTES
    q4, q6 = _lib.CODEC_ID["q4_k"], _lib.CODEC_ID["q6_k"]

    def ws(probs):
        arr = (P * len(probs))(*probs)
        return L.kq_matmul_workspace_bytes(arr, len(probs), _lib.DTYPE_F16)

    def prob(M, N, K, codec):
        return P(w=1 << 20, w_row_bytes=(210 if codec == q6 else 144) * (K // 256), x=1 << 21, x_row_stride=K,
                 y=1 << 22, y_row_stride=N, M=M, N=N, K=K, codec=codec)

    assert ws([prob(17, 4096, 12288, q6)]) == ctr + 256 * 5 * 2048
    assert ws([prob(64, 4096, 12288, q6)]) == ctr + 256 * 5 * 4096
    assert ws([prob(40, 4096, 4096, q4)]) == 0
    qkv = [prob(32, 4096, 4096, q4), prob(32, 1024, 4096, q4), prob(32, 1024, 4096, q6)]
    assert ws(qkv) == ctr + 384 * 3 * 2048
    assert ws([prob(64, 12288, 4096, q4), prob(64, 12288, 4096, q4)]) == 0
    monkeypatch.setenv("GMLX_KQ_MMS", "2")
    assert ws([prob(40, 4096, 4096, q4)]) == ctr + 256 * 4 * 4096
    monkeypatch.setenv("GMLX_KQ_MMS_S", "2")
    assert ws([prob(64, 4096, 4096, q4)]) == ctr + 256 * 2 * 4096
    monkeypatch.setenv("GMLX_KQ_MMS_S", "1")
    assert ws([prob(64, 4096, 4096, q4)]) == 0


def test_mixed_group_takes_two_k_slices():
    """A Q4_K + Q6_K group of K <= 16 super-blocks (the q|k|v of a Q4_K_M
    layer) is cut into two K slices: its workspace holds the counter region and
    two 512-byte partial tiles per 16-row tile; a one-codec group of the same
    K needs none."""
    from gmlx_amd import _lib
    L = _lib.lib()
    P = _lib.MatmulProblem
    base = dict(w=1 << 20, x=1 << 21, x_row_stride=4096, y=1 << 22, M=8, K=4096)
    q = P(**base, w_row_bytes=16 * 144, y_row_stride=4096, N=4096, codec=_lib.CODEC_ID["q4_k"])
    k = P(**base, w_row_bytes=16 * 144, y_row_stride=1024, N=1024, codec=_lib.CODEC_ID["q4_k"])
    v = P(**base, w_row_bytes=16 * 210, y_row_stride=1024, N=1024, codec=_lib.CODEC_ID["q6_k"])
    tiles = (4096 + 1024 + 1024) // 16
    assert L.kq_matmul_workspace_bytes((P * 3)(q, k, v), 3, _lib.DTYPE_F16) == \
        _lib.MATMUL_COUNTER_BYTES + tiles * 2 * 512
    assert L.kq_matmul_workspace_bytes((P * 2)(q, k), 2, _lib.DTYPE_F16) == 0


def test_ops_refuse_cpu_tensors():
    from gmlx_amd import ops
    x = torch.zeros(2, 256, dtype=torch.float16)
    w = torch.zeros(16, 144, dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU only"):
        ops.quantized_matmul(x, w, None, "q4_k")
    with pytest.raises(ValueError, match="GPU only"):
        ops.dequantize(w, None, "q4_k")


def test_ragged_attention_declines_like_the_reference():
    """Guard rails return None before any GPU work (gmlx/qwen35_attn.py:412-431)."""
    from gmlx_amd import ops
    q = torch.zeros(2, 16, 1, 80, dtype=torch.bfloat16)
    k = torch.zeros(2, 2, 512, 80, dtype=torch.bfloat16)
    assert ops.ragged_decode_attention(q, k, k, [0, 0], 80 ** -0.5) is None        # head dim 80
    q = torch.zeros(2, 16, 1, 128, dtype=torch.float16)
    k = torch.zeros(2, 2, 512, 128, dtype=torch.float16)
    assert ops.ragged_decode_attention(q, k, k, [0], 0.1) is None                    # pads != B
    assert ops.ragged_decode_attention(q, k, k, [0, -1], 0.1) is None                # negative pad
    assert ops.ragged_decode_attention(q, k, k, [0, 512], 0.1) is None               # pad >= L
    assert ops.ragged_decode_attention(q.float(), k.float(), k.float(), [0, 0], 0.1) is None
    q2 = torch.zeros(2, 16, 2, 128, dtype=torch.float16)
    assert ops.ragged_decode_attention(q2, k, k, [0, 0], 0.1) is None                # S != 1
    k3 = torch.zeros(2, 3, 512, 128, dtype=torch.float16)
    assert ops.ragged_decode_attention(q, k3, k3, [0, 0], 0.1) is None               # Hq % Hkv


def test_fault_injection(monkeypatch):
    from gmlx_amd import KQError, ops
    monkeypatch.setenv("GMLX_HIP_FAULT", "quantized_matmul,moe_router_topk")
    x = torch.zeros(2, 256, dtype=torch.float16)
    w = torch.zeros(16, 144, dtype=torch.uint8)
    with pytest.raises(KQError, match="fault injected"):
        ops.quantized_matmul(x, w, None, "q4_k")
    with pytest.raises(KQError):
        ops.moe_router_topk(torch.zeros(2, 8), 2)
    # an injected fault on the attention route reads as a decline upstream
    monkeypatch.setenv("GMLX_HIP_FAULT", "ragged_decode_attention")
    q = torch.zeros(1, 8, 1, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
    with pytest.raises(KQError):
        ops.ragged_decode_attention(q, k, k, [0], 0.1)


def test_wire_k_rule():
    from gmlx_amd.ops import wire_k
    assert wire_k(144 * 16, "q4_k") == 4096
    assert wire_k(210 * 48, "q6_k") == 12288
    assert wire_k(66 * 28, "iq2_xxs") == 7168
    assert wire_k(145, "q4_k") == -1


def test_install_kquant_modules_swaps_linear_leaves():
    from gmlx_amd.nn import KQuantLinear, install_kquant_modules
    model = torch.nn.Sequential(torch.nn.Linear(512, 64), torch.nn.ReLU(), torch.nn.Linear(64, 8))
    n = install_kquant_modules(model, {"0.weight": "q6_k"})
    assert n == 1
    assert isinstance(model[0], KQuantLinear) and model[0].kquant_type == "q6_k"
    assert tuple(model[0].weight.shape) == (64, 2 * 210) and model[0].bias is not None
    assert isinstance(model[2], torch.nn.Linear)
    with pytest.raises(ValueError, match="no recognized module"):
        install_kquant_modules(model, {"1.weight": "q4_k"})
    _ = np


def test_install_kquant_modules_swaps_embeddings_and_expert_stacks(monkeypatch):
    """The leaf swap's three kinds (gmlx/modules.py:1539-1552): nn.Embedding
    -> KQuantEmbedding with the activation dtype out, a 3-D expert stack
    (registered class, or a class named *SwitchLinear) -> KQuantSwitchLinear
    with its bias carried over."""
    from gmlx_amd import nn as knn

    class SwitchLinear(torch.nn.Module):
        def __init__(self, e, o, i, bias):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(e, o, i))
            self.bias = torch.nn.Parameter(torch.zeros(e, o)) if bias else None

    class Experts(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(4, 32, 256))
            self.bias = None

    model = torch.nn.ModuleDict({"emb": torch.nn.Embedding(100, 512), "sw": SwitchLinear(8, 64, 512, True),
                                 "ex": Experts(), "out": torch.nn.Linear(512, 16)})
    with pytest.raises(ValueError, match="no recognized module"):
        knn.install_kquant_modules(model, {"ex.weight": "q4_k"})
    knn.register_switch_linear(Experts)
    monkeypatch.setenv("GMLX_ACTIVATION_DTYPE", "float16")
    n = knn.install_kquant_modules(model, {"emb.weight": "q6_k", "sw.weight": "q4_k", "ex.weight": "q4_k"})
    assert n == 3
    assert isinstance(model["emb"], knn.KQuantEmbedding) and model["emb"].out_dtype == torch.float16
    assert tuple(model["emb"].weight.shape) == (100, 2 * 210)
    sw = model["sw"]
    assert isinstance(sw, knn.KQuantSwitchLinear) and tuple(sw.weight.shape) == (8, 64, 2 * 144)
    assert sw.bias is not None and tuple(sw.bias.shape) == (8, 64)
    assert isinstance(model["ex"], knn.KQuantSwitchLinear) and model["ex"].bias is None
    assert isinstance(model["out"], torch.nn.Linear)
    assert knn.install_kquant_modules(model, {"emb.weight": "q6_k"}) == 0   # already swapped
    monkeypatch.setenv("GMLX_ACTIVATION_DTYPE", "auto")
    assert knn.activation_dtype() == torch.bfloat16

"""K-quant ops on torch tensors, mirroring the mlx_kquant op surface gmlx binds.

Every op validates on the host, allocates its output with torch on the input's
device, and launches the gfx950 kernels of libgmlx_amd.so on the current torch
stream.  There is no CPU path: CPU tensors, a missing library or an
unsupported shape raise.  Reference call sites are cited per op.

Op names and argument orders follow the reference's calls:
  dequantize(w, scales, codec, dtype)            gmlx/modules.py:1461
  quantize(w, codec) -> (wire, scales)           tests/test_dequant_unattachable.py:36
  quantized_matmul(x, w, scales, codec, transpose=True)   gmlx/occupancy_fuse.py:162-165
  fused_mlp(x, gate_w, up_w, down_w, codec, down_codec, act)  _FusedMLP, gmlx/occupancy_fuse.py:270-316
  gather_qmm / KQuantSwitchLinear                tests/test_native_fp.py:420-428
  moe_glu_gather_kq(x, gate_w, up_w, codec, idx, act=, limit=, alpha=,
                    gate_bias=, up_bias=)        gmlx/modules.py:557-588
  gather_qmv_kq(h, down_w, codec, idx, bias=)    gmlx/modules.py:595-597
  gather_qmv_mix_ns_kq(h, down_w, codec, idx, scores)     gmlx/modules.py:591-593
  moe_router_topk(logits, k, norm_topk_prob, shared_gate=, per_expert_scale=,
                  bias=, scoring=, scale=)       gmlx/modules.py:750-752, 1043-1046;
                                                 gmlx/deepseek_v4_model.py:1179-1187
  sdpa_decode_gqa(q, k, v, scale, starts=)       gmlx/gemma4_batched_sdpa.py:221-222
  ragged_decode_attention(q, k, v, pads, scale)  gmlx/qwen35_attn.py:395-493
"""
from __future__ import annotations

import ctypes
import os
from collections import OrderedDict

import torch

from . import _lib
from ._lib import CODEC_ID, DTYPE_BF16, DTYPE_F16, DTYPE_F32, KQ_OK, KQError, MatmulProblem, check, lib

QK_K = 256
BLOCK_BYTES = {"q4_k": 144, "q6_k": 210, "iq2_xxs": 66}
_TORCH_DTYPE = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

__all__ = [
    "codecs", "codec_has_matmul", "codec_has_moe_glu", "dequantize", "quantize", "quantized_matmul",
    "quantized_matmul_grouped", "fused_mlp", "fused_mlp_status", "counts", "moe_route", "gather_qmm", "moe_glu_gather_kq", "gather_qmv_kq",
    "gather_qmv_mix_ns_kq", "moe_router_topk", "sdpa_decode_ragged", "sdpa_decode_gqa",
    "ragged_decode_attention", "wire_k",
]


# ------------------------------------------------------------------ helpers

def _fault(op):
    """GMLX_HIP_FAULT=<op>[,<op>...] makes that op reject the call before any
    launch (tests exercise the callers' decline paths on CPU with it)."""
    names = os.environ.get("GMLX_HIP_FAULT", "")
    if names and (op in names.split(",") or names == "all"):
        raise KQError(op, _lib.KQ_ERR_LAUNCH_FAILED, "fault injected by GMLX_HIP_FAULT")


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_gpu(*ts):
    for t in ts:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("gmlx_amd ops run on the GPU only: got a non-CUDA tensor")


def _codec_id(codec):
    try:
        return CODEC_ID[codec]
    except KeyError:
        raise ValueError(f"unsupported codec {codec!r}; have {tuple(CODEC_ID)}") from None


def _dt(dtype):
    try:
        return _TORCH_DTYPE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def wire_k(wire_cols, codec):
    """Logical K of a wire row of `wire_cols` bytes (-1 if not whole blocks);
    the rule of gmlx/modules.py:_kq_wire_k (:253-257)."""
    bpb = BLOCK_BYTES[codec]
    return (wire_cols // bpb) * QK_K if wire_cols % bpb == 0 else -1


def _rows_view(x):
    """2-D [M, K] view of x[..., K] with unit inner stride, 16-byte aligned
    base and 8-element aligned row stride (copying when needed)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if (x2.stride(1) != 1 or x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) % 8)
            or x2.stride(0) < K):
        x2 = x2.contiguous()
    return x2


class _Workspaces:
    """Scratch per (op family, device, stream), grown on demand.  Buffers
    start zeroed: a matmul / gather workspace begins with per-tile arrival
    counters that must be zero on a buffer's first use and that every call
    leaves zero; the rest (attention split partials, prepared activation
    rows, partial tiles) is written before it is read.  So one buffer serves
    every later call of its family on its stream; families keep their own,
    so a call of one never overwrites what a queued call of another still
    reads.

    A HIP graph captured from these calls holds the buffer's address, so a
    buffer is never freed once used: when a family's buffer must grow, the
    old one is kept (its counters left zero by its last call) for the graphs
    that replay it, and later calls use the new one.  A capture runs on its
    own stream, so it gets its own buffer (allocated in the capture, from the
    graph's pool, and zeroed by a fill kernel, not a memset)."""

    def __init__(self):
        self._ws = {}
        self._retired = []

    def get(self, kind, device, stream_handle, nbytes):
        key = (kind, device.index, stream_handle)
        cur = self._ws.get(key)
        if cur is None or cur.numel() < nbytes:
            if cur is not None:
                self._retired.append(cur)
            cur = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            self._ws[key] = cur
        return cur


_WS = _Workspaces()
_COUNTS = {"fused_mlp_launches": 0, "route_launches": 0}


# ------------------------------------------------------------ capabilities

def codecs():
    """Codecs with kernels here (kq.codecs(), gmlx/modules.py:179-181)."""
    return tuple(CODEC_ID)


def codec_has_matmul(codec):
    return codec in CODEC_ID and bool(lib().kq_supports(_lib.OP_MATMUL, CODEC_ID[codec], DTYPE_F16))


def codec_has_moe_glu(codec):
    return codec in CODEC_ID and bool(lib().kq_supports(_lib.OP_MOE_GLU, CODEC_ID[codec], DTYPE_F16))


# ------------------------------------------------------- dequant / quantize

def dequantize(w, scales=None, codec="q4_k", dtype=torch.float32):
    """Wire bytes [..., nb*bpb] -> [..., nb*256] of `dtype`.  float32 output is
    bit-exact to the GGML dequantize_row_* definition.  `scales` is the
    reference's vestigial placeholder and is ignored."""
    _fault("dequantize")
    _require_gpu(w)
    cid = _codec_id(codec)
    if w.dtype != torch.uint8:
        raise ValueError("wire bytes must be uint8")
    bpb = BLOCK_BYTES[codec]
    if w.shape[-1] % bpb:
        raise ValueError(f"wire width {w.shape[-1]} is not a whole number of {codec} blocks")
    w = w.contiguous()
    nb = w.numel() // bpb
    out = torch.empty((*w.shape[:-1], (w.shape[-1] // bpb) * QK_K), dtype=dtype, device=w.device)
    check("kq_dequantize", lib().kq_dequantize(w.data_ptr(), nb, cid, out.data_ptr(), _dt(dtype), _stream(w)))
    return out


def quantize(w, codec):
    """fp32 weights [..., K] -> (wire uint8 [..., K/256*bpb], scales placeholder
    uint8[1]) on the GPU.  Q4_K/Q6_K follow llama.cpp's reference quantizers."""
    _fault("quantize")
    _require_gpu(w)
    cid = _codec_id(codec)
    K = w.shape[-1]
    if K % QK_K:
        raise ValueError(f"K={K} is not a multiple of {QK_K}")
    w2 = w.reshape(-1, K).to(torch.float32).contiguous()
    rows = w2.shape[0]
    bpb = BLOCK_BYTES[codec]
    wire = torch.empty((rows, (K // QK_K) * bpb), dtype=torch.uint8, device=w.device)
    check("kq_quantize", lib().kq_quantize(w2.data_ptr(), rows, K, w2.stride(0), cid, wire.data_ptr(),
                                           _stream(w)))
    return wire.reshape(*w.shape[:-1], wire.shape[-1]), torch.zeros(1, dtype=torch.uint8, device=w.device)


# ------------------------------------------------------------------ matmul

def _problem(x2, w, codec, y2):
    N = w.shape[0]
    K = x2.shape[1]
    if wire_k(w.shape[-1], codec) != K:
        raise ValueError(f"x has K={K} but the {codec} wire rows hold {wire_k(w.shape[-1], codec)} values")
    if w.stride(-1) != 1:
        raise ValueError("wire rows must be contiguous bytes")
    return MatmulProblem(w.data_ptr(), w.stride(0), x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0),
                         x2.shape[0], N, K, _codec_id(codec))


def _launch_grouped(probs, x_dt, y_dt, device, stream):
    arr = (MatmulProblem * len(probs))(*probs)
    L = lib()
    need = L.kq_matmul_workspace_bytes(arr, len(probs), x_dt)
    ws_ptr, ws_len = None, 0
    if need:
        ws = _WS.get("matmul", device, stream.value, need)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    check("kq_quantized_matmul_grouped",
          L.kq_quantized_matmul_grouped(arr, len(probs), x_dt, y_dt, ws_ptr, ws_len, stream))


def quantized_matmul(x, w, scales=None, codec="q4_k", transpose=True, out_dtype=None):
    """y[..., N] = x[..., K] . dequant(w[N, K])^T with fp32 accumulation
    (KQuantLinear forward).  Output dtype = x dtype unless `out_dtype`."""
    _fault("quantized_matmul")
    if not transpose:
        raise ValueError("only transpose=True (y = x . W^T) is supported, as gmlx calls it")
    _require_gpu(x, w)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"activations must be float16, bfloat16 or float32, got {x.dtype}")
    if w.dim() != 2 or w.dtype != torch.uint8:
        raise ValueError("w must be a uint8 wire matrix [N, K/256*block_bytes]")
    x2 = _rows_view(x)
    out_dtype = out_dtype or x.dtype
    y = torch.empty((x2.shape[0], w.shape[0]), dtype=out_dtype, device=x.device)
    if x2.shape[0] > 0 and w.shape[0] > 0:
        s = _stream(x)
        _launch_grouped([_problem(x2, w, codec, y)], _dt(x.dtype), _dt(out_dtype), x.device, s)
    return y.reshape(*x.shape[:-1], w.shape[0])


def fused_mlp(x, gate_w, up_w, down_w, codec="q4_k", down_codec=None, act="silu", out_dtype=None):
    """gmlx's _FusedMLP forward (gmlx/occupancy_fuse.py:270-316):
    down_proj(swiglu(gate(x), up(x))), with h = act(x . Wg^T) * (x . Wu^T)
    computed in fp32 and held in the activation dtype (the dtype the
    reference's swiglu hands down_proj).  x [..., K]; gate / up wire
    [I, K/256*bpb] of `codec`; down wire [N, I/256*bpb] of `down_codec`
    (default `codec`).  fp16 activations of at most 8 rows with the served
    codecs and shapes (kq_fused_mlp) run in one launch; otherwise the same
    three steps run as the reference runs them: the grouped gate|up matmul,
    the GLU, the down matmul.""" 
    _fault("fused_mlp")
    _require_gpu(x, gate_w, up_w, down_w)
    down_codec = down_codec or codec
    if act not in ("silu", "gelu"):
        raise ValueError(f"act must be 'silu' or 'gelu', got {act!r}")
    if gate_w.shape != up_w.shape:
        raise ValueError("gate and up wires must have the same shape")
    x2 = _rows_view(x)
    M, K = x2.shape
    I, N = gate_w.shape[0], down_w.shape[0]
    if wire_k(gate_w.shape[-1], codec) != K or wire_k(down_w.shape[-1], down_codec) != I:
        raise ValueError("wire widths do not match x's K and gate's rows")
    out_dtype = out_dtype or x.dtype
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M == 0:
        return y.reshape(*x.shape[:-1], N)
    L = lib()
    s = _stream(x)
    need = L.kq_fused_mlp_workspace_bytes(M, K, I, N, _dt(x.dtype))
    ws = _WS.get("mlp", x.device, s.value, need)
    gate_w, up_w, down_w = gate_w.contiguous(), up_w.contiguous(), down_w.contiguous()
    rc = L.kq_fused_mlp(x2.data_ptr(), _dt(x.dtype), x2.stride(0), M, K, gate_w.data_ptr(), up_w.data_ptr(),
                        gate_w.stride(0), _codec_id(codec), I, down_w.data_ptr(), down_w.stride(0),
                        _codec_id(down_codec), N, _lib.ACT_ID[act], y.data_ptr(), _dt(out_dtype), y.stride(0),
                        ws.data_ptr(), ws.numel(), s)
    if rc == KQ_OK:
        _COUNTS["fused_mlp_launches"] += 1
    elif rc == _lib.KQ_ERR_BAD_SHAPE:
        g, u = quantized_matmul_grouped([(x2, gate_w, codec), (x2, up_w, codec)], out_dtype=torch.float32)
        gf = torch.nn.functional.silu(g) if act == "silu" else torch.nn.functional.gelu(g, approximate="tanh")
        h = (gf * u).to(x.dtype)
        y = quantized_matmul(h, down_w, None, down_codec, out_dtype=out_dtype)
    else:
        check("kq_fused_mlp", rc)
    return y.reshape(*x.shape[:-1], N)


def counts():
    """Launch counts since import: the single-launch fused MLP
    ("fused_mlp_launches") and the expert sorts ("route_launches")."""
    return dict(_COUNTS)


def fused_mlp_status(device=None):
    """1 if a fused MLP launch on this device's current stream gave up a
    wait (see kq_fused_mlp), else 0.  Synchronises the stream."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    s = torch.cuda.current_stream(device).cuda_stream
    ws = _WS._ws.get(("mlp", device.index, s))
    if ws is None:
        return 0
    off = _lib.FUSED_MLP_STATUS_OFFSET
    return int(ws[off:off + 4].view(torch.int32).item())


def quantized_matmul_grouped(items, out_dtype=None):
    """Run up to 8 independent quantized matmuls in ONE launch.

    items: sequence of (x, w, codec); every x shares one dtype (f16, bf16 or
    f32; bf16 / f32 rows are prepared as fp16 with a power of two per row).
    Returns the list of outputs.  This is the launch-level form of the
    reference's occupancy fusion (gmlx/occupancy_fuse.py:141-344, q|k|v and
    gate|up concatenated wires): codecs may differ (Q4_K q/k with Q6_K v) and
    no wire bytes are concatenated."""
    _fault("quantized_matmul")
    if not items or len(items) > _lib.MAX_GROUP:
        raise ValueError(f"need 1..{_lib.MAX_GROUP} problems")
    x0 = items[0][0]
    out_dtype = out_dtype or x0.dtype
    probs, outs = [], []
    for x, w, codec in items:
        _require_gpu(x, w)
        if x.dtype != x0.dtype:
            raise ValueError("all activations of a group must share a dtype")
        x2 = _rows_view(x)
        y = torch.empty((x2.shape[0], w.shape[0]), dtype=out_dtype, device=x.device)
        outs.append(y.reshape(*x.shape[:-1], w.shape[0]))
        if x2.shape[0] and w.shape[0]:
            probs.append(_problem(x2, w, codec, y))
    if probs:
        _launch_grouped(probs, _dt(x0.dtype), _dt(out_dtype), x0.device, _stream(x0))
    return outs


# --------------------------------------------------------------------- MoE

def moe_route(idx, n_experts):
    """Group (token, slot) pairs by expert on the device.  Returns (seg_info,
    pair_order) int32 tensors as documented for kq_moe_route."""
    _require_gpu(idx)
    idx32 = idx.reshape(-1).to(torch.int32).contiguous()
    P = idx32.numel()
    seg = torch.empty(2 + 2 * n_experts, dtype=torch.int32, device=idx.device)
    order = torch.empty(max(2 * P, 1), dtype=torch.int32, device=idx.device)
    check("kq_moe_route", lib().kq_moe_route(idx32.data_ptr(), P, n_experts, seg.data_ptr(), order.data_ptr(),
                                             _stream(idx)))
    _COUNTS["route_launches"] += 1
    return seg, order


class _RouteMemo:
    """Routing tables handed from one gather to the next.  A MoE layer passes
    one `idx` to its GLU gather and then to its down gather; grouping the
    pairs once serves both.  A gather that routes leaves its tables here;
    the next gather over the same index tensor (same storage, geometry and
    version counter, so not written in place since, on the same stream and
    on the same side of a graph capture) takes them and removes the entry,
    so a third call, or the next layer over a reused buffer, routes afresh.
    An entry keeps its index tensor alive, so its storage cannot be handed
    to another tensor while the entry exists."""

    def __init__(self, size=8):
        self._d = OrderedDict()
        self._size = size

    @staticmethod
    def _key(idx, n_experts, stream_handle):
        return (idx.data_ptr(), tuple(idx.shape), tuple(idx.stride()), idx.dtype, idx._version, n_experts,
                idx.device.index, stream_handle, torch.cuda.is_current_stream_capturing())

    def take(self, idx, n_experts, stream_handle):
        key = self._key(idx, n_experts, stream_handle)
        hit = self._d.get(key)
        if hit is None:
            return None
        if hit[3] > 1:
            self._d[key] = (hit[0], hit[1], hit[2], hit[3] - 1)
        else:
            del self._d[key]
        return hit[1], hit[2]

    def put(self, idx, n_experts, stream_handle, seg, order, uses=1):
        self._d[self._key(idx, n_experts, stream_handle)] = (idx, seg, order, uses)
        if len(self._d) > self._size:
            self._d.popitem(last=False)


_ROUTES = _RouteMemo()


def _routed(idx, n_experts):
    """(seg_info, pair_order) for idx: the tables the previous gather over
    the same idx left, else a fresh kq_moe_route (left for the next one)."""
    sh = _stream(idx).value
    hit = _ROUTES.take(idx, n_experts, sh)
    if hit is not None:
        return hit
    seg, order = moe_route(idx, n_experts)
    _ROUTES.put(idx, n_experts, sh, seg, order)
    return seg, order


def _expert_stack(w, codec, K):
    if w.dim() != 3 or w.dtype != torch.uint8:
        raise ValueError("expert weights must be a uint8 wire stack [E, N, K/256*block_bytes]")
    if wire_k(w.shape[-1], codec) != K:
        raise ValueError(f"activations have K={K} but the wire rows hold {wire_k(w.shape[-1], codec)}")
    if w.stride(-1) != 1 or w.stride(1) < w.shape[-1] or w.stride(0) < w.stride(1) * w.shape[1]:
        w = w.contiguous()
    return w


def _x_dt(x):
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"unsupported activation dtype {x.dtype}")
    return _dt(x.dtype)


def _bias_rows(b, E, N, name, device):
    """Per-expert fp32 bias rows [E, N] (the reference caches them as float32
    copies, gmlx/modules.py:625-633)."""
    if b is None:
        return None
    if not isinstance(b, torch.Tensor) or b.device != device:
        raise ValueError(f"{name} must be a tensor on the activations' device")
    if tuple(b.shape[-2:] if b.dim() >= 2 else (1,) + tuple(b.shape)) != (E, N):
        raise ValueError(f"{name} must be [{E}, {N}] (one row of N biases per expert)")
    return b.reshape(E, N).to(torch.float32).contiguous()


def _epilogue(act, limit, alpha, gate_bias, up_bias, E, N, device):
    """GatherEpilogue for act= / limit= / alpha= / gate_bias= / up_bias= of
    the fused GLU gathers (gmlx/modules.py:557-566), plus the tensors it
    points at (kept alive for the launch)."""
    if act not in _lib.ACT_ID:
        raise ValueError(f"act {act!r} has no kernel epilogue; have {tuple(_lib.ACT_ID)}")
    if act in ("silu_limit", "swiglu_clamp"):
        if limit is None:
            limit = 7.0 if act == "swiglu_clamp" else None
        if limit is None or not float(limit) > 0.0:
            raise ValueError(f"act {act!r} needs limit > 0")
    elif any(v is not None for v in (limit, alpha, gate_bias, up_bias)):
        raise ValueError(f"act {act!r} takes no limit / alpha / biases")
    if act != "swiglu_clamp" and (gate_bias is not None or up_bias is not None):
        raise ValueError("gate_bias / up_bias belong to act='swiglu_clamp'")
    gb = _bias_rows(gate_bias, E, N, "gate_bias", device)
    ub = _bias_rows(up_bias, E, N, "up_bias", device)
    ep = _lib.GatherEpilogue(_lib.ACT_ID[act], float(limit or 0.0),
                             float(1.702 if alpha is None and act == "swiglu_clamp" else (alpha or 0.0)),
                             None if gb is None else gb.data_ptr(), None if ub is None else ub.data_ptr(), N)
    return ep, (gb, ub)


def _gather_rows(x_ptr, x_dt, x_stride, x_pair_div, x_skip, w, w_up, codec, ep, seg, order, P, E, y_ptr, y_dt,
                 y_stride, y_skip, K, stream):
    L = lib()
    need = L.kq_gather_workspace_bytes(P, x_pair_div, x_skip, K, x_dt)
    ws_ptr, ws_len = None, 0
    if need:
        ws = _WS.get("gather", w.device, stream.value, need)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    rc = L.kq_moe_gather_rows(x_ptr, x_dt, x_stride, x_pair_div, x_skip, w.data_ptr(),
                              None if w_up is None else w_up.data_ptr(), w.stride(0), w.stride(1), w.shape[1],
                              K, _codec_id(codec), None if ep is None else ctypes.byref(ep), seg.data_ptr(),
                              order.data_ptr(), P, E, y_ptr, y_dt, y_stride, y_skip, ws_ptr, ws_len, stream)
    check("kq_moe_gather_rows", rc)


def gather_qmm(x, w, scales=None, codec="q4_k", indices=None, sorted_indices=False, out_dtype=None, bias=None):
    """KQuantSwitchLinear forward: x (T, 1, 1, K) or (T, K), indices (T, k)
    -> (T, k, 1, N) with y[t, s] = dequant(w[indices[t, s]]) . x[t]
    (+ bias[indices[t, s]], fp32 [E, N], added in the fp32 epilogue).
    `sorted_indices` is accepted for signature parity; grouping by expert
    always happens on the device."""
    _fault("gather_qmm")
    _require_gpu(x, w, indices)
    K = x.shape[-1]
    T, k = indices.shape[0], indices.shape[-1]
    x2 = _rows_view(x)
    if x2.shape[0] != T:
        raise ValueError(f"x has {x2.shape[0]} rows for {T} index rows")
    w = _expert_stack(w, codec, K)
    out_dtype = out_dtype or x.dtype
    E, N = w.shape[0], w.shape[1]
    y = torch.empty((T * k, N), dtype=out_dtype, device=x.device)
    b = _bias_rows(bias, E, N, "bias", x.device)
    ep = None if b is None else _lib.GatherEpilogue(_lib.ACT_ID["silu"], 0.0, 0.0, b.data_ptr(), None, N)
    if T * k:
        seg, order = _routed(indices, E)
        _gather_rows(x2.data_ptr(), _x_dt(x2), x2.stride(0), k, 0, w, None, codec, ep, seg, order, T * k, E,
                     y.data_ptr(), _dt(out_dtype), N, 0, K, _stream(x2))
    return y.reshape(T, k, 1, N)


def moe_glu_gather_kq(x, gate_w, up_w, codec, idx, act="silu", limit=None, alpha=None, gate_bias=None,
                      up_bias=None, out_dtype=torch.float32):
    """Fused MoE GLU gather (gmlx/modules.py:557-588): h[t, s] =
    act(Wg[e] . x[t], Wu[e] . x[t]), e = idx[t, s], computed in fp32 -> (t, k, I)
    of out_dtype.  act: "silu", "gelu" (tanh form), "silu_limit" (limit=) or
    "swiglu_clamp" (limit=, alpha=, gate_bias= / up_bias= fp32 [E, I]).
    out_dtype float32 (default) keeps any range; float16 / bfloat16 round h
    to the activation dtype the stock SwitchGLU path produces, so the down
    gather reads it without a preparation pass (an fp16 h rounds exactly as
    the prepared fp32 row does, and past 65504 it is inf, as in the stock
    fp16 path)."""
    _fault("moe_glu_gather_kq")
    _require_gpu(x, gate_w, up_w, idx)
    K = x.shape[-1]
    t, k = idx.shape[0], idx.shape[-1]
    x2 = _rows_view(x)
    gate_w = _expert_stack(gate_w, codec, K)
    up_w = _expert_stack(up_w, codec, K)
    if gate_w.shape != up_w.shape or gate_w.stride() != up_w.stride():
        raise ValueError("gate and up stacks must share shape and layout")
    E, I = gate_w.shape[0], gate_w.shape[1]
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError(f"out_dtype {out_dtype} is not float32, float16 or bfloat16")
    ep, keep = _epilogue(act, limit, alpha, gate_bias, up_bias, E, I, x.device)
    h = torch.empty((t * k, I), dtype=out_dtype, device=x.device)
    if t * k:
        seg, order = _routed(idx, E)
        _gather_rows(x2.data_ptr(), _x_dt(x2), x2.stride(0), k, 0, gate_w, up_w, codec, ep, seg, order, t * k, E,
                     h.data_ptr(), _dt(out_dtype), I, 0, K, _stream(x2))
    del keep
    return h.reshape(t, k, I)


def gather_qmv_kq(h, down_w, codec, idx, bias=None, out_dtype=torch.float32):
    """Per-pair down projection (gmlx/modules.py:595-597): y[t, s] =
    dequant(Wd[idx[t, s]]) . h[t, s] (+ bias[idx[t, s]], fp32 [E, N]) ->
    (t, k, N).  h (t, k, I) float32/float16/bfloat16."""
    _fault("gather_qmv_kq")
    _require_gpu(h, down_w, idx)
    t, k = idx.shape[0], idx.shape[-1]
    I = h.shape[-1]
    h2 = _rows_view(h)
    if h2.shape[0] != t * k:
        raise ValueError("h must hold one row per (token, slot) pair")
    down_w = _expert_stack(down_w, codec, I)
    E, N = down_w.shape[0], down_w.shape[1]
    b = _bias_rows(bias, E, N, "bias", h.device)
    ep = None if b is None else _lib.GatherEpilogue(0, 0.0, 0.0, b.data_ptr(), None, N)
    y = torch.empty((t * k, N), dtype=out_dtype, device=h.device)
    if t * k:
        seg, order = _routed(idx, E)
        _gather_rows(h2.data_ptr(), _x_dt(h2), h2.stride(0), 1, 0, down_w, None, codec, ep, seg, order, t * k, E,
                     y.data_ptr(), _dt(out_dtype), N, 0, I, _stream(h2))
    return y.reshape(t, k, N)


def gather_qmv_mix_ns_kq(h, down_w, codec, idx, scores, out_dtype=torch.float32):
    """Down projection with the routing mix folded in (gmlx/modules.py:
    591-593): y[t] = sum_s scores[t, s] * (Wd[idx[t, s]] . h[t, s]), fp32,
    slots summed in order."""
    _fault("gather_qmv_mix_ns_kq")
    _require_gpu(h, down_w, idx, scores)
    t, k = idx.shape[0], idx.shape[-1]
    yp = gather_qmv_kq(h, down_w, codec, idx, out_dtype=torch.float32).reshape(t * k, -1)
    N = yp.shape[1]
    sc = scores.reshape(t, k).to(torch.float32).contiguous()
    y = torch.empty((t, N), dtype=out_dtype, device=h.device)
    if t:
        check("kq_moe_mix", lib().kq_moe_mix(yp.data_ptr(), sc.data_ptr(), t, k, N, y.data_ptr(),
                                             _dt(out_dtype), _stream(h)))
    return y


_ONE_EXPERT = OrderedDict()  # (device, rows) -> routing tables sending every row to expert 0


def _one_expert_route(device, rows):
    """seg_info / pair_order (with its flags) of `rows` pairs all routed to
    expert 0, in kq_moe_route's layout; memoised per device and size."""
    key = (str(device), rows)
    hit = _ONE_EXPERT.get(key)
    if hit is not None:
        _ONE_EXPERT.move_to_end(key)
        return hit
    seg = torch.tensor([1, 0, 0, rows], dtype=torch.int32, device=device)
    order = torch.cat([torch.arange(rows, dtype=torch.int32), torch.zeros(rows, dtype=torch.int32)]).to(device)
    _ONE_EXPERT[key] = (seg, order)
    if len(_ONE_EXPERT) > 64:
        _ONE_EXPERT.popitem(last=False)
    return seg, order


def _shared_matrix(w, codec, K, name):
    """A shared expert's wire matrix [N, K/256 * block_bytes] as a one-expert stack."""
    if w.dim() != 2 or w.dtype != torch.uint8:
        raise ValueError(f"{name} must be a uint8 wire matrix [N, K/256*block_bytes]")
    if wire_k(w.shape[-1], codec) != K:
        raise ValueError(f"{name} rows hold K={wire_k(w.shape[-1], codec)}, activations have K={K}")
    return w.contiguous().unsqueeze(0)


def moe_glu_gather_shexp_kq(x, gate_w, up_w, shexp_gate_w, shexp_up_w, codec, idx, act="silu",
                            shexp_kquant_type=None, limit=None, alpha=None):
    """kq.moe_glu_gather_shexp_kq (gmlx/modules.py:571-574, 777-780): the
    routed GLU gather of moe_glu_gather_kq plus the shared expert's GLU on
    every token, h (t, k + 1, I) float32 with the shared expert in slot k.
    The shared matrices may use another codec (`shexp_kquant_type`); their
    intermediate size must equal the routed experts'.  Biased acts
    (swiglu_clamp) have no shared-expert form."""
    _fault("moe_glu_gather_shexp_kq")
    _require_gpu(x, gate_w, up_w, shexp_gate_w, shexp_up_w, idx)
    if act == "swiglu_clamp":
        raise ValueError("act 'swiglu_clamp' (biased experts) has no shared-expert form")
    K = x.shape[-1]
    t, k = idx.shape[0], idx.shape[-1]
    x2 = _rows_view(x)
    if x2.shape[0] != t:
        raise ValueError(f"x has {x2.shape[0]} rows for {t} index rows")
    gate_w = _expert_stack(gate_w, codec, K)
    up_w = _expert_stack(up_w, codec, K)
    if gate_w.shape != up_w.shape or gate_w.stride() != up_w.stride():
        raise ValueError("gate and up stacks must share shape and layout")
    scodec = shexp_kquant_type or codec
    sg = _shared_matrix(shexp_gate_w, scodec, K, "shexp_gate_w")
    su = _shared_matrix(shexp_up_w, scodec, K, "shexp_up_w")
    E, I = gate_w.shape[0], gate_w.shape[1]
    if sg.shape != su.shape or sg.shape[1] != I:
        raise ValueError(f"shared gate/up must both have {I} rows (the routed intermediate size)")
    ep, _ = _epilogue(act, limit, alpha, None, None, E, I, x.device)
    h = torch.empty((t, k + 1, I), dtype=torch.float32, device=x.device)
    if t == 0:
        return h
    s = _stream(x)
    xd = _x_dt(x2)
    if k:
        seg, order = _routed(idx, E)
        _gather_rows(x2.data_ptr(), xd, x2.stride(0), k, 0, gate_w, up_w, codec, ep, seg, order, t * k, E,
                     h.data_ptr(), DTYPE_F32, I, k, K, s)
    seg1, order1 = _one_expert_route(x.device, t)
    _gather_rows(x2.data_ptr(), xd, x2.stride(0), 1, 0, sg, su, scodec, ep, seg1, order1, t, 1,
                 h.data_ptr() + k * I * 4, DTYPE_F32, (k + 1) * I, 0, K, s)
    return h


def gather_qmv_mix_kq(h, down_w, shexp_down_w, codec, idx, scores, shexp_kquant_type=None,
                      out_dtype=torch.float32):
    """kq.gather_qmv_mix_kq (gmlx/modules.py:581-583, 784-786): h (t, k + 1, I)
    from moe_glu_gather_shexp_kq; y[t] = sum_s scores[t, s] * (Wd[idx[t, s]] .
    h[t, s]) + scores[t, k] * (Wsd . h[t, k]), the k + 1 products in fp32 and
    summed in slot order."""
    _fault("gather_qmv_mix_kq")
    _require_gpu(h, down_w, shexp_down_w, idx, scores)
    t, k = idx.shape[0], idx.shape[-1]
    if h.dim() != 3 or tuple(h.shape[:2]) != (t, k + 1):
        raise ValueError("h must be (t, k + 1, I): routed slots then the shared expert")
    if tuple(scores.reshape(t, -1).shape) != (t, k + 1):
        raise ValueError("scores must hold k + 1 mix weights per token (the shared expert's last)")
    I = h.shape[-1]
    h = h.contiguous()
    down_w = _expert_stack(down_w, codec, I)
    scodec = shexp_kquant_type or codec
    sd = _shared_matrix(shexp_down_w, scodec, I, "shexp_down_w")
    E, D = down_w.shape[0], down_w.shape[1]
    if sd.shape[1] != D:
        raise ValueError(f"shared down must have {D} rows (the routed output size)")
    y = torch.empty((t, D), dtype=out_dtype, device=h.device)
    if t == 0:
        return y
    s = _stream(h)
    hd = _x_dt(h)
    yp = torch.empty((t, k + 1, D), dtype=torch.float32, device=h.device)
    if k:
        seg, order = _routed(idx, E)
        _gather_rows(h.data_ptr(), hd, I, 1, k, down_w, None, codec, None, seg, order, t * k, E, yp.data_ptr(),
                     DTYPE_F32, D, k, I, s)
    seg1, order1 = _one_expert_route(h.device, t)
    _gather_rows(h.data_ptr() + k * I * h.element_size(), hd, (k + 1) * I, 1, 0, sd, None, scodec, None, seg1,
                 order1, t, 1, yp.data_ptr() + k * D * 4, DTYPE_F32, (k + 1) * D, 0, I, s)
    sc = scores.reshape(t, k + 1).to(torch.float32).contiguous()
    check("kq_moe_mix", lib().kq_moe_mix(yp.data_ptr(), sc.data_ptr(), t, k + 1, D, y.data_ptr(), _dt(out_dtype),
                                         s))
    return y


def _expert_vector(v, E, name, device):
    if v is None:
        return None, None
    if not isinstance(v, torch.Tensor) or v.device != device or v.numel() != E:
        raise ValueError(f"{name} must be a tensor of {E} values on the logits' device")
    v = v.reshape(E)
    if v.dtype not in _TORCH_DTYPE:
        v = v.to(torch.float32)
    return v.contiguous(), _dt(v.dtype if v.dtype in _TORCH_DTYPE else torch.float32)


def moe_router_topk(logits, k, norm_topk_prob=True, shared_gate=True, per_expert_scale=None, bias=None,
                    scoring="softmax", scale=1.0):
    """kq.moe_router_topk, in fp32 on the device (one wave per token).

    score_e = softmax over the routed logits / sigmoid / sqrt(softplus)
    (`scoring`, gmlx/deepseek_v4_model.py:690-697); the k experts with the
    largest score_e + bias[e] are picked (descending, ties to the lower id)
    with their unbiased scores; weights = picks / (sum + 1e-20) when
    `norm_topk_prob`, then times per_expert_scale[e] and `scale`
    (gmlx/deepseek_v4_model.py:700-717, gmlx/modules.py:1029-1046).
    shared_gate (the default, as gmlx/modules.py:750-752 calls it): the last
    logit column is the shared expert's gate (router-cat rows,
    gmlx/modules.py:300-312) and sigmoid(it) is appended as weight k (stock
    form gmlx/modules.py:754-763).  Returns (inds int32 (..., k), weights
    float32 (..., k + shared_gate))."""
    _fault("moe_router_topk")
    _require_gpu(logits)
    if scoring not in _lib.SCORE_ID:
        raise ValueError(f"scoring {scoring!r} not in {tuple(_lib.SCORE_ID)}")
    C = logits.shape[-1]
    sg = 1 if shared_gate else 0
    E = C - sg
    if E < 1 or not 1 <= k <= min(E, 32) or E > 1024:
        raise ValueError(f"router of {E} experts, top-{k}: need 1 <= k <= min(E, 32), E <= 1024")
    l2 = logits.reshape(-1, C)
    if l2.dtype not in _TORCH_DTYPE:
        l2 = l2.to(torch.float32)
    if l2.stride(-1) != 1 or (l2.shape[0] > 1 and l2.stride(0) < C):
        l2 = l2.contiguous()
    t = l2.shape[0]
    b, bdt = _expert_vector(bias, E, "bias", logits.device)
    pes, pdt = _expert_vector(per_expert_scale, E, "per_expert_scale", logits.device)
    opts = _lib.RouterOptions(int(bool(norm_topk_prob)), sg, _lib.SCORE_ID[scoring], float(scale),
                              None if b is None else b.data_ptr(), bdt or 0,
                              None if pes is None else pes.data_ptr(), pdt or 0)
    inds = torch.empty((t, k), dtype=torch.int32, device=logits.device)
    scores = torch.empty((t, k + sg), dtype=torch.float32, device=logits.device)
    lead = logits.shape[:-1]
    out = inds.reshape(*lead, k)
    if t:
        check("kq_moe_router_topk",
              lib().kq_moe_router_topk(l2.data_ptr(), _dt(l2.dtype), l2.stride(0) if t > 1 else C, t, E, k,
                                       ctypes.byref(opts), inds.data_ptr(), scores.data_ptr(), _stream(logits)))
    return out, scores.reshape(*lead, k + sg)


# --------------------------------------------------------------- attention

_TABLES = OrderedDict()  # memoised device row tables, like the reference's pads cache


def _row_tables(device, kv_off, head_stride, row_len):
    key = (device.index, tuple(kv_off), tuple(head_stride), tuple(row_len))
    hit = _TABLES.get(key)
    if hit is not None:
        _TABLES.move_to_end(key)
        return hit
    t = (torch.tensor(kv_off, dtype=torch.int64, device=device),
         torch.tensor(head_stride, dtype=torch.int64, device=device),
         torch.tensor(row_len, dtype=torch.int32, device=device))
    _TABLES[key] = t
    if len(_TABLES) > 128:
        _TABLES.popitem(last=False)
    return t


def sdpa_decode_ragged(q, k, v, kv_off, head_stride, row_len, n_kv_heads, scale, max_len):
    """Ragged GQA decode attention over per-row KV regions (device tables).

    q (B, Hq, D); k, v flat-addressable tensors of q's dtype sharing one
    layout; row b's kv head h tokens start at element
    kv_off[b] + h * head_stride[b], D contiguous elements per token,
    row_len[b] tokens (rows longer than max_len are clamped to it).
    kv_off / head_stride are int64 and row_len int32 device tensors.
    Returns (B, Hq, D) in q's dtype."""
    _fault("sdpa_decode_ragged")
    _require_gpu(q, k, v, kv_off, head_stride, row_len)
    B, Hq, D = q.shape
    dt = q.dtype
    if dt not in (torch.float16, torch.bfloat16) or k.dtype != dt or v.dtype != dt:
        raise ValueError("q, k, v must share dtype float16 or bfloat16")
    if Hq % n_kv_heads:
        raise ValueError("Hq must be a multiple of Hkv")
    if kv_off.dtype != torch.int64 or head_stride.dtype != torch.int64 or row_len.dtype != torch.int32:
        raise ValueError("kv_off / head_stride must be int64 and row_len int32")
    if kv_off.numel() != B or head_stride.numel() != B or row_len.numel() != B:
        raise ValueError("one table entry per row")
    q = q.contiguous()
    out = torch.empty_like(q)
    tabs = (kv_off.contiguous(), head_stride.contiguous(), row_len.contiguous())
    return _sdpa_launch(q, k, v, tabs, int(n_kv_heads), scale, int(max_len), out)


def _sdpa_launch(q, k, v, tabs, Hkv, scale, max_len, out):
    B, Hq, D = q.shape
    L = lib()
    need = L.kq_sdpa_workspace_bytes(B, Hq, Hkv, D, max_len)
    s = _stream(q)
    ws = _WS.get("sdpa", q.device, s.value, need)
    rc = L.kq_sdpa_decode_ragged(q.data_ptr(), k.data_ptr(), v.data_ptr(), tabs[0].data_ptr(),
                                 tabs[1].data_ptr(), tabs[2].data_ptr(), B, Hq, Hkv, D, max_len,
                                 float(scale), _dt(q.dtype), out.data_ptr(), ws.data_ptr(), ws.numel(), s)
    check("kq_sdpa_decode_ragged", rc)
    return out


def sdpa_decode_slabs(q, k_cache, v_cache, row_offsets, row_lens, n_kv_heads, scale, max_len=None,
                      k_scales=None, k_biases=None, v_scales=None, v_biases=None):
    """C-config layout: row b's KV is a contiguous slab [Hkv, len_b, D] at
    element offset row_offsets[b] of the flat caches.  row_offsets /
    row_lens are host sequences (memoised to device tables).  With the four
    scale / bias tensors the caches are 8-bit affine (uint8 values, one
    16-bit scale and bias per 64 consecutive values, flat beside them; slab
    offsets multiples of 64)."""
    _fault("sdpa_decode_ragged")
    _require_gpu(q, k_cache, v_cache)
    B, Hq, D = q.shape
    if Hq % n_kv_heads:
        raise ValueError("Hq must be a multiple of Hkv")
    row_lens = [int(x) for x in row_lens]
    offs = [int(x) for x in row_offsets]
    hstride = [l * D for l in row_lens]
    tabs = _row_tables(q.device, offs, hstride, row_lens)
    max_len = int(max_len if max_len is not None else (max(row_lens) if row_lens else 0))
    q = q.contiguous()
    out = torch.empty_like(q)
    q8 = (k_scales, k_biases, v_scales, v_biases)
    if all(t is None for t in q8):
        return _sdpa_launch(q, k_cache, v_cache, tabs, n_kv_heads, scale, max_len, out)
    if any(t is None for t in q8) or k_cache.dtype != torch.uint8 or v_cache.dtype != torch.uint8:
        raise ValueError("8-bit slabs: uint8 caches and all four scale / bias tensors")
    if any(o % 64 for o in offs) or D % 64 or any(t.dtype != q.dtype or not t.is_contiguous() for t in q8):
        raise ValueError("8-bit slabs: offsets and D multiples of 64, contiguous scales in q's dtype")
    _require_gpu(*q8)
    L = lib()
    need = L.kq_sdpa_workspace_bytes(B, Hq, n_kv_heads, D, max_len)
    s = _stream(q)
    ws = _WS.get("sdpa", q.device, s.value, need)
    rc = L.kq_sdpa_decode_ragged_q8(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *(t.data_ptr() for t in q8),
                                    tabs[0].data_ptr(), tabs[1].data_ptr(), tabs[2].data_ptr(), B, Hq, n_kv_heads,
                                    D, max_len, float(scale), _dt(q.dtype), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                    s)
    check("kq_sdpa_decode_ragged_q8", rc)
    return out


def _device_starts(starts, B, device):
    """Per-row starts as a device int32 [B] tensor (or None for all zeros)
    without a host synchronisation: a device tensor is used as is (cast on
    the device if need be); host sequences and CPU tensors are memoised by
    value, so a decode loop that keeps its pads copies them once."""
    if starts is None:
        return None
    if isinstance(starts, torch.Tensor) and starts.is_cuda:
        st = starts.reshape(-1)
        if st.dtype != torch.int32 or not st.is_contiguous():
            st = st.to(torch.int32).contiguous()
        if st.numel() != B:
            raise ValueError(f"one start per row: got {st.numel()} for {B} rows")
        return st
    vals = [int(x) for x in (starts.tolist() if isinstance(starts, torch.Tensor) else starts)]
    if len(vals) != B:
        raise ValueError(f"one start per row: got {len(vals)} for {B} rows")
    return _starts_table(device, vals)


def _kv_padded(k, v, name):
    """k / v [B, Hkv, L, D] as views with D contiguous elements per token,
    shared strides and 16-byte alignment (copying only when needed)."""
    if k.stride(3) != 1 or k.stride(2) != k.shape[3]:
        k = k.contiguous()
    if v.stride() != k.stride():
        v = v.contiguous()
        if v.stride() != k.stride():
            k = k.contiguous()
    if k.stride(0) % 8 or k.stride(1) % 8 or k.data_ptr() % 16 or v.data_ptr() % 16:
        k, v = k.contiguous(), v.contiguous()
        if k.data_ptr() % 16 or v.data_ptr() % 16:
            raise ValueError(f"{name}: K/V must be 16-byte aligned")
    return k, v


def _sdpa_padded(q, k, v, st, scale):
    """q (B, Hq, 1, D); k / v prepared by _kv_padded; st device int32 or None."""
    B, Hq, _, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    q3 = q.reshape(B, Hq, D).contiguous()
    out = torch.empty_like(q3)
    Lb = lib()
    need = Lb.kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L)
    s = _stream(q)
    ws = _WS.get("sdpa", q.device, s.value, need)
    # the batch stride of a single row is never used: give it its packed value
    bs = k.stride(0) if B > 1 else Hkv * k.stride(1)
    rc = Lb.kq_sdpa_decode_gqa(q3.data_ptr(), k.data_ptr(), v.data_ptr(), bs, k.stride(1), L,
                               None if st is None else st.data_ptr(), B, Hq, Hkv, D, float(scale), _dt(q.dtype),
                               out.data_ptr(), ws.data_ptr(), ws.numel(), s)
    check("kq_sdpa_decode_gqa", rc)
    return out.reshape(B, Hq, 1, D)


def sdpa_decode_gqa(q, k, v, scale, starts=None, k_scales=None, k_biases=None, v_scales=None, v_biases=None):
    """kq.sdpa_decode_gqa with per-row `starts` (gmlx/gemma4_batched_sdpa.py:
    210-226): q (B, Hq, 1, D), k/v (B, Hkv, L, D); row b attends keys
    [starts[b], L).  `starts` may be an int device tensor (read by the
    kernel: no host synchronisation, the reference's reason for passing
    device starts, gmlx/quantized_sdpa_fix.py:37-45, 88-93), a CPU tensor
    or a host sequence (memoised on the device by value).

    With k_scales / k_biases / v_scales / v_biases (the quantized-KV form,
    gmlx/quantized_sdpa_fix.py:170-182): k / v are an 8-bit affine cache,
    group 64 -- uint32 words of four values, lowest byte first (mlx's wire,
    (B, Hkv, L, D/4)) or uint8 (B, Hkv, L, D) -- and the scales / biases
    (B, Hkv, L, D/64) are in q's dtype; value = scale * q + bias."""
    q8 = (k_scales, k_biases, v_scales, v_biases)
    if any(t is not None for t in q8):
        if any(t is None for t in q8):
            raise ValueError("sdpa_decode_gqa: quantized KV needs k_scales, k_biases, v_scales and v_biases")
        return _sdpa_q8(q, k, v, q8, starts, scale)
    _fault("sdpa_decode_gqa")
    _require_gpu(q, k, v)
    if q.dim() != 4 or q.shape[2] != 1 or k.dim() != 4 or v.dim() != 4 or tuple(k.shape) != tuple(v.shape):
        raise ValueError("sdpa_decode_gqa: q (B, Hq, 1, D), k / v (B, Hkv, L, D) of one shape")
    B, Hq, _, D = q.shape
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("sdpa_decode_gqa: q, k, v must share dtype float16 or bfloat16")
    Hkv = k.shape[1]
    if k.shape[0] != B or k.shape[3] != D or Hq % Hkv or Hq // Hkv > 16 or D not in _GQA_HEAD_DIMS:
        raise ValueError("sdpa_decode_gqa: unsupported shape for the decode kernels")
    kk, vv = _kv_padded(k, v, "sdpa_decode_gqa")
    return _sdpa_padded(q, kk, vv, _device_starts(starts, B, q.device), scale)


def _q8_values(w, D, name):
    """An 8-bit KV wire tensor as uint8 (..., D): mlx's int32 / uint32 words
    (four values each, lowest byte first) or bytes."""
    if w.dtype in (torch.int32, getattr(torch, "uint32", torch.int32)):
        if w.stride(-1) != 1:
            w = w.contiguous()
        w = w.view(torch.uint8)
    elif w.dtype != torch.uint8:
        raise ValueError(f"{name}: 8-bit KV is uint8 or 32-bit words, got {w.dtype}")
    if w.shape[-1] != D:
        raise ValueError(f"{name}: rows of {w.shape[-1]} values, queries have D={D}")
    return w


def _q8_pair(w, sc, bi, D, dt, name):
    """(values, scales, biases) in layouts the kernel addresses together: the
    values' byte strides 64 x the scales' element strides, rows contiguous."""
    w = _q8_values(w, D, name)
    if D % 64 or sc.shape[-1] != D // 64 or tuple(sc.shape) != tuple(bi.shape) or \
            tuple(sc.shape[:-1]) != tuple(w.shape[:-1]):
        raise ValueError(f"{name}: scales / biases must be (..., D/64) beside (..., D) values (group 64)")
    if sc.dtype != dt or bi.dtype != dt:
        raise ValueError(f"{name}: scales / biases must be in the queries' dtype {dt}")

    def lined_up(a, b):
        return a.stride(-1) == 1 and b.stride(-1) == 1 and all(
            a.stride(i) == 64 * b.stride(i) for i in range(a.dim() - 1))
    if not (lined_up(w, sc) and lined_up(w, bi) and sc.stride() == bi.stride()):
        w, sc, bi = w.contiguous(), sc.contiguous(), bi.contiguous()
    if w.data_ptr() % 8:
        raise ValueError(f"{name}: 8-bit KV must be 8-byte aligned")
    return w, sc, bi


def _sdpa_q8(q, k, v, q8, starts, scale):
    _fault("sdpa_decode_gqa")
    _require_gpu(q, k, v, *q8)
    if q.dim() != 4 or q.shape[2] != 1 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("sdpa_decode_gqa: q (B, Hq, 1, D), k / v (B, Hkv, L, .)")
    B, Hq, _, D = q.shape
    dt = q.dtype
    if dt not in (torch.float16, torch.bfloat16):
        raise ValueError("queries must be float16 or bfloat16")
    k8, ks, kb = _q8_pair(k, q8[0], q8[1], D, dt, "k")
    v8, vs, vb = _q8_pair(v, q8[2], q8[3], D, dt, "v")
    if k8.shape != v8.shape or k8.stride() != v8.stride() or ks.stride() != vs.stride():
        k8, v8, ks, kb, vs, vb = (t.contiguous() for t in (k8, v8, ks, kb, vs, vb))
    Hkv, L = k8.shape[1], k8.shape[2]
    if k8.shape[0] != B or Hq % Hkv or Hq // Hkv > 16 or D not in _Q8_HEAD_DIMS:
        raise ValueError("unsupported quantized-KV attention shape")
    st = _device_starts(starts, B, q.device)
    q3 = q.reshape(B, Hq, D).contiguous()
    out = torch.empty_like(q3)
    Lb = lib()
    need = Lb.kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L)
    s = _stream(q)
    ws = _WS.get("sdpa", q.device, s.value, need)
    sc = (ctypes.c_void_p * 4)(ks.data_ptr(), kb.data_ptr(), vs.data_ptr(), vb.data_ptr())
    bs = k8.stride(0) if B > 1 else Hkv * k8.stride(1)
    rc = Lb.kq_sdpa_decode_gqa_q8(q3.data_ptr(), k8.data_ptr(), v8.data_ptr(), ctypes.cast(sc, ctypes.c_void_p), bs,
                                  k8.stride(1), L, None if st is None else st.data_ptr(), B, Hq, Hkv, D, float(scale),
                                  _dt(dt), out.data_ptr(), ws.data_ptr(), ws.numel(), s)
    check("kq_sdpa_decode_gqa_q8", rc)
    return out.reshape(B, Hq, 1, D)


# Head dims per route, as the reference's guards have them: the ragged route
# (gmlx/qwen35_attn.py:425-428), the batched starts= route and the cascade
# (512 too: gmlx/gemma4_batched_sdpa.py:172-177, gmlx/cascade_sdpa.py:66), the
# 8-bit KV route (whole 64-value scale groups: gmlx/quantized_sdpa_fix.py:66).
_SDPA_HEAD_DIMS = (64, 96, 128, 256)
_GQA_HEAD_DIMS = (64, 96, 128, 256, 512)
_Q8_HEAD_DIMS = (64, 128, 256, 512)


def ragged_decode_attention(queries, keys, values, pads, scale):
    """Ragged left-padded S=1 decode (gmlx/qwen35_attn.py:395-493).

    queries (B, Hq, 1, D); keys/values (B, Hkv, L, D); row b's visible keys
    are [pads[b], L).  Declines (returns None) exactly where the reference's
    guard rails do (:412-431): non-4-D inputs, S != 1, dtype other than
    float16/bfloat16 or mismatched, len(pads) != B, negative pads,
    Hq % Hkv != 0, D != V, D not in (64, 96, 128, 256), pad >= L.  The pads
    become device starts memoised by value, so the decode steps L, L + 1, ...
    of one batch copy nothing and build no tables."""
    if any(not isinstance(t, torch.Tensor) for t in (queries, keys, values)):
        return None
    if (queries.dim() != 4 or keys.dim() != 4 or values.dim() != 4 or queries.shape[2] != 1
            or queries.dtype not in (torch.float16, torch.bfloat16) or keys.dtype != queries.dtype
            or values.dtype != queries.dtype):
        return None
    B, Hq, _, D = queries.shape
    pads = tuple(int(p) for p in pads)
    if len(pads) != B or any(p < 0 for p in pads):
        return None
    Hkv, L = keys.shape[1], keys.shape[2]
    Dv = values.shape[-1]
    if Hq % Hkv != 0 or D != Dv or D not in _SDPA_HEAD_DIMS or any(p >= L for p in pads):
        return None
    if Hq // Hkv > 16 or tuple(values.shape) != tuple(keys.shape) or keys.shape[0] != B:
        return None
    _fault("ragged_decode_attention")
    _require_gpu(queries, keys, values)
    k, v = _kv_padded(keys, values, "ragged_decode_attention")
    st = None if not any(pads) else _starts_table(queries.device, pads)
    return _sdpa_padded(queries, k, v, st, scale)


_STARTS = OrderedDict()  # memoised device starts rows for host sequences


def _starts_table(device, starts):
    key = (str(device), tuple(starts))
    hit = _STARTS.get(key)
    if hit is not None:
        _STARTS.move_to_end(key)
        return hit
    t = torch.tensor(key[1], dtype=torch.int32, device=device)
    _STARTS[key] = t
    if len(_STARTS) > 128:
        _STARTS.popitem(last=False)
    return t


def _kv_pair(k, v, name):
    """k/v as views whose tokens are D contiguous elements and which share
    strides; copies only when they do not."""
    D = k.shape[-1]
    if k.stride(3) != 1 or k.stride(2) != D:
        k = k.contiguous()
    if v.stride() != k.stride():
        v = v.contiguous()
        if v.stride() != k.stride():
            k = k.contiguous()
    if any(int(x) % 8 for x in k.stride()[:2]) or k.data_ptr() % 16 or v.data_ptr() % 16:
        k, v = k.contiguous(), v.contiguous()
        if k.data_ptr() % 16 or v.data_ptr() % 16:
            raise ValueError(f"{name}: K/V must be 16-byte aligned")
    return k, v


_CASCADE_Q8_KEYS = ("k_shared_scales", "k_shared_biases", "v_shared_scales", "v_shared_biases",
                    "k_priv_scales", "k_priv_biases", "v_priv_scales", "v_priv_biases")


def sdpa_decode_gqa_cascade(queries, k_shared, v_shared, k_priv, v_priv, scale, starts=None,
                            **quant_kv):
    """kq.sdpa_decode_gqa_cascade (gmlx/cascade_sdpa.py:216-248): decode with
    a prefix shared by every sequence, held once.

    queries (B, Hq, qL, D); k_shared/v_shared (1, Hkv, P, D), the common
    prefix; k_priv/v_priv (B, Hkv, S, D), each sequence's keys after it.
    Query token i of sequence b attends the whole prefix and private keys
    [starts[b], S - qL + i] (left padding plus the end-aligned causal mask of
    a verify block, qL 2..8 in the reference).  `starts` is an int32 device
    tensor (read on the device, no host sync) or a host sequence; None = 0.
    Strided views (slices of a larger cache, as the reference passes) are
    used in place when the last two dims are contiguous.  Returns
    (B, Hq, qL, D) in the queries' dtype.

    The quantized-KV form takes k_shared_scales, k_shared_biases,
    v_shared_scales, v_shared_biases, k_priv_scales, k_priv_biases,
    v_priv_scales, v_priv_biases: K / V are then an 8-bit affine cache,
    group 64, as sdpa_decode_gqa's quantized form describes."""
    unknown = set(quant_kv) - set(_CASCADE_Q8_KEYS)
    if unknown:
        raise TypeError(f"sdpa_decode_gqa_cascade: unexpected keywords {sorted(unknown)}")
    q8 = bool(quant_kv)
    if q8 and any(quant_kv.get(k_) is None for k_ in _CASCADE_Q8_KEYS):
        raise ValueError("sdpa_decode_gqa_cascade: quantized KV needs all eight scale / bias tensors")
    _fault("sdpa_decode_gqa_cascade")
    _require_gpu(queries, k_shared, v_shared, k_priv, v_priv, *(quant_kv.values()))
    if queries.dim() != 4 or k_shared.dim() != 4 or k_priv.dim() != 4:
        raise ValueError("queries, k_shared, k_priv must be 4-D")
    B, Hq, qL, D = queries.shape
    dt = queries.dtype
    if dt not in (torch.float16, torch.bfloat16):
        raise ValueError("queries must be float16 or bfloat16")
    if q8:
        ks, kb, vs, vb = (quant_kv[k_] for k_ in _CASCADE_Q8_KEYS[:4])
        kps, kpb, vps, vpb = (quant_kv[k_] for k_ in _CASCADE_Q8_KEYS[4:])
        k_shared, ks, kb = _q8_pair(k_shared, ks, kb, D, dt, "k_shared")
        v_shared, vs, vb = _q8_pair(v_shared, vs, vb, D, dt, "v_shared")
        k_priv, kps, kpb = _q8_pair(k_priv, kps, kpb, D, dt, "k_priv")
        v_priv, vps, vpb = _q8_pair(v_priv, vps, vpb, D, dt, "v_priv")
    elif any(t.dtype != dt for t in (k_shared, v_shared, k_priv, v_priv)):
        raise ValueError("queries and K/V must share dtype float16 or bfloat16")
    if tuple(v_shared.shape) != tuple(k_shared.shape) or tuple(v_priv.shape) != tuple(k_priv.shape):
        raise ValueError("K and V shapes differ")
    if k_shared.shape[0] != 1 or k_priv.shape[0] != B:
        raise ValueError("k_shared must have batch 1 and k_priv batch B")
    Hkv, P = k_shared.shape[1], k_shared.shape[2]
    S = k_priv.shape[2]
    if k_priv.shape[1] != Hkv or k_shared.shape[3] != D or k_priv.shape[3] != D:
        raise ValueError("head count / head dim mismatch")
    if Hq % Hkv or Hq // Hkv > 16 or D not in (_Q8_HEAD_DIMS if q8 else _GQA_HEAD_DIMS) or not 1 <= qL <= 64:
        raise ValueError("unsupported cascade shape")
    if S < qL:
        raise ValueError("the private slab must hold the query block (S >= qL)")
    if q8:
        if k_shared.stride() != v_shared.stride() or ks.stride() != vs.stride():
            k_shared, v_shared, ks, kb, vs, vb = (t.contiguous() for t in (k_shared, v_shared, ks, kb, vs, vb))
        if k_priv.stride() != v_priv.stride() or kps.stride() != vps.stride():
            k_priv, v_priv, kps, kpb, vps, vpb = (t.contiguous() for t in (k_priv, v_priv, kps, kpb, vps, vpb))
        kS, vS, kP, vP = k_shared, v_shared, k_priv, v_priv
    else:
        kS, vS = _kv_pair(k_shared, v_shared, "sdpa_decode_gqa_cascade")
        kP, vP = _kv_pair(k_priv, v_priv, "sdpa_decode_gqa_cascade")
    if starts is None:
        st = None
    elif isinstance(starts, torch.Tensor):
        st = starts
        if not st.is_cuda:
            st = _starts_table(queries.device, [int(x) for x in st.tolist()])
        elif st.dtype != torch.int32 or not st.is_contiguous():
            st = st.to(torch.int32).contiguous()
        if st.numel() < B:
            raise ValueError("one start per sequence")
    else:
        st = _starts_table(queries.device, [int(x) for x in starts])
        if st.numel() < B:
            raise ValueError("one start per sequence")
    q = queries.contiguous()
    out = torch.empty_like(q)
    L = lib()
    need = L.kq_sdpa_cascade_workspace_bytes(B, qL, Hq, Hkv, D, P, S)
    s = _stream(q)
    ws = _WS.get("sdpa_cascade", q.device, s.value, need)
    # strides of size-1 dims are never used: give them their packed values
    shs = kS.stride(1) if Hkv > 1 else P * D
    phs = kP.stride(1) if Hkv > 1 else S * D
    pbs = kP.stride(0) if B > 1 else Hkv * phs
    common = (B, qL, Hq, Hkv, D, float(scale), _dt(dt), out.data_ptr(), ws.data_ptr(), ws.numel(), s)
    stp = None if st is None else st.data_ptr()
    if q8:
        sh = (ctypes.c_void_p * 4)(ks.data_ptr(), kb.data_ptr(), vs.data_ptr(), vb.data_ptr())
        pr = (ctypes.c_void_p * 4)(kps.data_ptr(), kpb.data_ptr(), vps.data_ptr(), vpb.data_ptr())
        rc = L.kq_sdpa_decode_gqa_cascade_q8(q.data_ptr(), kS.data_ptr(), vS.data_ptr(), ctypes.cast(sh, ctypes.c_void_p),
                                             shs, P, kP.data_ptr(), vP.data_ptr(), ctypes.cast(pr, ctypes.c_void_p),
                                             pbs, phs, S, stp, *common)
        check("kq_sdpa_decode_gqa_cascade_q8", rc)
        return out
    rc = L.kq_sdpa_decode_gqa_cascade(q.data_ptr(), kS.data_ptr(), vS.data_ptr(), shs, P, kP.data_ptr(),
                                      vP.data_ptr(), pbs, phs, S, stp, *common)
    check("kq_sdpa_decode_gqa_cascade", rc)
    return out

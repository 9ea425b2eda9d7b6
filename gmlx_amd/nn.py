"""torch leaf modules binding GGUF wire bytes to the K-quant kernels.

KQuantLinear / KQuantEmbedding / KQuantSwitchLinear mirror mlx_kquant.nn's
modules as gmlx constructs them (gmlx/modules.py:1539-1552): a uint8
``weight`` holding the GGUF wire rows unchanged, a vestigial ``scales``
placeholder (gmlx/transforms.py:65-66), ``kquant_type`` and an optional
``bias``.  ``install_kquant_modules`` is the leaf swap of
gmlx/modules.py:1473-1576 for torch models: ``nn.Linear`` leaves,
``nn.Embedding`` leaves (their output dtype is the activation dtype, which
seeds the graph), and expert stacks (3-D ``weight`` [n_experts, out, in];
classes registered with ``register_switch_linear`` or named
``*SwitchLinear``).
"""
from __future__ import annotations

import os

import torch
from torch import nn

from . import ops

BLOCK_BYTES = ops.BLOCK_BYTES


def _wire_cols(in_dims, codec):
    if in_dims % ops.QK_K:
        raise ValueError(f"in_dims={in_dims} is not a multiple of {ops.QK_K}")
    return in_dims // ops.QK_K * BLOCK_BYTES[codec]


class KQuantLinear(nn.Module):
    """y = x . dequant(weight)^T (+ bias); weight uint8 [out_dims, in_dims/256*bpb]."""

    def __init__(self, in_dims, out_dims, bias=False, codec="q4_k", device=None):
        super().__init__()
        if codec not in BLOCK_BYTES:
            raise ValueError(f"unsupported codec {codec!r}")
        self.in_dims, self.out_dims, self.kquant_type = in_dims, out_dims, codec
        self.register_buffer("weight", torch.zeros(out_dims, _wire_cols(in_dims, codec), dtype=torch.uint8,
                                                   device=device))
        self.register_buffer("scales", torch.zeros(1, dtype=torch.uint8, device=device))
        # inference leaf: the quantized matmul has no backward, so nothing here
        # takes part in autograd
        self.bias = nn.Parameter(torch.zeros(out_dims, device=device), requires_grad=False) if bias else None

    def forward(self, x):
        y = ops.quantized_matmul(x, self.weight, self.scales, self.kquant_type, transpose=True)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def extra_repr(self):
        return f"in_dims={self.in_dims}, out_dims={self.out_dims}, codec={self.kquant_type}"


def activation_dtype():
    """The graph's activation dtype (gmlx/dtypes.py): GMLX_ACTIVATION_DTYPE
    names float16 / bfloat16 / float32; "auto" (the default) is bfloat16, the
    reference's choice on every device but Apple GPUs before Apple9."""
    raw = os.environ.get("GMLX_ACTIVATION_DTYPE", "auto").strip().lower()
    return {"float16": torch.float16, "fp16": torch.float16, "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
            "float32": torch.float32, "fp32": torch.float32}.get(raw, torch.bfloat16)


class KQuantEmbedding(nn.Module):
    """Token embedding over GGUF wire rows: weight uint8 [num_embeddings,
    dims/256*bpb].  forward(ids) gathers the ids' wire rows and dequantizes
    them (the GGML definition, one rounding to out_dtype); as_linear(x) is the
    tied output head, x . dequant(weight)^T.  Ids must lie in
    [0, num_embeddings), as for torch.nn.Embedding."""

    def __init__(self, num_embeddings, dims, codec="q4_k", out_dtype=None, device=None):
        super().__init__()
        if codec not in BLOCK_BYTES:
            raise ValueError(f"unsupported codec {codec!r}")
        self.num_embeddings, self.dims, self.kquant_type = num_embeddings, dims, codec
        self.out_dtype = out_dtype or activation_dtype()
        self.register_buffer("weight", torch.zeros(num_embeddings, _wire_cols(dims, codec), dtype=torch.uint8,
                                                   device=device))
        self.register_buffer("scales", torch.zeros(1, dtype=torch.uint8, device=device))

    def forward(self, ids):
        rows = self.weight.index_select(0, ids.reshape(-1).to(torch.long))
        out = ops.dequantize(rows, self.scales, self.kquant_type, dtype=self.out_dtype)
        return out.reshape(*ids.shape, self.dims)

    def as_linear(self, x):
        return ops.quantized_matmul(x, self.weight, self.scales, self.kquant_type, transpose=True)

    def extra_repr(self):
        return f"num_embeddings={self.num_embeddings}, dims={self.dims}, codec={self.kquant_type}"


class KQuantSwitchLinear(nn.Module):
    """Expert stack: weight uint8 [n_experts, out_dims, in_dims/256*bpb], an
    optional fp32 bias [n_experts, out_dims].  forward(x (T, 1, 1, K),
    indices (T, k)) -> (T, k, 1, out_dims), the SwitchGLU calling convention
    (tests/test_native_fp.py:420-428); the bias of each pair's expert is added
    in the kernel's fp32 epilogue."""

    def __init__(self, n_experts, out_dims, in_dims, bias=False, codec="q4_k", device=None):
        super().__init__()
        if codec not in BLOCK_BYTES:
            raise ValueError(f"unsupported codec {codec!r}")
        self.n_experts, self.in_dims, self.out_dims, self.kquant_type = n_experts, in_dims, out_dims, codec
        self.register_buffer("weight", torch.zeros(n_experts, out_dims, _wire_cols(in_dims, codec),
                                                   dtype=torch.uint8, device=device))
        self.register_buffer("scales", torch.zeros(1, dtype=torch.uint8, device=device))
        self.bias = nn.Parameter(torch.zeros(n_experts, out_dims, device=device), requires_grad=False) \
            if bias else None

    def forward(self, x, indices, sorted_indices=False):
        return ops.gather_qmm(x, self.weight, self.scales, self.kquant_type, indices=indices,
                              sorted_indices=sorted_indices, bias=self.bias)


_SWITCH_LINEAR_TYPES = []


def register_switch_linear(cls):
    """Declare a module class an expert stack for the leaf swap (the
    reference asks mlx-lm / mlx-vlm for theirs, gmlx/modules.py:1503)."""
    if cls not in _SWITCH_LINEAR_TYPES:
        _SWITCH_LINEAR_TYPES.append(cls)
    return cls


def _is_switch_linear(module):
    w = getattr(module, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dim() != 3:
        return False
    return isinstance(module, tuple(_SWITCH_LINEAR_TYPES)) or type(module).__name__.endswith("SwitchLinear")


def _kquant_leaf(module, codec):
    """The K-quant module that takes `module`'s place, or None."""
    dev = module.weight.device if isinstance(getattr(module, "weight", None), torch.Tensor) else None
    if isinstance(module, nn.Linear):
        return KQuantLinear(module.in_features, module.out_features, module.bias is not None, codec, device=dev)
    if isinstance(module, nn.Embedding):
        return KQuantEmbedding(module.num_embeddings, module.embedding_dim, codec, out_dtype=activation_dtype(),
                               device=dev)
    if _is_switch_linear(module):
        n_experts, out_dims, in_dims = module.weight.shape
        return KQuantSwitchLinear(n_experts, out_dims, in_dims, getattr(module, "bias", None) is not None, codec,
                                  device=dev)
    return None


def install_kquant_modules(model: nn.Module, kquant_meta: dict) -> int:
    """Swap the leaves whose ``<path>.weight`` is in ``kquant_meta`` (name ->
    codec) for K-quant modules -- ``nn.Linear`` -> KQuantLinear,
    ``nn.Embedding`` -> KQuantEmbedding (activation dtype out), expert stacks
    -> KQuantSwitchLinear -- and return the number swapped.  A codec'd weight
    on a module this function cannot bind raises, as the reference does for
    unrecognised classes (gmlx/modules.py:1566-1574)."""
    n = 0
    unmatched = []
    for path, module in list(model.named_modules()):
        codec = kquant_meta.get(f"{path}.weight")
        if codec is None:
            continue
        if isinstance(module, (KQuantLinear, KQuantEmbedding, KQuantSwitchLinear)):
            continue
        new = _kquant_leaf(module, codec)
        if new is None:
            unmatched.append(f"{path} ({type(module).__name__}, codec {codec!r})")
            continue
        parent_path, _, leaf = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, leaf, new)
        n += 1
    if unmatched:
        raise ValueError(f"{len(unmatched)} quantized weights have no recognized module class: "
                         + ", ".join(unmatched[:3]))
    return n

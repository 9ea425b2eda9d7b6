"""torch leaf modules binding GGUF wire bytes to the K-quant kernels.

KQuantLinear / KQuantSwitchLinear mirror mlx_kquant.nn's modules as gmlx
constructs them (gmlx/modules.py:1539, :1552): a uint8 ``weight`` holding the
GGUF wire rows unchanged, a vestigial ``scales`` placeholder
(gmlx/transforms.py:65-66), ``kquant_type`` and an optional ``bias``.
``install_kquant_modules`` is the leaf swap of gmlx/modules.py:1473-1576 for
torch ``nn.Linear`` leaves.
"""
from __future__ import annotations

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


class KQuantSwitchLinear(nn.Module):
    """Expert stack: weight uint8 [n_experts, out_dims, in_dims/256*bpb].
    forward(x (T, 1, 1, K), indices (T, k)) -> (T, k, 1, out_dims), the
    SwitchGLU calling convention (tests/test_native_fp.py:420-428)."""

    def __init__(self, n_experts, out_dims, in_dims, bias=False, codec="q4_k", device=None):
        super().__init__()
        if bias:
            raise ValueError("biased K-quant expert stacks have no kernel")
        if codec not in BLOCK_BYTES:
            raise ValueError(f"unsupported codec {codec!r}")
        self.n_experts, self.in_dims, self.out_dims, self.kquant_type = n_experts, in_dims, out_dims, codec
        self.register_buffer("weight", torch.zeros(n_experts, out_dims, _wire_cols(in_dims, codec),
                                                   dtype=torch.uint8, device=device))
        self.register_buffer("scales", torch.zeros(1, dtype=torch.uint8, device=device))

    def forward(self, x, indices, sorted_indices=False):
        return ops.gather_qmm(x, self.weight, self.scales, self.kquant_type, indices=indices,
                              sorted_indices=sorted_indices)


def install_kquant_modules(model: nn.Module, kquant_meta: dict) -> int:
    """Swap ``nn.Linear`` leaves whose ``<path>.weight`` is in ``kquant_meta``
    (name -> codec) for KQuantLinear; returns the number swapped.  A codec'd
    weight on a module this function cannot bind raises, as the reference
    does for unrecognised classes (gmlx/modules.py:1566-1574)."""
    n = 0
    unmatched = []
    for path, module in list(model.named_modules()):
        codec = kquant_meta.get(f"{path}.weight")
        if codec is None:
            continue
        if isinstance(module, (KQuantLinear, KQuantSwitchLinear)):
            continue
        if isinstance(module, nn.Linear):
            dev = module.weight.device
            new = KQuantLinear(module.in_features, module.out_features, module.bias is not None, codec,
                               device=dev)
            parent_path, _, leaf = path.rpartition(".")
            parent = model.get_submodule(parent_path) if parent_path else model
            setattr(parent, leaf, new)
            n += 1
        else:
            unmatched.append(f"{path} ({type(module).__name__}, codec {codec!r})")
    if unmatched:
        raise ValueError(f"{len(unmatched)} quantized weights have no recognized module class: "
                         + ", ".join(unmatched[:3]))
    return n

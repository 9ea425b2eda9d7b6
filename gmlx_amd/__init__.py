"""gmlx_amd: MI355X (gfx950) K-quant batched-decode hot path.

GGUF Q4_K / Q6_K / IQ2_XXS dequant-fused matmuls (dense, grouped, MoE expert
gather) and ragged GQA decode attention, as hand-written HIP kernels behind
the C ABI of include/kq_capi.h (libgmlx_amd.so), driven from torch.
"""
from . import ops  # noqa: F401
from ._lib import KQError, KQLibraryError, lib, version  # noqa: F401

__all__ = ["ops", "nn", "lib", "version", "KQError", "KQLibraryError"]


def __getattr__(name):
    if name == "nn":
        from . import nn as _nn
        return _nn
    raise AttributeError(name)

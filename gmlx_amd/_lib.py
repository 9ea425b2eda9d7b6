"""ctypes binding of libgmlx_amd.so (the C ABI declared in include/kq_capi.h).

The library is loaded from the package directory (built in-tree by
``python -m gmlx_amd.build``).  There is no fallback: if the library is
missing or fails to load, every op raises ``KQLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgmlx_amd.so")

# kq_status codes (include/kq_capi.h)
KQ_OK = 0
KQ_ERR_NULL_POINTER = -1
KQ_ERR_BAD_SHAPE = -2
KQ_ERR_BAD_ALIGN = -3
KQ_ERR_UNSUPPORTED_CODEC = -4
KQ_ERR_UNSUPPORTED_DTYPE = -5
KQ_ERR_WORKSPACE_TOO_SMALL = -6
KQ_ERR_LAUNCH_FAILED = -7
KQ_ERR_TOO_MANY_PROBLEMS = -8
KQ_ERR_BAD_ARGUMENT = -9
KQ_ERR_IO = -10
KQ_ERR_BAD_FORMAT = -11

CODEC_ID = {"q4_k": 12, "q6_k": 14, "iq2_xxs": 16}
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
OP_DEQUANTIZE, OP_QUANTIZE, OP_MATMUL, OP_GATHER, OP_MOE_GLU, OP_SDPA = range(6)
MAX_GROUP = 8
SDPA_NOALLOC_SCRATCH_BYTES = 32 << 20  # KQ_SDPA_NOALLOC_SCRATCH_BYTES (include/kq_capi.h)
# KQ_MATMUL_COUNTER_BYTES: arrival counters at the start of every matmul / gather
# workspace (zero when allocated; the library leaves them zero)
MATMUL_COUNTER_BYTES = 16 << 10
# KQ_FUSED_MLP_STATUS_OFFSET: the fused MLP's give-up status word in its workspace
FUSED_MLP_STATUS_OFFSET = MATMUL_COUNTER_BYTES - 64

# every symbol include/kq_capi.h and include/kq_gguf.h declare, checked at load
EXPORTS = (
    "kq_version", "kq_strerror", "kq_codec_block_bytes", "kq_supports", "kq_iq2xxs_grid_host",
    "kq_dequantize", "kq_quantize", "kq_matmul_workspace_bytes", "kq_quantized_matmul_grouped",
    "kq_fused_mlp_workspace_bytes", "kq_fused_mlp",
    "kq_moe_route", "kq_gather_qmm", "kq_moe_glu_gather", "kq_moe_gather_rows", "kq_gather_workspace_bytes",
    "kq_moe_mix", "kq_moe_router_topk",
    "kq_sdpa_workspace_bytes", "kq_sdpa_decode_ragged", "kq_sdpa_decode_ragged_q8", "kq_sdpa_decode_gqa",
    "kq_sdpa_decode_gqa_q8", "kq_sdpa_decode_gqa_noalloc",
    "kq_sdpa_cascade_workspace_bytes", "kq_sdpa_decode_gqa_cascade", "kq_sdpa_decode_gqa_cascade_q8",
    "kq_gguf_open", "kq_gguf_close", "kq_gguf_header", "kq_gguf_kv", "kq_gguf_tensor", "kq_gguf_type_size",
)


class KQLibraryError(RuntimeError):
    """libgmlx_amd.so is missing, failed to load, or lacks a symbol."""


class KQError(RuntimeError):
    """A C-ABI call returned a non-zero kq_status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn}: {msg} (kq_status {code})")
        self.code = code


class MatmulProblem(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("w_row_bytes", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_row_stride", ctypes.c_int64),
        ("y", ctypes.c_void_p),
        ("y_row_stride", ctypes.c_int64),
        ("M", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("codec", ctypes.c_int32),
    ]


# GLU activations (KQ_ACT_*) and router scoring functions (KQ_SCORE_*)
ACT_ID = {"silu": 0, "gelu": 1, "silu_limit": 2, "swiglu_clamp": 3}
SCORE_ID = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}


class GatherEpilogue(ctypes.Structure):
    _fields_ = [
        ("act", ctypes.c_int32),
        ("limit", ctypes.c_float),
        ("alpha", ctypes.c_float),
        ("bias0", ctypes.c_void_p),
        ("bias1", ctypes.c_void_p),
        ("bias_expert_stride", ctypes.c_int64),
    ]


class RouterOptions(ctypes.Structure):
    _fields_ = [
        ("norm_topk_prob", ctypes.c_int32),
        ("shared_gate", ctypes.c_int32),
        ("scoring", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("bias", ctypes.c_void_p),
        ("bias_dtype", ctypes.c_int32),
        ("per_expert_scale", ctypes.c_void_p),
        ("per_expert_scale_dtype", ctypes.c_int32),
    ]


_lib = None
_lock = threading.Lock()

_vp, _i32, _i64, _f32, _sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_int = ctypes.c_int

_SIGS = {
    "kq_version": ([], ctypes.c_char_p),
    "kq_strerror": ([_int], ctypes.c_char_p),
    "kq_codec_block_bytes": ([_int], _int),
    "kq_supports": ([_int, _int, _int], _int),
    "kq_iq2xxs_grid_host": ([], ctypes.POINTER(ctypes.c_uint64)),
    "kq_dequantize": ([_vp, _i64, _int, _vp, _int, _vp], _int),
    "kq_quantize": ([_vp, _i64, _i64, _i64, _int, _vp, _vp], _int),
    "kq_matmul_workspace_bytes": ([ctypes.POINTER(MatmulProblem), _int, _int], _sz),
    "kq_quantized_matmul_grouped": ([ctypes.POINTER(MatmulProblem), _int, _int, _int, _vp, _sz, _vp], _int),
    "kq_fused_mlp_workspace_bytes": ([_i32, _i32, _i32, _i32, _int], _sz),
    "kq_fused_mlp": ([_vp, _int, _i64, _i32, _i32, _vp, _vp, _i64, _int, _i32, _vp, _i64, _int, _i32, _int, _vp,
                      _int, _i64, _vp, _sz, _vp], _int),
    "kq_moe_route": ([_vp, _i32, _i32, _vp, _vp, _vp], _int),
    "kq_gather_qmm": ([_vp, _int, _i64, _i32, _vp, _i64, _i64, _i32, _i32, _int, _vp, _vp, _i32, _i32,
                       _vp, _int, _i64, _vp, _sz, _vp], _int),
    "kq_moe_glu_gather": ([_vp, _int, _i64, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _int, _int, _vp, _vp,
                           _i32, _i32, _vp, _vp, _sz, _vp], _int),
    "kq_moe_gather_rows": ([_vp, _int, _i64, _i32, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _int,
                            ctypes.POINTER(GatherEpilogue), _vp, _vp, _i32, _i32, _vp, _int, _i64, _i32, _vp, _sz,
                            _vp], _int),
    "kq_gather_workspace_bytes": ([_i32, _i32, _i32, _i32, _int], _sz),
    "kq_moe_mix": ([_vp, _vp, _i32, _i32, _i32, _vp, _int, _vp], _int),
    "kq_moe_router_topk": ([_vp, _int, _i64, _i32, _i32, _i32, ctypes.POINTER(RouterOptions), _vp, _vp, _vp],
                           _int),
    "kq_sdpa_workspace_bytes": ([_i32, _i32, _i32, _i32, _i32], _sz),
    "kq_sdpa_decode_ragged": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _int, _vp,
                               _vp, _sz, _vp], _int),
    "kq_sdpa_decode_ragged_q8": ([_vp] * 10 + [_i32, _i32, _i32, _i32, _i32, _f32, _int, _vp, _vp, _sz, _vp], _int),
    "kq_sdpa_decode_gqa": ([_vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _f32, _int, _vp, _vp, _sz,
                            _vp], _int),
    "kq_sdpa_decode_gqa_q8": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _f32, _int, _vp,
                               _vp, _sz, _vp], _int),
    "kq_sdpa_decode_gqa_noalloc": ([_vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _f32, _int, _vp,
                                    _vp], _int),
    "kq_sdpa_cascade_workspace_bytes": ([_i32, _i32, _i32, _i32, _i32, _i32, _i32], _sz),
    "kq_sdpa_decode_gqa_cascade_q8": ([_vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32,
                                       _i32, _i32, _i32, _i32, _f32, _int, _vp, _vp, _sz, _vp], _int),
    "kq_sdpa_decode_gqa_cascade": ([_vp, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _i32,
                                    _i32, _i32, _i32, _f32, _int, _vp, _vp, _sz, _vp], _int),
    "kq_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_vp)], _int),
    "kq_gguf_close": ([_vp], None),
    "kq_gguf_header": ([_vp, ctypes.POINTER(ctypes.c_uint32)] + [ctypes.POINTER(_i64)] * 6, _int),
    "kq_gguf_kv": ([_vp, _i64, ctypes.POINTER(_vp), ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_uint32),
                    ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_i64), ctypes.POINTER(_vp)], _int),
    "kq_gguf_tensor": ([_vp, _i64, ctypes.POINTER(_vp), ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_uint32),
                        ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_i64),
                        ctypes.POINTER(_i64), ctypes.POINTER(_vp)], _int),
    "kq_gguf_type_size": ([ctypes.c_uint32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)], _int),
}


def lib():
    """Load (once) and return the ctypes library; raise KQLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise KQLibraryError(
                f"{LIB_PATH} not found: build it with `python -m gmlx_amd.build` "
                "(there is no CPU fallback)")
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise KQLibraryError(f"failed to load {LIB_PATH}: {e}") from e
        for name in EXPORTS:
            if not hasattr(L, name):
                raise KQLibraryError(f"{LIB_PATH} lacks symbol {name}")
            argtypes, restype = _SIGS[name]
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = L
    return _lib


def check(fn_name, code):
    if code != KQ_OK:
        msg = lib().kq_strerror(code).decode()
        raise KQError(fn_name, code, msg)


def version():
    return lib().kq_version().decode()

"""ctypes binding of libg5moe.so (the C ABI declared in include/g5moe.h).

The library is loaded from this package directory.  There is no fallback: if
the shared library is missing, `lib()` raises, so no caller can silently run a
CPU or PyTorch path in its place.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

# G5MOE_LIB may name another build of the same C ABI (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("G5MOE_LIB") or Path(__file__).resolve().parent / "libg5moe.so")

DTYPE_BF16 = 0
DTYPE_F32 = 1

STATUS_NAMES = {0: "OK", 1: "INVALID_ARG", 2: "UNSUPPORTED", 3: "HIP_ERROR"}

EXPORTED = (
    "g5moe_last_error",
    "g5moe_version",
    "g5moe_workspace_size",
    "g5moe_pack_gate_up",
    "g5moe_pack_gate_up_transposed",
    "g5moe_router_topk",
    "g5moe_dispatch",
    "g5moe_route",
    "g5moe_dispatch_noalloc",
    "g5moe_expert_gate_up",
    "g5moe_expert_gate_up_train",
    "g5moe_expert_gate_up_train_factors",
    "g5moe_dh_swiglu_backward",
    "g5moe_expert_down",
    "g5moe_expert_swiglu",
    "g5moe_combine",
    "g5moe_add_rmsnorm_router",
    "g5moe_add_rmsnorm_route",
    "g5moe_combine_residual",
    "g5moe_rmsnorm",
    "g5moe_transpose_experts",
    "g5moe_grouped_gemm",
    "g5moe_grouped_gemm_padded",
    "g5moe_gate_grad",
    "g5moe_gate_grad_padded",
    "g5moe_router_grad",
    "g5moe_expert_gate_up_raw",
    "g5moe_swiglu_backward",
    "g5moe_input_grad",
    "g5moe_pad_transpose",
    "g5moe_pad_rows",
    "g5moe_weight_grad",
    "g5moe_weight_grad_sorted_h",
    "g5moe_router_weight_grad_scratch",
    "g5moe_router_weight_grad",
    "g5moe_forward",
    "g5moe_attn_workspace_size",
    "g5moe_attn_varlen_fwd",
)


class Shape(ctypes.Structure):
    """Mirror of `g5moe_shape`."""

    _fields_ = [
        ("n_tokens", ctypes.c_int64),
        ("d_model", ctypes.c_int32),
        ("d_ff", ctypes.c_int32),
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("x_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class Dropout(ctypes.Structure):
    """Mirror of `g5moe_dropout`."""

    _fields_ = [
        ("p", ctypes.c_float),
        ("seed_lo", ctypes.c_uint32),
        ("seed_hi", ctypes.c_uint32),
        ("reserved", ctypes.c_int32),
    ]


def make_dropout(p: float, seed: int) -> Dropout:
    """g5moe_dropout for drop probability p and a 64-bit seed."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return Dropout(float(p), seed & 0xFFFFFFFF, seed >> 32, 0)


class AttnShape(ctypes.Structure):
    """Mirror of `g5moe_attn_shape`."""

    _fields_ = [
        ("n_seqs", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("total_tokens", ctypes.c_int64),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("q_token_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("k_token_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("v_token_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("o_token_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
    ]


class G5MoEError(RuntimeError):
    """A nonzero g5moe_status, with the library's message."""

    def __init__(self, status: int, func: str, message: str):
        self.status = status
        super().__init__(f"{func} failed with {STATUS_NAMES.get(status, status)}: {message}")


_P = ctypes.c_void_p
_SHAPE_P = ctypes.POINTER(Shape)
_DROP_P = ctypes.POINTER(Dropout)
_SIGS = {
    "g5moe_last_error": ([], ctypes.c_char_p),
    "g5moe_version": ([], ctypes.c_int32),
    "g5moe_workspace_size": ([_SHAPE_P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "g5moe_pack_gate_up": ([_P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_pack_gate_up_transposed": ([_P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_router_topk": ([_P, _P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_dispatch": ([_P, _P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_route": ([_P] * 11 + [_SHAPE_P, _P], ctypes.c_int),
    "g5moe_dispatch_noalloc": ([_P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_expert_gate_up": ([_P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_expert_gate_up_train": ([_P, _P, _P, _P, _P, _P, _DROP_P, _SHAPE_P, _P],
                                   ctypes.c_int),
    "g5moe_expert_gate_up_train_factors": ([_P, _P, _P, _P, _P, _P, _DROP_P, _SHAPE_P, _P],
                                           ctypes.c_int),
    "g5moe_dh_swiglu_backward": ([_P, ctypes.c_int32, _P, _P, _P, _P, _SHAPE_P, _P],
                                 ctypes.c_int),
    "g5moe_expert_down": ([_P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_expert_swiglu": ([_P, _P, _P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_combine": ([_P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_add_rmsnorm_router": ([_P, _P, _P, ctypes.c_float, _P, _P, _P, _P, _P, _P, _P,
                                  _SHAPE_P, _P], ctypes.c_int),
    "g5moe_add_rmsnorm_route": ([_P, _P, _P, ctypes.c_float] + [_P] * 12 + [_SHAPE_P, _P],
                                ctypes.c_int),
    "g5moe_combine_residual": ([_P, _P, _P, _P, ctypes.c_float, _P, _SHAPE_P, _P],
                               ctypes.c_int),
    "g5moe_rmsnorm": ([_P, _P, _P, ctypes.c_float, _P, _P, ctypes.c_int64, ctypes.c_int32,
                       ctypes.c_int32, _P], ctypes.c_int),
    "g5moe_transpose_experts": ([_P, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P],
                                ctypes.c_int),
    "g5moe_grouped_gemm": ([_P, _P, _P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                           ctypes.c_int32, _P], ctypes.c_int),
    "g5moe_grouped_gemm_padded": ([_P, ctypes.c_int32, _P, _P, _P, ctypes.c_int64,
                                   ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P],
                                  ctypes.c_int),
    "g5moe_gate_grad": ([_P, _P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_gate_grad_padded": ([_P, _P, _P, _P, _P, _P, _P, ctypes.c_int32, _SHAPE_P, _P],
                               ctypes.c_int),
    "g5moe_router_grad": ([_P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_expert_gate_up_raw": ([_P, _P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_swiglu_backward": ([_P, _P, _P, _P, _P, _P, _P, ctypes.c_int32, _DROP_P,
                               _SHAPE_P, _P], ctypes.c_int),
    "g5moe_pad_transpose": ([_P, _P, _P, _P, ctypes.c_int32, ctypes.c_int32, _SHAPE_P, _P],
                            ctypes.c_int),
    "g5moe_pad_rows": ([_P, _P, _P, _P, ctypes.c_int32, ctypes.c_int32, _SHAPE_P, _P],
                       ctypes.c_int),
    "g5moe_weight_grad": ([_P, _P, _P, _P, _P, _P, _P, ctypes.c_int32, _SHAPE_P, _P],
                          ctypes.c_int),
    "g5moe_weight_grad_sorted_h": ([_P] * 8 + [ctypes.c_int32, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_router_weight_grad_scratch": ([_SHAPE_P, ctypes.POINTER(ctypes.c_size_t)],
                                         ctypes.c_int),
    "g5moe_router_weight_grad": ([_P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_input_grad": ([_P, _P, _P, _P, _P, _SHAPE_P, _P], ctypes.c_int),
    "g5moe_forward": ([_P] * 13 + [_SHAPE_P, _P], ctypes.c_int),
    "g5moe_attn_workspace_size": ([ctypes.POINTER(AttnShape), ctypes.POINTER(ctypes.c_size_t)],
                                  ctypes.c_int),
    "g5moe_attn_varlen_fwd": ([_P, _P, _P, _P, _P, _P, ctypes.c_float, _P, _P,
                               ctypes.POINTER(AttnShape), _P], ctypes.c_int),
}

_lock = threading.Lock()
_lib = None
# the major version of include/g5moe.h these bindings follow (g5moe_version() >> 16)
ABI_MAJOR = 2


def lib() -> ctypes.CDLL:
    """Load (once) and return the shared library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m genet5_amd.build` "
                    "(there is no CPU fallback)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (argtypes, restype) in _SIGS.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = restype
            major = handle.g5moe_version() >> 16
            if major != ABI_MAJOR:
                raise ImportError(f"{LIB_PATH} has ABI major version {major}; these bindings "
                                  f"are for {ABI_MAJOR} (rebuild with python -m genet5_amd.build)")
            _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call `name` and raise G5MoEError on a nonzero status."""
    L = lib()
    st = getattr(L, name)(*args)
    if st != 0:
        msg = L.g5moe_last_error().decode(errors="replace")
        raise G5MoEError(st, name, msg)


def make_shape(n_tokens: int, d_model: int, d_ff: int, n_experts: int, top_k: int,
               x_dtype: int) -> Shape:
    return Shape(int(n_tokens), int(d_model), int(d_ff), int(n_experts), int(top_k),
                 int(x_dtype), 0)


def workspace_size(shape: Shape) -> int:
    n = ctypes.c_size_t(0)
    call("g5moe_workspace_size", ctypes.byref(shape), ctypes.byref(n))
    return int(n.value)

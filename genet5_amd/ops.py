"""Functional PyTorch wrappers over the C ABI (include/g5moe.h).

Each wrapper checks device, dtype, contiguity and shapes on the host (the C
ABI cannot see buffer sizes), allocates its outputs with the PyTorch caching
allocator, and enqueues the HIP kernels on the current stream of the input's
device.  Nothing here synchronises the host, and nothing falls back to a CPU
path: a missing library raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib

SUPPORTED_D_MODEL = (128, 256, 512, 768)
MAX_EXPERTS = 16
MAX_TOP_K = 4


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"g5moe supports bfloat16 and float32 activations, got {dt}")


def _require(t: torch.Tensor, name: str, shape, dtype, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_device(x: torch.Tensor) -> torch.device:
    if x.device.type != "cuda":
        raise RuntimeError(
            f"g5moe runs on the GPU only (got a tensor on {x.device}); there is no CPU path")
    return x.device


def make_shape(x2d: torch.Tensor, d_ff: int, n_experts: int, top_k: int) -> _lib.Shape:
    return _lib.make_shape(x2d.shape[0], x2d.shape[1], d_ff, n_experts, top_k,
                           _dtype_code(x2d.dtype))


def workspace(shape: _lib.Shape, device: torch.device) -> torch.Tensor:
    return torch.empty(_lib.workspace_size(shape), dtype=torch.uint8, device=device)


def pack_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[E, F, d] gate and up (bf16) -> interleaved [E, 2F, d] (32-row groups)."""
    dev = _check_device(w_gate)
    E, F, d = w_gate.shape
    _require(w_gate, "w_gate", (E, F, d), torch.bfloat16, dev)
    _require(w_up, "w_up", (E, F, d), torch.bfloat16, dev)
    out = torch.empty((E, 2 * F, d), dtype=torch.bfloat16, device=dev)
    shape = _lib.make_shape(0, d, F, E, 1, _lib.DTYPE_BF16)
    _lib.call("g5moe_pack_gate_up", _ptr(w_gate), _ptr(w_up), _ptr(out), ctypes.byref(shape),
              _stream(dev))
    return out


def pack_gate_up_transposed(w_gate: torch.Tensor, w_up: torch.Tensor):
    """(pack_gate_up(w_gate, w_up), its per-expert transpose [E, d, 2F]) in one pass."""
    dev = _check_device(w_gate)
    E, F, d = w_gate.shape
    _require(w_gate, "w_gate", (E, F, d), torch.bfloat16, dev)
    _require(w_up, "w_up", (E, F, d), torch.bfloat16, dev)
    out = torch.empty((E, 2 * F, d), dtype=torch.bfloat16, device=dev)
    out_t = torch.empty((E, d, 2 * F), dtype=torch.bfloat16, device=dev)
    shape = _lib.make_shape(0, d, F, E, 1, _lib.DTYPE_BF16)
    _lib.call("g5moe_pack_gate_up_transposed", _ptr(w_gate), _ptr(w_up), _ptr(out), _ptr(out_t),
              ctypes.byref(shape), _stream(dev))
    return out, out_t


def router_topk(x2d: torch.Tensor, w_router: torch.Tensor, top_k: int,
                bias: Optional[torch.Tensor] = None, return_logits: bool = False):
    """Router on [N, d] -> (topk_idx int32 [N, k], topk_w fp32 [N, k][, logits fp32 [N, E]])."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E = w_router.shape[0]
    _require(x2d, "x", (N, d), x2d.dtype, dev)
    _require(w_router, "w_router", (E, d), x2d.dtype, dev)
    if bias is not None:
        _require(bias, "bias", (E,), torch.float32, dev)
    shape = _lib.make_shape(N, d, 128, E, top_k, _dtype_code(x2d.dtype))
    idx = torch.empty((N, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((N, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev) if return_logits else None
    _lib.call("g5moe_router_topk", _ptr(x2d), _ptr(w_router), _ptr(bias), _ptr(idx), _ptr(w),
              _ptr(logits), ctypes.byref(shape), _stream(dev))
    return (idx, w, logits) if return_logits else (idx, w)


def dispatch(topk_idx: torch.Tensor, n_experts: int, d_model: int = 128):
    """topk_idx int32 [N, k] -> (counts [E], offsets [E+1], perm [N*k], inv_pos [N*k])."""
    dev = _check_device(topk_idx)
    N, k = topk_idx.shape
    _require(topk_idx, "topk_idx", (N, k), torch.int32, dev)
    shape = _lib.make_shape(N, d_model, 128, n_experts, k, _lib.DTYPE_BF16)
    counts = torch.empty((n_experts,), dtype=torch.int32, device=dev)
    offsets = torch.empty((n_experts + 1,), dtype=torch.int32, device=dev)
    perm = torch.empty((N * k,), dtype=torch.int32, device=dev)
    inv_pos = torch.empty((N * k,), dtype=torch.int32, device=dev)
    ws = workspace(shape, dev)
    _lib.call("g5moe_dispatch", _ptr(topk_idx), _ptr(counts), _ptr(offsets), _ptr(perm),
              _ptr(inv_pos), _ptr(ws), ctypes.byref(shape), _stream(dev))
    return counts, offsets, perm, inv_pos


def route(x2d: torch.Tensor, w_router: torch.Tensor, top_k: int,
          bias: Optional[torch.Tensor] = None, return_logits: bool = False,
          ws: Optional[torch.Tensor] = None, d_ff: int = 128):
    """router_topk then dispatch in two launches (g5moe_route: the router kernel
    forms the dispatch's ranks) -> (topk_idx, topk_w, counts, offsets, perm, inv_pos[,
    logits]), the same values as the two calls.  ws: a workspace for the shape
    (N, d, d_ff, E, top_k), allocated here when None."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E = w_router.shape[0]
    _require(x2d, "x", (N, d), x2d.dtype, dev)
    _require(w_router, "w_router", (E, d), x2d.dtype, dev)
    if bias is not None:
        _require(bias, "bias", (E,), torch.float32, dev)
    shape = _lib.make_shape(N, d, d_ff, E, top_k, _dtype_code(x2d.dtype))
    if ws is None:
        ws = workspace(shape, dev)
    elif ws.numel() < _lib.workspace_size(shape) or ws.device != dev:
        raise ValueError("ws is smaller than the shape's workspace or on another device")
    i32 = dict(dtype=torch.int32, device=dev)
    idx = torch.empty((N, top_k), **i32)
    w = torch.empty((N, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev) if return_logits else None
    counts = torch.empty((E,), **i32)
    offsets = torch.empty((E + 1,), **i32)
    perm = torch.empty((N * top_k,), **i32)
    inv_pos = torch.empty((N * top_k,), **i32)
    _lib.call("g5moe_route", _ptr(x2d), _ptr(w_router), _ptr(bias), _ptr(idx), _ptr(w),
              _ptr(logits), _ptr(counts), _ptr(offsets), _ptr(perm), _ptr(inv_pos), _ptr(ws),
              ctypes.byref(shape), _stream(dev))
    out = (idx, w, counts, offsets, perm, inv_pos)
    return out + (logits,) if return_logits else out


def expert_swiglu(x2d: torch.Tensor, perm: torch.Tensor, offsets: torch.Tensor,
                  w_gate_up: torch.Tensor, w_down: torch.Tensor, top_k: int,
                  return_h: bool = False):
    """Both grouped expert GEMMs -> y_perm bf16 [N*k, d] (and h bf16 [N*k, F] if asked)."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E, F2, _ = w_gate_up.shape
    F = F2 // 2
    _require(x2d, "x", (N, d), x2d.dtype, dev)
    _require(perm, "perm", (N * top_k,), torch.int32, dev)
    _require(offsets, "offsets", (E + 1,), torch.int32, dev)
    _require(w_gate_up, "w_gate_up", (E, 2 * F, d), torch.bfloat16, dev)
    _require(w_down, "w_down", (E, d, F), torch.bfloat16, dev)
    shape = _lib.make_shape(N, d, F, E, top_k, _dtype_code(x2d.dtype))
    ws = workspace(shape, dev)
    y_perm = torch.empty((N * top_k, d), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_expert_swiglu", _ptr(x2d), _ptr(perm), _ptr(offsets), _ptr(w_gate_up),
              _ptr(w_down), _ptr(y_perm), _ptr(ws), ctypes.byref(shape), _stream(dev))
    if return_h:
        off = _h_offset(shape)
        h = ws[off: off + N * top_k * F * 2].view(torch.bfloat16).view(N * top_k, F)
        return y_perm, h
    return y_perm


def _h_offset(shape: _lib.Shape) -> int:
    """Byte offset of h inside the workspace (mirrors WorkspaceLayout in g5moe_internal.h)."""
    a = lambda v: (v + 255) & ~255
    N, d, F, E, k = shape.n_tokens, shape.d_model, shape.d_ff, shape.n_experts, shape.top_k
    nblk = (N * k + 255) // 256
    off = a(N * d * 2 if shape.x_dtype == _lib.DTYPE_F32 else 0)
    off += a(nblk * E * 4)
    off += a(N * k * 4)
    return off


def combine(y_perm: torch.Tensor, inv_pos: torch.Tensor, topk_w: torch.Tensor,
            out_dtype: torch.dtype) -> torch.Tensor:
    """y[t] = sum_s w[t, s] * y_perm[inv_pos[t, s]] -> [N, d] in out_dtype."""
    dev = _check_device(y_perm)
    N, k = topk_w.shape
    d = y_perm.shape[1]
    _require(y_perm, "y_perm", (N * k, d), torch.bfloat16, dev)
    _require(inv_pos, "inv_pos", (N * k,), torch.int32, dev)
    _require(topk_w, "topk_w", (N, k), torch.float32, dev)
    shape = _lib.make_shape(N, d, 128, max(k, 1), k, _dtype_code(out_dtype))
    y = torch.empty((N, d), dtype=out_dtype, device=dev)
    _lib.call("g5moe_combine", _ptr(y_perm), _ptr(inv_pos), _ptr(topk_w), _ptr(y),
              ctypes.byref(shape), _stream(dev))
    return y


def add_rmsnorm_router(residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                       w_router: torch.Tensor, top_k: int,
                       x_add: Optional[torch.Tensor] = None,
                       bias: Optional[torch.Tensor] = None, return_logits: bool = False):
    """Residual add + RMSNorm + router on [N, d] rows (g5moe_add_rmsnorm_router).

    Mirrors fused_add_rmsnorm(X, R, W, eps) (lib/blocks/_component.py:17-20), which
    returns (rmsnorm(X + R), X + R), followed by the router on the normed rows.
    Returns (normed, sum_or_None, topk_idx, topk_w[, logits]); sum is x_add + residual
    (None without x_add: the residual itself is the sum)."""
    dev = _check_device(residual)
    N, d = residual.shape
    E = w_router.shape[0]
    dt = residual.dtype
    _require(residual, "residual", (N, d), dt, dev)
    if x_add is not None:
        _require(x_add, "x_add", (N, d), dt, dev)
    _require(norm_weight, "norm_weight", (d,), torch.float32, dev)
    _require(w_router, "w_router", (E, d), dt, dev)
    if bias is not None:
        _require(bias, "bias", (E,), torch.float32, dev)
    shape = _lib.make_shape(N, d, 128, E, top_k, _dtype_code(dt))
    normed = torch.empty((N, d), dtype=dt, device=dev)
    ssum = torch.empty((N, d), dtype=dt, device=dev) if x_add is not None else None
    idx = torch.empty((N, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((N, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev) if return_logits else None
    _lib.call("g5moe_add_rmsnorm_router", _ptr(x_add), _ptr(residual), _ptr(norm_weight),
              ctypes.c_float(eps), _ptr(w_router), _ptr(bias), _ptr(ssum), _ptr(normed),
              _ptr(idx), _ptr(w), _ptr(logits), ctypes.byref(shape), _stream(dev))
    out = (normed, ssum, idx, w)
    return out + (logits,) if return_logits else out


def add_rmsnorm_route(residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      w_router: torch.Tensor, top_k: int,
                      x_add: Optional[torch.Tensor] = None,
                      bias: Optional[torch.Tensor] = None, return_logits: bool = False,
                      ws: Optional[torch.Tensor] = None, d_ff: int = 128):
    """add_rmsnorm_router then dispatch in two launches (g5moe_add_rmsnorm_route: the
    norm-and-router kernel forms the dispatch's ranks) -> (normed, sum_or_None,
    topk_idx, topk_w, counts, offsets, perm, inv_pos[, logits]), the same values as
    the two calls.  ws: a workspace for the shape (N, d, d_ff, E, top_k), allocated
    here when None."""
    dev = _check_device(residual)
    N, d = residual.shape
    E = w_router.shape[0]
    dt = residual.dtype
    _require(residual, "residual", (N, d), dt, dev)
    if x_add is not None:
        _require(x_add, "x_add", (N, d), dt, dev)
    _require(norm_weight, "norm_weight", (d,), torch.float32, dev)
    _require(w_router, "w_router", (E, d), dt, dev)
    if bias is not None:
        _require(bias, "bias", (E,), torch.float32, dev)
    shape = _lib.make_shape(N, d, d_ff, E, top_k, _dtype_code(dt))
    if ws is None:
        ws = workspace(shape, dev)
    elif ws.numel() < _lib.workspace_size(shape) or ws.device != dev:
        raise ValueError("ws is smaller than the shape's workspace or on another device")
    i32 = dict(dtype=torch.int32, device=dev)
    normed = torch.empty((N, d), dtype=dt, device=dev)
    ssum = torch.empty((N, d), dtype=dt, device=dev) if x_add is not None else None
    idx = torch.empty((N, top_k), **i32)
    w = torch.empty((N, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev) if return_logits else None
    counts = torch.empty((E,), **i32)
    offsets = torch.empty((E + 1,), **i32)
    perm = torch.empty((N * top_k,), **i32)
    inv_pos = torch.empty((N * top_k,), **i32)
    _lib.call("g5moe_add_rmsnorm_route", _ptr(x_add), _ptr(residual), _ptr(norm_weight),
              ctypes.c_float(eps), _ptr(w_router), _ptr(bias), _ptr(ssum), _ptr(normed),
              _ptr(idx), _ptr(w), _ptr(logits), _ptr(counts), _ptr(offsets), _ptr(perm),
              _ptr(inv_pos), _ptr(ws), ctypes.byref(shape), _stream(dev))
    out = (normed, ssum, idx, w, counts, offsets, perm, inv_pos)
    return out + (logits,) if return_logits else out


def rmsnorm(residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
            x_add: Optional[torch.Tensor] = None, return_sum: bool = False):
    """(Residual add +) RMSNorm of [N, d] rows (g5moe_rmsnorm), the same arithmetic as
    add_rmsnorm_router's normed rows.  Returns normed, or (normed, x_add + residual)
    with return_sum (x_add given).  normed is allocated with empty_row_padded (it is
    the next projection's input)."""
    dev = _check_device(residual)
    N, d = residual.shape
    dt = residual.dtype
    _require(residual, "residual", (N, d), dt, dev)
    if x_add is not None:
        _require(x_add, "x_add", (N, d), dt, dev)
    elif return_sum:
        raise ValueError("return_sum needs x_add")
    _require(norm_weight, "norm_weight", (d,), torch.float32, dev)
    normed = empty_row_padded(N, d, dt, dev)
    ssum = torch.empty((N, d), dtype=dt, device=dev) if return_sum else None
    _lib.call("g5moe_rmsnorm", _ptr(x_add), _ptr(residual), _ptr(norm_weight), ctypes.c_float(eps),
              _ptr(ssum), _ptr(normed), N, d, _dtype_code(dt), _stream(dev))
    return (normed, ssum) if return_sum else normed


def combine_residual(y_perm: torch.Tensor, inv_pos: torch.Tensor, topk_w: torch.Tensor,
                     residual: torch.Tensor, alpha: float = 1.0,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """residual + alpha * combine(...) with the roundings of that composition in the
    residual's dtype (g5moe_combine_residual); `out` may be `residual` itself."""
    dev = _check_device(y_perm)
    N, k = topk_w.shape
    d = y_perm.shape[1]
    dt = residual.dtype
    _require(y_perm, "y_perm", (N * k, d), torch.bfloat16, dev)
    _require(inv_pos, "inv_pos", (N * k,), torch.int32, dev)
    _require(topk_w, "topk_w", (N, k), torch.float32, dev)
    _require(residual, "residual", (N, d), dt, dev)
    if out is None:
        out = torch.empty((N, d), dtype=dt, device=dev)
    else:
        _require(out, "out", (N, d), dt, dev)
    shape = _lib.make_shape(N, d, 128, max(k, 1), k, _dtype_code(dt))
    _lib.call("g5moe_combine_residual", _ptr(y_perm), _ptr(inv_pos), _ptr(topk_w),
              _ptr(residual), ctypes.c_float(alpha), _ptr(out), ctypes.byref(shape),
              _stream(dev))
    return out


@dataclass
class Routing:
    topk_idx: torch.Tensor  # int32 [N, k]
    topk_w: torch.Tensor    # fp32 [N, k]
    counts: torch.Tensor    # int32 [E]
    offsets: torch.Tensor   # int32 [E + 1]
    perm: torch.Tensor      # int32 [N*k]
    inv_pos: torch.Tensor   # int32 [N*k]


class ForwardBuffers:
    """Preallocated outputs + workspace for repeated g5moe_forward calls of one shape."""

    def __init__(self, n_tokens: int, d_model: int, d_ff: int, n_experts: int, top_k: int,
                 dtype: torch.dtype, device: torch.device):
        self.shape = _lib.make_shape(n_tokens, d_model, d_ff, n_experts, top_k,
                                     _dtype_code(dtype))
        dev = device
        self.y = torch.empty((n_tokens, d_model), dtype=dtype, device=dev)
        self.routing = Routing(
            topk_idx=torch.empty((n_tokens, top_k), dtype=torch.int32, device=dev),
            topk_w=torch.empty((n_tokens, top_k), dtype=torch.float32, device=dev),
            counts=torch.empty((n_experts,), dtype=torch.int32, device=dev),
            offsets=torch.empty((n_experts + 1,), dtype=torch.int32, device=dev),
            perm=torch.empty((n_tokens * top_k,), dtype=torch.int32, device=dev),
            inv_pos=torch.empty((n_tokens * top_k,), dtype=torch.int32, device=dev),
        )
        self.ws = workspace(self.shape, dev)


def moe_forward(x2d: torch.Tensor, w_router: torch.Tensor, w_gate_up: torch.Tensor,
                w_down: torch.Tensor, top_k: int, bias: Optional[torch.Tensor] = None,
                buffers: Optional[ForwardBuffers] = None, return_routing: bool = False):
    """Whole MoE layer forward on [N, d] through g5moe_forward."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E, F2, _ = w_gate_up.shape
    F = F2 // 2
    if not (1 <= top_k <= min(E, MAX_TOP_K)):
        raise ValueError(f"top_k={top_k} not in [1, min(E, {MAX_TOP_K})]")
    _require(x2d, "x", (N, d), x2d.dtype, dev)
    _require(w_router, "w_router", (E, d), x2d.dtype, dev)
    _require(w_gate_up, "w_gate_up", (E, 2 * F, d), torch.bfloat16, dev)
    _require(w_down, "w_down", (E, d, F), torch.bfloat16, dev)
    if bias is not None:
        _require(bias, "bias", (E,), torch.float32, dev)
    if buffers is None:
        buffers = ForwardBuffers(N, d, F, E, top_k, x2d.dtype, dev)
    else:
        s = buffers.shape
        if (s.n_tokens, s.d_model, s.d_ff, s.n_experts, s.top_k, s.x_dtype) != (
                N, d, F, E, top_k, _dtype_code(x2d.dtype)) or buffers.y.device != dev:
            raise ValueError("buffers were made for another shape, dtype or device")
    r = buffers.routing
    _lib.call("g5moe_forward", _ptr(x2d), _ptr(w_router), _ptr(bias), _ptr(w_gate_up),
              _ptr(w_down), _ptr(buffers.y), _ptr(r.topk_idx), _ptr(r.topk_w), _ptr(r.counts),
              _ptr(r.offsets), _ptr(r.perm), _ptr(r.inv_pos), _ptr(buffers.ws),
              ctypes.byref(buffers.shape), _stream(dev))
    return (buffers.y, r) if return_routing else buffers.y


# ---- training: forward that keeps what the backward needs, and the backward -----------

ROW_PAD = 256  # padding rows of buffers read as the A operand of the grouped GEMM
H_SLACK = 384  # rows after the workspace's h that the training gate|up zeroes
PACKED_SLACK = 384  # the packed padded layout holds at most N*k + PACKED_SLACK * E rows


def packed_rows(n_assignments: int, n_experts: int) -> int:
    """Rows of the packed per-expert padded layout (kmax = 0) for N*k assignments:
    expert e's max(384, 192 * ceil(M_e / 192)) rows laid end to end, at most this
    many in all (a bound that needs no expert counts)."""
    return n_assignments + PACKED_SLACK * n_experts


def _padded_rows(kmax: int, n_assignments: int, n_experts: int) -> int:
    return n_experts * kmax if kmax > 0 else packed_rows(n_assignments, n_experts)


def _dropout_arg(dropout: Optional[Tuple[float, int]]):
    """(p, seed) -> a g5moe_dropout reference for the C ABI (None: no dropout)."""
    if dropout is None or float(dropout[0]) == 0.0:
        return None
    p, seed = dropout
    if not (0.0 <= float(p) <= 1.0):
        raise ValueError(f"dropout p = {p} is not in [0, 1]")
    return ctypes.byref(_lib.make_dropout(p, seed))


def moe_forward_train(x2d: torch.Tensor, w_router: torch.Tensor, w_gate_up: torch.Tensor,
                      w_down: torch.Tensor, top_k: int, bias: Optional[torch.Tensor] = None,
                      offsets_host: Optional[torch.Tensor] = None,
                      offsets_ready: Optional["torch.cuda.Event"] = None,
                      dropout: Optional[Tuple[float, int]] = None, return_h: bool = False,
                      factors: bool = False):
    """The layer forward as stage calls, returning what the backward needs:
    (y, logits fp32 [N, E], topk_idx, topk_w, offsets, perm, inv_pos, y_perm, gu) with
    gu the raw gate|up products bf16 [N*k, 2F] (packed column order), which the
    gate|up GEMM stores beside h (g5moe_expert_gate_up_train) so that the backward
    does not recompute them.  return_h: h (bf16 [N*k + H_SLACK, F], a view of the
    workspace, the rows past N*k zero) is appended, for moe_backward(h=...).
    factors: the gu slot holds the SwiGLU derivative factors instead of the raw
    products (g5moe_expert_gate_up_train_factors), for moe_backward(factors=...).

    offsets_host (pinned int32 [E + 1] on the host): the expert offsets are copied
    there without blocking as soon as the dispatch has written them, and
    offsets_ready (if given) is recorded after the copy.  Once the event has
    completed, moe_backward(..., offsets_host=...) reads them without waiting for
    the rest of the forward.

    dropout = (p, seed): dropout with drop probability p on the expert hidden
    state, the mask of g5moe_dropout keyed on the 64-bit seed (pass the same pair
    to moe_backward)."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E, F2, _ = w_gate_up.shape
    F = F2 // 2
    _require(w_down, "w_down", (E, d, F), torch.bfloat16, dev)
    shape = _lib.make_shape(N, d, F, E, top_k, _dtype_code(x2d.dtype))
    ws = workspace(shape, dev)
    S = _stream(dev)
    idx, w, _, offsets, perm, inv_pos, logits = route(x2d, w_router, top_k, bias=bias,
                                                      return_logits=True, ws=ws, d_ff=F)
    if offsets_host is not None:
        if offsets_host.device.type != "cpu" or offsets_host.shape != (E + 1,) or \
                offsets_host.dtype != torch.int32 or not offsets_host.is_pinned():
            raise ValueError("offsets_host must be a pinned host int32 tensor of shape [E + 1]")
        offsets_host.copy_(offsets, non_blocking=True)
        if offsets_ready is not None:
            offsets_ready.record(torch.cuda.current_stream(dev))
    gu = torch.empty((N * top_k, F2), dtype=torch.bfloat16, device=dev)
    y_perm = torch.empty((N * top_k, d), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_expert_gate_up_train_factors" if factors else "g5moe_expert_gate_up_train",
              _ptr(x2d), _ptr(perm), _ptr(offsets), _ptr(w_gate_up), _ptr(gu), _ptr(ws),
              _dropout_arg(dropout), ctypes.byref(shape), S)
    _lib.call("g5moe_expert_down", _ptr(offsets), _ptr(w_down), _ptr(y_perm), _ptr(ws),
              ctypes.byref(shape), S)
    y = combine(y_perm, inv_pos, w, x2d.dtype)
    if not return_h:
        return y, logits, idx, w, offsets, perm, inv_pos, y_perm, gu
    off = _h_offset(shape)
    h = ws[off: off + (N * top_k + H_SLACK) * F * 2].view(torch.bfloat16).view(-1, F)
    return y, logits, idx, w, offsets, perm, inv_pos, y_perm, gu, h


def transpose_experts(w: torch.Tensor) -> torch.Tensor:
    """bf16 [E, R, C] -> [E, C, R]."""
    dev = _check_device(w)
    E, R, C = w.shape
    _require(w, "w", (E, R, C), torch.bfloat16, dev)
    out = torch.empty((E, C, R), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_transpose_experts", _ptr(w), _ptr(out), E, R, C, _stream(dev))
    return out


def grouped_gemm(a_padded: torch.Tensor, rows: int, offsets: torch.Tensor,
                 b: torch.Tensor) -> torch.Tensor:
    """c[p] = a[p] . b_e^T over expert-contiguous rows; a carries ROW_PAD padding rows."""
    dev = _check_device(a_padded)
    E, n_out, K = b.shape
    _require(a_padded, "a", (rows + ROW_PAD, K), torch.bfloat16, dev)
    _require(b, "b", (E, n_out, K), torch.bfloat16, dev)
    _require(offsets, "offsets", (E + 1,), torch.int32, dev)
    c = torch.empty((rows, n_out), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_grouped_gemm", _ptr(a_padded), _ptr(offsets), _ptr(b), _ptr(c), rows, K,
              n_out, E, _stream(dev))
    return c


def empty_row_padded(rows: int, cols: int, dtype: torch.dtype,
                     device: torch.device) -> torch.Tensor:
    """An uninitialised [rows, cols] tensor whose storage holds ROW_PAD more rows after
    its last, so that linear() can read it as its A operand without a copy."""
    return torch.empty((rows + ROW_PAD, cols), dtype=dtype, device=device)[:rows]


def _has_row_pad(x: torch.Tensor) -> bool:
    """x is a contiguous 2-D tensor whose storage extends ROW_PAD rows past its end."""
    if x.dim() != 2 or not x.is_contiguous():
        return False
    need = (x.storage_offset() + (x.shape[0] + ROW_PAD) * x.shape[1]) * x.element_size()
    return x.untyped_storage().nbytes() >= need


_ROW_OFFSETS: dict = {}


def linear(x2d: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x2d [M, K] @ weight[N, K]^T -> bf16 [M, N], as F.linear without bias, on the
    grouped GEMM with one expert (fp32 accumulate in a fixed k order, one rounding).
    K a multiple of 64 (>= 128), N a multiple of 128, bf16 operands.  The GEMM reads
    ROW_PAD rows past A's last one: a tensor from empty_row_padded (or any contiguous
    one whose storage extends that far) is read in place, any other is copied into
    such a buffer first.  No autograd."""
    dev = _check_device(x2d)
    M, K = x2d.shape
    N = weight.shape[0]
    _require(weight, "weight", (N, K), torch.bfloat16, dev)
    if x2d.dtype != torch.bfloat16:
        raise TypeError(f"x has dtype {x2d.dtype}; linear takes bfloat16")
    if not _has_row_pad(x2d):
        xp = empty_row_padded(M, K, torch.bfloat16, dev)
        xp.copy_(x2d)
        x2d = xp
    key = (dev, M)
    off = _ROW_OFFSETS.get(key)
    if off is None:
        # [0, M] written by fill kernels (no host-to-device copy, so a first call
        # under graph capture works too).  Under capture the fills are only
        # recorded (the graph writes the values before its GEMM reads them), so
        # that tensor is the graph's own and is not cached for eager calls.
        off = torch.empty((2,), dtype=torch.int32, device=dev)
        off[:1].fill_(0)
        off[1:].fill_(M)
        if not torch.cuda.is_current_stream_capturing():
            if len(_ROW_OFFSETS) > 64:
                _ROW_OFFSETS.clear()
            _ROW_OFFSETS[key] = off
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_grouped_gemm", _ptr(x2d), _ptr(off), _ptr(weight), _ptr(y), M, K, N, 1,
              _stream(dev))
    return y


def grouped_gemm_padded(a_pad: torch.Tensor, kmax: int, rows: int, offsets: torch.Tensor,
                        b: torch.Tensor) -> torch.Tensor:
    """c[offsets[e] + j] = a[start(e) + j] . b_e^T for j < M_e: the grouped product over
    a per-expert padded A: start(e) = e * kmax ([E * kmax + ROW_PAD, K]; kmax >= every
    M_e), or, kmax = 0, the packed layout ([packed_rows(rows, E) + ROW_PAD, K])."""
    dev = _check_device(a_pad)
    E, n_out, K = b.shape
    _require(a_pad, "a", (_padded_rows(kmax, rows, E) + ROW_PAD, K), torch.bfloat16, dev)
    _require(b, "b", (E, n_out, K), torch.bfloat16, dev)
    _require(offsets, "offsets", (E + 1,), torch.int32, dev)
    c = torch.empty((rows, n_out), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_grouped_gemm_padded", _ptr(a_pad), kmax, _ptr(offsets), _ptr(b), _ptr(c),
              rows, K, n_out, E, _stream(dev))
    return c


def moe_backward(dy: torch.Tensor, x2d: torch.Tensor, w_router: torch.Tensor,
                 w_gate_up: torch.Tensor, w_down: torch.Tensor, top_k: int,
                 topk_idx: torch.Tensor, topk_w: torch.Tensor, offsets: torch.Tensor,
                 perm: torch.Tensor, inv_pos: torch.Tensor, y_perm: torch.Tensor,
                 grad_logits: Optional[torch.Tensor] = None, w_down_t: Optional[torch.Tensor] = None,
                 w_gate_up_t: Optional[torch.Tensor] = None, gu: Optional[torch.Tensor] = None,
                 offsets_host: Optional[torch.Tensor] = None,
                 dropout: Optional[Tuple[float, int]] = None, h: Optional[torch.Tensor] = None,
                 split_gate_up: bool = False, factors: Optional[torch.Tensor] = None):
    """Gradients (dx, d_w_router, d_w_gate_up (packed layout), d_w_down) of the layer,
    or with split_gate_up (dx, d_w_router, d_w_gate, d_w_up, d_w_down).

    h: the forward's h (moe_forward_train(..., return_h=True)); the down weight
    gradient then reads it in sorted order (g5moe_weight_grad_sorted_h) instead of
    the SwiGLU backward writing a padded copy, and the gate and up gradients come
    out of the weight-gradient kernel unpacked.
    factors: the forward's SwiGLU derivative factors (moe_forward_train(...,
    factors=True), with h): the dh product then computes dGU in its epilogue
    (g5moe_dh_swiglu_backward) and gu and dropout are not used.

    offsets_host: for d or F not a multiple of 256 (the batched-product path, whose
    operands are padded to a common kmax), a completed host copy of offsets
    (moe_forward_train's, after its offsets_ready event); without it the offsets
    are read from the device there, which waits for every kernel queued before
    the call.  For d and F multiples of 256 (every GeneT5 shape) nothing is read
    on the host: the padded operands use the packed layout, whose expert starts
    the kernels compute from offsets and whose size N*k + 384 E the host knows.
    dropout: the forward's (p, seed); the SwiGLU backward regenerates its mask.

    HIP stages: gate gradient and dY (g5moe_gate_grad_padded: dY per expert
    padded), router-logit gradient (g5moe_router_grad, plus grad_logits), the
    gate|up recompute (g5moe_expert_gate_up_raw, unless gu or factors are given),
    dh = dY Wd_e with the SwiGLU backward (g5moe_dh_swiglu_backward with factors;
    otherwise g5moe_grouped_gemm_padded on Wd^T and g5moe_swiglu_backward: dGU
    per expert padded), dX_perm = dGU Wgu_e (g5moe_grouped_gemm_padded on the
    packed gate|up's transpose), dx (g5moe_input_grad), the gathered X rows padded
    (g5moe_pad_rows), the weight gradients dWd_e = dY_e^T h_e, dWgu_e = dGU_e^T X_e
    in one launch (g5moe_weight_grad[_sorted_h]) and dWr = dlogits^T x
    (g5moe_router_weight_grad).  For d or F not a multiple of 256 the expert
    weight gradients are batched torch products over transposed padded operands
    instead."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E, F2, _ = w_gate_up.shape
    F = F2 // 2
    k = top_k
    if x2d.dtype != torch.bfloat16:
        raise TypeError("the MoE backward takes bf16 activations")
    _require(dy, "dy", (N, d), torch.bfloat16, dev)
    _require(y_perm, "y_perm", (N * k, d), torch.bfloat16, dev)
    shape = _lib.make_shape(N, d, F, E, k, _lib.DTYPE_BF16)
    S = _stream(dev)
    hip_wgrad = d % 256 == 0 and F % 256 == 0
    if hip_wgrad:
        kmax = 0  # the packed padded layout: no host read of the offsets
    else:
        # the batched products need one row count for every expert: read the
        # offsets once on the host
        offs = (offsets_host if offsets_host is not None else offsets).tolist()
        if len(offs) != E + 1:
            raise ValueError(f"offsets_host has {len(offs)} entries, expected {E + 1}")
        m_max = max(b - a for a, b in zip(offs[:-1], offs[1:]))
        kmax = max(64, -(-m_max // 64) * 64)
    prows = _padded_rows(kmax, N * k, E)
    dw = torch.empty((N, k), dtype=torch.float32, device=dev)
    if hip_wgrad:
        # dY scaled by the gates, straight into the padded layout the dh product
        # and the weight-gradient kernel both read
        dy_buf = torch.empty((prows + ROW_PAD, d), dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_gate_grad_padded", _ptr(dy), _ptr(y_perm), _ptr(inv_pos),
                  _ptr(topk_w), _ptr(offsets), _ptr(dw), _ptr(dy_buf), kmax,
                  ctypes.byref(shape), S)
    else:
        dyp = torch.empty((N * k + ROW_PAD, d), dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_gate_grad", _ptr(dy), _ptr(y_perm), _ptr(inv_pos), _ptr(topk_w),
                  _ptr(dw), _ptr(dyp), ctypes.byref(shape), S)
    if grad_logits is not None:
        _require(grad_logits, "grad_logits", (N, E), torch.float32, dev)
    dlogits = torch.empty((N, E), dtype=torch.float32, device=dev)
    _lib.call("g5moe_router_grad", _ptr(dw), _ptr(topk_w), _ptr(topk_idx), _ptr(grad_logits),
              _ptr(dlogits), ctypes.byref(shape), S)
    sorted_h = h is not None and hip_wgrad
    if sorted_h:
        _require(h, "h", (N * k + H_SLACK, F), torch.bfloat16, dev)
    if w_down_t is None:
        w_down_t = transpose_experts(w_down)            # [E, F, d]
    # dGU per expert padded, with the grouped GEMM's ROW_PAD rows after the last
    dgu_buf = torch.empty((prows + ROW_PAD, 2 * F), dtype=torch.bfloat16, device=dev)
    dgu_pad = dgu_buf[:prows] if kmax == 0 else dgu_buf[:prows].view(E, kmax, 2 * F)
    h_pad = None
    if factors is not None:
        # the dh product with the SwiGLU backward in its epilogue (the forward's
        # derivative factors carry the dropout mask)
        if not (sorted_h and F % 256 == 0):
            raise ValueError("factors need the forward's h and d, F multiples of 256")
        _require(factors, "factors", (N * k, 2 * F), torch.bfloat16, dev)
        _lib.call("g5moe_dh_swiglu_backward", _ptr(dy_buf), kmax, _ptr(offsets),
                  _ptr(w_down_t), _ptr(factors), _ptr(dgu_buf), ctypes.byref(shape), S)
    else:
        if gu is None:
            # the forward's gate|up products were not kept: recompute them
            gu = torch.empty((N * k, 2 * F), dtype=torch.bfloat16, device=dev)
            ws = workspace(shape, dev)
            _lib.call("g5moe_expert_gate_up_raw", _ptr(x2d), _ptr(perm), _ptr(offsets),
                      _ptr(w_gate_up), _ptr(gu), _ptr(ws), ctypes.byref(shape), S)
            del ws
        else:
            _require(gu, "gu", (N * k, 2 * F), torch.bfloat16, dev)
        if hip_wgrad:
            dh = grouped_gemm_padded(dy_buf, kmax, N * k, offsets, w_down_t)   # [N*k, F]
        else:
            dh = grouped_gemm(dyp, N * k, offsets, w_down_t)
        if not sorted_h:
            h_pad = torch.empty((prows, F) if kmax == 0 else (E, kmax, F), dtype=torch.bfloat16,
                                device=dev)
        _lib.call("g5moe_swiglu_backward", _ptr(dh), _ptr(gu), _ptr(perm), _ptr(offsets), None,
                  _ptr(h_pad), _ptr(dgu_buf), kmax, _dropout_arg(dropout), ctypes.byref(shape),
                  S)
        del dh, gu
    if w_gate_up_t is None:
        w_gate_up_t = transpose_experts(w_gate_up)      # [E, d, 2F]
    dxp = grouped_gemm_padded(dgu_buf, kmax, N * k, offsets, w_gate_up_t)  # [N*k, d]
    dx = torch.empty((N, d), dtype=x2d.dtype, device=dev)
    _require(w_router, "w_router", (E, d), x2d.dtype, dev)
    _lib.call("g5moe_input_grad", _ptr(dxp), _ptr(inv_pos), _ptr(dlogits), _ptr(w_router),
              _ptr(dx), ctypes.byref(shape), S)
    del dxp
    d_wr = router_weight_grad(dlogits, x2d, shape)
    if hip_wgrad:
        # weight gradients on the HIP kernel over token-major padded operands
        dy_pad = dy_buf[:prows]
        x_pad = pad_rows(x2d, perm, offsets, E, kmax, k, n_assignments=N * k)
        if sorted_h:
            d_wd = torch.empty((E, d, F), dtype=torch.bfloat16, device=dev)
            d_wg = torch.empty((E, F, d), dtype=torch.bfloat16, device=dev)
            d_wu = torch.empty((E, F, d), dtype=torch.bfloat16, device=dev)
            _lib.call("g5moe_weight_grad_sorted_h", _ptr(dy_pad), _ptr(h), _ptr(d_wd),
                      _ptr(dgu_pad), _ptr(x_pad), _ptr(d_wg), _ptr(d_wu), _ptr(offsets), kmax,
                      ctypes.byref(shape), S)
            if split_gate_up:
                return dx, d_wr, d_wg, d_wu, d_wd
            return dx, d_wr, pack_gate_up(d_wg, d_wu), d_wd
        d_wd, d_wgu = weight_grad(dy_pad, h_pad, dgu_pad, x_pad, offsets, kmax, top_k=k)
        del dy_pad, dy_buf, x_pad, h_pad, dgu_buf
        if split_gate_up:
            return (dx, d_wr) + unpack_gate_up(d_wgu) + (d_wd,)
        return dx, d_wr, d_wgu, d_wd
    # other shapes: batched products over the per-expert padded operands (zero
    # rows past each expert's own): dWd_e = dY_e^T h_e, dWgu_e^T = X_e^T dGU_e
    dyT = torch.empty((E, d, kmax), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_pad_transpose", _ptr(dyp), None, _ptr(offsets), _ptr(dyT), d, kmax,
              ctypes.byref(shape), S)
    del dyp
    xT = torch.empty((E, d, kmax), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_pad_transpose", _ptr(x2d), _ptr(perm), _ptr(offsets), _ptr(xT), d, kmax,
              ctypes.byref(shape), S)
    d_wd = torch.bmm(dyT, h_pad)                       # [E, d, F]
    del dyT, h_pad
    d_wgu = transpose_experts(torch.bmm(xT, dgu_pad))  # [E, d, 2F] -> [E, 2F, d]
    if split_gate_up:
        return (dx, d_wr) + unpack_gate_up(d_wgu) + (d_wd,)
    return dx, d_wr, d_wgu, d_wd


def router_weight_grad(dlogits: torch.Tensor, x2d: torch.Tensor,
                       shape: "_lib.Shape") -> torch.Tensor:
    """d_w_router = dlogits^T x (fp32 accumulation, bf16 [E, d]) on the HIP kernel."""
    dev = _check_device(x2d)
    N, d = x2d.shape
    E = shape.n_experts
    _require(dlogits, "dlogits", (N, E), torch.float32, dev)
    n = ctypes.c_size_t(0)
    _lib.call("g5moe_router_weight_grad_scratch", ctypes.byref(shape), ctypes.byref(n))
    scratch = torch.empty((n.value // 4,), dtype=torch.float32, device=dev)
    out = torch.empty((E, d), dtype=torch.bfloat16, device=dev)
    _lib.call("g5moe_router_weight_grad", _ptr(dlogits), _ptr(x2d), _ptr(scratch), _ptr(out),
              ctypes.byref(shape), _stream(dev))
    return out


def wgrad_kmax(m_max: int) -> int:
    """Row count of the weight-gradient kernel's per-expert padded operands for a
    largest expert of m_max rows: a multiple of 192, at least 384."""
    return max(384, -(-m_max // 192) * 192)


def pad_rows(src: torch.Tensor, perm: Optional[torch.Tensor], offsets: torch.Tensor,
             n_experts: int, kmax: int, top_k: int = 1,
             n_assignments: Optional[int] = None) -> torch.Tensor:
    """out[e, j] = src row of expert e's j-th sorted position (src row p, or
    src row perm[p] // top_k with perm), zero for j >= M_e: [E, kmax, cols]; or,
    kmax = 0, the packed layout [packed_rows(n_assignments, E), cols] (expert e's
    wgrad rows from its packed start; rows past the last expert are left
    unwritten).  n_assignments: N*k (default: src's row count times top_k with
    perm, its row count without)."""
    dev = _check_device(src)
    cols = src.shape[1]
    if src.dtype != torch.bfloat16 or not src.is_contiguous():
        raise TypeError("pad_rows takes a contiguous bf16 source")
    _require(offsets, "offsets", (n_experts + 1,), torch.int32, dev)
    if n_assignments is None:
        n_assignments = src.shape[0] * (top_k if perm is not None else 1)
    if kmax > 0:
        out = torch.empty((n_experts, kmax, cols), dtype=torch.bfloat16, device=dev)
    else:
        out = torch.empty((packed_rows(n_assignments, n_experts), cols), dtype=torch.bfloat16,
                          device=dev)
    # n_tokens * top_k: the assignments (0 for an empty batch, when every output
    # row is a zero row); the kernel itself reads offsets and perm
    shape = _lib.make_shape(n_assignments // top_k, 256, 256, n_experts, top_k,
                            _lib.DTYPE_BF16)
    _lib.call("g5moe_pad_rows", _ptr(src), _ptr(perm), _ptr(offsets), _ptr(out), cols, kmax,
              ctypes.byref(shape), _stream(dev))
    return out


def weight_grad(dy_pad: torch.Tensor, h_pad: torch.Tensor, dgu_pad: torch.Tensor,
                x_pad: torch.Tensor, offsets: torch.Tensor, kmax: int, top_k: int = 2):
    """(d_w_down [E, d, F], d_w_gate_up [E, 2F, d] packed) = per-expert
    dy_pad[e]^T h_pad[e] and dgu_pad[e]^T x_pad[e] over token-major padded
    operands (zero rows past each expert's count): [E, kmax, .] with kmax from
    wgrad_kmax, or, kmax = 0, the packed layout ([rows, .], rows from packed_rows)."""
    dev = _check_device(dy_pad)
    E = offsets.shape[0] - 1
    d = dy_pad.shape[-1]
    F = h_pad.shape[-1]
    lead = (E, kmax) if kmax > 0 else (dy_pad.shape[0],)
    if kmax == 0 and (dy_pad.dim() != 2 or dy_pad.shape[0] < PACKED_SLACK * E):
        raise ValueError("packed weight-gradient operands are 2-D with at least 384 E rows")
    _require(dy_pad, "dy_pad", lead + (d,), torch.bfloat16, dev)
    _require(h_pad, "h_pad", lead + (F,), torch.bfloat16, dev)
    _require(dgu_pad, "dgu_pad", lead + (2 * F,), torch.bfloat16, dev)
    _require(x_pad, "x_pad", lead + (d,), torch.bfloat16, dev)
    _require(offsets, "offsets", (E + 1,), torch.int32, dev)
    d_wd = torch.empty((E, d, F), dtype=torch.bfloat16, device=dev)
    d_wgu = torch.empty((E, 2 * F, d), dtype=torch.bfloat16, device=dev)
    # n_tokens: the packed layout's bound is N*k + 384 E rows
    n_tok = 1 if kmax > 0 else max(0, lead[0] - PACKED_SLACK * E) // top_k
    shape = _lib.make_shape(n_tok, d, F, E, top_k, _lib.DTYPE_BF16)
    _lib.call("g5moe_weight_grad", _ptr(dy_pad), _ptr(h_pad), _ptr(d_wd), _ptr(dgu_pad),
              _ptr(x_pad), _ptr(d_wgu), _ptr(offsets), kmax, ctypes.byref(shape), _stream(dev))
    return d_wd, d_wgu


def unpack_gate_up(w_gate_up: torch.Tensor):
    """Inverse of pack_gate_up: packed [E, 2F, d] -> (gate [E, F, d], up [E, F, d])."""
    E, F2, d = w_gate_up.shape
    v = w_gate_up.view(E, F2 // 64, 2, 32, d)
    return v[:, :, 0].reshape(E, F2 // 2, d), v[:, :, 1].reshape(E, F2 // 2, d)

"""Varlen bidirectional ALiBi attention on the HIP kernel of libg5moe.so.

Reference interface: GeneT5's FlashAttention (lib/blocks/_flash_att.py:15-98)
calls flash-attn's

    flash_attn_varlen_func(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu,
                           max_seqlen_q=L, max_seqlen_k=L, dropout_p=p,
                           softmax_scale=1/sqrt(head_dim), causal=False)   (:76-88)
    flash_attn_func(q, k, v, dropout_p=p, softmax_scale=..., causal=False)  (:90-96)

with q [total, H, D] (varlen) or [B, L, H, D], GQA through fewer key/value
heads (:49-58).  This module keeps those two functions' signatures (and
flash-attn's `alibi_slopes` argument: bias[h, i, j] = -slope_h * |i - j| on
sequence-local positions) and a `FlashAttention`-shaped module whose
`forward(hidden_states, cu_seqlens=None, max_seqlen=None)` returns
`(out, None)` like the reference's.

Supported: bf16, head_dim 64, non-causal, no dropout, forward only.  Anything
else raises; there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn

from . import _lib, ops
from .ops import _check_device, _ptr, _stream

HEAD_DIM = 64


def alibi_slopes(n_heads: int) -> List[float]:
    """Head slopes of Press et al. (2022), "Train Short, Test Long": a geometric
    sequence starting at 2^(-8/n) for n a power of two; otherwise the slopes of
    the nearest lower power of two followed by every other slope of twice that
    count."""
    def pow2(n):
        start = 2.0 ** (-8.0 / n)
        return [start ** (i + 1) for i in range(n)]
    if n_heads & (n_heads - 1) == 0:
        return pow2(n_heads)
    m = 1 << int(math.floor(math.log2(n_heads)))
    return pow2(m) + pow2(2 * m)[0::2][: n_heads - m]


def _check_qkv(t: torch.Tensor, name: str, total: int, heads: int, dev: torch.device) -> None:
    if t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} has dtype {t.dtype}; the attention kernel takes bfloat16")
    if t.dim() != 3 or tuple(t.shape) != (total, heads, HEAD_DIM):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected ({total}, {heads}, "
                         f"{HEAD_DIM})")
    if t.stride(2) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.stride(0) < 0 \
            or t.stride(1) < 0:
        raise ValueError(f"{name}: head dims must be contiguous and the token/head strides "
                         f"multiples of 8 elements (strides {t.stride()})")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def attn_varlen_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    cu_seqlens: torch.Tensor, max_seqlen: int, softmax_scale: float,
                    alibi_slopes: Optional[torch.Tensor] = None, return_lse: bool = False,
                    key_bounds: bool = True):
    """g5moe_attn_varlen_fwd on the current stream.  q [T, H, 64], k/v [T, Hkv, 64]
    bf16 (head dims contiguous, other strides free); cu_seqlens int32 [n + 1] on
    the GPU; alibi_slopes fp32 [H] or None.  Returns out [T, H, 64] (and the
    natural-log softmax_lse [H, T] fp32 when return_lse).

    key_bounds: give the kernel a workspace for per-64-key-block norm maxima (one
    pre-pass over k).  With them it (a) leaves out, under ALiBi, the key blocks whose
    probabilities are provably below 2^-64 of each row's largest (a key-norm bound
    against the ALiBi distance), and (b) uses a fixed per-query reference maximum
    instead of the online running maximum where the bounds keep every score term
    within 32 of zero (base 2).  The result equals the plain online computation over
    every block (key_bounds=False) to fp32 rounding of the probabilities."""
    dev = _check_device(q)
    T, H = q.shape[0], q.shape[1]
    Hkv = k.shape[1] if k.dim() == 3 else -1
    _check_qkv(q, "q", T, H, dev)
    _check_qkv(k, "k", T, Hkv, dev)
    _check_qkv(v, "v", T, Hkv, dev)
    if H % Hkv:
        raise ValueError(f"key/value heads {Hkv} must divide query heads {H}")
    if cu_seqlens.device != dev or cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 \
            or cu_seqlens.numel() < 1 or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be a contiguous int32 vector [n_seqs + 1] on "
                         f"{dev}")
    if alibi_slopes is not None:
        if alibi_slopes.device != dev or alibi_slopes.dtype != torch.float32 \
                or tuple(alibi_slopes.shape) != (H,) or not alibi_slopes.is_contiguous():
            raise ValueError(f"alibi_slopes must be a contiguous float32 [{H}] tensor on {dev}")
    # ops.ROW_PAD rows of slack after the output, so that the output projection's
    # grouped GEMM (ops.linear) reads it in place
    out = torch.empty((T + ops.ROW_PAD, H, HEAD_DIM), dtype=torch.bfloat16, device=dev)[:T]
    lse = torch.empty((H, T), dtype=torch.float32, device=dev) if return_lse else None
    shape = _lib.AttnShape(
        cu_seqlens.numel() - 1, int(max_seqlen), T, H, Hkv, HEAD_DIM, 0,
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1))
    ws = None
    if key_bounds:
        n = ctypes.c_size_t(0)
        _lib.call("g5moe_attn_workspace_size", ctypes.byref(shape), ctypes.byref(n))
        ws = torch.empty(int(n.value), dtype=torch.uint8, device=dev)
    _lib.call("g5moe_attn_varlen_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(cu_seqlens),
              _ptr(alibi_slopes), ctypes.c_float(softmax_scale), _ptr(lse), _ptr(ws),
              ctypes.byref(shape), _stream(dev))
    return (out, lse) if return_lse else out


@torch.library.custom_op("g5moe::attn_varlen_fwd", mutates_args=())
def _attn_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
             max_seqlen: int, softmax_scale: float, alibi_slopes: Optional[torch.Tensor],
             return_lse: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(out, softmax_lse [H, T]) with return_lse, else (out, an empty [0] tensor): the
    kernel keeps the fp32 row sums lse needs only when it is asked for."""
    if return_lse:
        return attn_varlen_fwd(q, k, v, cu_seqlens, max_seqlen, softmax_scale, alibi_slopes,
                               return_lse=True)
    out = attn_varlen_fwd(q, k, v, cu_seqlens, max_seqlen, softmax_scale, alibi_slopes)
    return out, out.new_empty((0,), dtype=torch.float32)


@_attn_op.register_fake
def _(q, k, v, cu_seqlens, max_seqlen, softmax_scale, alibi_slopes, return_lse):
    T, H, D = q.shape
    lse_shape = (H, T) if return_lse else (0,)
    return q.new_empty((T, H, D)), q.new_empty(lse_shape, dtype=torch.float32)


def _no_backward(ctx, *grads):
    raise NotImplementedError("g5moe::attn_varlen_fwd has no backward (inference kernel)")


_attn_op.register_autograd(_no_backward)


def _unsupported(dropout_p, causal, window_size):
    if dropout_p:
        raise NotImplementedError("attention dropout is not supported (dropout_p must be 0)")
    if causal:
        raise NotImplementedError("causal attention is not supported (GeneT5's encoder is "
                                  "bidirectional)")
    if tuple(window_size) != (-1, -1):
        raise NotImplementedError("local (windowed) attention is not supported")


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False,
                           window_size=(-1, -1), alibi_slopes=None, deterministic=False,
                           return_attn_probs=False):
    """flash-attn's varlen entry point over the HIP kernel (self-attention: the
    query and key segmentations must be the same).  Returns out [T, H, D], or
    (out, softmax_lse, None) with return_attn_probs."""
    _unsupported(dropout_p, causal, window_size)
    if cu_seqlens_k is not cu_seqlens_q and not torch.equal(cu_seqlens_k, cu_seqlens_q):
        raise NotImplementedError("cu_seqlens_k must equal cu_seqlens_q (self-attention)")
    if max_seqlen_q is None:
        max_seqlen_q = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) \
            if cu_seqlens_q.numel() > 1 else 0
    if max_seqlen_k is not None and max_seqlen_k != max_seqlen_q:
        raise NotImplementedError("max_seqlen_k must equal max_seqlen_q (self-attention)")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise NotImplementedError("the HIP attention kernel is forward-only; call it under "
                                  "torch.no_grad()")
    out, lse = _attn_op(q, k, v, cu_seqlens_q, int(max_seqlen_q), float(softmax_scale),
                        alibi_slopes, bool(return_attn_probs))
    return (out, lse, None) if return_attn_probs else out


_CU_CACHE: dict = {}


def _uniform_cu_seqlens(batch: int, seqlen: int, device: torch.device) -> torch.Tensor:
    key = (batch, seqlen, device)
    cu = _CU_CACHE.get(key)
    if cu is None:
        cu = torch.arange(0, (batch + 1) * seqlen, seqlen, dtype=torch.int32, device=device)
        _CU_CACHE.clear()
        _CU_CACHE[key] = cu
    return cu


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                    window_size=(-1, -1), alibi_slopes=None, deterministic=False,
                    return_attn_probs=False):
    """flash-attn's fixed-length entry point: q [B, L, H, D], k/v [B, L, Hkv, D]."""
    _unsupported(dropout_p, causal, window_size)
    B, L = q.shape[0], q.shape[1]
    cu = _uniform_cu_seqlens(B, L, q.device)
    res = flash_attn_varlen_func(q.reshape(B * L, *q.shape[2:]), k.reshape(B * L, *k.shape[2:]),
                                 v.reshape(B * L, *v.shape[2:]), cu, cu, L, L, 0.0,
                                 softmax_scale, False, (-1, -1), alibi_slopes, deterministic,
                                 return_attn_probs)
    if return_attn_probs:
        out, lse, _ = res
        return out.view(B, L, *out.shape[1:]), lse, None
    return res.view(B, L, *res.shape[1:])


@dataclass
class FlashAttentionConfig:
    """Fields of the reference's FlashAttentionConfig (lib/blocks/_flash_att.py:15-30)
    plus `alibi` (slopes of Press et al. per head when True)."""
    embed_dim: int = 768
    num_heads: int = 12
    num_kv_heads: int = None
    head_dim: int = None
    dropout: float = 0.0
    window_size: tuple = (-1, -1)
    alibi: bool = True

    def __post_init__(self):
        if self.num_kv_heads is None:
            self.num_kv_heads = self.num_heads
        if self.head_dim is None:
            self.head_dim = self.embed_dim // self.num_heads


class FlashAttention(nn.Module):
    """Bidirectional attention with optional varlen packing and ALiBi, mirroring
    the reference's FlashAttention (lib/blocks/_flash_att.py:38-98): bias-free
    q/k/v/o projections, GQA, softmax scale 1/sqrt(head_dim); forward returns
    (out, None)."""

    def __init__(self, config: FlashAttentionConfig):
        super().__init__()
        if config.head_dim != HEAD_DIM:
            raise NotImplementedError(f"head_dim {config.head_dim}: the kernel supports "
                                      f"{HEAD_DIM}")
        if config.num_heads % config.num_kv_heads:
            raise ValueError("num_kv_heads must divide num_heads")
        self.config = config
        self.embed_dim = config.embed_dim
        self.num_heads = config.num_heads
        self.num_kv_heads = config.num_kv_heads
        self.head_dim = config.head_dim
        self.kv_dim = config.head_dim * config.num_kv_heads
        self.softmax_scale = 1.0 / math.sqrt(self.head_dim)
        self.q = nn.Linear(config.embed_dim, config.num_heads * self.head_dim, bias=False)
        self.k = nn.Linear(config.embed_dim, self.kv_dim, bias=False)
        self.v = nn.Linear(config.embed_dim, self.kv_dim, bias=False)
        self.o = nn.Linear(config.num_heads * self.head_dim, config.embed_dim, bias=False)
        self.dropout = nn.Dropout(config.dropout)
        # fp32 slopes kept outside the module's buffers, so that casting the model
        # to bf16 does not round them
        self._slopes = alibi_slopes(config.num_heads) if config.alibi else None
        self._slopes_dev: dict = {}

    def alibi_slopes(self, device: torch.device) -> Optional[torch.Tensor]:
        """The per-head slopes as a float32 tensor on `device` (None without ALiBi)."""
        if self._slopes is None:
            return None
        t = self._slopes_dev.get(device)
        if t is None:
            t = torch.tensor(self._slopes, dtype=torch.float32, device=device)
            self._slopes_dev[device] = t
        return t

    def qkv_weight(self) -> torch.Tensor:
        """[H*hd + 2*Hkv*hd, D] concatenation of the q, k and v weights, rebuilt when
        any of them changes."""
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in
                    (self.q.weight, self.k.weight, self.v.weight))
        if getattr(self, "_qkv_key", None) != key:
            self._qkv = torch.cat([self.q.weight, self.k.weight, self.v.weight]).detach()
            self._qkv_key = key
        return self._qkv

    def _fused_projections(self, hidden_states: torch.Tensor) -> bool:
        """In inference (no gradient) with bf16 on the GPU, q, k and v come from one
        product and o from another on the grouped GEMM (ops.linear), faster than
        three nn.Linear calls at GeneT5's shapes; the module's parameters, outputs'
        shapes and meaning are unchanged (values differ from nn.Linear's only by the
        bf16 rounding of a different fp32 summation order)."""
        D = hidden_states.shape[-1]
        nq = self.num_heads * self.head_dim + 2 * self.kv_dim
        needs_grad = torch.is_grad_enabled() and (
            hidden_states.requires_grad or any(p.requires_grad for p in self.parameters()))
        return (not needs_grad and hidden_states.is_cuda
                and hidden_states.dtype == torch.bfloat16
                and all(p.dtype == torch.bfloat16 for p in self.parameters())
                and D % 64 == 0 and D >= 128 and nq % 128 == 0 and D % 128 == 0
                and self.num_heads * self.head_dim >= 128)

    def forward(self, hidden_states, cu_seqlens=None, max_seqlen=None):
        B, L, _ = hidden_states.shape
        fused = self._fused_projections(hidden_states)
        if fused:
            hq = self.num_heads * self.head_dim
            qkv = ops.linear(hidden_states.reshape(B * L, -1), self.qkv_weight())
            q = qkv[:, :hq].view(B * L, self.num_heads, self.head_dim)
            k = qkv[:, hq:hq + self.kv_dim].view(B * L, self.num_kv_heads, self.head_dim)
            v = qkv[:, hq + self.kv_dim:].view(B * L, self.num_kv_heads, self.head_dim)
        else:
            q = self.q(hidden_states).view(B * L, self.num_heads, self.head_dim)
            k = self.k(hidden_states).view(B * L, self.num_kv_heads, self.head_dim)
            v = self.v(hidden_states).view(B * L, self.num_kv_heads, self.head_dim)
        drop_p = self.dropout.p if self.training else 0.0
        if cu_seqlens is None:
            cu_seqlens = _uniform_cu_seqlens(B, L, hidden_states.device)
            max_seqlen = L
        out = flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen,
                                     dropout_p=drop_p, softmax_scale=self.softmax_scale,
                                     causal=False,
                                     alibi_slopes=self.alibi_slopes(hidden_states.device))
        if fused:
            out = ops.linear(out.reshape(B * L, self.num_heads * self.head_dim),
                             self.o.weight).view(B, L, -1)
        else:
            out = self.o(out.reshape(B, L, self.num_heads * self.head_dim))
        return self.dropout(out), None

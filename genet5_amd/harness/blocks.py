"""Pre-norm MoE block and block stack.

Reference: EncoderBlock.forward (lib/blocks/encoder.py:73-90) is
    normed = norm2(h); h = h + dropout(ff(normed)) * alpha
with alpha = 1/sqrt(i+1) under depth_scaling (encoder.py:118), else 1.  Config 4
keeps that shape with the attention half removed: h <- h + MoE(RMSNorm(h)).
RMSNorm is LigerRMSNorm in the reference (lib/blocks/_component.py:14, eps 1e-6
at :17-20); here it is the textbook form with the reduction in fp32.  Liger's
exact bf16 casting is not reproduced (parity unpinned for RMSNorm itself; the
MoE's inputs are whatever this RMSNorm produces, and the MoE is checked on them).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch
import torch.nn as nn

from ..moe import MoEFeedForward


class RMSNorm(nn.Module):
    """y = x * rsqrt(mean(x^2) + eps) * weight, computed in fp32, returned in x's dtype.

    hip = True: the HIP kernel g5moe_rmsnorm (the fused norm+router kernel's
    arithmetic: fixed reduction order, correctly rounded sqrt and division);
    otherwise the torch composition.  The kernel builds no autograd graph, so
    when a gradient is needed (grad enabled and x or the weight requiring grad)
    the torch composition runs even with hip = True."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.variance_epsilon = eps
        self.hip = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        needs_grad = torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad)
        if self.hip and not needs_grad:
            from .. import ops
            d = x.shape[-1]
            w = self.weight.detach().to(torch.float32).contiguous()
            return ops.rmsnorm(x.reshape(-1, d).contiguous(), w,
                               self.variance_epsilon).view(x.shape)
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return (y * self.weight.float()).to(x.dtype)


class MoEBlock(nn.Module):
    """h <- h + alpha * MoE(RMSNorm(h)).

    fused (default): MoEFeedForward.residual_block — the RMSNorm, the router and
    the dispatch's ranks in one pass (g5moe_add_rmsnorm_route) and the residual add
    inside the combine
    (g5moe_combine_residual).  fused = False: the reference-shaped composition of
    this module's torch RMSNorm, the MoE module and a torch residual add."""

    def __init__(self, embed_dim: int, ff_dim: int, num_experts: int = 16, top_k: int = 2,
                 residual_scale: float = 1.0, eps: float = 1e-6):
        super().__init__()
        self.norm = RMSNorm(embed_dim, eps)
        self.ff = MoEFeedForward(embed_dim, ff_dim, 0.0, "silu", num_experts, top_k)
        self.residual_scale = residual_scale
        self.fused = True

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        if self.fused:
            return self.ff.residual_block(h, self.norm.weight, self.norm.variance_epsilon,
                                          alpha=self.residual_scale)
        return h + self.ff(self.norm(h)) * self.residual_scale


class MoEStack(nn.Module):
    def __init__(self, num_layers: int, embed_dim: int, ff_dim: int, num_experts: int = 16,
                 top_k: int = 2, depth_scaling: bool = False):
        super().__init__()
        self.layers = nn.ModuleList([
            MoEBlock(embed_dim, ff_dim, num_experts, top_k,
                     (1.0 / math.sqrt(i + 1)) if depth_scaling else 1.0)
            for i in range(num_layers)])

    def set_fused(self, fused: bool) -> "MoEStack":
        for layer in self.layers:
            layer.fused = fused
        return self

    def forward(self, h: torch.Tensor, return_all: bool = False):
        outs = [h]
        for layer in self.layers:
            h = layer(h)
            if return_all:
                outs.append(h)
        return outs if return_all else h


@dataclass
class Config4:
    """Inputs of BASELINE config 4: packed variable-length sequences, 12 seeded layers."""
    x: np.ndarray                # bf16 bits [1, T, d]
    cu_seqlens: np.ndarray       # int32 [n_seq + 1] (recorded; the MoE and RMSNorm are token-wise)
    layer_seeds: List[int]


def packed_lengths(total: int, lo: int, hi: int, rng: np.random.Generator) -> np.ndarray:
    """Lengths ~ U[lo, hi] drawn until they cover `total`, the last one truncated."""
    lens = []
    acc = 0
    while acc < total:
        n = int(rng.integers(lo, hi + 1))
        n = min(n, total - acc)
        lens.append(n)
        acc += n
    return np.array(lens, dtype=np.int64)


def make_config4(n_tokens: int = 45500, d_model: int = 768, n_layers: int = 12,
                 seed: int = 0) -> Config4:
    from .. import synth
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = packed_lengths(n_tokens, 1000, 9000, rng)
    cu = np.zeros(len(lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(lens)
    x = synth.f32_to_bf16_bits(rng.standard_normal((1, n_tokens, d_model), dtype=np.float32))
    return Config4(x=x, cu_seqlens=cu, layer_seeds=[seed + i for i in range(n_layers)])


@torch.no_grad()
def load_layer_weights(stack: MoEStack, seeds: List[int], d_ff: int) -> None:
    """Independent seeded N(0, 0.02) weights per layer (synth.make_layer's draw order)."""
    from .. import synth
    for layer, s in zip(stack.layers, seeds):
        w = synth.make_layer(0, d_model=layer.ff.embed_dim, d_ff=d_ff,
                             n_experts=layer.ff.num_experts, top_k=layer.ff.top_k, seed=s,
                             dtype="bf16")
        dev = layer.ff.w_gate.device
        as_t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16).to(dev)
        layer.ff.router.weight.copy_(as_t(w.w_router).to(layer.ff.router.weight.dtype))
        layer.ff.w_gate.copy_(as_t(w.w_gate).to(layer.ff.w_gate.dtype))
        layer.ff.w_up.copy_(as_t(w.w_up).to(layer.ff.w_up.dtype))
        layer.ff.w_down.copy_(as_t(w.w_down).to(layer.ff.w_down.dtype))

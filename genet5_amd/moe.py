"""MoEFeedForward — drop-in for GeneT5's FeedForward with 16 SwiGLU experts, top-2.

Reference interface (lib/blocks/_component.py:35-52): `FeedForward(embed_dim,
ff_dim, dropout=0.0, activation='gelu_new')`, constructed positionally as
`FeedForward(embed_dim, ff_dim, dropout)` at lib/blocks/encoder.py:69 and called
as `self.ff(normed)` at lib/blocks/encoder.py:88, whose single tensor result
(same shape and dtype as the input) is added into the residual at :89.  The
expert body is that module's formula with activation='silu':
`wo(silu(wi_0 x) * wi_1 x)`, bias-free (:42-44, :48-52).

This module keeps that constructor prefix and forward contract and adds
`num_experts` and `top_k`.  Every forward runs the HIP kernels of
libg5moe.so on the input's GPU; there is no CPU or eager-PyTorch fallback.
Parameters, in nn.Linear orientation [out, in]:
    router.weight  [E, d]      (dtype of the model)
    w_gate         [E, F, d]   expert gate projections  (wi_0 of each expert)
    w_up           [E, F, d]   expert up projections    (wi_1 of each expert)
    w_down         [E, d, F]   expert down projections  (wo of each expert)
    router_bias    [E] fp32 buffer, optional (added to the logits before top-k)
The expert GEMMs run in bf16 with fp32 accumulation whatever the parameter
dtype; the interleaved gate|up copy they read is cached and rebuilt only when a
weight changes.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import ops


@torch.library.custom_op("g5moe::moe_forward", mutates_args=())
def _moe_forward_op(x: torch.Tensor, w_router: torch.Tensor, bias: Optional[torch.Tensor],
                    w_gate_up: torch.Tensor, w_down: torch.Tensor, top_k: int) -> torch.Tensor:
    return ops.moe_forward(x, w_router, w_gate_up, w_down, top_k, bias=bias)


@_moe_forward_op.register_fake
def _(x, w_router, bias, w_gate_up, w_down, top_k):
    return torch.empty_like(x)


@torch.library.custom_op("g5moe::pack_gate_up", mutates_args=())
def _pack_gate_up_op(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    return ops.pack_gate_up(w_gate, w_up)


@_pack_gate_up_op.register_fake
def _(w_gate, w_up):
    E, F, d = w_gate.shape
    return w_gate.new_empty((E, 2 * F, d))


def _no_backward(ctx, grad):
    raise NotImplementedError(
        "g5moe::moe_forward is the inference op; MoEFeedForward runs "
        "g5moe::moe_forward_train (which has a backward) whenever gradients are needed")


_moe_forward_op.register_autograd(_no_backward)


def _pack_backward(ctx, grad):
    return ops.unpack_gate_up(grad.contiguous())


_pack_gate_up_op.register_autograd(_pack_backward)


@torch.library.custom_op("g5moe::transpose_experts", mutates_args=())
def _transpose_experts_op(w: torch.Tensor) -> torch.Tensor:
    return ops.transpose_experts(w)


@_transpose_experts_op.register_fake
def _(w):
    E, R, C = w.shape
    return w.new_empty((E, C, R))


# Host copies of the expert offsets made by the training forward, waiting for
# their autograd node: offsets' storage address -> (pinned int32 [E + 1], event
# recorded after the non-blocking copy).  The backward needs the largest expert
# count on the host (it sizes the padded operands); with the copy issued right
# after the dispatch, reading it waits for that point of the forward only, not
# for the device to drain.  Entries of forwards whose node never comes (no
# gradient) are dropped oldest first.
_HOST_OFFSETS: "OrderedDict[int, Tuple[torch.Tensor, torch.cuda.Event]]" = OrderedDict()
_HOST_OFFSETS_MAX = 256


def _fused_swiglu_backward(w_gate_up: torch.Tensor) -> bool:
    """Whether the training op keeps the SwiGLU derivative factors (the fused dh +
    SwiGLU backward, d and F multiples of 256) or the raw gate|up products."""
    F2, d = w_gate_up.shape[1], w_gate_up.shape[2]
    return d % 256 == 0 and (F2 // 2) % 256 == 0


@torch.library.custom_op("g5moe::moe_forward_train", mutates_args=())
def _moe_forward_train_op(x: torch.Tensor, w_router: torch.Tensor, bias: Optional[torch.Tensor],
                          w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                          w_gate_up: torch.Tensor, w_gate_up_t: torch.Tensor,
                          w_down_t: torch.Tensor, top_k: int, dropout_p: float, seed: int
                          ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                     torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                     torch.Tensor, torch.Tensor]:
    """Training forward.  w_gate / w_up / w_down are the differentiable parameters
    (bf16); the kernels read w_gate_up (their packed copy) and w_down, and the
    backward the transposed copies w_gate_up_t [E, d, 2F] and w_down_t [E, F, d].
    The last output is the forward's h [N*k + 384, F] (zero rows past N*k), which
    the backward's down-weight gradient reads; the one before it the SwiGLU
    derivative factors (or, for d or F not a multiple of 256, the raw gate|up
    products), the backward's SwiGLU operand."""
    E = w_router.shape[0]
    host = torch.empty((E + 1,), dtype=torch.int32, pin_memory=True)
    ready = torch.cuda.Event()
    outs = ops.moe_forward_train(x, w_router, w_gate_up, w_down, top_k, bias=bias,
                                 offsets_host=host, offsets_ready=ready,
                                 dropout=(dropout_p, seed) if dropout_p > 0 else None,
                                 return_h=True, factors=_fused_swiglu_backward(w_gate_up))
    _HOST_OFFSETS[outs[4].data_ptr()] = (host, ready)
    while len(_HOST_OFFSETS) > _HOST_OFFSETS_MAX:
        _HOST_OFFSETS.popitem(last=False)
    return tuple(t.contiguous() for t in outs)


@_moe_forward_train_op.register_fake
def _(x, w_router, bias, w_gate, w_up, w_down, w_gate_up, w_gate_up_t, w_down_t, top_k,
      dropout_p, seed):
    N, d = x.shape
    E = w_router.shape[0]
    i32 = dict(dtype=torch.int32, device=x.device)
    f32 = dict(dtype=torch.float32, device=x.device)
    return (torch.empty_like(x), torch.empty((N, E), **f32), torch.empty((N, top_k), **i32),
            torch.empty((N, top_k), **f32), torch.empty((E + 1,), **i32),
            torch.empty((N * top_k,), **i32), torch.empty((N * top_k,), **i32),
            torch.empty((N * top_k, d), dtype=torch.bfloat16, device=x.device),
            torch.empty((N * top_k, w_gate_up.shape[1]), dtype=torch.bfloat16, device=x.device),
            torch.empty((N * top_k + ops.H_SLACK, w_gate_up.shape[1] // 2), dtype=torch.bfloat16,
                        device=x.device))


def _train_setup(ctx, inputs, output):
    (x, w_router, bias, w_gate, w_up, w_down, w_gate_up, w_gate_up_t, w_down_t, top_k,
     dropout_p, seed) = inputs
    _, _, idx, w, offsets, perm, inv_pos, y_perm, gu, h = output
    ctx.top_k = top_k
    ctx.dropout = (dropout_p, seed) if dropout_p > 0 else None
    # gradients of the outputs nobody differentiates (gu alone is 894 MB at 36,400
    # tokens) stay None instead of being filled with zeros
    ctx.set_materialize_grads(False)
    try:
        ctx.host_offsets = _HOST_OFFSETS.pop(offsets.data_ptr(), None)
    except Exception:  # traced (fake) tensors have no storage: read on the device later
        ctx.host_offsets = None
    # gu: the forward's SwiGLU derivative factors (or raw gate|up products), kept
    # so the backward does not recompute them (894 MB at 36,400 tokens: HBM for
    # time); h: the forward's SwiGLU outputs, the down-weight gradient's operand
    # (447 MB)
    ctx.save_for_backward(x, w_router, w_gate_up, w_down, w_gate_up_t, w_down_t, idx, w,
                          offsets, perm, inv_pos, y_perm, gu, h)
    ctx.mark_non_differentiable(idx, w, offsets, perm, inv_pos, y_perm, gu, h)


def _train_backward(ctx, dy, dlogits, *unused):
    (x, w_router, w_gate_up, w_down, w_gate_up_t, w_down_t, idx, w, offsets, perm, inv_pos,
     y_perm, gu, h) = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros_like(x)
    offsets_host = None
    if ctx.host_offsets is not None:
        offsets_host, ready = ctx.host_offsets
        ready.synchronize()  # the copy issued right after the forward's dispatch
    dx, d_wr, d_wg, d_wu, d_wd = ops.moe_backward(
        dy.to(torch.bfloat16).contiguous(), x, w_router, w_gate_up, w_down, ctx.top_k, idx, w,
        offsets, perm, inv_pos, y_perm,
        grad_logits=None if dlogits is None else dlogits.float().contiguous(),
        w_down_t=w_down_t, w_gate_up_t=w_gate_up_t, offsets_host=offsets_host, h=h,
        split_gate_up=True,
        **(dict(factors=gu) if _fused_swiglu_backward(w_gate_up) else
           dict(gu=gu, dropout=ctx.dropout)))
    return dx, d_wr, None, d_wg, d_wu, d_wd, None, None, None, None, None, None


_moe_forward_train_op.register_autograd(_train_backward, setup_context=_train_setup)


class MoEFeedForward(nn.Module):
    """Top-k routed mixture of SwiGLU experts.

    Inference (no gradient needed): the custom op g5moe::moe_forward.  Training
    (grad enabled and x or a parameter requiring grad): g5moe::moe_forward_train,
    whose registered backward runs the HIP backward kernels."""

    def __init__(self, embed_dim: int, ff_dim: int, dropout: float = 0.0,
                 activation: str = "silu", num_experts: int = 16, top_k: int = 2,
                 router_bias: bool = False):
        super().__init__()
        if activation != "silu":
            raise ValueError(
                f"MoEFeedForward experts are SwiGLU (activation='silu'); got {activation!r}")
        if embed_dim not in ops.SUPPORTED_D_MODEL:
            raise ValueError(f"embed_dim {embed_dim} not in {ops.SUPPORTED_D_MODEL}")
        if ff_dim % 128 != 0 or ff_dim <= 0:
            raise ValueError(f"ff_dim {ff_dim} must be a positive multiple of 128")
        if not (1 <= num_experts <= ops.MAX_EXPERTS):
            raise ValueError(f"num_experts {num_experts} not in [1, {ops.MAX_EXPERTS}]")
        if not (1 <= top_k <= min(num_experts, ops.MAX_TOP_K)):
            raise ValueError(f"top_k {top_k} not in [1, min(num_experts, {ops.MAX_TOP_K})]")
        self.embed_dim = embed_dim
        self.ff_dim = ff_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.dropout = float(dropout)
        self.router = nn.Linear(embed_dim, num_experts, bias=False)
        self.w_gate = nn.Parameter(torch.empty(num_experts, ff_dim, embed_dim))
        self.w_up = nn.Parameter(torch.empty(num_experts, ff_dim, embed_dim))
        self.w_down = nn.Parameter(torch.empty(num_experts, embed_dim, ff_dim))
        if router_bias:
            self.register_buffer("router_bias", torch.zeros(num_experts, dtype=torch.float32))
        else:
            self.router_bias = None
        self.reset_parameters()
        self._packed_key = None
        self._packed = None
        self._transposed = None
        # Switch-style load-balancing loss weight (0 = off); the loss of the last
        # differentiable forward is left in self.aux_loss.
        self.aux_loss_coef = 0.0
        self.aux_loss = None

    def reset_parameters(self) -> None:
        # nn.Linear's default init, per expert matrix.
        for w in (self.w_gate, self.w_up, self.w_down):
            bound = 1.0 / math.sqrt(w.shape[-1])
            nn.init.uniform_(w, -bound, bound)
        self.router.reset_parameters()

    @torch.no_grad()
    def load_dense(self, wi_0: torch.Tensor, wi_1: torch.Tensor, wo: torch.Tensor) -> None:
        """Upcycle a dense FeedForward (wi_0/wi_1/wo weights) into every expert."""
        self.w_gate.copy_(wi_0.unsqueeze(0).expand_as(self.w_gate))
        self.w_up.copy_(wi_1.unsqueeze(0).expand_as(self.w_up))
        self.w_down.copy_(wo.unsqueeze(0).expand_as(self.w_down))

    def _expert_weights(self, transposed: bool = False):
        """bf16 packed gate|up [E, 2F, d] and bf16 down [E, d, F] (with transposed:
        also their per-expert transposes [E, d, 2F] and [E, F, d], the backward's
        operands), cached by the parameters' versions: rebuilt only when a weight
        changes, so forwards and backwards between two optimizer steps (gradient
        accumulation) share one copy.  Under torch.compile the cache (Python-side
        state) is bypassed and the copies are made by custom ops on every call, from
        detached parameters: the copies are kernel operands, and the gradients reach
        the parameters through the training op's own inputs."""
        if torch.compiler.is_compiling():
            wgu = _pack_gate_up_op(self.w_gate.detach().to(torch.bfloat16),
                                   self.w_up.detach().to(torch.bfloat16))
            wd = self.w_down.detach().to(torch.bfloat16)
            if not transposed:
                return wgu, wd
            return wgu, wd, _transpose_experts_op(wgu), _transpose_experts_op(wd)
        key = (self.w_gate.data_ptr(), self.w_gate._version, self.w_up.data_ptr(),
               self.w_up._version, self.w_down.data_ptr(), self.w_down._version,
               self.w_gate.device, self.w_gate.dtype)
        if self._packed_key != key:
            with torch.no_grad():
                wg = self.w_gate.detach().to(torch.bfloat16).contiguous()
                wu = self.w_up.detach().to(torch.bfloat16).contiguous()
                wd = self.w_down.detach().to(torch.bfloat16).contiguous()
                if transposed:
                    # the packed copy and its transpose in one pass over gate and up
                    wgu, wgu_t = ops.pack_gate_up_transposed(wg, wu)
                    self._packed = (wgu, wd)
                    self._transposed = (wgu_t, ops.transpose_experts(wd))
                else:
                    self._packed = (ops.pack_gate_up(wg, wu), wd)
                    self._transposed = None
            self._packed_key = key
        if not transposed:
            return self._packed
        if self._transposed is None:
            with torch.no_grad():
                self._transposed = tuple(ops.transpose_experts(w) for w in self._packed)
        return self._packed + self._transposed

    def _block_needs_grad(self, residual: torch.Tensor, norm_weight: torch.Tensor,
                          x_add: Optional[torch.Tensor]) -> bool:
        return torch.is_grad_enabled() and (
            residual.requires_grad or norm_weight.requires_grad
            or (x_add is not None and x_add.requires_grad)
            or any(p.requires_grad for p in
                   (self.router.weight, self.w_gate, self.w_up, self.w_down)))

    def _needs_grad(self, x: torch.Tensor) -> bool:
        return torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in
                                   (self.router.weight, self.w_gate, self.w_up, self.w_down)))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.embed_dim:
            raise ValueError(f"last dim {x.shape[-1]} != embed_dim {self.embed_dim}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.embed_dim)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        w_router = self.router.weight
        if w_router.dtype != x2.dtype:
            w_router = w_router.to(x2.dtype)
        if self._needs_grad(x2) or (self.training and self.dropout > 0.0):
            return self._forward_train(x2, w_router.contiguous()).view(*lead, self.embed_dim)
        wgu, wd = self._expert_weights()
        y = _moe_forward_op(x2, w_router.contiguous(), self.router_bias, wgu, wd, self.top_k)
        return y.view(*lead, self.embed_dim)

    def _forward_train(self, x2: torch.Tensor, w_router: torch.Tensor) -> torch.Tensor:
        """Training forward (bf16 activations), differentiable in x, the router and
        the expert weights.  In training mode with dropout > 0 the expert hidden
        state gets dropout (FeedForward.forward's `self.dropout(hidden)`,
        lib/blocks/_component.py:51) with the counter-based mask of g5moe_dropout,
        seeded by a 64-bit draw from torch's default CPU generator (so
        torch.manual_seed makes it reproducible); the backward regenerates the
        mask.  With aux_loss_coef > 0 the Switch-style load-balancing loss
        coef * E * sum_e f_e * P_e (f_e: share of assignments routed to e, P_e:
        mean softmax probability of e) is left in self.aux_loss for the caller
        to add to its loss (the module's output stays one tensor)."""
        if x2.dtype != torch.bfloat16:
            raise TypeError("MoEFeedForward trains on bf16 activations (the model's autocast "
                            "dtype); got " + str(x2.dtype))
        p = self.dropout if self.training else 0.0
        seed = int(torch.randint(0, 2 ** 62, (1,)).item()) if p > 0.0 else 0
        wgu, wd, wgu_t, wd_t = self._expert_weights(transposed=True)
        y, logits, idx, _, offsets, _, _, _, _, _ = _moe_forward_train_op(
            x2, w_router, self.router_bias, self.w_gate.to(torch.bfloat16),
            self.w_up.to(torch.bfloat16), self.w_down.to(torch.bfloat16), wgu, wgu_t, wd_t,
            self.top_k, p, seed)
        self.aux_loss = None
        if self.aux_loss_coef > 0:
            counts = (offsets[1:] - offsets[:-1]).float()
            f = counts / max(1, idx.numel())
            p_mean = torch.softmax(logits, dim=-1).mean(dim=0)
            self.aux_loss = self.aux_loss_coef * self.num_experts * (f * p_mean).sum()
        return y

    def residual_block(self, residual: torch.Tensor, norm_weight: torch.Tensor,
                       eps: float = 1e-6, x_add: Optional[torch.Tensor] = None,
                       alpha: float = 1.0) -> torch.Tensor:
        """The MoE half of GeneT5's encoder block, fused around the experts:

            h = residual + x_add                 (or residual alone)
            return h + alpha * self(rmsnorm(h) * norm_weight)

        i.e. `fused_add_rmsnorm(x_add, residual, norm2.weight, eps)` then
        `hidden + ff(normed) * alpha` (lib/blocks/encoder.py:80-89,
        lib/blocks/_component.py:17-20), as g5moe_add_rmsnorm_router ->
        g5moe_dispatch -> g5moe_expert_swiglu -> g5moe_combine_residual: the
        normalised rows feed the router in the same pass, and the layer output is
        added into the residual inside the combine.  The RMSNorm follows the C
        ABI's reduction order (fp32, correctly rounded sqrt and division).

        The fused kernels build no autograd graph and apply no dropout.  When a
        gradient is needed (grad enabled and residual, x_add, norm_weight or a
        parameter of this module requiring grad), or in training mode with
        dropout > 0, the block runs as the differentiable composition instead:
        torch's add and fp32 RMSNorm, this module's training forward (its own
        backward kernels and dropout) and torch's residual add, all on the GPU."""
        d = self.embed_dim
        if residual.shape[-1] != d:
            raise ValueError(f"last dim {residual.shape[-1]} != embed_dim {d}")
        if self._block_needs_grad(residual, norm_weight, x_add) or (
                self.training and self.dropout > 0.0):
            h = residual if x_add is None else residual + x_add.to(residual.dtype)
            hf = h.float()
            normed = hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps)
            normed = (normed * norm_weight.float()).to(h.dtype)
            return h + self(normed) * alpha
        lead = residual.shape[:-1]
        r2 = residual.reshape(-1, d).contiguous()
        xa2 = None if x_add is None else x_add.reshape(-1, d).to(r2.dtype).contiguous()
        w_router = self.router.weight.to(r2.dtype).contiguous()
        nw = norm_weight.detach().to(torch.float32).contiguous()
        normed, ssum, idx, w = ops.add_rmsnorm_router(r2, nw, eps, w_router, self.top_k,
                                                      x_add=xa2, bias=self.router_bias)
        base = ssum if xa2 is not None else r2
        _, offsets, perm, inv_pos = ops.dispatch(idx, self.num_experts, d)
        wgu, wd = self._expert_weights()
        y_perm = ops.expert_swiglu(normed, perm, offsets, wgu, wd, self.top_k)
        out = ops.combine_residual(y_perm, inv_pos, w, base, alpha)
        return out.view(*lead, d)

    def forward_with_routing(self, x: torch.Tensor):
        """Forward that also returns the routing tensors (ops.Routing)."""
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.embed_dim).contiguous()
        w_router = self.router.weight.to(x2.dtype).contiguous()
        wgu, wd = self._expert_weights()
        y, r = ops.moe_forward(x2, w_router, wgu, wd, self.top_k, bias=self.router_bias,
                               return_routing=True)
        return y.view(*lead, self.embed_dim), r

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
import weakref
from collections import OrderedDict
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import ops


class _ExpertWeightCache:
    """The expert GEMMs' copies of one (w_gate, w_up, w_down) parameter set: the
    bf16 packed gate|up [E, 2F, d] and bf16 down [E, d, F], and on request their
    per-expert transposes [E, d, 2F] and [E, F, d] (the backward's operands).

    An entry is keyed by the parameters' storage addresses and holds weak
    references to the parameter objects; it is used while every reference still
    names the very tensor passed in and each parameter's version counter (bumped by
    every in-place update, such as an optimizer step) is unchanged, and rebuilt
    otherwise.  So forwards and backwards between two optimizer steps (gradient
    accumulation) share one copy, eager or compiled: torch.compile hands the
    custom ops the parameter objects themselves.  An entry is dropped when one of
    its parameters is freed, and when the same parameter objects get a new entry
    (their storage was replaced, e.g. `p.data = ...` by a checkpoint loader).
    `builds` counts the rebuilds."""

    def __init__(self, max_entries: int = 64):
        self._entries: "OrderedDict[tuple, tuple]" = OrderedDict()
        self.max_entries = max_entries
        self.builds = 0

    @staticmethod
    def _state(ws):
        return tuple((w._version, w.dtype, tuple(w.shape), w.stride()) for w in ws)

    def _drop(self, key):
        def cb(_ref):
            self._entries.pop(key, None)
        return cb

    def clear(self) -> None:
        self._entries.clear()

    def get(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
            transposed: bool = False):
        ws = (w_gate, w_up, w_down)
        key = tuple(w.data_ptr() for w in ws) + (w_gate.device,)
        state = self._state(ws)
        ent = self._entries.get(key)
        if ent is not None:
            refs, st, wgu, wd, tr = ent
            if st == state and all(r() is w for r, w in zip(refs, ws)):
                wd = w_down if wd is None else wd
                if transposed and tr is None:
                    with torch.no_grad():
                        tr = (ops.transpose_experts(wgu), ops.transpose_experts(wd))
                    self._entries[key] = (refs, st, wgu, ent[3], tr)
                self._entries.move_to_end(key)
                return (wgu, wd) + tr if transposed else (wgu, wd)
        # the same parameter objects under an older storage address: that copy is stale
        for k2 in [k2 for k2, e2 in self._entries.items()
                   if k2 != key and all(r() is w for r, w in zip(e2[0], ws))]:
            del self._entries[k2]
        with torch.no_grad():
            wg = w_gate.detach().to(torch.bfloat16).contiguous()
            wu = w_up.detach().to(torch.bfloat16).contiguous()
            wd = w_down.detach().to(torch.bfloat16).contiguous()
            if transposed:
                # the packed copy and its transpose in one pass over gate and up
                wgu, wgu_t = ops.pack_gate_up_transposed(wg, wu)
                tr = (wgu_t, ops.transpose_experts(wd))
            else:
                wgu, tr = ops.pack_gate_up(wg, wu), None
        self.builds += 1
        # a bf16 contiguous w_down is its own copy: not kept here, so the entry
        # holds no strong reference to a parameter
        own_wd = None if wd.data_ptr() == w_down.data_ptr() else wd
        refs = tuple(weakref.ref(w, self._drop(key)) for w in ws)
        self._entries[key] = (refs, state, wgu, own_wd, tr)
        self._entries.move_to_end(key)
        while len(self._entries) > self.max_entries:
            self._entries.popitem(last=False)
        return (wgu, wd) + tr if transposed else (wgu, wd)


_WEIGHTS = _ExpertWeightCache()


def clear_weight_cache() -> None:
    """Drop every cached packed / transposed expert weight copy."""
    _WEIGHTS.clear()


@torch.library.custom_op("g5moe::moe_forward", mutates_args=())
def _moe_forward_op(x: torch.Tensor, w_router: torch.Tensor, bias: Optional[torch.Tensor],
                    w_gate_up: torch.Tensor, w_down: torch.Tensor, top_k: int) -> torch.Tensor:
    """Inference forward on already packed bf16 expert weights."""
    return ops.moe_forward(x, w_router, w_gate_up, w_down, top_k, bias=bias)


@_moe_forward_op.register_fake
def _(x, w_router, bias, w_gate_up, w_down, top_k):
    return torch.empty_like(x)


@torch.library.custom_op("g5moe::moe_forward_params", mutates_args=())
def _moe_forward_params_op(x: torch.Tensor, w_router: torch.Tensor,
                           bias: Optional[torch.Tensor], w_gate: torch.Tensor,
                           w_up: torch.Tensor, w_down: torch.Tensor,
                           top_k: int) -> torch.Tensor:
    """Inference forward on the expert parameters themselves ([E, F, d], [E, F, d],
    [E, d, F], any float dtype): their packed bf16 copies come from the weight
    cache, eager or compiled."""
    wgu, wd = _WEIGHTS.get(w_gate, w_up, w_down)
    return ops.moe_forward(x, w_router, wgu, wd, top_k, bias=bias)


@_moe_forward_params_op.register_fake
def _(x, w_router, bias, w_gate, w_up, w_down, top_k):
    return torch.empty_like(x)


def _no_backward(ctx, grad):
    raise NotImplementedError(
        "g5moe::moe_forward is the inference op; MoEFeedForward runs "
        "g5moe::moe_forward_train (which has a backward) whenever gradients are needed")


_moe_forward_op.register_autograd(_no_backward)
_moe_forward_params_op.register_autograd(_no_backward)


def _fused_swiglu_backward(d: int, F: int) -> bool:
    """Whether the training op keeps the SwiGLU derivative factors (the fused dh +
    SwiGLU backward, d and F multiples of 256) or the raw gate|up products."""
    return d % 256 == 0 and F % 256 == 0


@torch.library.custom_op("g5moe::moe_forward_train", mutates_args=())
def _moe_forward_train_op(x: torch.Tensor, w_router: torch.Tensor, bias: Optional[torch.Tensor],
                          w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                          top_k: int, dropout_p: float
                          ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                     torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                     torch.Tensor, torch.Tensor, torch.Tensor]:
    """Training forward on the expert parameters (their bf16 packed copy and its
    transpose come from the weight cache).  Outputs: y, logits fp32 [N, E], topk_idx,
    topk_w, offsets, perm, inv_pos, y_perm, the SwiGLU operand of the backward (the
    derivative factors, or, for d or F not a multiple of 256, the raw gate|up
    products; [N*k, 2F]), the forward's h [N*k + 384, F] (zero rows past N*k), which
    the down-weight gradient reads, and the dropout seed (int64 [1] on the host).

    With dropout_p > 0 the op draws the mask's 64-bit seed from torch's default CPU
    generator (one draw per call, so torch.manual_seed makes it reproducible, and
    activation checkpointing's recompute, which restores the generator, draws the
    same one); the backward regenerates the mask from it.  Nothing is copied from
    the device to the host."""
    seed = int(torch.randint(0, 2 ** 62, (1,)).item()) if dropout_p > 0 else 0
    wgu, wd, _, _ = _WEIGHTS.get(w_gate, w_up, w_down, transposed=True)
    outs = ops.moe_forward_train(x, w_router, wgu, wd, top_k, bias=bias,
                                 dropout=(dropout_p, seed) if dropout_p > 0 else None,
                                 return_h=True,
                                 factors=_fused_swiglu_backward(x.shape[1], w_gate.shape[1]))
    return tuple(t.contiguous() for t in outs) + (torch.tensor([seed], dtype=torch.int64),)


@_moe_forward_train_op.register_fake
def _(x, w_router, bias, w_gate, w_up, w_down, top_k, dropout_p):
    N, d = x.shape
    E, F, _ = w_gate.shape
    i32 = dict(dtype=torch.int32, device=x.device)
    f32 = dict(dtype=torch.float32, device=x.device)
    bf = dict(dtype=torch.bfloat16, device=x.device)
    return (torch.empty_like(x), torch.empty((N, E), **f32), torch.empty((N, top_k), **i32),
            torch.empty((N, top_k), **f32), torch.empty((E + 1,), **i32),
            torch.empty((N * top_k,), **i32), torch.empty((N * top_k,), **i32),
            torch.empty((N * top_k, d), **bf), torch.empty((N * top_k, 2 * F), **bf),
            torch.empty((N * top_k + ops.H_SLACK, F), **bf),
            torch.empty((1,), dtype=torch.int64, device="cpu"))


@torch.library.custom_op("g5moe::moe_backward", mutates_args=())
def _moe_backward_op(dy: torch.Tensor, dlogits: Optional[torch.Tensor], x: torch.Tensor,
                     w_router: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                     w_down: torch.Tensor, idx: torch.Tensor, w: torch.Tensor,
                     offsets: torch.Tensor, perm: torch.Tensor, inv_pos: torch.Tensor,
                     y_perm: torch.Tensor, gu: torch.Tensor, h: torch.Tensor, top_k: int,
                     dropout_p: float, seed: torch.Tensor
                     ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                torch.Tensor]:
    """The training op's backward as one op (AOT autograd records it as a single
    node and never looks inside): (dx, d_w_router, d_w_gate, d_w_up, d_w_down), the
    expert gradients in their parameters' dtypes.  dy: bf16 [N, d]; dlogits: the
    fp32 gradient of the logits output (the load-balancing loss's) or None; seed:
    the forward's dropout seed (host int64 [1])."""
    wgu, wd, wgu_t, wd_t = _WEIGHTS.get(w_gate, w_up, w_down, transposed=True)
    fused = _fused_swiglu_backward(x.shape[1], w_gate.shape[1])
    dx, d_wr, d_wg, d_wu, d_wd = ops.moe_backward(
        dy, x, w_router, wgu, wd, top_k, idx, w, offsets, perm, inv_pos, y_perm,
        grad_logits=dlogits, w_down_t=wd_t, w_gate_up_t=wgu_t, h=h, split_gate_up=True,
        **(dict(factors=gu) if fused else
           dict(gu=gu, dropout=(dropout_p, int(seed[0])) if dropout_p > 0 else None)))
    return (dx, d_wr, d_wg.to(w_gate.dtype), d_wu.to(w_up.dtype), d_wd.to(w_down.dtype))


@_moe_backward_op.register_fake
def _(dy, dlogits, x, w_router, w_gate, w_up, w_down, idx, w, offsets, perm, inv_pos, y_perm,
      gu, h, top_k, dropout_p, seed):
    return (torch.empty_like(x), torch.empty_like(w_router), torch.empty_like(w_gate),
            torch.empty_like(w_up), torch.empty_like(w_down))


def _train_setup(ctx, inputs, output):
    (x, w_router, bias, w_gate, w_up, w_down, top_k, dropout_p) = inputs
    _, _, idx, w, offsets, perm, inv_pos, y_perm, gu, h, seed = output
    ctx.top_k = top_k
    ctx.dropout_p = dropout_p
    # gradients of the outputs nobody differentiates (gu alone is 894 MB at 36,400
    # tokens) stay None instead of being filled with zeros
    ctx.set_materialize_grads(False)
    # gu: the forward's SwiGLU derivative factors (or raw gate|up products), kept
    # so the backward does not recompute them (894 MB at 36,400 tokens: HBM for
    # time); h: the forward's SwiGLU outputs, the down-weight gradient's operand
    # (447 MB)
    ctx.save_for_backward(x, w_router, w_gate, w_up, w_down, idx, w, offsets, perm, inv_pos,
                          y_perm, gu, h, seed)
    ctx.mark_non_differentiable(idx, w, offsets, perm, inv_pos, y_perm, gu, h, seed)


def _train_backward(ctx, dy, dlogits, *unused):
    (x, w_router, w_gate, w_up, w_down, idx, w, offsets, perm, inv_pos, y_perm, gu, h,
     seed) = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros_like(x)
    dx, d_wr, d_wg, d_wu, d_wd = _moe_backward_op(
        dy.to(torch.bfloat16).contiguous(),
        None if dlogits is None else dlogits.float().contiguous(), x, w_router, w_gate, w_up,
        w_down, idx, w, offsets, perm, inv_pos, y_perm, gu, h, ctx.top_k, ctx.dropout_p,
        seed)
    return dx, d_wr, None, d_wg, d_wu, d_wd, None, None


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
        operands), from the weight cache: rebuilt only when a weight changes, so
        forwards and backwards between two optimizer steps (gradient accumulation)
        share one copy.  The custom ops consult the same cache themselves."""
        return _WEIGHTS.get(self.w_gate, self.w_up, self.w_down, transposed)

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
        y = _moe_forward_params_op(x2, w_router.contiguous(), self.router_bias, self.w_gate,
                                   self.w_up, self.w_down, self.top_k)
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
        y, logits, idx, _, offsets, _, _, _, _, _, _ = _moe_forward_train_op(
            x2, w_router, self.router_bias, self.w_gate, self.w_up, self.w_down, self.top_k, p)
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
        lib/blocks/_component.py:17-20), as g5moe_add_rmsnorm_route (add + norm +
        router with the dispatch's ranks, then the placement) ->
        g5moe_expert_swiglu -> g5moe_combine_residual: the normalised rows feed the
        router in the same pass, and the layer output is added into the residual
        inside the combine.  The RMSNorm follows the C
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
        normed, ssum, idx, w, _, offsets, perm, inv_pos = ops.add_rmsnorm_route(
            r2, nw, eps, w_router, self.top_k, x_add=xa2, bias=self.router_bias)
        base = ssum if xa2 is not None else r2
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

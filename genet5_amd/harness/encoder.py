"""GeneT5-shaped encoder with the HIP MoE in every layer, and the MDLM unmasking driver
(BASELINE config 5).

Reference shapes followed:
  * GeneT5.forward (lib/model/genet5.py:49-59): embed -> Encoder -> tied lm_head,
    returning {"logits": ...}; vocab 4,096, d 768, 12 layers, 12 heads; depth
    scaling off (genet5.py:22).
  * EncoderBlock.forward (lib/blocks/encoder.py:73-90), non-fused path:
    h = h + attn(norm1(h)); h = h + ff(norm2(h)); Encoder adds a final norm
    (encoder.py:148).  Here ff is MoEFeedForward (HIP) and attention is the
    HIP varlen ALiBi kernel (genet5_amd.attention); backend "torch" keeps the
    PyTorch SDPA composition as the reference.
  * Attention projections q/k/v/o bias-free (lib/blocks/_sdpa_att.py:68-71),
    bidirectional, scale 1/sqrt(head_dim).  No reference attention backend adds
    a positional bias (lib/blocks/_sdpa_att.py, _flash_att.py); following the
    DNABERT-2 lineage this one adds
    symmetric ALiBi, bias[h, i, j] = -slope_h * |i - j|, with the slopes of
    Press et al. (2022), "Train Short, Test Long".  Packed inputs with
    cu_seqlens attend within each sequence only (a block-diagonal mask per
    row, unlike the global-offset mask of the reference SDPA fallback,
    lib/blocks/_sdpa_att.py:36-43).
  * diffusion_generate (lib/inference/diffusion_engine.py:18-95): linear unmask
    schedule, mask/pad logits suppressed, argmax (temperature 0) or sampling,
    confidence = log-prob of the prediction (strategy "confidence") or the gap
    between the two largest logits ("margin"), per-sample top-n unmasking of the
    most confident masked positions, final fill pass.  The per-sample Python
    loop with host syncs (diffusion_engine.py:69-82) is replaced by one
    sort-based selection on the device; among equal confidences the lower
    position is unmasked first.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import attention, ops
from ..attention import alibi_slopes  # noqa: F401  (re-exported for the harness)
from ..moe import MoEFeedForward
from .blocks import RMSNorm


class ALiBiSelfAttention(nn.Module):
    """Bidirectional self-attention with symmetric ALiBi, bias-free q/k/v/o.

    backend "hip" (default): the HIP kernel through genet5_amd.attention's
    flash_attn_varlen_func (the call GeneT5's FlashAttention makes,
    lib/blocks/_flash_att.py:76-88), forward-only, head_dim 64.
    backend "torch": the reference composition in PyTorch, SDPA with the ALiBi
    bias as an explicit mask, one call per packed sequence."""

    def __init__(self, embed_dim: int, num_heads: int, backend: str = "hip"):
        super().__init__()
        if backend not in ("hip", "torch"):
            raise ValueError(f"attention backend {backend!r} is neither 'hip' nor 'torch'")
        self.backend = backend
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.q = nn.Linear(embed_dim, embed_dim, bias=False)
        self.k = nn.Linear(embed_dim, embed_dim, bias=False)
        self.v = nn.Linear(embed_dim, embed_dim, bias=False)
        self.o = nn.Linear(embed_dim, embed_dim, bias=False)
        # fp32 slopes outside the module's buffers (a bf16 cast of the model must
        # not round them)
        self._slopes = alibi_slopes(num_heads)
        self._slopes_dev: Dict[torch.device, torch.Tensor] = {}
        self._bias_cache: Dict[tuple, torch.Tensor] = {}
        self._cu_cache: Dict[tuple, torch.Tensor] = {}

    @property
    def slopes(self) -> torch.Tensor:
        return torch.tensor(self._slopes, dtype=torch.float32)

    def slopes_on(self, device: torch.device) -> torch.Tensor:
        t = self._slopes_dev.get(device)
        if t is None:
            t = torch.tensor(self._slopes, dtype=torch.float32, device=device)
            self._slopes_dev[device] = t
        return t

    def alibi_bias(self, L: int, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
        key = (L, dtype, device)
        b = self._bias_cache.get(key)
        if b is None:
            pos = torch.arange(L, device=device, dtype=torch.float32)
            dist = (pos[None, :] - pos[:, None]).abs()
            b = (-self.slopes_on(device)[:, None, None] * dist[None]).to(dtype).unsqueeze(0)
            self._bias_cache = {key: b}  # keep only the latest length
        return b

    def _attend(self, h: torch.Tensor) -> torch.Tensor:
        B, L, D = h.shape
        q = self.q(h).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k(h).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        v = self.v(h).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=self.alibi_bias(L, q.dtype, q.device),
                                             scale=1.0 / math.sqrt(self.head_dim))
        return self.o(out.transpose(1, 2).reshape(B, L, D))

    def project(self, x2d: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """x2d @ weight^T (no bias): the grouped GEMM as a one-expert product
        (ops.linear) for bf16 rows on the GPU when no gradient is needed, F.linear
        (hipBLASLt) otherwise.  At this encoder's shapes the grouped GEMM is the
        faster of the two (36,400 rows, K = 768: N = 2,304 in 127 against 140 us,
        N = 768 in 47 against 55 us)."""
        needs_grad = torch.is_grad_enabled() and (x2d.requires_grad or weight.requires_grad)
        K, N = x2d.shape[1], weight.shape[0]
        if (not needs_grad and x2d.is_cuda and x2d.dtype == torch.bfloat16
                and weight.dtype == torch.bfloat16 and K % 64 == 0 and K >= 128
                and N % 128 == 0 and weight.is_contiguous()):
            return ops.linear(x2d, weight)
        return F.linear(x2d, weight)

    def qkv_weight(self) -> torch.Tensor:
        """[3D, D] concatenation of the q, k and v weights, rebuilt when any changes."""
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in
                    (self.q.weight, self.k.weight, self.v.weight))
        if getattr(self, "_qkv_key", None) != key:
            self._qkv = torch.cat([self.q.weight, self.k.weight, self.v.weight]).detach()
            self._qkv_key = key
        return self._qkv

    def _attend_hip(self, h: torch.Tensor, cu_seqlens: Optional[torch.Tensor]) -> torch.Tensor:
        B, L, D = h.shape
        H, hd = self.num_heads, self.head_dim
        # one projection for q, k and v; the kernel reads them as strided views
        qkv = self.project(h.reshape(B * L, D), self.qkv_weight()).view(B * L, 3, H, hd)
        q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
        if cu_seqlens is None:
            key = (B, L, h.device)
            cu = self._cu_cache.get(key)
            if cu is None:
                cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=h.device)
                self._cu_cache = {key: cu}
            max_len = L
        else:
            bounds = cu_seqlens.tolist()
            cu = torch.tensor(bounds, dtype=torch.int32, device=h.device)
            max_len = max((b - a for a, b in zip(bounds[:-1], bounds[1:])), default=0)
        out = attention.flash_attn_varlen_func(q, k, v, cu, cu, max_len, max_len,
                                               softmax_scale=1.0 / math.sqrt(hd),
                                               alibi_slopes=self.slopes_on(h.device))
        return self.project(out.view(B * L, D), self.o.weight).view(B, L, D)

    def forward(self, h: torch.Tensor, cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.backend == "hip":
            return self._attend_hip(h, cu_seqlens)
        if cu_seqlens is None:
            return self._attend(h)
        # packed [1, T, D]: attend within each sequence
        bounds = cu_seqlens.tolist()
        parts = [self._attend(h[:, a:b]) for a, b in zip(bounds[:-1], bounds[1:])]
        return torch.cat(parts, dim=1)


class MoEEncoderBlock(nn.Module):
    """fused (default): the attention output, the residual add, norm2, the router and
    the MoE's own residual add run as MoEFeedForward.residual_block (the
    fused_add_norm path of encoder.py:80-83).  fused = False: the non-fused path of
    encoder.py:84-89 in torch around the MoE module."""

    def __init__(self, embed_dim: int, num_heads: int, ff_dim: int, num_experts: int = 16,
                 top_k: int = 2, attention_backend: str = "hip"):
        super().__init__()
        self.norm1 = RMSNorm(embed_dim)
        self.self_attn = ALiBiSelfAttention(embed_dim, num_heads, attention_backend)
        self.norm2 = RMSNorm(embed_dim)
        self.ff = MoEFeedForward(embed_dim, ff_dim, 0.0, "silu", num_experts, top_k)
        self.fused = True

    def forward(self, h: torch.Tensor, cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = self.self_attn(self.norm1(h), cu_seqlens)
        if self.fused:
            return self.ff.residual_block(h, self.norm2.weight, self.norm2.variance_epsilon,
                                          x_add=a)
        h = h + a
        return h + self.ff(self.norm2(h))


class GeneT5MoE(nn.Module):
    """embed -> 12 x (ALiBi attention + MoE) -> final RMSNorm -> tied lm_head."""

    def __init__(self, vocab_size: int = 4096, embed_dim: int = 768, num_layers: int = 12,
                 num_heads: int = 12, ff_dim: int = 3072, num_experts: int = 16,
                 top_k: int = 2, attention_backend: str = "hip"):
        super().__init__()
        self.embed = nn.Embedding(vocab_size, embed_dim)
        self.layers = nn.ModuleList([
            MoEEncoderBlock(embed_dim, num_heads, ff_dim, num_experts, top_k, attention_backend)
            for _ in range(num_layers)])
        self.final_norm = RMSNorm(embed_dim)
        self.lm_head = nn.Linear(embed_dim, vocab_size, bias=False)
        self.lm_head.weight = self.embed.weight
        self.set_fused(True)

    def set_fused(self, fused: bool) -> "GeneT5MoE":
        """fused: every block's MoE half as MoEFeedForward.residual_block, and the
        attention pre-norms and the final norm as the HIP RMSNorm; otherwise the
        torch composition around the MoE module."""
        for layer in self.layers:
            layer.fused = fused
            layer.norm1.hip = fused
        self.final_norm.hip = fused
        return self

    def set_attention_backend(self, backend: str) -> "GeneT5MoE":
        if backend not in ("hip", "torch"):
            raise ValueError(f"attention backend {backend!r} is neither 'hip' nor 'torch'")
        for layer in self.layers:
            layer.self_attn.backend = backend
        return self

    def forward(self, input_ids: torch.Tensor, cu_seqlens: Optional[torch.Tensor] = None):
        h = self.embed(input_ids)
        for layer in self.layers:
            h = layer(h, cu_seqlens)
        hn = self.final_norm(h)
        if self.layers and self.layers[0].self_attn.backend == "hip":
            # the tied LM head through the same projection as the attention's
            lead = hn.shape[:-1]
            w = self.lm_head.weight
            return {"logits": self.layers[0].self_attn.project(hn.reshape(-1, hn.shape[-1]),
                                                               w).view(*lead, w.shape[0])}
        return {"logits": self.lm_head(hn)}


def linear_unmask_schedule(num_steps: int, eps: float = 1e-3) -> List[float]:
    """Fraction of the target unmasked at each step: differences of linspace(1, eps, T+1)."""
    t = torch.linspace(1.0, eps, num_steps + 1)
    return [(t[i] - t[i + 1]).item() for i in range(num_steps)]


def unmask_confidence(logits: torch.Tensor, preds: torch.Tensor, strategy: str) -> torch.Tensor:
    """Per-position confidence [B, L] of logits [B, L, V] (mask and pad already -inf):
    "confidence" = log-softmax of the prediction (lib/inference/diffusion_engine.py:58-60),
    "margin" = largest minus second-largest logit (:54-56)."""
    if strategy == "margin":
        top2 = logits.topk(2, dim=-1).values
        return top2[..., 0] - top2[..., 1]
    if strategy == "confidence":
        return F.log_softmax(logits, dim=-1).gather(-1, preds.unsqueeze(-1)).squeeze(-1)
    raise ValueError(f"strategy {strategy!r} is neither 'confidence' nor 'margin'")


def select_unmask(conf: torch.Tensor, is_masked: torch.Tensor,
                  n_unmask: torch.Tensor) -> torch.Tensor:
    """Boolean [B, L]: in each row i, the n_unmask[i] still-masked positions of largest
    confidence (n_unmask[i] <= masked count of the row).

    The reference takes a per-row topk over the masked positions
    (diffusion_engine.py:70-82, a Python loop over rows); here every row at once:
    unmasked positions carry -inf, a stable descending sort ranks the row, and
    the first n_unmask[i] ranks are taken.  On distinct confidences both give the
    same set (the topk's order among equal values is unspecified, the stable sort
    takes the lower position)."""
    B, L = conf.shape
    conf = conf.masked_fill(~is_masked, float("-inf"))
    order = torch.sort(conf, dim=1, descending=True, stable=True).indices
    rank = torch.empty_like(order)
    rank.scatter_(1, order, torch.arange(L, device=conf.device).expand(B, -1))
    return (rank < n_unmask[:, None]) & is_masked


@torch.no_grad()
def diffusion_generate(model, prefix_ids: torch.Tensor, target_len: int, mask_token_id: int,
                       pad_token_id: int, num_steps: int = 16, temperature: float = 0.0,
                       generator: Optional[torch.Generator] = None,
                       stats: Optional[dict] = None,
                       strategy: str = "confidence") -> torch.Tensor:
    """Iterative unmasking of a fully masked target appended to prefix_ids [B, P]
    (lib/inference/diffusion_engine.py:18-95): per step the model runs once, the
    mask and pad tokens are suppressed, each position's prediction (argmax, or a
    sample at temperature > 0) gets a confidence (`strategy` "confidence" or
    "margin"), and the scheduled count of most confident masked positions takes
    its predictions; a last pass fills what is still masked.  The logits are taken
    in fp32 (the reference uses the logits' own dtype), so confidences of a bf16
    model do not collapse into ties."""
    if strategy not in ("confidence", "margin"):
        raise ValueError(f"strategy {strategy!r} is neither 'confidence' nor 'margin'")
    device = prefix_ids.device
    B, P = prefix_ids.shape
    target = torch.full((B, target_len), mask_token_id, dtype=torch.long, device=device)
    input_ids = torch.cat([prefix_ids, target], dim=1)
    is_masked = torch.ones(B, target_len, dtype=torch.bool, device=device)
    n_forward = 0
    for frac in linear_unmask_schedule(num_steps):
        logits = model(input_ids)["logits"][:, P:].float()
        n_forward += 1
        logits[:, :, mask_token_id] = float("-inf")
        logits[:, :, pad_token_id] = float("-inf")
        if temperature > 0:
            probs = F.softmax(logits / temperature, dim=-1)
            preds = torch.multinomial(probs.view(-1, probs.size(-1)), 1,
                                      generator=generator).view(B, target_len)
        else:
            preds = logits.argmax(dim=-1)
        conf = unmask_confidence(logits, preds, strategy)
        # same float32 product and truncation as diffusion_engine.py:63-64
        n_unmask = torch.minimum(
            (frac * target_len * torch.ones(B, device=device)).long(), is_masked.sum(dim=1))
        unmask = select_unmask(conf, is_masked, n_unmask)
        input_ids[:, P:] = torch.where(unmask, preds, input_ids[:, P:])
        is_masked &= ~unmask
    if bool(is_masked.any()):
        logits = model(input_ids)["logits"][:, P:].float()
        n_forward += 1
        logits[:, :, mask_token_id] = float("-inf")
        final = logits.argmax(dim=-1)
        input_ids[:, P:] = torch.where(is_masked, final, input_ids[:, P:])
    if stats is not None:
        stats["forwards"] = n_forward
    return input_ids

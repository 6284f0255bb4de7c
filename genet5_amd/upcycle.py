"""Sparse upcycling of a dense GeneT5 checkpoint into the MoE model.

README.md:12 describes GeneT5's MoE as "16 experts top-2, upcycled from DNABERT-2
dense FFN": every expert starts as a copy of the dense gated MLP of its layer.
The dense MLP is FeedForward (lib/blocks/_component.py:35-52) with parameters
`wi_0` (gate), `wi_1` (up) and `wo` (down), which lib/model/build.py:29-35 fills
from DNABERT-2's fused `gated_layers` (gate first) and `wo`.  A GeneT5
checkpoint is `torch.save({"embed", "encoder", "lm_head"})` of the three
state dicts (lib/model/genet5.py:71-84, read back at :86-95 with
`weights_only=True`; "decoder" is accepted for "encoder" as at :90), and the
encoder's keys are `layers.{i}.ff.wi_0.weight` and so on.

Differences from the reference loader, on purpose:
  * the reference loads each part with `load_state_dict(strict=False)`
    (genet5.py:92-94), so a renamed or missing key is silently skipped; here
    every missing, unexpected or mis-shaped key is reported by name, raised by
    default (`strict=True`) and warned about otherwise;
  * the dense FFN of each layer becomes `w_gate` / `w_up` / `w_down` stacks of
    MoEFeedForward, and the router weight, which the dense model does not
    have, is drawn N(0, router_std^2) from a seeded generator per layer (with
    identical experts the layer output does not depend on the routing, because
    the top-k gates sum to 1).
"""
from __future__ import annotations

import re
import warnings
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Mapping, Optional, Union

import torch
import torch.nn as nn

_DENSE_FF = re.compile(r"^layers\.(\d+)\.ff\.(wi_0|wi_1|wo)\.weight$")


def upcycle_encoder_state_dict(dense: Mapping[str, torch.Tensor], num_experts: int = 16,
                               router_std: float = 0.006, seed: int = 0,
                               router_dtype: Optional[torch.dtype] = None
                               ) -> Dict[str, torch.Tensor]:
    """Dense encoder state dict -> MoE encoder state dict.

    `layers.{i}.ff.wi_0/wi_1/wo.weight` become `layers.{i}.ff.w_gate/w_up/w_down`
    ([E, F, d], [E, F, d], [E, d, F], every expert a copy) plus
    `layers.{i}.ff.router.weight` [E, d]; every other key passes through.
    Raises ValueError if a layer has only part of its FFN or inconsistent shapes."""
    out: Dict[str, torch.Tensor] = {}
    ffn: Dict[int, Dict[str, torch.Tensor]] = {}
    for k, v in dense.items():
        m = _DENSE_FF.match(k)
        if m:
            ffn.setdefault(int(m.group(1)), {})[m.group(2)] = v
        else:
            out[k] = v
    for i in sorted(ffn):
        parts = ffn[i]
        missing = sorted({"wi_0", "wi_1", "wo"} - set(parts))
        if missing:
            raise ValueError(f"layer {i}: dense FFN is missing {missing} "
                             f"(has {sorted(parts)})")
        wi0, wi1, wo = parts["wi_0"], parts["wi_1"], parts["wo"]
        if wi0.dim() != 2 or wi0.shape != wi1.shape or wo.shape != (wi0.shape[1], wi0.shape[0]):
            raise ValueError(f"layer {i}: inconsistent dense FFN shapes wi_0 {tuple(wi0.shape)}, "
                             f"wi_1 {tuple(wi1.shape)}, wo {tuple(wo.shape)}")
        F, d = wi0.shape
        pre = f"layers.{i}.ff."
        out[pre + "w_gate"] = wi0.unsqueeze(0).expand(num_experts, F, d).clone()
        out[pre + "w_up"] = wi1.unsqueeze(0).expand(num_experts, F, d).clone()
        out[pre + "w_down"] = wo.unsqueeze(0).expand(num_experts, d, F).clone()
        g = torch.Generator(device="cpu").manual_seed(seed + i)
        router = torch.randn(num_experts, d, generator=g, dtype=torch.float32) * router_std
        out[pre + "router.weight"] = router.to(router_dtype or wi0.dtype)
    return out


@dataclass
class LoadReport:
    missing: List[str] = field(default_factory=list)
    unexpected: List[str] = field(default_factory=list)
    mismatched: List[str] = field(default_factory=list)
    upcycled_layers: List[int] = field(default_factory=list)

    @property
    def clean(self) -> bool:
        return not (self.missing or self.unexpected or self.mismatched)

    def describe(self) -> str:
        lines = []
        for name, keys in (("missing", self.missing), ("unexpected", self.unexpected),
                           ("shape-mismatched", self.mismatched)):
            if keys:
                lines.append(f"{len(keys)} {name} key(s): " + ", ".join(keys))
        return "; ".join(lines) if lines else "clean"


def load_upcycled(model: nn.Module, checkpoint: Union[str, Path, Mapping],
                  num_experts: Optional[int] = None, router_std: float = 0.006,
                  seed: int = 0, strict: bool = True) -> LoadReport:
    """Load a dense GeneT5 checkpoint into a MoE model (harness.encoder.GeneT5MoE,
    whose top level holds embed / layers / final_norm / lm_head like the
    reference's embed / encoder.* / lm_head).

    `checkpoint` is a path (read with torch.load(weights_only=True)) or the dict
    {"embed": ..., "encoder" | "decoder": ..., "lm_head": ...}.  The model's
    own expert count is used unless num_experts is given.  Every key the model
    does not receive, every key it does not know and every shape mismatch is
    reported; strict=True raises KeyError, strict=False warns."""
    if isinstance(checkpoint, (str, Path)):
        checkpoint = torch.load(checkpoint, map_location="cpu", weights_only=True)
    enc_key = "encoder" if "encoder" in checkpoint else "decoder"
    for part in ("embed", enc_key, "lm_head"):
        if part not in checkpoint:
            raise KeyError(f"checkpoint has no {part!r} part (parts: {sorted(checkpoint)})")
    if num_experts is None:
        ffs = [m for m in model.modules() if hasattr(m, "num_experts")]
        if not ffs:
            raise ValueError("model has no MoE layer; pass num_experts")
        num_experts = ffs[0].num_experts
    sd: Dict[str, torch.Tensor] = {}
    sd.update({f"embed.{k}": v for k, v in checkpoint["embed"].items()})
    enc = upcycle_encoder_state_dict(checkpoint[enc_key], num_experts, router_std, seed)
    sd.update(enc)
    sd.update({f"lm_head.{k}": v for k, v in checkpoint["lm_head"].items()})
    report = LoadReport(upcycled_layers=sorted({int(k.split(".")[1]) for k in enc
                                                if k.endswith(".ff.w_gate")}))
    own = model.state_dict()
    for k, v in list(sd.items()):
        if k in own and tuple(own[k].shape) != tuple(v.shape):
            report.mismatched.append(f"{k} {tuple(v.shape)} != model {tuple(own[k].shape)}")
            del sd[k]
    result = model.load_state_dict(sd, strict=False)
    # buffers the dense model cannot hold (the optional router bias) are not "missing"
    report.missing = sorted(k for k in result.missing_keys if not k.endswith("router_bias"))
    report.unexpected = sorted(result.unexpected_keys)
    if not report.clean:
        msg = f"dense -> MoE checkpoint load: {report.describe()}"
        if strict:
            raise KeyError(msg)
        warnings.warn(msg, stacklevel=2)
    return report

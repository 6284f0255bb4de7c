"""Synthetic MoE layer inputs for the benchmark configurations (numpy, host side).

Inputs are drawn with numpy's PCG64 generator, so the same seed gives the same
bits on every machine with this numpy; bf16 tensors are fp32 draws rounded to
nearest-even and kept as raw uint16 bit patterns.  Draw order (one generator):
x [N, d] ~ N(0, 1), router [E, d], gate [E, F, d], up [E, F, d], down [E, d, F],
all weights ~ N(0, 0.02).

Configurations (the reference's BASELINE configs; d = 768, F = 3072, E = 16, k = 2):
  1  2,048 tokens, fp32                          (the CPU oracle's own case)
  2  36,400 tokens (8 x 4,550 packed), bf16      (the benchmark workload)
  3  config 2 + Zipf(s=1.2) router bias b_e = 0.5 ln p_e, p_e ∝ (e+1)^-1.2
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

D_MODEL = 768
D_FF = 3072
N_EXPERTS = 16
TOP_K = 2


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest-even), returned as uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def zipf_router_bias(n_experts: int = N_EXPERTS, s: float = 1.2) -> np.ndarray:
    p = (np.arange(1, n_experts + 1, dtype=np.float64)) ** (-s)
    p /= p.sum()
    return (0.5 * np.log(p)).astype(np.float32)


@dataclass
class LayerInputs:
    """One MoE layer call.  Arrays are fp32 (dtype 'f32') or uint16 bf16 bits ('bf16')."""
    dtype: str                 # 'bf16' or 'f32' — dtype of x and the router weight
    x: np.ndarray              # [N, d]
    w_router: np.ndarray       # [E, d]
    w_gate: np.ndarray         # [E, F, d]  (always bf16 bits: expert GEMMs are bf16)
    w_up: np.ndarray           # [E, F, d]
    w_down: np.ndarray         # [E, d, F]
    bias: Optional[np.ndarray]  # fp32 [E] or None
    top_k: int

    @property
    def n_tokens(self) -> int:
        return self.x.shape[0]

    def x_f32(self) -> np.ndarray:
        return self.x if self.dtype == "f32" else bf16_bits_to_f32(self.x)

    def w_router_f32(self) -> np.ndarray:
        return self.w_router if self.dtype == "f32" else bf16_bits_to_f32(self.w_router)


def make_layer(n_tokens: int, d_model: int = D_MODEL, d_ff: int = D_FF,
               n_experts: int = N_EXPERTS, top_k: int = TOP_K, seed: int = 0,
               dtype: str = "bf16", bias: Optional[str] = None,
               expert_f32: bool = False) -> LayerInputs:
    """Draw one layer's inputs.  Expert weights are rounded to bf16 unless expert_f32."""
    if dtype not in ("bf16", "f32"):
        raise ValueError(dtype)
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((n_tokens, d_model), dtype=np.float32)
    wr = rng.standard_normal((n_experts, d_model), dtype=np.float32) * np.float32(0.02)
    wg = rng.standard_normal((n_experts, d_ff, d_model), dtype=np.float32) * np.float32(0.02)
    wu = rng.standard_normal((n_experts, d_ff, d_model), dtype=np.float32) * np.float32(0.02)
    wd = rng.standard_normal((n_experts, d_model, d_ff), dtype=np.float32) * np.float32(0.02)
    if dtype == "bf16":
        x = f32_to_bf16_bits(x)
        wr = f32_to_bf16_bits(wr)
    if not expert_f32:
        wg, wu, wd = f32_to_bf16_bits(wg), f32_to_bf16_bits(wu), f32_to_bf16_bits(wd)
    b = None
    if bias == "zipf":
        b = zipf_router_bias(n_experts)
    elif bias is not None:
        raise ValueError(bias)
    return LayerInputs(dtype, x, wr, wg, wu, wd, b, top_k)


CONFIGS = {
    1: dict(n_tokens=2048, dtype="f32", bias=None,
            name="cfg1: 2,048 tok fp32, d=768, F=3072, E=16, top-2"),
    2: dict(n_tokens=36400, dtype="bf16", bias=None,
            name="cfg2: 36,400 tok (8x4,550) bf16, d=768, F=3072, E=16, top-2, uniform routing"),
    3: dict(n_tokens=36400, dtype="bf16", bias="zipf",
            name="cfg3: cfg2 + Zipf(1.2) router bias (skewed routing)"),
}


def make_config(cfg: int, seed: int = 0, n_tokens: Optional[int] = None) -> LayerInputs:
    c = CONFIGS[cfg]
    return make_layer(n_tokens if n_tokens is not None else c["n_tokens"], seed=seed,
                      dtype=c["dtype"], bias=c["bias"])


def expert_gemm_flops(n_tokens: int, d_model: int = D_MODEL, d_ff: int = D_FF,
                      top_k: int = TOP_K) -> int:
    """Algorithmic FLOP of the expert GEMMs: 6 * d * F per routed row."""
    return 6 * d_model * d_ff * n_tokens * top_k


def to_torch(inp: LayerInputs, device):
    """Move a LayerInputs to torch tensors on `device` (bf16 bits -> torch.bfloat16)."""
    import torch

    def t(a, bf16):
        tt = torch.from_numpy(np.ascontiguousarray(a))
        if bf16:
            tt = tt.view(torch.bfloat16)
        return tt.to(device)

    xb = inp.dtype == "bf16"
    out = dict(
        x=t(inp.x, xb), w_router=t(inp.w_router, xb),
        w_gate=t(inp.w_gate, inp.w_gate.dtype == np.uint16),
        w_up=t(inp.w_up, inp.w_up.dtype == np.uint16),
        w_down=t(inp.w_down, inp.w_down.dtype == np.uint16),
        bias=None if inp.bias is None else t(inp.bias, False),
    )
    return out

"""Seeded synthetic weights and inputs for the benchmark configurations.

Weights are N(0, 0.02) and activations N(0, 1), drawn on the CPU from
torch.Generator streams so every consumer (GPU path, CPU checker) sees the same
bits: weights from `seed` in the fixed order Wg, then per expert gate/up/down,
then shared gate/up/down; activations from their own stream `seed + 1`.
There are no checkpoints: the layers are random-init of the DeepSeek-V2-Lite
architecture (hidden 2048, 64 routed experts top-6, 2 shared, intermediate 1408).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

HIDDEN = 2048
N_EXPERTS = 64
TOP_K = 6
INTERMEDIATE = 1408
N_SHARED = 2


@dataclass
class MoEWeights:
    wg: torch.Tensor        # [E, H]
    gates: torch.Tensor     # [E, I, H]
    ups: torch.Tensor       # [E, I, H]
    downs: torch.Tensor     # [E, H, I]
    shared_gate: Optional[torch.Tensor]  # [nI, H]
    shared_up: Optional[torch.Tensor]    # [nI, H]
    shared_down: Optional[torch.Tensor]  # [H, nI]

    @property
    def shared(self):
        if self.shared_gate is None:
            return None
        return (self.shared_gate, self.shared_up, self.shared_down)

    def to(self, dtype=None, device=None) -> "MoEWeights":
        f = lambda t: None if t is None else t.to(device=device, dtype=dtype)  # noqa: E731
        return MoEWeights(f(self.wg), f(self.gates), f(self.ups), f(self.downs),
                          f(self.shared_gate), f(self.shared_up), f(self.shared_down))


def _randn_(t: torch.Tensor, g: torch.Generator, std: float) -> torch.Tensor:
    torch.randn(t.shape, generator=g, out=t)
    return t.mul_(std)


def moe_weights(E: int = N_EXPERTS, H: int = HIDDEN, I: int = INTERMEDIATE,
                n_shared: int = N_SHARED, seed: int = 42, std: float = 0.02) -> MoEWeights:
    """fp32 CPU weights of one DeepSeekMoE layer (moe.py:46-75 shapes)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    wg = _randn_(torch.empty(E, H), g, std)
    gates = torch.empty(E, I, H)
    ups = torch.empty(E, I, H)
    downs = torch.empty(E, H, I)
    for e in range(E):
        _randn_(gates[e], g, std)
        _randn_(ups[e], g, std)
        _randn_(downs[e], g, std)
    sg = su = sd = None
    if n_shared > 0:
        sg = _randn_(torch.empty(n_shared * I, H), g, std)
        su = _randn_(torch.empty(n_shared * I, H), g, std)
        sd = _randn_(torch.empty(H, n_shared * I), g, std)
    return MoEWeights(wg, gates, ups, downs, sg, su, sd)


def tokens(T: int, H: int = HIDDEN, seed: int = 42) -> torch.Tensor:
    """fp32 CPU activations [T, H] ~ N(0, 1) from the stream seed + 1."""
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    return torch.randn(T, H, generator=g)


def zipf_router_bias(E: int = N_EXPERTS, s: float = 1.1) -> torch.Tensor:
    """Decode configuration's router logit bias b_e = 2 ln((e+1)^-s)."""
    return torch.tensor([2.0 * math.log((e + 1) ** (-s)) for e in range(E)], dtype=torch.float32)


def mla_weights(H: int = HIDDEN, n_heads: int = 16, nope: int = 128, rope_dim: int = 64,
                v_dim: int = 128, kv_lora: int = 512, seed: int = 7, std: float = 0.02) -> dict:
    """fp32 CPU weights of the MLA projection block (mla.py:251-276); norm = ones."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return {
        "q": _randn_(torch.empty(n_heads * (nope + rope_dim), H), g, std),
        "kva": _randn_(torch.empty(kv_lora + rope_dim, H), g, std),
        "kva_norm": torch.ones(kv_lora),
        "kvb": _randn_(torch.empty(n_heads * (nope + v_dim), kv_lora), g, std),
        "o": _randn_(torch.empty(H, n_heads * v_dim), g, std),
    }

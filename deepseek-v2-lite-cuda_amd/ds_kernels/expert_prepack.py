"""Expert weight packing (reference: src/kernels/expert_prepack.py:47-132).

Layouts consumed by the grouped GEMMs (nn.Linear [out, in] order, K-contiguous):
  packed_w1[g] = cat(gate_proj.weight, up_proj.weight)   [G, 2I, H]
  w2[g]        = down_proj.weight                          [G, H, I]

tile_weights() rewrites either into the fragment-tiled layout the fused layer
also accepts (DSK_LAYOUT_TILED in include/dsk.h): [G, N/32, K/16, 64, 8], one
1 KB MFMA fragment (32 rows x 16 columns, lane l = row l % 32, columns
8*(l // 32) .. +7) per [64, 8] slice, so a wave loads a fragment as 1 KB of
consecutive bytes. It is a pure permutation of the same elements.

prepack_with_shared() appends the shared expert (intermediate n_sh * I) as n_sh
extra groups of width I: group E + j takes gate/up rows [j*I, (j+1)*I) and the
matching down columns. Since down(silu(gate x) * up x) splits exactly over
those intermediate slices, the shared expert's output is the sum of the n_sh
group outputs, which the fused combine adds with weight 1.0.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch


def _weights(expert) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    for attr in ("gate_proj", "up_proj", "down_proj"):
        if not hasattr(expert, attr):
            raise AttributeError(
                f"prepack_experts: expert module is missing attribute '{attr}'. "
                "Expected an ExpertMLP with gate_proj, up_proj, and down_proj.")
    return expert.gate_proj.weight, expert.up_proj.weight, expert.down_proj.weight


def pack_tensors(gates: Sequence[torch.Tensor], ups: Sequence[torch.Tensor],
                 downs: Sequence[torch.Tensor], device: Optional[torch.device] = None,
                 shared: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
                 ) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Pack per-expert [I,H], [I,H], [H,I] weights (+ optional shared expert
    [nI,H], [nI,H], [H,nI]) into bf16 (w1 [G,2I,H], w2 [G,H,I], n_shared_groups)."""
    if len(gates) == 0:
        raise ValueError("prepack_experts: experts list is empty.")
    I, H = gates[0].shape
    E = len(gates)
    dev = device if device is not None else gates[0].device
    nsh = 0
    if shared is not None:
        sg, su, sd = shared
        if sg.shape[0] % I != 0 or sg.shape[1] != H:
            raise ValueError(f"shared expert gate shape {tuple(sg.shape)} is not [n*{I}, {H}]")
        nsh = sg.shape[0] // I
    G = E + nsh
    w1 = torch.empty((G, 2 * I, H), dtype=torch.bfloat16, device=dev)
    w2 = torch.empty((G, H, I), dtype=torch.bfloat16, device=dev)
    for i in range(E):
        g, u, d = gates[i], ups[i], downs[i]
        assert tuple(g.shape) == (I, H), f"Expert {i} gate_proj shape mismatch: {tuple(g.shape)}"
        assert tuple(u.shape) == (I, H), f"Expert {i} up_proj shape mismatch: {tuple(u.shape)}"
        assert tuple(d.shape) == (H, I), f"Expert {i} down_proj shape mismatch: {tuple(d.shape)}"
        w1[i, :I] = g.to(device=dev, dtype=torch.bfloat16)
        w1[i, I:] = u.to(device=dev, dtype=torch.bfloat16)
        w2[i] = d.to(device=dev, dtype=torch.bfloat16)
    for j in range(nsh):
        sl = slice(j * I, (j + 1) * I)
        w1[E + j, :I] = sg[sl].to(device=dev, dtype=torch.bfloat16)
        w1[E + j, I:] = su[sl].to(device=dev, dtype=torch.bfloat16)
        w2[E + j] = sd[:, sl].to(device=dev, dtype=torch.bfloat16)
    return w1, w2, nsh


def tile_weights(w: torch.Tensor) -> torch.Tensor:
    """[G, N, K] row-major -> [G, N/32, K/16, 64, 8] fragment-tiled (same dtype/device)."""
    G, N, K = w.shape
    if N % 32 or K % 16:
        raise ValueError(f"tile_weights: [{G}, {N}, {K}] needs N % 32 == 0 and K % 16 == 0")
    return (w.reshape(G, N // 32, 32, K // 16, 2, 8).permute(0, 1, 3, 4, 2, 5)
            .reshape(G, N // 32, K // 16, 64, 8).contiguous())


def untile_weights(wt: torch.Tensor) -> torch.Tensor:
    """Inverse of tile_weights: [G, N/32, K/16, 64, 8] -> [G, N, K]."""
    G, NB, KS = wt.shape[:3]
    return (wt.reshape(G, NB, KS, 2, 32, 8).permute(0, 1, 4, 2, 3, 5)
            .reshape(G, NB * 32, KS * 16).contiguous())


def prepack_experts(experts: List) -> Tuple[torch.Tensor, torch.Tensor]:
    """Reference-compatible packing: (packed_w1 [E,2I,H], w2 [E,H,I]) in bf16 on
    the experts' (CUDA) device."""
    if len(experts) == 0:
        raise ValueError("prepack_experts: experts list is empty.")
    ws = [_weights(e) for e in experts]
    device = ws[0][0].device
    if device.type != "cuda":
        raise RuntimeError(
            "prepack_experts: expert weights must be on a CUDA device. "
            f"Got device: {device}")
    w1, w2, _ = pack_tensors([w[0] for w in ws], [w[1] for w in ws], [w[2] for w in ws])
    return w1, w2


def prepack_with_shared(experts: List, shared_expert=None,
                        device: Optional[torch.device] = None, tiled: bool = True
                        ) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Packing for the fused layer: routed experts then the shared expert split
    into width-I groups, fragment-tiled unless tiled=False.
    Returns (w1, w2, n_shared_groups)."""
    ws = [_weights(e) for e in experts]
    shared = _weights(shared_expert) if shared_expert is not None else None
    w1, w2, nsh = pack_tensors([w[0] for w in ws], [w[1] for w in ws], [w[2] for w in ws],
                               device=device, shared=shared)
    if tiled:
        w1, w2 = tile_weights(w1), tile_weights(w2)
    return w1, w2, nsh


def verify_prepack(experts: List) -> bool:
    """Checks packed_w1 / w2 against the expert weights (expert_prepack.py:135-161)."""
    packed_w1, w2 = prepack_experts(experts)
    for i, e in enumerate(experts):
        g, u, d = (t.to(torch.bfloat16) for t in _weights(e))
        I = g.shape[0]
        assert torch.equal(packed_w1[i, :I], g), f"Expert {i}: packed_w1 gate rows differ"
        assert torch.equal(packed_w1[i, I:], u), f"Expert {i}: packed_w1 up rows differ"
        assert torch.equal(w2[i], d), f"Expert {i}: w2 differs from down_proj.weight"
    return True

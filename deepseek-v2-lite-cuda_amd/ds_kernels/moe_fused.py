"""Fused MoE forward on MI355X (reference host orchestrator:
src/kernels/moe_fused.py:89-272).

Two levels are offered, as in the reference:
  * the op-by-op pipeline `route_dispatch_combine` — the reference's seven-op
    call sequence (moe_fused.py:118-154) built from this package's ops, plus the
    shared expert the reference omits;
  * the fused entry `moe_fused_forward_logits` / `FusedMoELayer` /
    `fused_moe_forward` — one C call (dsk_moe_fused_forward) that enqueues
    route -> permutation -> GEMM1+SwiGLU -> GEMM2 -> combine with the shared
    expert folded into the grouped GEMMs, and no host synchronisation.

Gate logits: with a bf16 gate weight they come from the library's gate kernel
(ops.moe_gate: bf16 products, fp32 accumulation, as F.linear(x.float(),
w.float()) at moe_fused.py:131 up to fp32 summation order); with an fp32 gate
weight they stay the torch fp32 linear.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from ._lib import check, lib, stream_handle
from .expert_prepack import prepack_experts, prepack_with_shared, tile_weights


def _expert_shapes(op: str, w1: torch.Tensor, w2: torch.Tensor):
    """(tiled, G, 2I, H, w2 logical shape) of row-major or fragment-tiled weights."""
    tiled = w1.dim() == 5
    if tiled:
        if w2.dim() != 5 or tuple(w1.shape[3:]) != (64, 8) or tuple(w2.shape[3:]) != (64, 8):
            raise RuntimeError(f"{op}: tiled w1/w2 must both be [G, N/32, K/16, 64, 8]")
        G, N2, Hw = w1.shape[0], w1.shape[1] * 32, w1.shape[2] * 16
        w2_shape = (w2.shape[0], w2.shape[1] * 32, w2.shape[2] * 16)
    else:
        if w1.dim() != 3 or w2.dim() != 3:
            raise RuntimeError(f"{op}: w1/w2 must be [G, 2I, H] / [G, H, I] (or tiled)")
        G, N2, Hw = w1.shape
        w2_shape = tuple(w2.shape)
    return tiled, G, N2, Hw, w2_shape


def _routing_outputs(return_routing: bool, T: int, top_k: int, E: int, dev):
    if not return_routing:
        return None, None, None
    return (torch.empty((T, top_k), dtype=torch.int32, device=dev),
            torch.empty((T, top_k), dtype=torch.float32, device=dev),
            torch.empty((E + 1,), dtype=torch.int32, device=dev))


def _ptr(t: Optional[torch.Tensor]):
    return t.data_ptr() if t is not None else None


def _events(stage_events):
    if stage_events is not None and not isinstance(stage_events, int):
        return ctypes.cast(stage_events, ctypes.c_void_p).value
    return stage_events


def moe_fused_forward_logits(logits: torch.Tensor, hidden_states: torch.Tensor,
                             w1: torch.Tensor, w2: torch.Tensor, top_k: int,
                             n_shared_groups: int, num_experts: Optional[int] = None,
                             return_routing: bool = False, stage_events=None,
                             workspace: Optional[torch.Tensor] = None):
    """Whole MoE layer from precomputed fp32 gate logits [T, E].

    w1: [E + n_shared_groups, 2I, H] bf16, w2: [E + n_shared_groups, H, I] bf16,
    row-major, or both fragment-tiled by expert_prepack.tile_weights
    ([G, 2I/32, H/16, 64, 8] and [G, H/32, I/16, 64, 8]).
    Returns out [T, H] bf16 (and (topk_idx, topk_w, expert_offsets) if asked).
    stage_events: optional ctypes array of 5 hipEvent_t handles recorded at the
    stage boundaries (instrumentation for benchmarks). workspace: optional
    preallocated uint8 CUDA buffer of at least dsk_moe_fused_workspace_size bytes."""
    op = "moe_fused_forward"
    T, H = hidden_states.shape
    E = logits.shape[1] if num_experts is None else num_experts
    tiled, G, N2, Hw, w2_shape = _expert_shapes(op, w1, w2)
    I = N2 // 2
    for t, n, dt in ((logits, "logits", torch.float32), (hidden_states, "hidden_states", torch.bfloat16),
                     (w1, "w1", torch.bfloat16), (w2, "w2", torch.bfloat16)):
        if not (t.is_cuda and t.is_contiguous() and t.dtype == dt):
            raise RuntimeError(f"{op}: {n} must be a contiguous CUDA {dt} tensor")
    if logits.shape != (T, E) or G != E + n_shared_groups or Hw != H or w2_shape != (G, H, I):
        raise RuntimeError(f"{op}: inconsistent shapes logits={tuple(logits.shape)} "
                           f"x={tuple(hidden_states.shape)} w1={tuple(w1.shape)} w2={tuple(w2.shape)}")
    dev = hidden_states.device
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    if T == 0:
        return (out, (None, None, None)) if return_routing else out
    nws = lib.dsk_moe_fused_workspace_size(T, E, top_k, n_shared_groups, H, I)
    ws = workspace if workspace is not None and workspace.numel() >= nws else \
        torch.empty(nws, dtype=torch.uint8, device=dev)
    idx, w, offs = _routing_outputs(return_routing, T, top_k, E, dev)
    with torch.cuda.device(dev):
        check(lib.dsk_moe_fused_forward(
            logits.data_ptr(), hidden_states.data_ptr(), w1.data_ptr(), w2.data_ptr(),
            out.data_ptr(), T, E, top_k, n_shared_groups, H, I, 1 if tiled else 0,
            _ptr(idx), _ptr(w), _ptr(offs), ws.data_ptr(), ws.numel(), _events(stage_events),
            stream_handle(dev)), op)
    if return_routing:
        return out, (idx, w, offs)
    return out


def moe_layer_forward(hidden_states: torch.Tensor, gate_weight: torch.Tensor,
                      w1: torch.Tensor, w2: torch.Tensor, top_k: int, n_shared_groups: int,
                      gate_bias: Optional[torch.Tensor] = None, return_routing: bool = False,
                      stage_events=None, workspace: Optional[torch.Tensor] = None):
    """Whole MoE layer from the hidden states, router included (one C call:
    partial gate sums -> route -> permutation -> GEMM1+SwiGLU -> GEMM2 -> combine).

    gate_weight: bf16 [E, H], in the same layout as w1/w2 (tile_weights(w[None])[0]
    when they are tiled); gate_bias: optional fp32 [E] added to the logits."""
    op = "moe_layer_forward"
    T, H = hidden_states.shape
    tiled, G, N2, Hw, w2_shape = _expert_shapes(op, w1, w2)
    I = N2 // 2
    if tiled:
        if gate_weight.dim() != 4 or tuple(gate_weight.shape[2:]) != (64, 8):
            raise RuntimeError(f"{op}: with tiled experts the gate weight must be tiled too")
        E, Hg = gate_weight.shape[0] * 32, gate_weight.shape[1] * 16
    else:
        if gate_weight.dim() != 2:
            raise RuntimeError(f"{op}: gate_weight must be [experts, hidden]")
        E, Hg = gate_weight.shape
    for t, n, dt in ((hidden_states, "hidden_states", torch.bfloat16),
                     (gate_weight, "gate_weight", torch.bfloat16),
                     (w1, "w1", torch.bfloat16), (w2, "w2", torch.bfloat16)):
        if not (t.is_cuda and t.is_contiguous() and t.dtype == dt):
            raise RuntimeError(f"{op}: {n} must be a contiguous CUDA {dt} tensor")
    if gate_bias is not None and not (gate_bias.is_cuda and gate_bias.dtype == torch.float32
                                      and tuple(gate_bias.shape) == (E,)):
        raise RuntimeError(f"{op}: gate_bias must be a CUDA float32 tensor of shape [{E}]")
    if Hg != H or G != E + n_shared_groups or Hw != H or w2_shape != (G, H, I):
        raise RuntimeError(f"{op}: inconsistent shapes x={tuple(hidden_states.shape)} "
                           f"gate={tuple(gate_weight.shape)} w1={tuple(w1.shape)} "
                           f"w2={tuple(w2.shape)}")
    dev = hidden_states.device
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    if T == 0:
        return (out, (None, None, None)) if return_routing else out
    nws = lib.dsk_moe_layer_workspace_size(T, E, top_k, n_shared_groups, H, I)
    ws = workspace if workspace is not None and workspace.numel() >= nws else \
        torch.empty(nws, dtype=torch.uint8, device=dev)
    idx, w, offs = _routing_outputs(return_routing, T, top_k, E, dev)
    bias = gate_bias.contiguous() if gate_bias is not None else None
    with torch.cuda.device(dev):
        check(lib.dsk_moe_layer_forward(
            hidden_states.data_ptr(), gate_weight.data_ptr(), _ptr(bias), w1.data_ptr(),
            w2.data_ptr(), out.data_ptr(), T, E, top_k, n_shared_groups, H, I,
            1 if tiled else 0, _ptr(idx), _ptr(w), _ptr(offs), ws.data_ptr(), ws.numel(),
            _events(stage_events), stream_handle(dev)), op)
    if return_routing:
        return out, (idx, w, offs)
    return out


def gate_logits(hidden_states: torch.Tensor, gate_weight: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 router logits [T, E]: the gate kernel for a bf16 gate weight, else
    torch's fp32 linear (the reference's own formula)."""
    if gate_weight.dtype == torch.bfloat16 and hidden_states.dtype == torch.bfloat16:
        return ops.moe_gate(hidden_states, gate_weight, bias)   # row-major or tiled weight
    logits = F.linear(hidden_states.float(), gate_weight.float(), None)
    return logits + bias if bias is not None else logits


def route_dispatch_combine(hidden_states: torch.Tensor, gate_weight: torch.Tensor,
                           packed_w1: torch.Tensor, w2: torch.Tensor, top_k: int,
                           fuse_swiglu: bool = False) -> torch.Tensor:
    """The reference op sequence (moe_fused.py:118-154) over this package's ops:
    routing -> scan -> dispatch -> gemm1 -> swiglu -> gemm2 -> combine."""
    T = hidden_states.shape[0]
    logits = F.linear(hidden_states.float(), gate_weight.float(), None)
    topk_indices, topk_weights, expert_counts = ops.moe_routing(logits, top_k)
    expert_offsets = ops.moe_scan(expert_counts)
    dispatched, token_map, dispatched_weights = ops.moe_dispatch(
        hidden_states, topk_indices, topk_weights, expert_offsets)
    if fuse_swiglu:
        swiglu_out = ops.moe_gemm1_swiglu(dispatched, packed_w1, expert_offsets)
    else:
        swiglu_out = ops.swiglu(ops.moe_gemm1(dispatched, packed_w1, expert_offsets))
    expert_out = ops.moe_gemm2(swiglu_out, w2, expert_offsets)
    return ops.moe_combine(expert_out, token_map, dispatched_weights, T)


class FusedMoELayer(nn.Module):
    """Drop-in for DeepSeekMoE (moe.py:46-109; reference wrapper
    moe_fused.py:161-216) that runs the fused device pipeline, shared expert
    included. `moe_module` needs .gate.weight, .experts (gate_proj/up_proj/
    down_proj each), .num_experts_per_tok and optionally .shared_experts."""

    def __init__(self, moe_module: nn.Module, device: Optional[torch.device] = None):
        super().__init__()
        if not hasattr(moe_module, "gate") or not hasattr(moe_module, "experts"):
            raise ValueError("FusedMoELayer: moe_module must have 'gate' and 'experts' attributes.")
        dev = device if device is not None else moe_module.gate.weight.device
        self.gate_weight = moe_module.gate.weight.detach().to(dev)
        if self.gate_weight.dtype == torch.bfloat16 and self.gate_weight.shape[0] % 32 == 0:
            # fragment-tiled for the gate kernel (coalesced weight loads)
            self.gate_weight = tile_weights(self.gate_weight[None])[0]
        self.top_k = int(moe_module.num_experts_per_tok)
        self.num_experts = len(moe_module.experts)
        shared = getattr(moe_module, "shared_experts", None)
        self.w1, self.w2, self.n_shared_groups = prepack_with_shared(
            list(moe_module.experts), shared, device=dev)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        assert hidden_states.is_cuda, "hidden_states must be on CUDA."
        assert hidden_states.dtype == torch.bfloat16, "hidden_states must be BF16."
        orig = hidden_states.shape
        x = hidden_states.reshape(-1, orig[-1]).contiguous()
        if self.gate_weight.dtype == torch.bfloat16 and (self.w1.dim() == 5) == (
                self.gate_weight.dim() == 4):
            out = moe_layer_forward(x, self.gate_weight, self.w1, self.w2, self.top_k,
                                    self.n_shared_groups)   # gate + layer, one call
        else:
            logits = gate_logits(x, self.gate_weight)
            out = moe_fused_forward_logits(logits, x, self.w1, self.w2, self.top_k,
                                           self.n_shared_groups, self.num_experts)
        return out.view(orig)


# id(experts) -> (w1, w2) packed on first use, as the reference caches
# (moe_fused.py:224); held fragment-tiled, the layout the layer kernels stream
# fastest (the reference layout [E, 2I, H] / [E, H, I] is what prepack_experts
# returns and what explicitly passed packed_w1 / w2 keep)
_WEIGHT_CACHE: dict = {}


def fused_moe_forward(hidden_states: torch.Tensor, gate_weight: torch.Tensor, experts: list,
                      top_k: int = 6, packed_w1: Optional[torch.Tensor] = None,
                      w2: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Functional form (moe_fused.py:227-272): routed experts only, like the
    reference; weights are packed on first use and cached by id(experts).
    packed_w1 / w2, when given, may be in the reference layout (prepack_experts)
    or fragment-tiled (tile_weights of it); the cached pack is tiled. Both
    layouts give the same bits."""
    assert hidden_states.is_cuda, "hidden_states must be on CUDA."
    assert hidden_states.dim() == 2, "hidden_states must be [num_tokens, hidden_size]."
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be BF16."
    if packed_w1 is None or w2 is None:
        key = id(experts)
        if key not in _WEIGHT_CACHE:
            rw1, rw2 = prepack_experts(experts)
            _WEIGHT_CACHE[key] = (tile_weights(rw1), tile_weights(rw2))
            del rw1, rw2
        packed_w1, w2 = _WEIGHT_CACHE[key]
    logits = gate_logits(hidden_states.contiguous(), gate_weight)
    return moe_fused_forward_logits(logits, hidden_states.contiguous(), packed_w1, w2, top_k, 0,
                                    packed_w1.shape[0])

"""numpy restatement of the reference MoE layer (TEST INFRASTRUCTURE ONLY).

References (sahan974/DeepSeek-V2-Lite-CUDA):
  src/reference/moe.py:6-19    ExpertMLP: down(silu(gate x) * up x)
  src/reference/moe.py:33-43   MoEGate: fp32 logits, softmax, top-k, no renormalisation
  src/reference/moe.py:77-109  DeepSeekMoE.forward: per-expert loop, ascending tokens,
                               accumulation in expert order, then shared experts
  src/kernels/moe/routing.cu:139-198  top-k emitted in descending order
  src/kernels/moe/scan.cu:104-127     offsets[E+1] with the total as sentinel
  src/kernels/moe/dispatch.cu:76-100  slot rows, token_map, dispatched weights
  src/kernels/moe/gemm1.cu:105-154, gemm2.cu:94-123  per-expert X @ W^T, zeros elsewhere
  src/kernels/moe/swiglu.cu:50-52     silu(x) = x / (1 + exp(-x))
  src/kernels/moe/combine.cu:57-60    out[token_map[s]] += y[s] * w[s]
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    u = np.asarray(a, dtype=f32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(f32)


def gate_logits(x: np.ndarray, wg: np.ndarray) -> np.ndarray:
    """moe.py:35 / moe_fused.py:131: F.linear(x.float(), W.float())."""
    return np.asarray(x, f32) @ np.asarray(wg, f32).T


def softmax(logits: np.ndarray) -> np.ndarray:
    """moe.py:36 (fp32, max-subtracted)."""
    l = np.asarray(logits, f32)
    e = np.exp(l - l.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(f32)


def route(logits: np.ndarray, top_k: int):
    """moe.py:33-43 with the canonical order of routing.cu:139-198.

    Selection ranks the fp32 logits (softmax is monotone) in descending order,
    ties to the lower expert index (a stable sort of -logits); weights are the
    softmax probabilities of the winners, not renormalised.
    Returns (idx int32 [T,K], w fp32 [T,K], counts int32 [E])."""
    l = np.asarray(logits, f32)
    T, E = l.shape
    order = np.argsort(-l, axis=1, kind="stable")
    idx = order[:, :top_k].astype(np.int32)
    w = np.take_along_axis(softmax(l), idx, axis=1).astype(f32)
    counts = np.bincount(idx.ravel(), minlength=E).astype(np.int32) if T else np.zeros(E, np.int32)
    return idx, w, counts


def scan(counts: np.ndarray) -> np.ndarray:
    """scan.cu:104-127: exclusive prefix sum, offsets[E] = total."""
    c = np.asarray(counts, np.int64)
    out = np.zeros(c.shape[0] + 1, np.int64)
    for e in range(c.shape[0]):
        out[e + 1] = out[e] + c[e]
    return out.astype(np.int32)


def permute(idx: np.ndarray, w: np.ndarray, offsets: np.ndarray, num_experts: int):
    """Slot order of the oracle loop (moe.py:90-95): for expert e, the tokens
    routed to it in ascending order fill [offsets[e], offsets[e+1]).
    Returns (token_map int32 [S], dispatched_weights fp32 [S], slot_of int32 [T,K])."""
    idx = np.asarray(idx)
    T, K = idx.shape
    S = T * K
    token_map = np.full(S, -1, np.int32)
    dw = np.zeros(S, f32)
    slot_of = np.full((T, K), -1, np.int32)
    for e in range(num_experts):
        rows, ks = np.nonzero(idx == e)  # row-major: ascending token
        base = int(offsets[e])
        for j, (t, k) in enumerate(zip(rows, ks)):
            s = base + j
            token_map[s] = t
            dw[s] = w[t, k]
            slot_of[t, k] = s
    return token_map, dw, slot_of


def dispatch(x: np.ndarray, idx: np.ndarray, w: np.ndarray, offsets: np.ndarray,
             num_experts: int):
    """dispatch.cu:76-100 with the stable slot order of permute()."""
    token_map, dw, _ = permute(idx, w, offsets, num_experts)
    x = np.asarray(x)
    dispatched = np.zeros((token_map.shape[0], x.shape[1]), x.dtype)
    ok = token_map >= 0
    dispatched[ok] = x[token_map[ok]]
    return dispatched, token_map, dw


def grouped_linear(a: np.ndarray, w: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    """gemm1.cu:105-154 / gemm2.cu:94-123: out[s] = a[s] @ w[e]^T for s in
    [offsets[e], offsets[e+1]); other rows 0. fp32 accumulation."""
    a = np.asarray(a, f32)
    S = a.shape[0]
    out = np.zeros((S, w.shape[1]), f32)
    for e in range(w.shape[0]):
        s0, s1 = int(offsets[e]), int(offsets[e + 1])
        if s1 > s0:
            out[s0:s1] = a[s0:s1] @ np.asarray(w[e], f32).T
    return out


def silu(x: np.ndarray) -> np.ndarray:
    """swiglu.cu:50-52."""
    x = np.asarray(x, f32)
    return (x / (f32(1) + np.exp(-x))).astype(f32)


def swiglu(gu: np.ndarray) -> np.ndarray:
    """swiglu.cu:86-105: silu(gu[:, :I]) * gu[:, I:]."""
    gu = np.asarray(gu, f32)
    I = gu.shape[1] // 2
    return (silu(gu[:, :I]) * gu[:, I:]).astype(f32)


def combine(y: np.ndarray, token_map: np.ndarray, dw: np.ndarray, num_tokens: int) -> np.ndarray:
    """combine.cu:57-60 in fixed order: for each token, its slots in ascending
    slot order, w * y accumulated in fp32."""
    y = np.asarray(y, f32)
    out = np.zeros((num_tokens, y.shape[1]), f32)
    for s in np.argsort(token_map, kind="stable"):  # groups by token, ascending s inside
        t = int(token_map[s])
        if 0 <= t < num_tokens:
            out[t] += f32(dw[s]) * y[s]
    return out


def expert_mlp(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """moe.py:18-19."""
    x = np.asarray(x, f32)
    h = silu(x @ np.asarray(gate, f32).T) * (x @ np.asarray(up, f32).T)
    return (h @ np.asarray(down, f32).T).astype(f32)


def moe_layer(x: np.ndarray, wg: np.ndarray, gates, ups, downs, top_k: int,
              shared=None, logits: np.ndarray | None = None) -> np.ndarray:
    """DeepSeekMoE.forward (moe.py:77-109), fp32.

    gates/ups/downs: per-expert [I,H], [I,H], [H,I] (sequences or stacked arrays);
    shared: optional (gate [nI,H], up [nI,H], down [H,nI]). If `logits` is given
    it replaces x @ wg^T (used when the harness biases the router logits)."""
    x = np.asarray(x, f32)
    if logits is None:
        logits = gate_logits(x, wg)
    idx, w, _ = route(logits, top_k)
    out = np.zeros_like(x)
    for e in range(len(gates)):
        mask = idx == e
        if not mask.any():
            continue
        tok = np.nonzero(mask.any(axis=1))[0]                       # moe.py:95
        we = w[tok][mask[tok]][:, None]                             # moe.py:98-99
        out[tok] += expert_mlp(x[tok], gates[e], ups[e], downs[e]) * we  # moe.py:102-103
    if shared is not None:
        out += expert_mlp(x, *shared)                               # moe.py:106-107
    return out

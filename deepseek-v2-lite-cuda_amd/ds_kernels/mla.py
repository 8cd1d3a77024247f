"""DeepSeek-V2-Lite MLA projection block and decoder layer composed from this
package's kernels (reference: src/reference/mla.py:251-393 DeepSeekMLA,
src/reference/decoder_layer.py:108-139 DeepSeekDecoderLayer).

Kernels used: `linear` (MFMA GEMM, weights prepacked in the fragment-tiled
layout) for q_proj, kv_a_proj_with_mqa and o_proj, `rms_norm` straight on the
512-wide latent slice of the 576-wide kv_a output (row-strided, no copy),
`kv_upproj`, `rope` on strided q_pe / k_pe views with the position tables
broadcast over the batch (no materialised copies), and the fused MoE layer
(`moe_layer_forward`). In the causal attention core the two batched products
stay torch (the attention core is outside the kernel scope); the scale, causal mask, fp32 softmax and
bf16 rounding between them are one pass of `attn_softmax_`, at the reference's
precision.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import ops
from .expert_prepack import pack_tensors, tile_weights
from .moe_fused import moe_layer_forward


# ------------------------------------------------------------- YaRN tables --
def _yarn_correction_dim(num_rotations: float, dim: int, base: float, max_pos: int) -> float:
    return (dim * math.log(max_pos / (num_rotations * 2 * math.pi))) / (2 * math.log(base))


def _yarn_mscale(scale: float, mscale: float) -> float:
    return 1.0 if scale <= 1 else 0.1 * mscale * math.log(scale) + 1.0


def yarn_cos_sin(seq_len: int, dim: int = 64, base: float = 10000.0, factor: float = 40.0,
                 original_max_position: int = 4096, beta_fast: int = 32, beta_slow: int = 1,
                 mscale: float = 0.707, mscale_all_dim: float = 0.707,
                 device: Optional[torch.device] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq_len, dim] fp32 of YaRNRotaryEmbedding (mla.py:108-165):
    inv_freq blends base^(-2i/d) and base^(-2i/d)/factor over the linear ramp
    between the correction dims of beta_fast and beta_slow; emb = cat(freqs,
    freqs); the tables are scaled by mscale(factor, mscale)/mscale(factor, all)."""
    pos = torch.arange(0, dim, 2, dtype=torch.float32) / dim
    extra = 1.0 / (base ** pos)
    inter = 1.0 / (factor * base ** pos)
    lo = max(math.floor(_yarn_correction_dim(beta_fast, dim, base, original_max_position)), 0)
    hi = min(math.ceil(_yarn_correction_dim(beta_slow, dim, base, original_max_position)),
             dim - 1)
    if lo == hi:
        hi += 0.001
    ramp = ((torch.arange(dim // 2, dtype=torch.float32) - lo) / (hi - lo)).clamp(0, 1)
    keep = 1.0 - ramp
    inv_freq = inter * (1.0 - keep) + extra * keep
    m = _yarn_mscale(factor, mscale) / _yarn_mscale(factor, mscale_all_dim)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos() * m, emb.sin() * m
    if device is not None:
        cos, sin = cos.to(device), sin.to(device)
    return cos, sin


# ----------------------------------------------------------------- weights --
@dataclass
class MLAWeights:
    """bf16 projection weights ([out, in], nn.Linear order, or that matrix in the
    fragment-tiled layout [out/32, in/16, 64, 8]) and the fp32 latent norm."""
    q: torch.Tensor          # [heads*(nope+rope), H]
    kva: torch.Tensor        # [kv_lora+rope, H]
    kva_norm: torch.Tensor   # [kv_lora] fp32
    kvb: torch.Tensor        # [heads*(nope+v), kv_lora]
    o: torch.Tensor          # [H, heads*v]
    # optional [q rows; kva rows] in one matrix (q and kva then view into it),
    # so that the prefill projections run as one GEMM launch
    q_kva: Optional[torch.Tensor] = None
    # optional kv_b weight with the latent norm weight folded into its input
    # columns (tiled), for the RMSNorm carried by the projection epilogues
    kvb_w: Optional[torch.Tensor] = None
    n_heads: int = 16
    nope: int = 128
    rope_dim: int = 64
    v_dim: int = 128
    kv_lora: int = 512
    factor: float = 40.0     # YaRN scaling factor of DeepSeek-V2-Lite

    @staticmethod
    def from_tensors(w: dict, device: torch.device, tiled: bool = True) -> "MLAWeights":
        """tiled: prepack the four projections once into the fragment-tiled
        layout, which the projection GEMMs stream straight into registers."""
        def bf(t):
            t = t.to(device=device, dtype=torch.bfloat16).contiguous()
            return tile_weights(t[None])[0] if tiled else t
        # q and kva share one matrix: the tiled layout keeps 32-row blocks in
        # order along its first dimension, so both are leading-dim slices of it
        nq = w["q"].shape[0]
        q_kva = bf(torch.cat([w["q"], w["kva"]]))
        split = nq // 32 if tiled else nq
        norm = w["kva_norm"].to(torch.float32)
        # kv_b(w * xhat) = (kv_b * w) xhat: the norm weight scales kv_b's input
        # columns (rounded to bf16 once)
        kvb_w = bf(w["kvb"].to(torch.float32) * norm[None, :]) if tiled else None
        return MLAWeights(q=q_kva[:split], kva=q_kva[split:],
                          kva_norm=norm.to(device=device),
                          kvb=bf(w["kvb"]), o=bf(w["o"]), q_kva=q_kva, kvb_w=kvb_w)

    @property
    def softmax_scale(self) -> float:
        """mla.py:287-288: (nope + rope)^-0.5 * mscale(factor, 0.707)^2."""
        m = _yarn_mscale(self.factor, 0.707)
        return (self.nope + self.rope_dim) ** -0.5 * m * m


# ------------------------------------------------------------- projections --
def _projection_rows(x: torch.Tensor, W: MLAWeights, eps: float, with_latent: bool):
    """q_proj, kv_a_proj and kv_b_proj (mla.py:318-346) as token rows: q [b, s,
    h*(nope+rope)], kv [b, s, h*(nope+v)], kva [b, s, kv_lora+rope] (column
    slices of the projection outputs, no copies) and the normalised latent (None
    unless with_latent or needed by the unfused path)."""
    h, nope, r, lora = W.n_heads, W.nope, W.rope_dim, W.kv_lora
    nq = h * (nope + r)
    fused_norm = W.q_kva is not None and W.kvb_w is not None and nq % 256 == 0 and lora % 256 == 0
    if fused_norm:
        y, ss = ops.linear_rowsq(x, W.q_kva, nq, nq + lora)            # [b,s,3072+576], [2, b*s]
        q, kva = y[..., :nq], y[..., nq:]
    elif W.q_kva is not None:
        # one GEMM for both projections (q_proj alone leaves no partial round of
        # tiles for kv_a's 576 columns to fill); q and kva are column slices
        y = ops.linear(x, W.q_kva)                                     # [b,s,3072+576]
        q, kva = y[..., :nq], y[..., nq:]
    else:
        q, kva = ops.linear(x, W.q), ops.linear(x, W.kva)
    if fused_norm:
        kv = ops.linear_rowscale(kva[..., :lora], W.kvb_w, ss, lora, eps)
        latent = ops.rms_norm(kva[..., :lora], W.kva_norm, eps) if with_latent else None
    else:
        latent = ops.rms_norm(kva[..., :lora], W.kva_norm, eps)        # strided rows, no copy
        kv = ops.kv_upproj(latent, W.kvb)
    return q, kv, kva, latent


def mla_projections(x: torch.Tensor, W: MLAWeights, cos: torch.Tensor, sin: torch.Tensor,
                    eps: float = 1e-6, with_latent: bool = True):
    """The projection block of DeepSeekMLA.forward (mla.py:318-352, BASELINE
    config 3). x: bf16 [b, s, H]; cos/sin: [>= s, rope_dim] for positions 0..s-1,
    or [b, s, rope_dim] per batch entry (tables indexed by position_ids).
    Returns (q_nope [b,h,s,nope], q_rot [b,h,s,r], k_nope [b,h,s,nope],
    v [b,h,s,v], k_rot [b,1,s,r], latent_normed [b,s,kv_lora]); q_nope, k_nope
    and v are strided views of the projection outputs.

    With the merged q/kv_a weight and the folded kv_b weight (MLAWeights.from_tensors
    with tiled weights), the latent RMSNorm rides the projections' epilogues: the
    q/kv_a GEMM also returns each row's sum of squares over the 512 latent
    columns, and kv_b runs on the raw latent with the row scale applied to its
    outputs, so the normalised latent is never materialised. latent_normed
    (the reference module's intermediate, not an output of the block) is then
    computed by the rms_norm kernel only if with_latent; otherwise it is None."""
    b, s, _ = x.shape
    h, nope, r, vd, lora = W.n_heads, W.nope, W.rope_dim, W.v_dim, W.kv_lora
    q, kv, kva, latent = _projection_rows(x, W, eps, with_latent)
    q = q.view(b, s, h, nope + r).transpose(1, 2)                      # [b,h,s,192] view
    kv = kv.view(b, s, h, nope + vd).transpose(1, 2)
    k_pe = kva[..., lora:].view(b, s, 1, r).transpose(1, 2)           # [b,1,s,64] view
    if cos.dim() == 3:        # per batch entry (tables indexed by position_ids)
        cb = cos.to(torch.bfloat16)[:, None, :s]
        sb = sin.to(torch.bfloat16)[:, None, :s]
    else:                     # shared by the batch: batch stride 0
        cb = cos[:s].to(torch.bfloat16)[None, None].expand(b, 1, s, r)
        sb = sin[:s].to(torch.bfloat16)[None, None].expand(b, 1, s, r)
    q_rot, k_rot = ops.rope(q[..., nope:], k_pe, cb, sb)
    return q[..., :nope], q_rot, kv[..., :nope], kv[..., nope:], k_rot, latent


def rope_tables_for(cos: torch.Tensor, sin: torch.Tensor, s: int,
                    position_ids: Optional[torch.Tensor]):
    """The tables apply_rotary_pos_emb uses (mla.py:186-187, 349-351): the
    module's cos/sin cut to the sequence length, indexed by position_ids
    [b, s] when given -> bf16 [s, d] (shared by the batch) or [b, s, d].
    position_ids index the first s rows, as `cos[:q_len][position_ids]` does
    in the reference; an index outside them raises IndexError here (torch
    raises it there)."""
    cs, sn = cos[:s].to(torch.bfloat16), sin[:s].to(torch.bfloat16)
    if position_ids is None:
        return cs, sn
    pid = position_ids.to(device=cos.device, dtype=torch.long)
    ops._req(pid.dim() == 2 and pid.shape[1] == s,
             f"position_ids must be [bsz, {s}], got {tuple(position_ids.shape)}.")
    if pid.numel() and bool(((pid < -s) | (pid >= s)).any()):
        raise IndexError(f"position_ids must index the {s} table rows (positions -{s}..{s - 1}).")
    return cs[pid].contiguous(), sn[pid].contiguous()


def mla_forward(x: torch.Tensor, W: MLAWeights, cos: torch.Tensor, sin: torch.Tensor,
                eps: float = 1e-6, attention_mask: Optional[torch.Tensor] = None,
                position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """DeepSeekMLA.forward (mla.py:295-393): projections on this package's
    kernels, o_proj on the MFMA GEMM, and the attention core at the
    reference's precision (mla.py:366-384): bf16 Q.K^T and .V in torch
    (right-hand operands contiguous), the scale, mask, fp32 softmax and bf16
    rounding in one pass of attn_softmax_.
    x: bf16 [b, s, H] -> bf16 [b, s, H], any s >= 1. cos/sin: the YaRN tables
    for positions 0.. (at least s rows). attention_mask: additive [b, 1, s, s]
    (bf16 or fp32, -inf where masked; anything broadcastable to it) used instead
    of the causal mask, as in the reference; position_ids: [b, s] rows of the
    tables for each token (default 0..s-1). With s % 8 != 0 the key dimension of
    K^T, the scores and V is padded to a multiple of 8 with zeros."""
    b, s, H = x.shape
    h, nope, r = W.n_heads, W.nope, W.rope_dim
    cs, sn = rope_tables_for(cos, sin, s, position_ids)
    sp = (s + 7) // 8 * 8
    if (nope, r, W.v_dim) == (128, 64, 128):
        # Q, K^T and V packed head-major in one pass from the projection rows
        # (RoPE of q_pe and k_pe included); other head dims assemble them by copies
        qr, kv, kva, _ = _projection_rows(x, W, eps, with_latent=False)
        q, kT, v = ops.mla_attn_pack(qr, kv, kva[..., W.kv_lora:], cs, sn, heads=h, pad=True)
    else:
        q, kT, v = _assemble_attention_operands(x, W, cs, sn, eps, sp)
    scores = torch.matmul(q, kT)                                       # bf16 [b,h,s,sp]
    p = ops.attn_softmax_(scores, W.softmax_scale, causal=attention_mask is None, kv_len=s,
                          mask=attention_mask)
    o = torch.matmul(p, v)                                             # [b,h,s,v]
    o = o.transpose(1, 2).reshape(b, s, W.n_heads * W.v_dim)
    return ops.linear(o, W.o)


def _assemble_attention_operands(x, W: MLAWeights, cs, sn, eps, sp):
    """Q [b,h,s,nope+r], K^T [b,h,nope+r,sp] and V [b,h,sp,v] by copies, for head
    dims the pack kernel does not take; K^T columns and V rows past s are zero."""
    b, s, _ = x.shape
    h, nope, r = W.n_heads, W.nope, W.rope_dim
    q_nope, q_rot, k_nope, v, k_rot, _ = mla_projections(x, W, cs, sn, eps, with_latent=False)
    q = torch.cat([q_nope, q_rot], dim=-1)                             # [b,h,s,192]
    kT = torch.zeros((b, h, nope + r, sp), dtype=torch.bfloat16, device=x.device)
    kT[:, :, :nope, :s].copy_(k_nope.transpose(-1, -2))
    kT[:, :, nope:, :s].copy_(k_rot.transpose(-1, -2).expand(b, h, r, s))
    vp = torch.zeros((b, h, sp, W.v_dim), dtype=torch.bfloat16, device=x.device)
    vp[:, :, :s].copy_(v)
    return q, kT, vp


# ------------------------------------------------------------ decoder layer --
@dataclass
class DecoderLayerWeights:
    mla: MLAWeights
    in_norm: torch.Tensor      # [H] fp32
    post_norm: torch.Tensor    # [H] fp32
    gate: torch.Tensor         # tiled bf16 router weight
    w1: torch.Tensor           # tiled [G, 2I/32, H/16, 64, 8]
    w2: torch.Tensor           # tiled [G, H/32, I/16, 64, 8]
    n_shared_groups: int
    top_k: int = 6

    @staticmethod
    def from_tensors(mla_w: dict, moe_w, device: torch.device,
                     in_norm: Optional[torch.Tensor] = None,
                     post_norm: Optional[torch.Tensor] = None) -> "DecoderLayerWeights":
        """mla_w: synthetic.mla_weights() layout; moe_w: synthetic.moe_weights()."""
        H = moe_w.wg.shape[1]
        w1, w2, nsh = pack_tensors(moe_w.gates, moe_w.ups, moe_w.downs, device=device,
                                   shared=moe_w.shared)
        gate = tile_weights(moe_w.wg.to(torch.bfloat16)[None])[0].to(device)
        ones = torch.ones(H, dtype=torch.float32)
        return DecoderLayerWeights(
            mla=MLAWeights.from_tensors(mla_w, device),
            in_norm=(in_norm if in_norm is not None else ones).to(device, torch.float32),
            post_norm=(post_norm if post_norm is not None else ones).to(device, torch.float32),
            gate=gate, w1=tile_weights(w1), w2=tile_weights(w2), n_shared_groups=nsh)


def decoder_layer_forward(x: torch.Tensor, P: DecoderLayerWeights, cos: torch.Tensor,
                          sin: torch.Tensor, eps: float = 1e-6,
                          attention_mask: Optional[torch.Tensor] = None,
                          position_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """DeepSeekDecoderLayer.forward (decoder_layer.py:108-139), BASELINE config 4:
    RMSNorm -> MLA -> residual -> RMSNorm -> MoE (routed + shared) -> residual.
    x: bf16 [b, s, H]; attention_mask / position_ids as in mla_forward (causal
    and positions 0..s-1 by default)."""
    b, s, H = x.shape
    h = ops.rms_norm(x, P.in_norm, eps)
    x = x + mla_forward(h, P.mla, cos, sin, eps, attention_mask=attention_mask,
                        position_ids=position_ids)
    h = ops.rms_norm(x, P.post_norm, eps)
    m = moe_layer_forward(h.reshape(-1, H), P.gate, P.w1, P.w2, P.top_k, P.n_shared_groups)
    return x + m.view(b, s, H)

"""numpy restatement of the reference MLA helpers and decoder layer
(TEST INFRASTRUCTURE ONLY).

References (sahan974/DeepSeek-V2-Lite-CUDA):
  src/reference/mla.py:53-64    RMSNorm (fp32 math, x_hat rounded to the input dtype, * w)
  src/reference/mla.py:70-96    YaRN helpers (correction dim/range, mscale, ramp mask)
  src/reference/mla.py:108-165  YaRN tables: inv_freq blend, emb = cat(freqs, freqs), cos/sin * mscale
  src/reference/mla.py:176-206  rotate_half + deinterleave + (x*cos) + (rotate_half(x)*sin)
  src/reference/mla.py:295-393  DeepSeekMLA.forward (eager attention; causal or an additive
                                attention_mask; position_ids index the RoPE tables)
  src/reference/decoder_layer.py:108-139  pre-norm -> MLA -> residual -> pre-norm -> MoE -> residual
"""
from __future__ import annotations

import math

import numpy as np

from .moe import bf16_round, moe_layer

f32 = np.float32


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, round_bf16: bool = False) -> np.ndarray:
    """mla.py:59-64: x * rsqrt(mean(x^2) + eps), optionally rounded to bf16 (the
    module's `.to(input_dtype)` for bf16 inputs), then * w."""
    x = np.asarray(x, f32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=f32)
    xh = (x * (f32(1) / np.sqrt(var + f32(eps)))).astype(f32)
    if round_bf16:
        xh = bf16_round(xh)
    return (np.asarray(w, f32) * xh).astype(f32)


def yarn_find_correction_dim(num_rotations, dim, base=10000, max_pos=2048):
    """mla.py:70-73."""
    return (dim * math.log(max_pos / (num_rotations * 2 * math.pi))) / (2 * math.log(base))


def yarn_find_correction_range(low_rot, high_rot, dim, base=10000, max_pos=2048):
    """mla.py:75-78."""
    low = math.floor(yarn_find_correction_dim(low_rot, dim, base, max_pos))
    high = math.ceil(yarn_find_correction_dim(high_rot, dim, base, max_pos))
    return max(low, 0), min(high, dim - 1)


def yarn_get_mscale(scale: float = 1.0, mscale: float = 1.0) -> float:
    """mla.py:80-83."""
    if scale <= 1:
        return 1.0
    return 0.1 * mscale * math.log(scale) + 1.0


def yarn_linear_ramp_mask(lo, hi, n):
    """mla.py:85-89."""
    if lo == hi:
        hi += 0.001
    r = (np.arange(n, dtype=f32) - f32(lo)) / f32(hi - lo)
    return np.clip(r, 0, 1).astype(f32)


def yarn_inv_freq(dim=64, base=10000.0, factor=40.0, orig_max=4096, beta_fast=32, beta_slow=1):
    """mla.py:137-155: blend of extrapolated (base^-2i/d) and interpolated
    (base^-2i/d / factor) frequencies over the correction ramp."""
    pos = np.arange(0, dim, 2, dtype=f32) / f32(dim)
    freq_extra = (f32(1) / (f32(base) ** pos)).astype(f32)
    freq_inter = (f32(1) / (f32(factor) * f32(base) ** pos)).astype(f32)
    lo, hi = yarn_find_correction_range(beta_fast, beta_slow, dim, base, orig_max)
    mask = f32(1) - yarn_linear_ramp_mask(lo, hi, dim // 2)
    return (freq_inter * (f32(1) - mask) + freq_extra * mask).astype(f32)


def yarn_cos_sin(seq_len, dim=64, base=10000.0, factor=40.0, orig_max=4096, beta_fast=32,
                 beta_slow=1, mscale=0.707, mscale_all_dim=0.707):
    """mla.py:157-165: cos/sin [seq_len, dim] = cos/sin(cat(freqs, freqs)) * m,
    with m = mscale(factor, mscale) / mscale(factor, mscale_all_dim)."""
    inv = yarn_inv_freq(dim, base, factor, orig_max, beta_fast, beta_slow)
    m = float(yarn_get_mscale(factor, mscale) / yarn_get_mscale(factor, mscale_all_dim))
    t = np.arange(seq_len, dtype=f32)
    freqs = np.outer(t, inv).astype(f32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return (np.cos(emb) * f32(m)).astype(f32), (np.sin(emb) * f32(m)).astype(f32)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """mla.py:176-180."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """mla.py:196-205 for one tensor x [..., d] with cos/sin broadcastable to it:
    deinterleave (pairs (2k, 2k+1) -> k, k+d/2), then x*cos + rotate_half(x)*sin."""
    x = np.asarray(x, f32)
    d = x.shape[-1]
    xd = np.concatenate([x[..., 0::2], x[..., 1::2]], axis=-1)
    return (xd * cos + rotate_half(xd) * sin).astype(f32)


def linear(x, w):
    return (np.asarray(x, f32) @ np.asarray(w, f32).T).astype(f32)


def mla_projections(x, w_q, w_kva, w_kva_norm, w_kvb, cos, sin, n_heads=16, nope=128,
                    rope_dim=64, v_dim=128, kv_lora=512, eps=1e-6):
    """mla.py:318-352: the projection block of config 3.

    x [b, s, H]; cos/sin [s, rope_dim] (positions 0..s-1).
    Returns q_nope [b,h,s,nope], q_rot [b,h,s,r], k_nope [b,h,s,nope],
    v [b,h,s,v], k_rot [b,1,s,r], latent_normed [b,s,kv_lora]."""
    b, s, _ = x.shape
    q = linear(x, w_q).reshape(b, s, n_heads, nope + rope_dim).transpose(0, 2, 1, 3)
    q_nope, q_pe = q[..., :nope], q[..., nope:]
    kv_a = linear(x, w_kva)
    latent, k_pe = kv_a[..., :kv_lora], kv_a[..., kv_lora:]
    k_pe = k_pe.reshape(b, s, 1, rope_dim).transpose(0, 2, 1, 3)
    ln = rms_norm(latent, w_kva_norm, eps)
    kv = linear(ln, w_kvb).reshape(b, s, n_heads, nope + v_dim).transpose(0, 2, 1, 3)
    k_nope, v = kv[..., :nope], kv[..., nope:]
    c = cos[None, None]
    sn = sin[None, None]
    return q_nope, rope(q_pe, c, sn), k_nope, v, rope(k_pe, c, sn), ln


def attention(q, k, v, scale, mask=None):
    """mla.py:356-384: softmax(q k^T * scale + mask) v in fp32, per (batch, head)
    to bound memory. mask None: the causal mask (mla.py:368-373); otherwise the
    additive attention_mask broadcast to [b, h, s, s] (mla.py:374-375)."""
    b, h, s = q.shape[0], q.shape[1], q.shape[-2]
    causal = np.triu(np.ones((s, s), bool), k=1) if mask is None else None
    mk = None if mask is None else np.broadcast_to(np.asarray(mask, f32), (b, h, s, k.shape[-2]))
    out = np.empty(q.shape[:-1] + (v.shape[-1],), f32)
    for bi in range(b):
        for hi in range(h):
            kk = k[bi, hi if k.shape[1] > 1 else 0]
            sc = (q[bi, hi] @ kk.T).astype(f32) * f32(scale)
            sc = np.where(causal, -np.inf, sc) if mk is None else sc + mk[bi, hi]
            sc = sc - sc.max(axis=-1, keepdims=True)
            p = np.exp(sc)
            p = p / p.sum(axis=-1, keepdims=True)
            out[bi, hi] = p @ v[bi, hi if v.shape[1] > 1 else 0]
    return out


def tables_at(cos, sin, position_ids):
    """mla.py:186-187: cos[position_ids], sin[position_ids] -> [b, 1, s, d] (or the
    [1, 1, s, d] tables for positions 0..s-1 when position_ids is None)."""
    if position_ids is None:
        return cos[None, None], sin[None, None]
    pid = np.asarray(position_ids)
    return cos[pid][:, None], sin[pid][:, None]


def mla_forward(x, w_q, w_kva, w_kva_norm, w_kvb, w_o, n_heads=16, nope=128, rope_dim=64,
                v_dim=128, kv_lora=512, eps=1e-6, factor=40.0, attention_mask=None,
                position_ids=None):
    """DeepSeekMLA.forward (mla.py:295-393), fp32. position_ids [b, s] index the
    tables of the first s positions (default 0..s-1, mla.py:310-312);
    attention_mask: additive [b, 1, s, s] replacing the causal mask."""
    b, s, _ = x.shape
    cos, sin = yarn_cos_sin(s, rope_dim, factor=factor)
    c, sn = tables_at(cos, sin, position_ids)
    q = linear(x, w_q).reshape(b, s, n_heads, nope + rope_dim).transpose(0, 2, 1, 3)
    kv_a = linear(x, w_kva)
    k_pe = kv_a[..., kv_lora:].reshape(b, s, 1, rope_dim).transpose(0, 2, 1, 3)
    ln = rms_norm(kv_a[..., :kv_lora], w_kva_norm, eps)
    kv = linear(ln, w_kvb).reshape(b, s, n_heads, nope + v_dim).transpose(0, 2, 1, 3)
    q_rot, k_rot = rope(q[..., nope:], c, sn), rope(k_pe, c, sn)
    qf = np.concatenate([q[..., :nope], q_rot], axis=-1)
    k = np.concatenate([kv[..., :nope], np.broadcast_to(k_rot, (b, n_heads, s, rope_dim))],
                       axis=-1)
    m = yarn_get_mscale(factor, 0.707)
    scale = (nope + rope_dim) ** -0.5 * m * m                      # mla.py:287-288
    o = attention(qf, k, kv[..., nope:], scale, attention_mask)
    o = o.transpose(0, 2, 1, 3).reshape(b, s, n_heads * v_dim)
    return linear(o, w_o)


def decoder_layer(x, p: dict, top_k=6, eps=1e-6, attention_mask=None, position_ids=None):
    """DeepSeekDecoderLayer.forward (decoder_layer.py:108-139), fp32.
    p: dict with in_norm, q, kva, kva_norm, kvb, o, post_norm, wg, gates, ups,
    downs, shared (tuple or None)."""
    h = rms_norm(x, p["in_norm"], eps)
    h = mla_forward(h, p["q"], p["kva"], p["kva_norm"], p["kvb"], p["o"], eps=eps,
                    attention_mask=attention_mask, position_ids=position_ids)
    x = x + h
    h = rms_norm(x, p["post_norm"], eps)
    b, s, H = h.shape
    m = moe_layer(h.reshape(-1, H), p["wg"], p["gates"], p["ups"], p["downs"], top_k,
                  shared=p.get("shared")).reshape(b, s, H)
    return (x + m).astype(f32)

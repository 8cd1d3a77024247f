"""Pins the numpy MLA oracle (CPU only): library routines, closed forms of the
YaRN bands, complex-number RoPE, and torch SDPA for the attention core."""
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import mla as ol


def test_rms_norm_matches_torch():
    x = np.random.default_rng(0).standard_normal((33, 512)).astype(np.float32) * 3
    w = np.random.default_rng(1).uniform(0.5, 1.5, 512).astype(np.float32)
    ref = F.rms_norm(torch.from_numpy(x), (512,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(ol.rms_norm(x, w, 1e-6), ref, rtol=1e-5, atol=1e-6)


def test_rms_norm_bf16_rounding_point():
    x = np.random.default_rng(2).standard_normal((4, 64)).astype(np.float32)
    w = np.full(64, 3.0, np.float32)
    xt = torch.from_numpy(x)
    xh = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).float()
    np.testing.assert_allclose(ol.rms_norm(x, w, 1e-6, round_bf16=True), 3.0 * xh.numpy(),
                               rtol=1e-6, atol=1e-6)


def test_yarn_correction_range_and_bands():
    lo, hi = ol.yarn_find_correction_range(32, 1, 64, 10000, 4096)
    assert (lo, hi) == (10, 23)
    inv = ol.yarn_inv_freq(64, 10000.0, 40.0, 4096, 32, 1)
    i = np.arange(32)
    extra = 1.0 / 10000.0 ** (2 * i / 64)
    # below the ramp: pure extrapolation; above it: interpolation by the factor
    np.testing.assert_allclose(inv[:lo + 1], extra[:lo + 1], rtol=1e-6)
    np.testing.assert_allclose(inv[hi:], extra[hi:] / 40.0, rtol=1e-6)
    # inside the ramp the value lies strictly between the two
    mid = slice(lo + 1, hi)
    assert np.all(inv[mid] < extra[mid]) and np.all(inv[mid] > extra[mid] / 40.0)
    assert ol.yarn_get_mscale(40, 0.707) / ol.yarn_get_mscale(40, 0.707) == 1.0


def test_yarn_ramp_interior_is_linear():
    """Inside the correction range the YaRN blend (mla.py:85-91,137-155) moves
    linearly from extrapolation to interpolation: with the blend weight
    t_i = (extra_i - inv_i) / (extra_i - extra_i / factor) recovered from the
    table, t rises by the same step 1 / (hi - lo) at every index of the ramp,
    is 0 at lo and 1 at hi. A clipped, reversed or non-linear ramp fails."""
    lo, hi = ol.yarn_find_correction_range(32, 1, 64, 10000, 4096)
    inv = ol.yarn_inv_freq(64, 10000.0, 40.0, 4096, 32, 1).astype(np.float64)
    i = np.arange(32)
    extra = 1.0 / 10000.0 ** (2 * i / 64)
    t = (extra - inv) / (extra - extra / 40.0)
    np.testing.assert_allclose(t[lo], 0.0, atol=1e-6)
    np.testing.assert_allclose(t[hi], 1.0, atol=1e-6)
    steps = np.diff(t[lo:hi + 1])
    np.testing.assert_allclose(steps, 1.0 / (hi - lo), rtol=1e-4, atol=1e-6)
    m = ol.yarn_linear_ramp_mask(lo, hi, 32)
    assert m[0] == 0 and m[-1] == 1 and np.all(np.diff(m) >= 0)


def test_yarn_tables_shape_and_symmetry():
    cos, sin = ol.yarn_cos_sin(128)
    assert cos.shape == (128, 64)
    np.testing.assert_array_equal(cos[:, :32], cos[:, 32:])
    np.testing.assert_array_equal(sin[:, :32], sin[:, 32:])
    np.testing.assert_allclose(cos[0], 1.0)
    np.testing.assert_allclose(sin[0], 0.0)


def test_rope_is_complex_rotation():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 5, 64)).astype(np.float32)
    theta = rng.uniform(-3, 3, (5, 32)).astype(np.float32)
    cos = np.concatenate([np.cos(theta)] * 2, -1)
    sin = np.concatenate([np.sin(theta)] * 2, -1)
    out = ol.rope(x, cos, sin)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * theta)
    np.testing.assert_allclose(out[..., :32], z.real, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out[..., 32:], z.imag, rtol=1e-5, atol=1e-5)


def test_attention_matches_torch_sdpa():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, 3, 17, 24)).astype(np.float32) for _ in range(3))
    out = ol.attention(q, k, v, 0.3)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                         torch.from_numpy(v), is_causal=True, scale=0.3)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-5)


def test_mla_forward_causal_and_shapes():
    """Small-shape MLA: causality (reference test_reference_mla.py:71-96)."""
    rng = np.random.default_rng(5)
    H, nh, nope, r, vd, kl = 64, 2, 16, 8, 16, 32
    p = dict(w_q=rng.standard_normal((nh * (nope + r), H)) * 0.1,
             w_kva=rng.standard_normal((kl + r, H)) * 0.1, w_kva_norm=np.ones(kl),
             w_kvb=rng.standard_normal((nh * (nope + vd), kl)) * 0.1,
             w_o=rng.standard_normal((H, nh * vd)) * 0.1)
    p = {k: v.astype(np.float32) for k, v in p.items()}
    x = rng.standard_normal((1, 9, H)).astype(np.float32)
    kw = dict(n_heads=nh, nope=nope, rope_dim=r, v_dim=vd, kv_lora=kl)
    y = ol.mla_forward(x, **p, **kw)
    assert y.shape == (1, 9, H)
    x2 = x.copy()
    x2[:, 5:] += 1.0
    y2 = ol.mla_forward(x2, **p, **kw)
    np.testing.assert_allclose(y[:, :5], y2[:, :5], rtol=1e-5, atol=1e-5)
    assert not np.allclose(y[:, 5:], y2[:, 5:])


def test_attention_additive_mask_matches_torch_sdpa():
    """The additive-mask branch (mla.py:374-375) against SDPA's float attn_mask,
    with a [b, 1, s, s] mask broadcast over the heads and -inf entries."""
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((2, 3, 11, 24)).astype(np.float32) for _ in range(3))
    m = rng.standard_normal((2, 1, 11, 11)).astype(np.float32)
    m[0, 0, :, 7:] = -np.inf
    m[1, 0, 3, :5] = -np.inf
    out = ol.attention(q, k, v, 0.25, m)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                         torch.from_numpy(v), attn_mask=torch.from_numpy(m),
                                         scale=0.25)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-5)


def _small_mla():
    rng = np.random.default_rng(8)
    H, nh, nope, r, vd, kl = 64, 2, 16, 8, 16, 32
    p = dict(w_q=rng.standard_normal((nh * (nope + r), H)) * 0.1,
             w_kva=rng.standard_normal((kl + r, H)) * 0.1, w_kva_norm=np.ones(kl),
             w_kvb=rng.standard_normal((nh * (nope + vd), kl)) * 0.1,
             w_o=rng.standard_normal((H, nh * vd)) * 0.1)
    p = {k: v.astype(np.float32) for k, v in p.items()}
    return rng, H, p, dict(n_heads=nh, nope=nope, rope_dim=r, v_dim=vd, kv_lora=kl)


def test_mla_forward_position_ids_and_mask_relabel_invariance():
    """Tokens presented in a shuffled order with position_ids = their original
    positions and the causal mask of those positions give the original rows,
    shuffled: pins the position_ids table lookup (mla.py:186-187) and the
    additive-mask path together against the default causal forward."""
    rng, H, p, kw = _small_mla()
    s = 12
    x = rng.standard_normal((1, s, H)).astype(np.float32)
    y = ol.mla_forward(x, **p, **kw)
    perm = rng.permutation(s)
    pid = perm[None, :]
    m = np.where(perm[None, :] > perm[:, None], -np.inf, 0.0).astype(np.float32)[None, None]
    y2 = ol.mla_forward(x[:, perm], **p, **kw, attention_mask=m, position_ids=pid)
    np.testing.assert_allclose(y2, y[:, perm], rtol=1e-4, atol=1e-5)
    # the explicit causal mask and arange positions are the defaults
    causal = np.triu(np.full((s, s), -np.inf, np.float32), 1)[None, None]
    y3 = ol.mla_forward(x, **p, **kw, attention_mask=causal, position_ids=np.arange(s)[None])
    np.testing.assert_allclose(y3, y, rtol=1e-6, atol=1e-6)


def test_mla_forward_positions_shift_invariance():
    """RoPE makes q.k depend on the position difference only: shifting every
    position of a sequence by the same amount (inside the table) leaves the
    attention output unchanged up to rounding, while a non-uniform change does
    not (mla.py:196-205 with tables indexed by position_ids)."""
    rng, H, p, kw = _small_mla()
    s = 16
    x = rng.standard_normal((1, s, H)).astype(np.float32)
    base = np.concatenate([np.arange(8), np.full(8, 7)])[None]    # 8 tokens, then padding
    i = np.arange(s)
    m = np.where(i[None, :] > i[:, None], -np.inf, 0.0).astype(np.float32)
    m[:, 8:] = -np.inf
    m = m[None, None]
    y = ol.mla_forward(x, **p, **kw, attention_mask=m, position_ids=base)
    y_shift = ol.mla_forward(x, **p, **kw, attention_mask=m, position_ids=base + 5)
    np.testing.assert_allclose(y_shift[:, :8], y[:, :8], rtol=1e-4, atol=1e-5)
    y_bad = ol.mla_forward(x, **p, **kw, attention_mask=m,
                           position_ids=base * np.array([[1] * 4 + [2] * 12]))
    assert not np.allclose(y_bad[:, :8], y[:, :8], rtol=1e-4, atol=1e-5)

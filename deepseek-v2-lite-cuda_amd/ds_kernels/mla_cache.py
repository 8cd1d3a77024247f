"""Latent KV cache and absorbed-MLA decode on it.

LatentKVCache mirrors src/kernels/mla_cache.py:29-219 (same constructor,
properties, update/get/reset, errors and repr): per token it keeps the raw
compressed latent (kv_lora_rank, before the RMSNorm) and the raw shared RoPE
key (rope_head_dim, before RoPE), 576 bf16 values instead of the 5120 of the
up-projected K and V. Both live in one [bsz, max_seq, 640] buffer, in the
layout kv_a_proj_with_mqa produces, followed by the RoPE key after RoPE
(`k_rope`, 64 more values per token, written once per token by the first
attention that reads it): the attention kernel reads the latent and the rotated
key of a token (1152 bytes) and no angle tables. `kv_latent` and `k_pe_cache`
are views with the reference's shapes.

mla_decode_forward runs DeepSeekMLA.forward (src/reference/mla.py:295-393) for
new tokens against the cache in the absorbed form: the kv_b up-projection is
folded into the query (q_abs = (W_UK * w)^T q_nope per head) and into the
output ((W_UV * w) o_lat per head), and `ops.mla_decode_attention` attends
straight over the cached raw latents, computing each key's RMS scale and RoPE
on the fly and rotating each cached key once. The reference itself has no
attention over its cache (mla.py:7 recomputes K and V for the whole sequence).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import ops
from .expert_prepack import tile_weights, untile_weights
from .mla import MLAWeights


class LatentKVCache:
    """Pre-allocated compressed KV cache for MLA (mla_cache.py:29-96).

    kv_latent  [bsz, max_seq, kv_lora_rank]   raw latent (pre-norm), a view
    k_pe_cache [bsz, max_seq, rope_head_dim]  raw shared RoPE key, a view
    k_rope     [bsz, max_seq, rope_head_dim]  the RoPE key after RoPE (positions
                                              < rope_len hold it), a view

    The rotated keys are valid for the cos/sin tables that produced them: a
    decode step given other tables (another storage or layout, or the same
    tensors modified in place) rotates every cached key again; views of the
    same rows with a different position count are the same tables. A
    caller that writes kv_latent or k_pe_cache directly (not through update()
    or a decode step) must call reset_rope() (or reset()) afterwards, or the
    rotated keys of the rewritten positions stay stale.
    """

    def __init__(self, bsz: int, max_seq: int, kv_lora_rank: int = 512, rope_head_dim: int = 64,
                 device="cuda", dtype: torch.dtype = torch.bfloat16):
        if not isinstance(bsz, int) or bsz < 1:
            raise ValueError(f"bsz must be a positive integer, got {bsz}")
        if not isinstance(max_seq, int) or max_seq < 1:
            raise ValueError(f"max_seq must be a positive integer, got {max_seq}")
        self.bsz = bsz
        self.max_seq = max_seq
        self.kv_lora_rank = kv_lora_rank
        self.rope_head_dim = rope_head_dim
        self.device = torch.device(device)
        self.dtype = dtype
        self._len = 0
        self._rope_len = 0   # leading positions whose k_rope is valid
        self._rope_tables = None   # (identity, cos, sin) of the tables that rotated them
        w = kv_lora_rank + rope_head_dim
        self.rows = torch.zeros((bsz, max_seq, w + rope_head_dim), dtype=dtype,
                                device=self.device)
        self.kv_latent = self.rows[..., :kv_lora_rank]
        self.k_pe_cache = self.rows[..., kv_lora_rank:w]
        self.k_rope = self.rows[..., w:]

    @property
    def current_len(self) -> int:
        """Number of tokens currently stored."""
        return self._len

    @property
    def remaining_capacity(self) -> int:
        """Number of tokens that can still be appended."""
        return self.max_seq - self._len

    @property
    def rope_len(self) -> int:
        """Leading positions whose rotated key (k_rope) is valid."""
        return min(self._rope_len, self._len)

    @property
    def memory_bytes(self) -> int:
        """Bytes held by the latent and RoPE-key planes (mla_cache.py:92-98); the
        rotated keys take rope_head_dim more values per token beside them."""
        return (self.kv_latent.numel() + self.k_pe_cache.numel()) * self.rows.element_size()

    def update(self, compressed_kv: torch.Tensor, k_pe: torch.Tensor) -> None:
        """Append new tokens (mla_cache.py:102-143): compressed_kv [bsz, n,
        kv_lora_rank] and k_pe [bsz, n, rope_head_dim], converted to the cache's
        device and dtype. ValueError for non-3-D inputs, RuntimeError when the
        cache would exceed max_seq (nothing is written then)."""
        if compressed_kv.dim() != 3:
            raise ValueError("compressed_kv must be 3D [bsz, new_tokens, kv_lora_rank], "
                             f"got shape {tuple(compressed_kv.shape)}")
        if k_pe.dim() != 3:
            raise ValueError("k_pe must be 3D [bsz, new_tokens, rope_head_dim], "
                             f"got shape {tuple(k_pe.shape)}")
        n = compressed_kv.shape[1]
        if self._len + n > self.max_seq:
            raise RuntimeError(f"KV cache overflow: current_len={self._len}, new_tokens={n}, "
                               f"max_seq={self.max_seq}. Increase max_seq or reset the cache.")
        slot = slice(self._len, self._len + n)
        self._rope_len = self.rope_len   # rows from _len on are rewritten
        self.kv_latent[:, slot, :] = compressed_kv.to(self.device, self.dtype)
        self.k_pe_cache[:, slot, :] = k_pe.to(self.device, self.dtype)
        self._len += n

    def append_slots(self, n: int) -> torch.Tensor:
        """Reserve the next n token slots and return them as a [bsz, n, 576] view of
        the cache rows (raw latent, then raw RoPE key), for a producer that writes
        them in place (the kv_a projection of a decode step). Same overflow error as
        `update`; not part of the reference API."""
        if self._len + n > self.max_seq:
            raise RuntimeError(f"KV cache overflow: current_len={self._len}, new_tokens={n}, "
                               f"max_seq={self.max_seq}. Increase max_seq or reset the cache.")
        self._rope_len = self.rope_len   # rows from _len on are rewritten
        rows = self.rows[:, self._len:self._len + n, :self.kv_lora_rank + self.rope_head_dim]
        self._len += n
        return rows

    def get(self, seq_len: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Views of the first seq_len tokens (default: all stored), mla_cache.py:145-169.
        ValueError if more tokens are asked for than are stored."""
        if seq_len is None:
            seq_len = self._len
        if seq_len > self._len:
            raise ValueError(f"Requested seq_len={seq_len} but cache only has {self._len} tokens.")
        return self.kv_latent[:, :seq_len, :], self.k_pe_cache[:, :seq_len, :]

    def reset(self) -> None:
        """Start a new sequence; keeps the buffers (mla_cache.py:171-176)."""
        self._len = 0
        self._rope_len = 0

    def reset_rope(self) -> None:
        """Mark every rotated key stale (after direct writes into kv_latent or
        k_pe_cache): the next decode step rotates them again."""
        self._rope_len = 0

    def use_rope_tables(self, cos: torch.Tensor, sin: torch.Tensor) -> None:
        """Called by a decode step with its tables: rotated keys made with other
        tables (another storage, other strides, or these modified in place) are
        dropped. The cache holds the tables it last saw, so their memory cannot be
        handed to another tensor while their address identifies them; a view of
        the same rows with another length (cos[:seq_len] as the reference passes
        it, growing every step) is the same table, and keeps the rotated keys."""
        def ident(t):
            # everything but the position count: batch dims, row width, layout
            return (t.data_ptr(), t.stride(), tuple(t.shape[:-2]), t.shape[-1], t.dtype,
                    t._version)
        key = (ident(cos), ident(sin))
        if self._rope_tables is None or key != self._rope_tables[0]:
            self._rope_len = 0
        self._rope_tables = (key, cos, sin)

    def __repr__(self) -> str:
        used = (self._len * (self.kv_lora_rank + self.rope_head_dim) * self.rows.element_size()
                * self.bsz) / (1024 ** 2)
        total = self.memory_bytes / (1024 ** 2)
        return (f"LatentKVCache(bsz={self.bsz}, tokens={self._len}/{self.max_seq}, "
                f"used={used:.2f}MB/{total:.2f}MB, device={self.device}, dtype={self.dtype})")

    @classmethod
    def for_inference(cls, bsz: int, max_seq: int = 4096, device="cuda") -> "LatentKVCache":
        """bf16 cache with DeepSeek-V2-Lite's widths (512 + 64), mla_cache.py:201-219."""
        return cls(bsz=bsz, max_seq=max_seq, kv_lora_rank=512, rope_head_dim=64, device=device,
                   dtype=torch.bfloat16)


@dataclass
class AbsorbedMLAWeights:
    """kv_b folded for the absorbed form, with the latent RMSNorm weight w in it:
    w_uk[h] = W_UK[h] * w (the k_nope rows of head h, [nope, kv_lora]) and
    w_uv_t[h] = (W_UV[h] * w)^T ([kv_lora, v_dim]), bf16 contiguous for torch's
    batched products; and the same two per-head matrices in the operand order
    and fragment-tiled layout of `linear_batched`: uk_tiled = tile of the
    [16, kv_lora, nope] stack w_uk^T, uv_tiled = tile of [16, v_dim, kv_lora]."""
    w_uk: torch.Tensor
    w_uv_t: torch.Tensor
    uk_tiled: Optional[torch.Tensor] = None
    uv_tiled: Optional[torch.Tensor] = None

    @staticmethod
    def from_mla(W: MLAWeights) -> "AbsorbedMLAWeights":
        kvb = W.kvb if W.kvb.dim() == 2 else untile_weights(W.kvb[None])[0]
        h, nope, vd = W.n_heads, W.nope, W.v_dim
        kv = kvb.float().view(h, nope + vd, W.kv_lora) * W.kva_norm.float()[None, None, :]
        uk = kv[:, :nope].to(torch.bfloat16)        # [h, nope, lora]
        uv = kv[:, nope:].to(torch.bfloat16)        # [h, v, lora]
        return AbsorbedMLAWeights(
            w_uk=uk.contiguous(), w_uv_t=uv.transpose(1, 2).contiguous(),
            uk_tiled=tile_weights(uk.transpose(1, 2).contiguous()),
            uv_tiled=tile_weights(uv.contiguous()))


# A step of at least this many new tokens (a prompt) attends through up-projected
# K and V, like DeepSeekMLA.forward: the absorbed kernel reads every cached row
# once per new token, which a long step cannot amortise.
UP_PROJECTED_MIN_TOKENS = 128

# Decode steps of at most this many tokens run their projections on the
# vector-ALU row kernel (dsk_linear_rows); longer ones on the small-group MFMA
# kernel.
ROWS_MAX_TOKENS = 4


def _attend_up_projected(q: torch.Tensor, cache: LatentKVCache, W: MLAWeights, cos: torch.Tensor,
                         sin: torch.Tensor, eps: float) -> torch.Tensor:
    """The attention of mla.py:338-384 for the last n of the L cached positions:
    RMSNorm of the cached latents, kv_b, RoPE of the cached keys and the new
    queries, bf16 Q.K^T, attn_softmax_ (scale, causal mask offset by L - n, fp32
    softmax), .V. q: [b, n, h, nope + rope] view of the q projection. Returns
    bf16 [b, n, h * v_dim]."""
    b, n, h, _ = q.shape
    nope, r, vd = W.nope, W.rope_dim, W.v_dim
    L = cache.current_len
    lat, pe = cache.get(L)
    kv = ops.kv_upproj(ops.rms_norm(lat, W.kva_norm, eps), W.kvb).view(b, L, h, nope + vd)
    kv = kv.transpose(1, 2)                                       # [b, h, L, 256] view
    cq = cos[L - n:L][None, None].expand(b, 1, n, r)
    sq = sin[L - n:L][None, None].expand(b, 1, n, r)
    ck = cos[:L][None, None].expand(b, 1, L, r)
    sk = sin[:L][None, None].expand(b, 1, L, r)
    q_rot = ops.rope_single(q[..., nope:].transpose(1, 2), cq, sq)        # [b, h, n, r]
    k_rot = ops.rope_single(pe[:, None], ck, sk)                          # [b, 1, L, r]
    cache.k_rope[:, :L].copy_(k_rot[:, 0])       # every cached key rotated once
    cache._rope_len = L
    qf = torch.cat([q[..., :nope].transpose(1, 2), q_rot], dim=-1)       # [b, h, n, 192]
    # K^T and V with the key dimension padded to a multiple of 8 (zeros), so the
    # score rows are 16-byte aligned for any L and the padding adds exact zeros
    Lp = (L + 7) // 8 * 8
    kT = torch.zeros((b, h, nope + r, Lp), dtype=torch.bfloat16, device=q.device)
    kT[..., :nope, :L].copy_(kv[..., :nope].transpose(-1, -2))
    kT[..., nope:, :L].copy_(k_rot.transpose(-1, -2).expand(b, h, r, L))
    vp = torch.zeros((b, h, Lp, vd), dtype=torch.bfloat16, device=q.device)
    vp[:, :, :L].copy_(kv[..., nope:])
    scores = torch.matmul(qf, kT)                                          # bf16 [b, h, n, Lp]
    p = ops.attn_softmax_(scores, W.softmax_scale, causal=True, kv_len=L)
    o = torch.matmul(p, vp)                                                # [b, h, n, v]
    return o.transpose(1, 2).reshape(b, n, h * vd)


def mla_decode_forward(x: torch.Tensor, W: MLAWeights, cache: LatentKVCache, cos: torch.Tensor,
                       sin: torch.Tensor, absorbed: Optional[AbsorbedMLAWeights] = None,
                       eps: float = 1e-6) -> torch.Tensor:
    """DeepSeekMLA.forward (mla.py:295-393) for new tokens x: bf16 [bsz, n, H] at
    positions cache.current_len .. + n - 1, causal over the cached prefix and
    among themselves. Appends their raw latent and k_pe to the cache and
    returns bf16 [bsz, n, H]. cos/sin: bf16 [positions, rope_dim] tables
    indexed by position (yarn_cos_sin of at least the final length).
    Steps of fewer than UP_PROJECTED_MIN_TOKENS tokens use the absorbed
    attention kernel over the raw cache; longer ones (prompts) up-project the
    cached latents as the reference forward does."""
    op = "mla_decode_forward"
    ops._req(x.dim() == 3 and x.dtype == torch.bfloat16, f"{op}: x must be bf16 [bsz, n, H].")
    b, n, H = x.shape
    ops._req(b == cache.bsz, f"{op}: x has batch {b}, the cache {cache.bsz}.")
    ops._req(cache.kv_lora_rank == W.kv_lora and cache.rope_head_dim == W.rope_dim,
             f"{op}: cache widths do not match the weights.")
    h, nope, r, vd, lora = W.n_heads, W.nope, W.rope_dim, W.v_dim, W.kv_lora
    # everything a later step would reject is checked before the cache advances
    w_in = W.kva.shape[1] * 16 if W.kva.dim() == 4 else W.kva.shape[1]
    ops._req(H == w_in, f"{op}: x has hidden size {H}, the projections take {w_in}.")
    end = cache.current_len + n
    for t, name in ((cos, "cos"), (sin, "sin")):
        ops._req(t.dim() == 2 and t.shape[1] == r and t.shape[0] >= end,
                 f"{op}: {name} must be [positions >= {end}, {r}], got {tuple(t.shape)}.")
    ops._req(n <= cache.remaining_capacity,
             f"KV cache overflow: current_len={cache.current_len}, new_tokens={n}, "
             f"max_seq={cache.max_seq}. Increase max_seq or reset the cache.")
    A = absorbed if absorbed is not None else AbsorbedMLAWeights.from_mla(W)
    cache.use_rope_tables(cos, sin)
    len0 = cache.current_len
    rows = cache.append_slots(n)                           # [b, n, 576] slots
    try:
        return _decode_step(x, W, cache, rows, cos, sin, A, eps)
    except Exception:
        cache._len = len0      # the rows were not (all) written: do not count them
        raise


def _decode_step(x: torch.Tensor, W: MLAWeights, cache: LatentKVCache, rows: torch.Tensor,
                 cos: torch.Tensor, sin: torch.Tensor, A: AbsorbedMLAWeights,
                 eps: float) -> torch.Tensor:
    """mla_decode_forward after the cache slots of the new tokens are reserved."""
    b, n, H = x.shape
    h, nope, r, vd, lora = W.n_heads, W.nope, W.rope_dim, W.v_dim, W.kv_lora
    T = b * n
    x2 = x.reshape(T, H)
    nq = h * (nope + r)
    # up to 4 tokens: every projection on the vector-ALU row kernel, which
    # spreads a one-token projection over N/8 lane groups
    few = (T <= ROWS_MAX_TOKENS and W.q_kva is not None and W.q_kva.dim() == 4 and
           W.o.dim() == 4 and A.uk_tiled is not None)
    if (b == 1 or n == 1) and W.q_kva is not None and W.q_kva.dim() == 4 and T <= 64:
        # q_proj and kv_a_proj in one launch, kv_a's rows straight into the slots
        q = torch.empty((T, nq), dtype=torch.bfloat16, device=x.device)
        dst = rows[0] if b == 1 else rows[:, 0]
        if few:
            ops.linear_rows(x2, W.q_kva, out=q, out1=dst, n_split=nq)
        else:
            ops.linear_split(x2, W.q_kva, q, dst)
        q = q.view(T, h, nope + r)                         # [T, h, 192]
    else:
        q = ops.linear(x, W.q).view(T, h, nope + r)
        if b == 1 or n == 1:                               # one row stride: project in place
            ops.linear(x2, W.kva, out=rows[0] if b == 1 else rows[:, 0])
        else:
            rows.copy_(ops.linear(x2, W.kva).view(b, n, lora + r))
    L = cache.current_len
    if n >= UP_PROJECTED_MIN_TOKENS:
        o = _attend_up_projected(q.view(b, n, h, nope + r), cache, W, cos, sin, eps)
        return ops.linear(o, W.o)
    latent, k_pe = cache.get(L)
    small = T <= 64 and A.uk_tiled is not None
    if few:
        q_abs = ops.linear_rows(q[..., :nope].transpose(0, 1), A.uk_tiled)     # [h, T, lora]
    elif small:   # per-head products on strided views, one launch each
        q_abs = ops.linear_batched(q[..., :nope].transpose(0, 1), A.uk_tiled)  # [h, T, lora]
    else:
        q_abs = torch.bmm(q[..., :nope].transpose(0, 1).contiguous(), A.w_uk)
    o_lat = torch.empty((h, T, lora), dtype=torch.bfloat16, device=x.device)
    ops.mla_decode_attention(q_abs.transpose(0, 1), q[..., nope:], latent, k_pe, cos, sin,
                             W.softmax_scale, eps, out=o_lat.transpose(0, 1),
                             k_rope=cache.k_rope[:, :L], rope_len=cache.rope_len)
    cache._rope_len = L          # the kernel rotated and stored the new keys
    if small:   # o[t, h*v:(h+1)*v] = o_lat[h, t] @ (W_UV[h] * w)^T, written token-major
        o = torch.empty((T, h * vd), dtype=torch.bfloat16, device=x.device)
        (ops.linear_rows if few else ops.linear_batched)(o_lat, A.uv_tiled,
                                                         out=o.view(T, h, vd).transpose(0, 1))
    else:
        o = torch.bmm(o_lat, A.w_uv_t).transpose(0, 1).reshape(T, h * vd)
    if few:
        return ops.linear_rows(o, W.o).view(b, n, -1)
    return ops.linear(o, W.o).view(b, n, -1)

"""GPU parity of decode over the latent KV cache: mla_decode_forward (absorbed
MLA attention on the raw cached latents, dsk_mla_decode_attention) against the
oracle's full-sequence DeepSeekMLA.forward (oracle/mla.py mla_forward, fp32,
causal), whose rows for the positions of the new tokens are what incremental
decoding must reproduce. Prefix fills (through the absorbed kernel and, for
long steps, through up-projected K and V), single-token steps, multi-token
steps, batches, block-boundary lengths and the empty-cache start are covered;
the bar is the bf16 one (max relative error <= 2e-2)."""
import numpy as np
import pytest
import torch

from gpu_util import BF16_TOL, max_rel_err, np32
from oracle import mla as ol

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def setup():
    import ds_kernels as dsk
    from ds_kernels import mla as dm
    from ds_kernels import synthetic as syn
    w = syn.mla_weights()
    W = dm.MLAWeights.from_tensors(w, torch.device(DEV))
    A = dsk.AbsorbedMLAWeights.from_mla(W)
    wn = {k: (np32(v.to(torch.bfloat16)) if k != "kva_norm" else v.numpy()) for k, v in w.items()}
    cos, sin = dm.yarn_cos_sin(2048)
    return dsk, W, A, wn, cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)


def _oracle(x, wn):
    return ol.mla_forward(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], wn["o"])


def _run_steps(setup, x, steps):
    """Feed x [b, S, H] to a fresh cache in consecutive pieces of the given sizes."""
    dsk, W, A, _, cos, sin = setup
    b, S, _ = x.shape
    cache = dsk.LatentKVCache(b, S + 3, device=DEV)
    outs, pos = [], 0
    for n in steps:
        outs.append(dsk.mla_decode_forward(x[:, pos:pos + n].to(DEV), W, cache, cos, sin, A))
        pos += n
    assert pos == S and cache.current_len == S
    torch.cuda.synchronize()
    return torch.cat(outs, 1).cpu(), cache


@pytest.mark.parametrize("b,steps", [
    (1, [1, 1, 1, 1]),                 # starts from an empty cache
    (1, [50, 1, 1, 1, 7, 1]),          # prefill, single steps, a multi-token step
    (2, [127, 1, 1, 1]),               # crosses the 64-key chunk boundary at 128
    (2, [63, 2, 64, 1]),
    (1, [700, 1, 5]),                  # 700 keys, not a multiple of 8: padded prompt path
    (2, [256, 1, 130]),                # prompt through up-projected K/V, then the kernel (merge)
    (1, [1, 255, 8]),                  # up-projected step over a one-token prefix
    (3, [40, 1, 1]),                   # 3 sequences: the few-row projections at 3 rows
    (4, [100, 1, 1]),                  # 4 sequences: the few-row projections at 4 rows
    (1, [30, 3, 4, 5]),                # 3 and 4 new tokens of one sequence, then 5 (MFMA path)
])
def test_decode_matches_full_sequence_oracle(setup, b, steps):
    S = sum(steps)
    g = torch.Generator().manual_seed(7 * S + b)
    x = torch.randn(b, S, 2048, generator=g).to(torch.bfloat16)
    out, _ = _run_steps(setup, x, steps)
    ref = _oracle(x, setup[3])
    assert out.shape == (b, S, 2048)
    err = max_rel_err(np32(out), ref)
    assert err <= BF16_TOL, f"max rel err {err:.3e}"
    # every step's rows on their own (a late step must not hide in the global max)
    pos = 0
    for n in steps:
        e = max_rel_err(np32(out[:, pos:pos + n]), ref[:, pos:pos + n])
        assert e <= BF16_TOL, f"rows {pos}..{pos + n}: {e:.3e}"
        pos += n


def test_decode_prompt_longer_than_4096(setup):
    """A 4100-token prompt through the up-projected path (keys padded to 4104,
    the two-pass softmax beyond 4096 keys), then one decode step through the
    absorbed kernel over 4101 cached tokens, against the oracle's full-sequence
    forward at 4101 positions."""
    dsk, W, A, wn, _, _ = setup
    from ds_kernels import mla as dm
    S = 4101
    cos, sin = dm.yarn_cos_sin(S)
    cos, sin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    g = torch.Generator().manual_seed(4100)
    x = torch.randn(1, S, 2048, generator=g).to(torch.bfloat16)
    cache = dsk.LatentKVCache(1, S, device=DEV)
    o1 = dsk.mla_decode_forward(x[:, :S - 1].to(DEV), W, cache, cos, sin, A)
    o2 = dsk.mla_decode_forward(x[:, S - 1:].to(DEV), W, cache, cos, sin, A)
    out = torch.cat([o1, o2], 1).cpu()
    ref = _oracle(x, wn)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    assert max_rel_err(np32(out[:, S - 1:]), ref[:, S - 1:]) <= BF16_TOL


def test_decode_step_with_new_tables_rotates_again(setup):
    """Keys rotated with one pair of tables are not reused with another: a step
    given new tables equals the same step on a fresh cache filled with the new
    tables, bit for bit."""
    dsk, W, A, wn, cos, sin = setup
    cos2, sin2 = torch.roll(cos, 3, 0).contiguous(), torch.roll(sin, 3, 0).contiguous()
    g = torch.Generator().manual_seed(91)
    x = torch.randn(1, 40, 2048, generator=g).to(torch.bfloat16).to(DEV)
    c1 = dsk.LatentKVCache(1, 64, device=DEV)
    dsk.mla_decode_forward(x[:, :39], W, c1, cos, sin, A)
    o1 = dsk.mla_decode_forward(x[:, 39:], W, c1, cos2, sin2, A)
    c2 = dsk.LatentKVCache(1, 64, device=DEV)
    dsk.mla_decode_forward(x[:, :39], W, c2, cos2, sin2, A)
    o2 = dsk.mla_decode_forward(x[:, 39:], W, c2, cos2, sin2, A)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_decode_attention_rejects_overlapping_k_rope(setup):
    """k_rope is written while latent and k_pe are read: a k_rope view on the
    raw keys (a natural 'rotate in place' call) is refused before any launch."""
    dsk, W, A, wn, cos, sin = setup
    rows = torch.randn(1, 16, 640).to(torch.bfloat16).to(DEV)
    q_abs = torch.zeros(1, 16, 512, dtype=torch.bfloat16, device=DEV)
    q_pe = torch.zeros(1, 16, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="overlaps"):
        dsk.mla_decode_attention(q_abs, q_pe, rows[..., :512], rows[..., 512:576], cos, sin,
                                 0.1, k_rope=rows[..., 512:576])
    with pytest.raises(RuntimeError, match="overlaps"):
        dsk.mla_decode_attention(q_abs, q_pe, rows[..., :512], rows[..., 512:576], cos, sin,
                                 0.1, k_rope=rows[..., 448:512])
    out = dsk.mla_decode_attention(q_abs, q_pe, rows[..., :512], rows[..., 512:576], cos, sin,
                                   0.1)       # scratch keys: no overlap
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())


def test_cache_holds_raw_projection_rows(setup):
    """The cache stores kv_a_proj_with_mqa's raw output (pre-norm latent,
    pre-RoPE key), as mla_cache.py:33-35 documents."""
    dsk, W, A, wn, cos, sin = setup
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 9, 2048, generator=g).to(torch.bfloat16)
    _, cache = _run_steps(setup, x, [4, 5])
    lat, pe = cache.get()
    kva = ol.linear(np32(x), wn["kva"])
    assert max_rel_err(np32(lat), kva[..., :512]) <= BF16_TOL
    assert max_rel_err(np32(pe), kva[..., 512:]) <= BF16_TOL


def _rotated_rows(dsk, rows, cos, sin):
    """[b, L, 640] cache rows from raw [b, L, 576] ones: the RoPE key after
    dsk_rope (the prompt path's rotation) in columns 576..639."""
    b, L, _ = rows.shape
    out = torch.zeros(b, L, 640, dtype=torch.bfloat16, device=DEV)
    out[..., :576] = rows
    c = cos[:L][None, None].expand(b, 1, L, 64)
    s = sin[:L][None, None].expand(b, 1, L, 64)
    from ds_kernels import ops
    out[..., 576:] = ops.rope_single(rows[:, None, :, 512:], c, s)[:, 0]
    return out


def test_decode_attention_op_rotated_keys(setup):
    """The op over cached rotated keys (rope_len = L), over none (rope_len = 0:
    every key rotated in the kernel from k_pe and stored), over the last few
    (rope_len = L - 5, a decode step) and on separately allocated planes with
    equal strides and a strided output: all give the same bits, the kernel's
    rotation equals dsk_rope's bit for bit, and rows below rope_len are not
    written."""
    dsk, W, A, wn, cos, sin = setup
    g = torch.Generator().manual_seed(9)
    b, n, L = 2, 3, 150
    raw = torch.randn(b, L, 576, generator=g).to(torch.bfloat16).to(DEV)
    q_abs = (torch.randn(b * n, 16, 512, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    q_pe = torch.randn(b * n, 16, 64, generator=g).to(torch.bfloat16).to(DEV)
    scale = W.softmax_scale
    rows = _rotated_rows(dsk, raw, cos, sin)
    krot = rows[..., 576:].clone()

    def run(rows_, rope_len, out=None):
        return dsk.mla_decode_attention(q_abs, q_pe, rows_[..., :512], rows_[..., 512:576], cos,
                                        sin, scale, out=out, k_rope=rows_[..., 576:640],
                                        rope_len=rope_len)
    a = run(rows, L)
    fresh = rows.clone()
    fresh[..., 576:] = 0
    b0 = run(fresh, 0)
    part = rows.clone()
    part[:, L - 5:, 576:] = 0
    b5 = run(part, L - 5)
    torch.cuda.synchronize()
    assert torch.equal(b0.cpu(), a.cpu()) and torch.equal(b5.cpu(), a.cpu())
    assert torch.equal(fresh[..., 576:].cpu(), krot.cpu())
    assert torch.equal(part[..., 576:].cpu(), krot.cpu())
    # separate planes (row pitch 576 in each) and a strided output view
    lat = torch.zeros(b, L, 576, dtype=torch.bfloat16, device=DEV)
    pe = torch.zeros(b, L, 576, dtype=torch.bfloat16, device=DEV)
    kr = torch.zeros(b, L, 576, dtype=torch.bfloat16, device=DEV)
    lat[..., :512] = raw[..., :512]
    pe[..., :64] = raw[..., 512:]
    kr[..., :64] = krot
    out = torch.zeros(16, b * n, 512, dtype=torch.bfloat16, device=DEV)
    dsk.mla_decode_attention(q_abs, q_pe, lat[..., :512], pe[..., :64], cos, sin, scale,
                             out=out.transpose(0, 1), k_rope=kr[..., :64], rope_len=L)
    # without k_rope the op rotates every key into a scratch buffer
    c = dsk.mla_decode_attention(q_abs, q_pe, raw[..., :512], raw[..., 512:], cos, sin, scale)
    torch.cuda.synchronize()
    assert torch.equal(out.transpose(0, 1).cpu(), a.cpu()) and torch.equal(c.cpu(), a.cpu())


@pytest.mark.parametrize("b,n", [(1, 1), (4, 1), (8, 1), (16, 1), (1, 8), (2, 4)])
def test_decode_attention_op_split_plans(setup, b, n):
    """The op over a 4096-token cache at the batch shapes whose key-split plans
    differ (64 splits of one 64-key block at b = 1, 32 of two at b = 4 and 8 and
    for 8 new tokens, 16 of four at b = 16) against an fp32 torch restatement of
    absorbed attention (RMS-scaled latents, rotated keys, causal over the new
    tokens), and one sequence of the batch against the same sequence alone,
    which runs under the one-sequence plan."""
    dsk, W, A, wn, _, _ = setup
    from ds_kernels import mla as dm
    L = 4096
    cos, sin = dm.yarn_cos_sin(L)
    cos, sin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    g = torch.Generator().manual_seed(100 * b + n)
    raw = torch.randn(b, L, 576, generator=g).to(torch.bfloat16).to(DEV)
    q_abs = (torch.randn(b * n, 16, 512, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    q_pe = torch.randn(b * n, 16, 64, generator=g).to(torch.bfloat16).to(DEV)
    rows = _rotated_rows(dsk, raw, cos, sin)
    scale = W.softmax_scale
    got = dsk.mla_decode_attention(q_abs, q_pe, rows[..., :512], rows[..., 512:576], cos, sin,
                                   scale, k_rope=rows[..., 576:640], rope_len=L)
    # fp32 reference: the query rotated at its position L - n + j as the keys are
    from ds_kernels import ops
    c = cos[L - n:L][None, None].expand(b, 1, n, 64)
    s = sin[L - n:L][None, None].expand(b, 1, n, 64)
    q_rot = ops.rope_single(q_pe.view(b, n, 16, 64).permute(0, 2, 1, 3), c, s)
    q_rot = q_rot.permute(0, 2, 1, 3).reshape(b, n * 16, 64).float()
    x = rows[..., :512].float()
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    kr = rows[..., 576:640].float()
    sc = (torch.matmul(q_abs.view(b, n * 16, 512).float(), xn.transpose(1, 2).contiguous())
          + torch.matmul(q_rot, kr.transpose(1, 2).contiguous())) * scale
    pos = (L - n + torch.arange(n, device=DEV)).repeat_interleave(16)     # [n * 16]
    sc = sc.masked_fill(torch.arange(L, device=DEV)[None, None, :] > pos[None, :, None],
                        float("-inf"))
    ref = torch.matmul(torch.softmax(sc, -1), xn).view(b * n, 16, 512)
    torch.cuda.synchronize()
    assert max_rel_err(np32(got), np32(ref)) <= BF16_TOL
    i = b - 1
    alone = dsk.mla_decode_attention(q_abs[i * n:(i + 1) * n], q_pe[i * n:(i + 1) * n],
                                     rows[i:i + 1, :, :512], rows[i:i + 1, :, 512:576], cos, sin,
                                     scale, k_rope=rows[i:i + 1, :, 576:640], rope_len=L)
    torch.cuda.synchronize()
    assert max_rel_err(np32(alone), np32(ref[i * n:(i + 1) * n])) <= BF16_TOL
    assert max_rel_err(np32(alone), np32(got[i * n:(i + 1) * n])) <= 1e-2


def test_decode_after_reference_update(setup):
    """A cache filled through the reference API (update() with raw rows, nothing
    rotated) and then a decode step: the kernel rotates the whole prefix, and the
    new token's output matches the full-sequence oracle."""
    dsk, W, A, wn, cos, sin = setup
    g = torch.Generator().manual_seed(21)
    b, S = 2, 200
    x = torch.randn(b, S, 2048, generator=g).to(torch.bfloat16)
    kva = torch.from_numpy(ol.linear(np32(x[:, :S - 1]), wn["kva"])).to(torch.bfloat16)
    cache = dsk.LatentKVCache(b, S, device=DEV)
    cache.update(kva[..., :512], kva[..., 512:])
    assert cache.rope_len == 0
    out = dsk.mla_decode_forward(x[:, S - 1:].to(DEV), W, cache, cos, sin, A)
    torch.cuda.synchronize()
    assert cache.rope_len == S
    ref = _oracle(x, wn)[:, S - 1:]
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def test_decode_op_rejects_bad_shapes(setup):
    dsk, W, A, wn, cos, sin = setup
    rows = torch.zeros(1, 8, 576, dtype=torch.bfloat16, device=DEV)
    q_abs = torch.zeros(9, 16, 512, dtype=torch.bfloat16, device=DEV)
    q_pe = torch.zeros(9, 16, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="new tokens"):
        dsk.mla_decode_attention(q_abs, q_pe, rows[..., :512], rows[..., 512:], cos, sin, 0.1)
    with pytest.raises(RuntimeError, match="cos/sin"):
        dsk.mla_decode_attention(q_abs[:2], q_pe[:2], rows[..., :512], rows[..., 512:],
                                 cos[:4], sin[:4], 0.1)


@pytest.mark.parametrize("M,K,N", [(1, 128, 512), (5, 128, 512), (64, 512, 128), (3, 512, 128)])
def test_linear_batched_strided_views(setup, M, K, N):
    """The per-head products of the decode step: 16 entries on strided views (the
    q_nope slice of the q projection in, a token-major output slice out),
    against an fp32 reference of the same bf16 operands."""
    dsk = setup[0]
    g = torch.Generator().manual_seed(M * 7 + K)
    big = torch.randn(M, 16, K + 64, generator=g).to(torch.bfloat16)   # [tokens, heads, K + pad]
    w = (torch.randn(16, N, K, generator=g) * 0.05).to(torch.bfloat16)
    x = big.to(DEV)[..., :K].transpose(0, 1)                            # [16, M, K] strided
    out_full = torch.zeros(M, 16, N + 8, dtype=torch.bfloat16, device=DEV)
    out = out_full[..., :N].transpose(0, 1)                              # [16, M, N] strided
    dsk.linear_batched(x, dsk.tile_weights(w.to(DEV)), out=out)
    ref = torch.einsum("hmk,hnk->hmn", big[..., :K].transpose(0, 1).float(), w.float())
    assert max_rel_err(np32(out), ref.numpy()) <= BF16_TOL
    assert torch.count_nonzero(out_full[..., N:]) == 0   # nothing written past the slice


@pytest.mark.parametrize("M,K,N", [(1, 2048, 3648), (2, 2048, 2048), (4, 2048, 64), (3, 512, 128),
                                   (1, 128, 512), (4, 128, 96), (1, 640, 32)])
def test_linear_rows_matches_fp32(setup, M, K, N):
    """dsk_linear_rows (vector ALU, 8 weight rows per lane group) against an fp32
    reference of the same bf16 operands: one entry with x rows strided inside a
    wider buffer, and 3 batched entries on strided views; the same bits on a
    second call; one weight shared by 3 batched entries; K = 128 and 640 take the
    16-lane path (four row groups per wave; K = 640 with five K chunks per lane)."""
    dsk = setup[0]
    g = torch.Generator().manual_seed(M * 31 + K + N)
    xb = torch.randn(M, K + 32, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    x = xb.to(DEV)[:, :K]
    out = dsk.linear_rows(x, dsk.tile_weights(w[None].to(DEV))[0])
    ref = xb[:, :K].float() @ w.float().T
    assert out.shape == (M, N)
    assert max_rel_err(np32(out), ref.numpy()) <= BF16_TOL
    again = dsk.linear_rows(x, dsk.tile_weights(w[None].to(DEV))[0])
    assert torch.equal(out, again)
    # batched, strided in and out
    big = torch.randn(M, 3, K + 64, generator=g).to(torch.bfloat16)
    wb = (torch.randn(3, N, K, generator=g) * 0.05).to(torch.bfloat16)
    xs = big.to(DEV)[..., :K].transpose(0, 1)                       # [3, M, K] strided
    out_full = torch.zeros(M, 3, N + 8, dtype=torch.bfloat16, device=DEV)
    o = out_full[..., :N].transpose(0, 1)                            # [3, M, N] strided
    dsk.linear_rows(xs, dsk.tile_weights(wb.to(DEV)), out=o)
    refb = torch.einsum("hmk,hnk->hmn", big[..., :K].transpose(0, 1).float(), wb.float())
    assert max_rel_err(np32(o), refb.numpy()) <= BF16_TOL
    assert torch.count_nonzero(out_full[..., N:]) == 0
    # batched x with one weight shared by every entry (weight batch stride 0)
    shared = dsk.linear_rows(xs, dsk.tile_weights(w[None].to(DEV))[0])
    refs = big[..., :K].transpose(0, 1).float() @ w.float().T
    assert shared.shape == (3, M, N)
    assert max_rel_err(np32(shared), refs.numpy()) <= BF16_TOL
    assert torch.equal(shared[0], dsk.linear_rows(xs[0], dsk.tile_weights(w[None].to(DEV))[0]))


@pytest.mark.parametrize("M,n0", [(1, 3072), (4, 64), (2, 0)])
def test_linear_rows_split_output(setup, M, n0):
    """The two-destination form used for q_proj + kv_a_proj: columns from n0 go to
    a strided second buffer; equal to the one-output call bit for bit."""
    dsk = setup[0]
    g = torch.Generator().manual_seed(M + n0)
    x = torch.randn(M, 2048, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(3648, 2048, generator=g) * 0.02).to(torch.bfloat16)
    wt = dsk.tile_weights(w[None])[0].to(DEV)
    full = dsk.linear_rows(x, wt)
    out0 = torch.empty(M, n0, dtype=torch.bfloat16, device=DEV)
    pad = torch.zeros(M, 3648 - n0 + 64, dtype=torch.bfloat16, device=DEV)
    dsk.linear_rows(x, wt, out=out0, out1=pad[:, :3648 - n0], n_split=n0)
    assert torch.equal(out0, full[:, :n0])
    assert torch.equal(pad[:, :3648 - n0], full[:, n0:])
    assert torch.count_nonzero(pad[:, 3648 - n0:]) == 0


@pytest.mark.parametrize("M,n0", [(1, 3072), (16, 3072), (64, 64), (100, 3072)])
def test_linear_split_matches_linear(setup, M, n0):
    """dsk_linear_split (one small-group launch for M <= 64, two launches over the
    weight's row blocks above) equals the one-output projection bit for bit; out1
    is a strided view (rows of a wider buffer), and nothing lands past its columns."""
    dsk = setup[0]
    g = torch.Generator().manual_seed(M + n0)
    x = torch.randn(M, 2048, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(3648, 2048, generator=g) * 0.02).to(torch.bfloat16)
    wt = dsk.tile_weights(w[None])[0].to(DEV)
    full = dsk.linear(x, wt)
    out0 = torch.empty(M, n0, dtype=torch.bfloat16, device=DEV)
    pad = torch.zeros(M, 3648 - n0 + 64, dtype=torch.bfloat16, device=DEV)
    dsk.linear_split(x, wt, out0, pad[:, :3648 - n0])
    torch.cuda.synchronize()
    assert torch.equal(out0, full[:, :n0])
    assert torch.equal(pad[:, :3648 - n0], full[:, n0:])
    assert torch.count_nonzero(pad[:, 3648 - n0:]) == 0

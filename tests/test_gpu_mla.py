"""GPU parity of the MLA helper kernels (rms_norm, rope, kv_upproj) and the
dense MFMA linear against the numpy oracle."""
import numpy as np
import pytest
import torch

from gpu_util import BF16_TOL, F32_TOL, max_rel_err, np32
from oracle import mla as ol
from oracle import moe as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def dsk():
    import ds_kernels
    return ds_kernels


@pytest.mark.parametrize("rows,H", [(4, 512), (64, 512), (1000, 512), (33, 2048), (8, 6),
                                    (5, 4096), (3, 5000), (20001, 512), (9001, 1024)])
def test_rms_norm_bf16(dsk, rows, H):
    g = torch.Generator().manual_seed(rows + H)
    x = (torch.randn(rows, H, generator=g) * 0.5).to(torch.bfloat16)
    w = torch.rand(H, generator=g) + 0.5
    out = dsk.rms_norm(x.to(DEV), w.to(DEV), 1e-6)
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    ref = ol.rms_norm(np32(x), w.numpy(), 1e-6)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    np.testing.assert_allclose(np32(out), ref, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("rows,H", [(16, 512), (300, 2048), (7, 2050)])
def test_rms_norm_f32(dsk, rows, H):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, H, generator=g) * 3
    w = torch.rand(H, generator=g) + 0.5
    out = dsk.rms_norm(x.to(DEV), w.to(DEV), 1e-6)
    ref = ol.rms_norm(x.numpy(), w.numpy(), 1e-6)
    assert max_rel_err(np32(out), ref) <= F32_TOL
    np.testing.assert_allclose(np32(out), ref, rtol=F32_TOL, atol=1e-6)


@pytest.mark.parametrize("scale", [1.0, 1e4, 1e-4])
def test_rms_norm_3d_input_and_magnitudes(dsk, scale):
    """[bsz, seq, hidden] input (the reference test's 3-D case, flattened rows),
    at ordinary, large and small magnitudes (the normalised output has the same
    scale whatever the input's), plus an all-zero row (eps keeps it finite: 0)."""
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(2, 32, 512, generator=g) * scale).to(torch.bfloat16)
    x[1, 5] = 0
    w = torch.rand(512, generator=g) + 0.5
    out = dsk.rms_norm(x.to(DEV), w.to(DEV), 1e-6)
    assert out.shape == (2, 32, 512) and out.dtype == torch.bfloat16
    o = np32(out)
    assert np.isfinite(o).all()
    assert (o[1, 5] == 0).all()
    ref = ol.rms_norm(np32(x).reshape(-1, 512), w.numpy(), 1e-6).reshape(2, 32, 512)
    assert max_rel_err(o, ref) <= BF16_TOL


def test_rms_norm_strided_latent_view(dsk):
    """Normalise the 512-wide latent inside the 576-wide kv_a output in place."""
    g = torch.Generator().manual_seed(3)
    kva = torch.randn(2, 40, 576, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.ones(512, device=DEV)
    out = dsk.rms_norm(kva[..., :512], w)
    ref = ol.rms_norm(np32(kva[..., :512]), np.ones(512, np.float32))
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def _rope_inputs(b, s, seed, strided=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, 16, 192, generator=g).to(torch.bfloat16)
    kva = torch.randn(b, s, 576, generator=g).to(torch.bfloat16)
    cos, sin = ol.yarn_cos_sin(s)
    if strided:   # views straight out of the projections, as DeepSeekMLA makes them
        q_pe = q.to(DEV).transpose(1, 2)[..., 128:]
        k_pe = kva.to(DEV)[..., 512:].view(b, s, 1, 64).transpose(1, 2)
    else:
        q_pe = q.transpose(1, 2)[..., 128:].contiguous().to(DEV)
        k_pe = kva[..., 512:].reshape(b, s, 1, 64).transpose(1, 2).contiguous().to(DEV)
    cb = torch.from_numpy(cos).to(torch.bfloat16)[None, None].expand(b, 1, s, 64).contiguous()
    sb = torch.from_numpy(sin).to(torch.bfloat16)[None, None].expand(b, 1, s, 64).contiguous()
    return q_pe, k_pe, cb.to(DEV), sb.to(DEV)


@pytest.mark.parametrize("b,s,strided", [(1, 16, False), (2, 64, False), (2, 64, True),
                                         (1, 1, False), (8, 256, True)])
def test_rope_matches_oracle(dsk, b, s, strided):
    q_pe, k_pe, cos, sin = _rope_inputs(b, s, b * 1000 + s, strided)
    q_rot, k_rot = dsk.rope(q_pe, k_pe, cos, sin)
    assert q_rot.shape == (b, 16, s, 64) and k_rot.shape == (b, 1, s, 64)
    c, sn = np32(cos), np32(sin)
    rq = ol.rope(np32(q_pe), c, sn)
    rk = ol.rope(np32(k_pe), c, sn)
    assert max_rel_err(np32(q_rot), rq) <= BF16_TOL
    assert max_rel_err(np32(k_rot), rk) <= BF16_TOL
    np.testing.assert_allclose(np32(q_rot), rq, rtol=2 ** -7, atol=2e-3)


@pytest.mark.parametrize("d,hq,s", [(8, 3, 37), (24, 3, 37), (32, 16, 5), (48, 2, 64),
                                    (128, 5, 9), (64, 12, 33), (64, 20, 7), (16, 9, 3)])
def test_rope_other_dims(dsk, d, hq, s):
    """Rope dims other than 64: 4 pairs per thread when d is not a multiple of 16
    (8, 24), 8 pairs otherwise; odd head counts and sequence lengths exercise the
    multiply-shift index split. A thread rotates up to 8 heads at one position, so
    head counts of 9, 12 and 20 leave a partial last group. The cos/sin tables are
    random, not duplicated halves, so the first- and second-half table reads are
    told apart."""
    b = 2
    g = torch.Generator().manual_seed(d * 100 + hq + s)
    q = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, 1, s, d, generator=g).to(torch.bfloat16)
    cos = (torch.rand(b, 1, s, d, generator=g) * 2 - 1).to(torch.bfloat16)
    sin = (torch.rand(b, 1, s, d, generator=g) * 2 - 1).to(torch.bfloat16)
    q_rot, k_rot = dsk.rope(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV))
    c, sn = np32(cos), np32(sin)
    np.testing.assert_allclose(np32(q_rot), ol.rope(np32(q), c, sn), rtol=2 ** -7, atol=2e-3)
    np.testing.assert_allclose(np32(k_rot), ol.rope(np32(k), c, sn), rtol=2 ** -7, atol=2e-3)


@pytest.mark.parametrize("rows", [1, 64, 4096])
def test_kv_upproj(dsk, rows):
    g = torch.Generator().manual_seed(rows)
    n = (torch.randn(rows, 512, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(4096, 512, generator=g) * 0.02).to(torch.bfloat16)
    out = dsk.kv_upproj(n.to(DEV), w.to(DEV))
    ref = om.grouped_linear(np32(n), np32(w)[None], np.array([0, rows], np.int32))
    assert out.shape == (rows, 4096)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def test_kv_upproj_3d_input(dsk):
    """[bsz, seq, 512] in, [bsz, seq, 4096] out (the reference test's 3-D case),
    the same rows as the 2-D call bit for bit, and against fp32 products."""
    g = torch.Generator().manual_seed(5)
    n = (torch.randn(2, 32, 512, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(4096, 512, generator=g) * 0.02).to(torch.bfloat16)
    out = dsk.kv_upproj(n.to(DEV), w.to(DEV))
    assert out.shape == (2, 32, 4096)
    flat = dsk.kv_upproj(n.reshape(64, 512).to(DEV), w.to(DEV))
    assert torch.equal(out.reshape(64, 4096), flat)
    ref = np32(n).reshape(64, 512) @ np32(w).T
    assert max_rel_err(np32(out).reshape(64, 4096), ref) <= BF16_TOL


@pytest.mark.parametrize("M,K,N", [(8, 2048, 3072), (130, 2048, 576), (1000, 512, 4096),
                                   (77, 128, 100)])
def test_linear(dsk, M, K, N):
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    out = dsk.linear(x.to(DEV), w.to(DEV))
    ref = np32(x) @ np32(w).T
    assert max_rel_err(np32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("N,ld_out", [(200, 216), (200, 204), (136, 140), (1000, 1000)])
def test_linear_strided_output_rows(dsk, N, ld_out):
    """The 256-row tile kernel's row stores into an output view whose row
    pitch is ld_out: 16-byte stores when the pitch is a multiple of 8
    elements, 8-byte stores otherwise, and a per-element tail when N is not
    a multiple of 16. Columns N .. ld_out-1 must stay untouched."""
    M, K = 300, 256
    g = torch.Generator().manual_seed(N + ld_out)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    full = torch.full((M, ld_out), 7.0, dtype=torch.bfloat16, device=DEV)
    out = full[:, :N]
    dsk.linear(x.to(DEV), w.to(DEV), out=out)
    torch.cuda.synchronize()
    assert max_rel_err(np32(out), np32(x) @ np32(w).T) <= BF16_TOL
    assert bool((full[:, N:] == 7.0).all())


@pytest.mark.parametrize("M,K,N", [(8, 2048, 3072), (130, 2048, 576), (1000, 512, 4096),
                                   (300, 2048, 2048), (77, 128, 96), (50, 192, 64)])
def test_linear_tiled_weight(dsk, M, K, N):
    """The fragment-tiled weight path (one wave per SIMD, weights straight to
    registers when K % 128 == 0; the 8-wave kernel otherwise) against fp32."""
    g = torch.Generator().manual_seed(3 * M + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wt = dsk.tile_weights(w[None])[0].to(DEV)
    out = dsk.linear(x.to(DEV), wt)
    ref = np32(x) @ np32(w).T
    assert out.shape == (M, N)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    # same rounding as the row-major path: both accumulate in fp32 and round once
    out_rm = dsk.linear(x.to(DEV), w.to(DEV))
    assert max_rel_err(np32(out), np32(out_rm)) <= BF16_TOL


@pytest.mark.parametrize("rows", [1, 64, 4096])
def test_kv_upproj_tiled_weight(dsk, rows):
    g = torch.Generator().manual_seed(rows + 7)
    n = (torch.randn(rows, 512, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(4096, 512, generator=g) * 0.02).to(torch.bfloat16)
    out = dsk.kv_upproj(n.to(DEV), dsk.tile_weights(w[None])[0].to(DEV))
    ref = om.grouped_linear(np32(n), np32(w)[None], np.array([0, rows], np.int32))
    assert out.shape == (rows, 4096)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("M", [1, 300, 4096])
def test_linear_rowsq_matches_torch(dsk, M):
    """q/kv_a projection with the latent rows' sums of squares from its epilogue:
    the output is bit-identical to the plain tiled projection, and each 256-column
    partial equals the fp64 sum of squares of those bf16 outputs to fp32 rounding
    (1e-5). Columns [3072, 3584) of a 3648-wide output, as in config 3."""
    K, N, c0, c1 = 2048, 3648, 3072, 3584
    g = torch.Generator().manual_seed(M + 5)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wt = dsk.tile_weights(w[None])[0].to(DEV)
    out, ss = dsk.linear_rowsq(x, wt, c0, c1)
    assert torch.equal(out, dsk.linear(x, wt))
    assert tuple(ss.shape) == ((c1 - c0) // 256, M)
    o64 = out.double().cpu()
    ref = torch.stack([(o64[:, c0 + 256 * p:c0 + 256 * (p + 1)] ** 2).sum(1)
                       for p in range((c1 - c0) // 256)])
    np.testing.assert_allclose(ss.double().cpu().numpy(), ref.numpy(), rtol=F32_TOL, atol=0)
    out2, ss2 = dsk.linear_rowsq(x, wt, c0, c1)
    assert torch.equal(ss, ss2) and torch.equal(out, out2)


@pytest.mark.parametrize("M", [1, 300, 4096])
def test_linear_rowscale_is_rms_norm_then_projection(dsk, M):
    """kv_b on the raw latent with the RMS row scale in its epilogue against the
    reference order of operations (mla.py:338-346: RMSNorm with weight w, then
    kv_b) in fp32 on the same bf16 inputs: within the bf16 bar. The latent is a
    strided view (row pitch 576 inside the kv_a output), the statistics come from
    linear_rowsq, and the norm weight is folded into kv_b's input columns."""
    from ds_kernels import mla as dm
    g = torch.Generator().manual_seed(M + 9)
    K, Hq = 2048, 3072
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w_qkva = (torch.randn(Hq + 576, K, generator=g) * 0.02).to(torch.bfloat16)
    kvb = (torch.randn(4096, 512, generator=g) * 0.02).to(torch.bfloat16)
    nw = 1.0 + 0.1 * torch.randn(512, generator=g)   # a non-trivial norm weight
    y, ss = dsk.linear_rowsq(x, dsk.tile_weights(w_qkva[None])[0].to(DEV), Hq, Hq + 512)
    lat = y[:, Hq:Hq + 512]                            # strided view, pitch 3648
    kvb_w = dsk.tile_weights((kvb.float() * nw[None, :]).to(torch.bfloat16)[None])[0].to(DEV)
    out = dsk.linear_rowscale(lat, kvb_w, ss, 512, 1e-6)
    l32 = lat.float().cpu()
    normed = l32 * torch.rsqrt((l32 * l32).mean(-1, keepdim=True) + 1e-6) * nw[None, :]
    ref = normed @ kvb.float().T
    assert out.shape == (M, 4096)
    assert max_rel_err(np32(out), ref.numpy()) <= BF16_TOL
    # and against this library's unfused pair (rms_norm kernel, then kv_upproj)
    sep = dsk.kv_upproj(dsk.rms_norm(lat, nw.to(DEV)), dsk.tile_weights(kvb[None])[0].to(DEV))
    assert max_rel_err(np32(out), np32(sep)) <= BF16_TOL
    assert torch.equal(out, dsk.linear_rowscale(lat, kvb_w, ss, 512, 1e-6))


def test_mla_projections_fused_norm_matches_separate_pass(mla_setup):
    """The projection block with the latent norm in the epilogues against the
    same block with the norm as its own pass (MLAWeights without the folded
    kv_b weight): q and k_rot bit-identical, k_nope and v within the bf16 bar."""
    import dataclasses
    dm, w, W, wn = mla_setup
    assert W.kvb_w is not None
    b, s = 2, 256
    g = torch.Generator().manual_seed(17)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16).to(DEV)
    cos, sin = dm.yarn_cos_sin(s, device=torch.device(DEV))
    fused = dm.mla_projections(x, W, cos, sin, with_latent=False)
    sep = dm.mla_projections(x, dataclasses.replace(W, kvb_w=None), cos, sin)
    assert fused[5] is None
    for i in (0, 1, 4):
        assert torch.equal(fused[i], sep[i])
    for i in (2, 3):
        assert max_rel_err(np32(fused[i]), np32(sep[i])) <= BF16_TOL


def _softmax_ref(sc: torch.Tensor, scale: float, causal: bool, mask=None) -> torch.Tensor:
    """CPU fp32 restatement of mla.py:366-381 on the same bf16 scores: scores *
    scale rounded to bf16, causal mask (query i of the last q_len positions sees
    keys j <= i + kv_len - q_len) or the additive mask added in the dtype torch
    promotes bf16 + mask to, softmax in fp32 (torch), rounded to bf16."""
    q_len, kv_len = sc.shape[-2:]
    x = (sc.float() * scale).to(torch.bfloat16)
    if mask is not None:
        x = x + mask                    # bf16 + bf16 -> bf16, bf16 + fp32 -> fp32
    x = x.float()
    if causal:
        i = torch.arange(q_len)[:, None]
        j = torch.arange(kv_len)[None, :]
        x = x.masked_fill(j > i + (kv_len - q_len), float("-inf"))
    return torch.softmax(x, dim=-1).to(torch.bfloat16)


@pytest.mark.parametrize("shape,causal", [((2, 3, 64, 64), True), ((1, 2, 40, 520), True),
                                          ((2, 16, 128, 2048), True), ((1, 1, 8, 4096), True),
                                          ((3, 5, 16, 1024), False), ((4, 7, 72), False),
                                          ((1, 2, 24, 4104), True), ((2, 1, 5, 6000), False),
                                          ((1, 1, 3, 9000), True)])
def test_attn_softmax_matches_torch(dsk, shape, causal):
    g = torch.Generator().manual_seed(sum(shape))
    sc = (torch.randn(*shape, generator=g) * 6).to(torch.bfloat16)
    scale = 0.1147
    ref = _softmax_ref(sc, scale, causal)
    out = dsk.attn_softmax_(sc.to(DEV), scale, causal=causal).cpu()
    # bf16 outputs of the same fp32 softmax: at most one bf16 ulp apart
    diff = (out.float() - ref.float()).abs()
    assert float(diff.max()) <= 2 ** -7 * float(ref.float().abs().max())
    assert max_rel_err(np32(out), np32(ref)) <= BF16_TOL
    if causal:  # masked keys are exactly zero, every row sums to one
        q_len, kv_len = shape[-2:]
        i = torch.arange(q_len)[:, None]
        j = torch.arange(kv_len)[None, :]
        assert bool((out.float()[..., j > i + (kv_len - q_len)] == 0).all())
    np.testing.assert_allclose(out.float().sum(-1).numpy(), 1.0, atol=2e-2)


@pytest.mark.parametrize("kv_len,causal", [(100, True), (1, False), (4099, True), (13, False)])
def test_attn_softmax_padded_rows(dsk, kv_len, causal):
    """kv_len keys in rows padded to a multiple of 8: the probabilities of the
    first kv_len columns as the unpadded reference, the padding columns exactly 0
    (a P.V product over zero-padded V rows then adds nothing)."""
    L = (kv_len + 7) // 8 * 8
    q_len = min(kv_len, 24) if causal else 7
    g = torch.Generator().manual_seed(kv_len)
    sc = (torch.randn(2, 3, q_len, L, generator=g) * 4).to(torch.bfloat16)
    ref = _softmax_ref(sc[..., :kv_len], 0.13, causal)
    out = dsk.attn_softmax_(sc.to(DEV), 0.13, causal=causal, kv_len=kv_len).cpu()
    assert float((out[..., :kv_len].float() - ref.float()).abs().max()) <= \
        2 ** -7 * float(ref.float().abs().max())
    assert bool((out[..., kv_len:] == 0).all())


@pytest.mark.parametrize("mdtype,shape", [(torch.bfloat16, (2, 3, 40, 40)),
                                          (torch.float32, (2, 3, 40, 40)),
                                          (torch.float32, (1, 4, 17, 4100)),
                                          (torch.bfloat16, (2, 2, 33, 33))])
def test_attn_softmax_additive_mask(dsk, mdtype, shape):
    """The additive attention_mask of mla.py:374 ([b, 1, q, kv], broadcast over
    the heads): a causal-plus-padding mask with -inf entries and finite biases,
    added in the promoted dtype, against torch's fp32 softmax of the same sum."""
    b, h, q_len, kv_len = shape
    g = torch.Generator().manual_seed(q_len * 7 + kv_len)
    L = (kv_len + 7) // 8 * 8
    sc = (torch.randn(b, h, q_len, L, generator=g) * 5).to(torch.bfloat16)
    i = torch.arange(q_len)[:, None] + (kv_len - q_len)
    j = torch.arange(kv_len)[None, :]
    m = torch.randn(b, 1, q_len, kv_len, generator=g) * 2        # finite biases
    m = m.masked_fill(j > i, float("-inf"))                      # causal
    m[-1, :, :, kv_len - kv_len // 4:] = float("-inf")           # last sequence padded
    m[-1, :, :, 0] = 0.0                                         # no row fully masked
    m = m.to(mdtype)
    ref = _softmax_ref(sc[..., :kv_len], 0.2, False, mask=m)
    out = dsk.attn_softmax_(sc.to(DEV), 0.2, causal=False, kv_len=kv_len, mask=m.to(DEV)).cpu()
    assert float((out[..., :kv_len].float() - ref.float()).abs().max()) <= \
        2 ** -7 * float(ref.float().abs().max())
    assert bool((out[..., :kv_len][ref == 0] == 0).all())
    assert bool((out[..., kv_len:] == 0).all())


# ------------------------------------------- configs 3 and 4 (composition) --
def _bf(t):
    return t.to(torch.bfloat16).float().numpy()


@pytest.fixture(scope="module")
def mla_setup(dsk):
    from ds_kernels import mla as dm
    from ds_kernels import synthetic as syn
    w = syn.mla_weights()
    W = dm.MLAWeights.from_tensors(w, torch.device(DEV))
    wn = {k: (_bf(v) if k != "kva_norm" else v.numpy()) for k, v in w.items()}
    return dm, w, W, wn


def test_mla_projections_match_oracle(mla_setup):
    """Config 3's projection block (b=2, s=128 here): every output within the bf16 bar."""
    dm, w, W, wn = mla_setup
    b, s = 2, 128
    g = torch.Generator().manual_seed(11)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    outs = dm.mla_projections(x.to(DEV), W, cos.to(DEV), sin.to(DEV))
    cb, sb = _bf(cos), _bf(sin)
    refs = ol.mla_projections(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], cb, sb)
    names = ["q_nope", "q_rot", "k_nope", "v", "k_rot", "latent"]
    for name, o, r in zip(names, outs, refs):
        assert tuple(o.shape) == r.shape, name
        assert max_rel_err(np32(o), r) <= BF16_TOL, name


@pytest.mark.parametrize("b,s", [(1, 8), (2, 64), (2, 72), (3, 200)])
def test_attn_pack_is_rope_and_head_major_copies(dsk, b, s):
    """mla_attn_pack against the composition it replaces, bitwise: Q = cat(q_nope,
    rope(q_pe)), K^T = cat(k_nope, rope(k_pe) over heads)^T and V = v made
    contiguous, from strided projection rows (q and k_pe slices of one
    [b, s, 3648] buffer, kv rows padded to 4104). Lengths that are not multiples
    of the 64-position block cover the partial last block. Q's rope part is also
    checked against the oracle's RoPE."""
    g = torch.Generator().manual_seed(b * 1000 + s)
    y = torch.randn(b, s, 3648, generator=g).to(torch.bfloat16).to(DEV)
    kvb = torch.randn(b, s, 4104, generator=g).to(torch.bfloat16).to(DEV)
    cos = (torch.rand(s + 5, 64, generator=g) * 2 - 1)
    sin = (torch.rand(s + 5, 64, generator=g) * 2 - 1)
    q, kv, k_pe = y[..., :3072], kvb[..., :4096], y[..., 3584:]
    Q, KT, V = dsk.mla_attn_pack(q, kv, k_pe, cos.to(DEV), sin.to(DEV))
    qh = q.view(b, s, 16, 192).transpose(1, 2)
    kvh = kv.view(b, s, 16, 256).transpose(1, 2)
    cb = cos[:s].to(torch.bfloat16).to(DEV)[None, None].expand(b, 1, s, 64)
    sb = sin[:s].to(torch.bfloat16).to(DEV)[None, None].expand(b, 1, s, 64)
    q_rot, k_rot = dsk.rope(qh[..., 128:], k_pe.view(b, s, 1, 64).transpose(1, 2), cb, sb)
    q_ref = torch.cat([qh[..., :128], q_rot], dim=-1)
    k_ref = torch.cat([kvh[..., :128], k_rot.expand(b, 16, s, 64)], dim=-1)
    assert Q.is_contiguous() and KT.is_contiguous() and V.is_contiguous()
    assert torch.equal(Q, q_ref)
    assert torch.equal(KT, k_ref.transpose(-1, -2))
    assert torch.equal(V, kvh[..., 128:])
    rq = ol.rope(np32(qh[..., 128:]), np32(cb), np32(sb))
    np.testing.assert_allclose(np32(Q[..., 128:]), rq, rtol=2 ** -7, atol=2e-3)


def test_mla_forward_matches_oracle(mla_setup):
    dm, w, W, wn = mla_setup
    b, s = 1, 128
    g = torch.Generator().manual_seed(12)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.mla_forward(x.to(DEV), W, cos.to(DEV), sin.to(DEV))
    ref = ol.mla_forward(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], wn["o"])
    assert out.shape == (b, s, 2048)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def test_decoder_layer_matches_oracle(mla_setup):
    """Config 4's layer at b=1, s=64: RMSNorm -> MLA -> residual -> RMSNorm ->
    MoE (64 routed top-6 + 2 shared) -> residual, against the fp32 oracle."""
    dm, w, W, wn = mla_setup
    from ds_kernels import synthetic as syn
    M = syn.moe_weights()
    P = dm.DecoderLayerWeights.from_tensors(w, M, torch.device(DEV))
    b, s = 1, 64
    g = torch.Generator().manual_seed(13)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.decoder_layer_forward(x.to(DEV), P, cos.to(DEV), sin.to(DEV))
    p = {"in_norm": np.ones(2048, np.float32), "post_norm": np.ones(2048, np.float32),
         "q": wn["q"], "kva": wn["kva"], "kva_norm": wn["kva_norm"], "kvb": wn["kvb"],
         "o": wn["o"], "wg": _bf(M.wg), "gates": _bf(M.gates), "ups": _bf(M.ups),
         "downs": _bf(M.downs), "shared": tuple(_bf(t) for t in M.shared)}
    ref = ol.decoder_layer(np32(x), p)
    assert out.shape == (b, s, 2048)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def test_decoder_layer_causality(mla_setup):
    """Causality of the layer (the property the reference checks on its module,
    test_reference_decoder_layer.py:80): changing the tokens from position p on
    leaves every output before p bit for bit as it was. The attention masks the
    later keys to exact zeros, and every MoE row is computed from its own token
    in a fixed order, whichever rows share its groups."""
    dm, w, W, wn = mla_setup
    from ds_kernels import synthetic as syn
    P = dm.DecoderLayerWeights.from_tensors(w, syn.moe_weights(), torch.device(DEV))
    b, s, p = 2, 96, 40
    g = torch.Generator().manual_seed(17)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    x2 = x.clone()
    x2[:, p:] = torch.randn(b, s - p, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    cos, sin = cos.to(DEV), sin.to(DEV)
    out = dm.decoder_layer_forward(x.to(DEV), P, cos, sin)
    out2 = dm.decoder_layer_forward(x2.to(DEV), P, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :p], out2[:, :p])
    assert not torch.equal(out[:, p:], out2[:, p:])


def test_decoder_layer_matches_oracle_large_groups(mla_setup):
    """Config 4's layer at b=2, s=512 (1024 tokens) against the fp32 oracle: the
    MoE inside runs the T > 64 routing (route, then scan and permutation in one
    kernel), the large-group GEMMs (routed groups of ~100 rows, shared groups of
    1024) and the attention softmax over up to 512 causal keys.
    Reference composition: decoder_layer.py:108-139."""
    dm, w, W, wn = mla_setup
    from ds_kernels import synthetic as syn
    M = syn.moe_weights()
    P = dm.DecoderLayerWeights.from_tensors(w, M, torch.device(DEV))
    b, s = 2, 512
    g = torch.Generator().manual_seed(14)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.decoder_layer_forward(x.to(DEV), P, cos.to(DEV), sin.to(DEV))
    p = {"in_norm": np.ones(2048, np.float32), "post_norm": np.ones(2048, np.float32),
         "q": wn["q"], "kva": wn["kva"], "kva_norm": wn["kva_norm"], "kvb": wn["kvb"],
         "o": wn["o"], "wg": _bf(M.wg), "gates": _bf(M.gates), "ups": _bf(M.ups),
         "downs": _bf(M.downs), "shared": tuple(_bf(t) for t in M.shared)}
    ref = ol.decoder_layer(np32(x), p)
    assert out.shape == (b, s, 2048)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    # the layer's residual stream dominates max|ref|: check the update the layer
    # adds (attention + MoE) on its own scale too
    upd, rupd = np32(out) - np32(x), ref - np32(x)
    assert max_rel_err(upd, rupd) <= 4 * BF16_TOL


def test_config3_projection_block_full_size(mla_setup):
    """BASELINE config 3 at its full size (b=8, s=2048): every output of the
    projection block against the oracle."""
    dm, w, W, wn = mla_setup
    b, s = 8, 2048
    g = torch.Generator().manual_seed(31)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    outs = dm.mla_projections(x.to(DEV), W, cos.to(DEV), sin.to(DEV))
    refs = ol.mla_projections(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], _bf(cos),
                              _bf(sin))
    for name, o, r in zip(["q_nope", "q_rot", "k_nope", "v", "k_rot", "latent"], outs, refs):
        assert max_rel_err(np32(o), r) <= BF16_TOL, name


def test_config4_decoder_layer_full_size_properties(mla_setup):
    """BASELINE config 4 at its full size (b=4, s=2048), through properties that
    hold at any size: the layer is deterministic (two runs bit-identical), its
    output is finite, and each sequence's rows match the layer run on that
    sequence alone (attention never mixes sequences; routing is per token)."""
    dm, w, W, wn = mla_setup
    from ds_kernels import synthetic as syn
    P = dm.DecoderLayerWeights.from_tensors(w, syn.moe_weights(), torch.device(DEV))
    b, s = 4, 2048
    g = torch.Generator().manual_seed(41)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16).to(DEV)
    cos, sin = dm.yarn_cos_sin(s, device=DEV)
    out1 = dm.decoder_layer_forward(x, P, cos, sin)
    out2 = dm.decoder_layer_forward(x, P, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.isfinite(out1.float()).all()
    one = dm.decoder_layer_forward(x[2:3].contiguous(), P, cos, sin)
    torch.cuda.synchronize()
    assert max_rel_err(np32(one), np32(out1[2:3])) <= BF16_TOL


def _decoder_params(M, wn):
    return {"in_norm": np.ones(2048, np.float32), "post_norm": np.ones(2048, np.float32),
            "q": wn["q"], "kva": wn["kva"], "kva_norm": wn["kva_norm"], "kvb": wn["kvb"],
            "o": wn["o"], "wg": _bf(M.wg), "gates": _bf(M.gates), "ups": _bf(M.ups),
            "downs": _bf(M.downs), "shared": tuple(_bf(t) for t in M.shared)}


@pytest.mark.parametrize("b,s", [(2, 100), (1, 13), (1, 1)])
def test_mla_forward_any_length(mla_setup, b, s):
    """DeepSeekMLA.forward at sequence lengths that are not multiples of 8
    (K^T, scores and V padded to 16-byte rows with zeros) against the oracle."""
    dm, w, W, wn = mla_setup
    g = torch.Generator().manual_seed(100 + s)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.mla_forward(x.to(DEV), W, cos.to(DEV), sin.to(DEV))
    ref = ol.mla_forward(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], wn["o"])
    assert out.shape == (b, s, 2048)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def _padding_mask(b, s, pad, dtype):
    """Additive [b, 1, s, s]: causal, and the last `pad` positions of sequence
    b-1 are padding no query attends to (mla.py:295-315 attention_mask)."""
    i = torch.arange(s)[:, None]
    j = torch.arange(s)[None, :]
    m = torch.zeros(b, 1, s, s).masked_fill(j > i, float("-inf"))
    m[b - 1, :, :, s - pad:] = float("-inf")
    m[b - 1, :, s - pad:, 0] = 0.0          # padded queries still see key 0
    return m.to(dtype)


@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float32])
def test_mla_forward_padded_batch_mask_and_positions(mla_setup, mdtype):
    """A padded batch as a serving stack builds it: an additive mask that hides
    the second sequence's padding, and per-sequence position_ids (the padded
    sequence's positions restart after a left shift), against the oracle's
    forward with the same mask and positions (mla.py:295-315, 349-352, 374)."""
    dm, w, W, wn = mla_setup
    b, s, pad = 2, 64, 16
    g = torch.Generator().manual_seed(71)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    m = _padding_mask(b, s, pad, mdtype)
    pid = torch.stack([torch.arange(s), torch.cat([torch.arange(s - pad),
                                                   torch.zeros(pad, dtype=torch.long)])])
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.mla_forward(x.to(DEV), W, cos.to(DEV), sin.to(DEV), attention_mask=m.to(DEV),
                         position_ids=pid.to(DEV))
    ref = ol.mla_forward(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], wn["o"],
                         attention_mask=m.float().numpy(), position_ids=pid.numpy())
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    # the unpadded rows of sequence 1 do not depend on what sits in its padding
    x2 = x.clone()
    x2[1, s - pad:] = torch.randn(pad, 2048, generator=g).to(torch.bfloat16)
    out2 = dm.mla_forward(x2.to(DEV), W, cos.to(DEV), sin.to(DEV), attention_mask=m.to(DEV),
                          position_ids=pid.to(DEV))
    assert max_rel_err(np32(out2[1, :s - pad]), np32(out[1, :s - pad])) <= BF16_TOL / 4


def test_mla_forward_position_ids_out_of_range(mla_setup):
    dm, w, W, wn = mla_setup
    x = torch.zeros(1, 8, 2048, dtype=torch.bfloat16, device=DEV)
    cos, sin = dm.yarn_cos_sin(8, device=DEV)
    with pytest.raises(IndexError):
        dm.mla_forward(x, W, cos, sin, position_ids=torch.full((1, 8), 8, device=DEV))


def test_decoder_layer_mask_and_positions(mla_setup):
    """Config 4's layer with an attention_mask and position_ids (b=2, s=40)
    against the oracle decoder layer (decoder_layer.py:108-130)."""
    dm, w, W, wn = mla_setup
    from ds_kernels import synthetic as syn
    M = syn.moe_weights()
    P = dm.DecoderLayerWeights.from_tensors(w, M, torch.device(DEV))
    b, s, pad = 2, 40, 8
    g = torch.Generator().manual_seed(72)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    m = _padding_mask(b, s, pad, torch.bfloat16)
    pid = torch.stack([torch.arange(s), torch.arange(s).flip(0)])
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.decoder_layer_forward(x.to(DEV), P, cos.to(DEV), sin.to(DEV),
                                   attention_mask=m.to(DEV), position_ids=pid.to(DEV))
    ref = ol.decoder_layer(np32(x), _decoder_params(M, wn), attention_mask=m.float().numpy(),
                           position_ids=pid.numpy())
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    upd, rupd = np32(out) - np32(x), ref - np32(x)
    assert max_rel_err(upd, rupd) <= 4 * BF16_TOL


def test_mla_forward_longer_than_4096(mla_setup):
    """s = 4100 > 4096 (score rows take the two-pass softmax, keys padded to
    4104) against the oracle forward."""
    dm, w, W, wn = mla_setup
    b, s = 1, 4100
    g = torch.Generator().manual_seed(73)
    x = torch.randn(b, s, 2048, generator=g).to(torch.bfloat16)
    cos, sin = dm.yarn_cos_sin(s)
    out = dm.mla_forward(x.to(DEV), W, cos.to(DEV), sin.to(DEV))
    ref = ol.mla_forward(np32(x), wn["q"], wn["kva"], wn["kva_norm"], wn["kvb"], wn["o"])
    assert max_rel_err(np32(out), ref) <= BF16_TOL

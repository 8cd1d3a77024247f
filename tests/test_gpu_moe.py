"""GPU parity of the MoE ops and the fused layer against the numpy oracle.

Bars: routing indices, counts, offsets, token_map, dispatched rows and weights
bit-exact; bf16 outputs max|d|/max|ref| <= 2e-2 against the fp32 oracle on the
same bf16-rounded inputs; fp32 routing weights <= 1e-5; every output bitwise
identical run to run."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_util import BF16_TOL, F32_TOL, max_rel_err, np32
from oracle import moe as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


@pytest.fixture(scope="module")
def dsk():
    import ds_kernels
    return ds_kernels


# -------------------------------------------------------------- gate logits --
@pytest.mark.parametrize("T,E,H,bias", [(1, 64, 2048, True), (16, 64, 2048, True),
                                        (64, 64, 2048, False), (100, 40, 512, True),
                                        (4096, 64, 2048, False)])
def test_gate_logits_match_fp64(dsk, T, E, H, bias):
    """fp32 logits of bf16 x and gate weight vs the same dot products in fp64
    (the products are exact; only the fp32 summation differs): <= 1e-5."""
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wg = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(E, generator=g)).float() if bias else None
    xd = x.contiguous().to(DEV)
    out = dsk.moe_gate(xd, wg.to(DEV), b.to(DEV) if b is not None else None)
    ref = x.double().numpy() @ wg.double().numpy().T
    if b is not None:
        ref = ref + b.double().numpy()
    assert out.shape == (T, E) and out.dtype == torch.float32
    err = np.abs(out.cpu().double().numpy() - ref).max() / np.abs(ref).max()
    assert err <= F32_TOL, err
    assert torch.equal(out, dsk.moe_gate(xd, wg.to(DEV), b.to(DEV) if b is not None else None))
    if E % 32 == 0:   # fragment-tiled gate weight: same sums, same bits
        wt = dsk.tile_weights(wg[None])[0].to(DEV)
        assert torch.equal(out, dsk.moe_gate(xd, wt, b.to(DEV) if b is not None else None))


def test_gate_logits_strided_rows(dsk):
    g = torch.Generator().manual_seed(5)
    big = torch.randn(48, 2048 + 256, generator=g).to(torch.bfloat16).to(DEV)
    x = big[:, 128:128 + 2048]          # row stride 2304
    wg = (torch.randn(64, 2048, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    out = dsk.moe_gate(x, wg)
    ref = x.double().cpu().numpy() @ wg.double().cpu().numpy().T
    assert np.abs(out.cpu().double().numpy() - ref).max() / np.abs(ref).max() <= F32_TOL


# ------------------------------------------------------------------ routing --
@pytest.mark.parametrize("T,E,K", [(1, 64, 6), (32, 64, 6), (128, 64, 6), (4096, 64, 6),
                                   (100, 16, 4), (65, 64, 1)])
def test_routing_matches_oracle(dsk, T, E, K):
    g = torch.Generator().manual_seed(T * 131 + E)
    logits = torch.randn(T, E, generator=g)
    idx, w, counts = dsk.moe_routing(logits.to(DEV), K)
    ridx, rw, rcounts = om.route(logits.numpy(), K)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(counts.cpu().numpy(), rcounts)
    assert max_rel_err(np32(w), rw) <= F32_TOL
    np.testing.assert_allclose(np32(w), rw, rtol=F32_TOL, atol=1e-7)


def test_routing_all_zero_kat(dsk):
    kat = GOLD["routing_all_zero"]
    logits = torch.zeros(kat["num_tokens"], kat["num_experts"], device=DEV)
    idx, w, counts = dsk.moe_routing(logits, kat["top_k"])
    assert all(r == kat["topk_indices_row"] for r in idx.cpu().tolist())
    assert torch.all(w.cpu() == kat["topk_weight"])
    assert counts.cpu().tolist() == kat["expert_counts"]


def test_routing_ties_and_determinism(dsk):
    logits = torch.randint(-2, 3, (300, 64)).float()   # heavy ties
    a = dsk.moe_routing(logits.to(DEV), 6)
    b = dsk.moe_routing(logits.to(DEV), 6)
    ridx, _, _ = om.route(logits.numpy(), 6)
    np.testing.assert_array_equal(a[0].cpu().numpy(), ridx)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


# --------------------------------------------------------------------- scan --
@pytest.mark.parametrize("case", GOLD["scan"], ids=lambda c: c["name"])
def test_scan_kat(dsk, case):
    counts = torch.tensor(case["counts"], dtype=torch.int32, device=DEV)
    assert dsk.moe_scan(counts).cpu().tolist() == case["offsets"]


# ----------------------------------------------------------------- dispatch --
@pytest.mark.parametrize("T", [1, 32, 128, 1000])
def test_dispatch_matches_oracle(dsk, T):
    g = torch.Generator().manual_seed(T)
    logits = torch.randn(T, 64, generator=g)
    x = torch.randn(T, 2048, generator=g).to(torch.bfloat16)
    idx, w, counts = dsk.moe_routing(logits.to(DEV), 6)
    off = dsk.moe_scan(counts)
    disp, tm, dw = dsk.moe_dispatch(x.to(DEV), idx, w, off)
    ridx, rw, rcounts = om.route(logits.numpy(), 6)
    roff = om.scan(rcounts)
    np.testing.assert_array_equal(off.cpu().numpy(), roff)
    rdisp, rtm, rdw = om.dispatch(np32(x), ridx, np32(w), roff, 64)
    np.testing.assert_array_equal(tm.cpu().numpy(), rtm)
    np.testing.assert_array_equal(np32(dw), rdw)
    np.testing.assert_array_equal(np32(disp), rdisp)
    np.testing.assert_array_equal(np.bincount(rtm, minlength=T), np.full(T, 6))


# ------------------------------------------------------------------ combine --
def _combine_case(dsk, y, tm, dw, T):
    out = dsk.moe_combine(y.to(DEV), tm.to(DEV), dw.to(DEV), T)
    ref = om.combine(np32(y), tm.numpy(), dw.numpy(), T)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    # one rounding of the fp32 sum: within one bf16 ulp of the oracle everywhere
    np.testing.assert_allclose(np32(out), ref, rtol=2 ** -7, atol=1e-6)
    out2 = dsk.moe_combine(y.to(DEV), tm.to(DEV), dw.to(DEV), T)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("T", [1, 7, 128])
def test_combine_random_token_map(dsk, T):
    g = torch.Generator().manual_seed(10 + T)
    S = T * 6
    y = torch.randn(S, 2048, generator=g).to(torch.bfloat16)
    tm = torch.randint(0, T, (S,), generator=g, dtype=torch.int32)
    dw = torch.rand(S, generator=g)
    _combine_case(dsk, y, tm, dw, T)


def test_combine_single_and_multi_slot(dsk):
    g = torch.Generator().manual_seed(0)
    T = 64
    y = torch.randn(T, 2048, generator=g).to(torch.bfloat16)
    _combine_case(dsk, y, torch.arange(T, dtype=torch.int32), torch.rand(T, generator=g), T)
    y6 = torch.randn(T * 6, 2048, generator=g).to(torch.bfloat16)
    tm6 = torch.repeat_interleave(torch.arange(T, dtype=torch.int32), 6)
    _combine_case(dsk, y6, tm6, torch.rand(T * 6, generator=g), T)


def test_combine_zero_weights_and_empty_tokens(dsk):
    g = torch.Generator().manual_seed(1)
    y = torch.randn(60, 2048, generator=g).to(torch.bfloat16)
    tm = torch.randint(0, 5, (60,), generator=g, dtype=torch.int32)   # tokens 5..9 get nothing
    out = dsk.moe_combine(y.to(DEV), tm.to(DEV), torch.zeros(60, device=DEV), 10)
    assert torch.all(out == 0)
    out = dsk.moe_combine(y.to(DEV), tm.to(DEV), torch.rand(60, device=DEV), 10)
    assert torch.all(out[5:] == 0)


# ------------------------------------------------------------------- swiglu --
@pytest.mark.parametrize("rows", [0, 1, 8, 256])
def test_swiglu(dsk, rows):
    g = torch.Generator().manual_seed(rows)
    x = (torch.rand(rows, 2816, generator=g) * 4 - 2).to(torch.bfloat16)
    out = dsk.swiglu(x.to(DEV))
    assert out.shape == (rows, 1408)
    if rows:
        ref = om.swiglu(np32(x))
        assert max_rel_err(np32(out), ref) <= BF16_TOL
        np.testing.assert_allclose(np32(out), ref, rtol=1e-2, atol=1e-2)


# -------------------------------------------------------------------- GEMMs --
def _round_robin_offsets(S, E):
    counts = np.array([len(range(e, S, E)) for e in range(E)], np.int32)
    return om.scan(counts)


def _gemm_inputs(S, N, K, E, seed):
    g = torch.Generator().manual_seed(seed)
    a = (torch.rand(S, K, generator=g) * 2 - 1).to(torch.bfloat16)
    w = (torch.rand(E, N, K, generator=g) * 0.1).to(torch.bfloat16)
    return a, w


@pytest.mark.parametrize("T", [1, 8, 32, 128])
def test_gemm1_round_robin(dsk, T):
    """test_moe_gemm1.py:58-119 shapes: 2048 -> 2816, round-robin offsets."""
    S, E = T * 6, 64
    a, w = _gemm_inputs(S, 2816, 2048, E, T)
    off = _round_robin_offsets(S, E)
    out = dsk.moe_gemm1(a.to(DEV), w.to(DEV), torch.from_numpy(off).to(DEV))
    ref = om.grouped_linear(np32(a), np32(w), off)
    assert out.shape == (S, 2816)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("T", [1, 32, 128])
def test_gemm2_round_robin(dsk, T):
    S, E = T * 6, 64
    a, w = _gemm_inputs(S, 2048, 1408, E, 100 + T)
    off = _round_robin_offsets(S, E)
    out = dsk.moe_gemm2(a.to(DEV), w.to(DEV), torch.from_numpy(off).to(DEV))
    ref = om.grouped_linear(np32(a), np32(w), off)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


def test_gemm_skewed_groups_and_uncovered_rows(dsk):
    """Empty experts, one big expert, partial tiles, rows past offsets[E] = 0."""
    E = 8
    counts = np.array([0, 300, 1, 0, 33, 129, 0, 64], np.int32)
    off = om.scan(counts)
    S = int(off[-1]) + 5
    a, w = _gemm_inputs(S, 512, 256, E, 7)
    out = dsk.moe_gemm2(a.to(DEV), w.to(DEV), torch.from_numpy(off).to(DEV))
    ref = om.grouped_linear(np32(a), np32(w), off)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    assert torch.all(out[int(off[-1]):] == 0)


@pytest.mark.parametrize("counts", [[64], [33, 0, 31], [1, 0, 0, 17, 32, 0, 14], [0, 0, 5]])
def test_gemm_small_groups(dsk, counts):
    """At most 64 slots in total: the small-group (decode) kernel, with 1 and 2
    token blocks, empty groups, and rows past the last group left at zero."""
    E = len(counts)
    off = om.scan(np.array(counts, np.int32))
    S = int(off[-1]) + 2
    offd = torch.from_numpy(off).to(DEV)
    a, w = _gemm_inputs(S, 2816, 2048, E, 300 + S)
    ref1 = om.grouped_linear(np32(a), np32(w), off)
    out = dsk.moe_gemm1(a.to(DEV), w.to(DEV), offd)
    assert max_rel_err(np32(out), ref1) <= BF16_TOL
    assert torch.all(out[int(off[-1]):] == 0)
    sw = dsk.moe_gemm1_swiglu(a.to(DEV), w.to(DEV), offd)
    assert max_rel_err(np32(sw), om.swiglu(ref1)) <= BF16_TOL
    h, w2 = _gemm_inputs(S, 2048, 1408, E, 400 + S)
    out2 = dsk.moe_gemm2(h.to(DEV), w2.to(DEV), offd)
    assert max_rel_err(np32(out2), om.grouped_linear(np32(h), np32(w2), off)) <= BF16_TOL


@pytest.mark.parametrize("I", [1400, 100])
def test_gemm1_swiglu_few_groups_ragged_width(dsk, I):
    """Few busy groups (the grid of a one-token step) run SwiGLU in 16-column
    units; with an intermediate size that is not a multiple of 16 the last unit
    reads clamped weight rows and writes only the columns below I."""
    counts = [1, 0, 3, 2]
    E = len(counts)
    off = om.scan(np.array(counts, np.int32))
    S = int(off[-1])
    offd = torch.from_numpy(off).to(DEV)
    a, w = _gemm_inputs(S, 2 * I, 2048, E, 500 + I)
    ref = om.swiglu(om.grouped_linear(np32(a), np32(w), off))
    out = dsk.moe_gemm1_swiglu(a.to(DEV), w.to(DEV), offd)
    assert out.shape == (S, I)
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    unfused = dsk.swiglu(dsk.moe_gemm1(a.to(DEV), w.to(DEV), offd))
    assert max_rel_err(np32(unfused), ref) <= BF16_TOL


def test_gemm_small_groups_caller_offsets_not_sorted(dsk):
    """Offsets from a caller need not increase: here busy groups (3) outnumber
    the rows (2), group 4 alone covers row 1, and groups 0, 2 and 4 (identical
    weights) all cover row 0. Every busy group must run on the small-group
    path (none dropped), so both rows equal x @ W^T (the reference loops over
    every expert's range, gemm1.cu:94-123)."""
    g = torch.Generator().manual_seed(77)
    H, N = 2048, 2816
    a = torch.randn(2, H, generator=g).to(torch.bfloat16)
    w0 = (torch.randn(N, H, generator=g) * 0.02).to(torch.bfloat16)
    w = torch.stack([w0 if e % 2 == 0 else torch.zeros_like(w0) for e in range(5)])
    off = torch.tensor([0, 1, 0, 1, 0, 2], dtype=torch.int32)
    out = dsk.moe_gemm1(a.to(DEV), w.to(DEV), off.to(DEV))
    ref = np32(a) @ np32(w0).T
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    out2 = dsk.moe_gemm2(a[:, :1408].contiguous().to(DEV), w[:, :, :1408].contiguous().to(DEV),
                         off.to(DEV))
    ref2 = np32(a[:, :1408]) @ np32(w0[:, :1408]).T
    assert max_rel_err(np32(out2), ref2) <= BF16_TOL


def test_gemm_zero_slots(dsk):
    out = dsk.moe_gemm1(torch.empty(0, 2048, dtype=torch.bfloat16, device=DEV),
                        torch.zeros(64, 2816, 2048, dtype=torch.bfloat16, device=DEV),
                        torch.zeros(65, dtype=torch.int32, device=DEV))
    assert out.shape == (0, 2816)


@pytest.mark.parametrize("T", [1, 64, 512])
def test_gemm1_swiglu_fused(dsk, T):
    S, E = T * 6, 64
    a, w = _gemm_inputs(S, 2816, 2048, E, 200 + T)
    off = _round_robin_offsets(S, E)
    offd = torch.from_numpy(off).to(DEV)
    out = dsk.moe_gemm1_swiglu(a.to(DEV), w.to(DEV), offd)
    ref = om.swiglu(om.grouped_linear(np32(a), np32(w), off))
    assert max_rel_err(np32(out), ref) <= BF16_TOL
    unfused = dsk.swiglu(dsk.moe_gemm1(a.to(DEV), w.to(DEV), offd))
    assert max_rel_err(np32(unfused), ref) <= BF16_TOL


# ------------------------------------------------------------- fused layer --
def _oracle_layer(Wn, x_bf, logits, K, shared=True):
    return om.moe_layer(np32(x_bf), None, Wn["gates"], Wn["ups"], Wn["downs"], K,
                        shared=Wn["shared"] if shared else None, logits=logits)


@pytest.fixture(scope="module")
def full_layer(dsk):
    """Layer weights on the GPU (bf16, packed) and their bf16-rounded fp32
    numpy copies for the oracle."""
    from ds_kernels import synthetic as syn
    W = syn.moe_weights()
    w1, w2, nsh = dsk.pack_tensors(W.gates, W.ups, W.downs, device=torch.device(DEV),
                                   shared=W.shared)
    wb = lambda t: t.to(torch.bfloat16).float().numpy()  # noqa: E731
    Wn = {"gates": wb(W.gates), "ups": wb(W.ups), "downs": wb(W.downs),
          "shared": tuple(wb(t) for t in W.shared)}
    return W, w1, w2, nsh, Wn


@pytest.fixture(scope="module")
def tiled_layer(dsk, full_layer):
    W, w1, w2, nsh, Wn = full_layer
    return dsk.tile_weights(w1), dsk.tile_weights(w2)


@pytest.mark.parametrize("layout", ["row_major", "tiled"])
@pytest.mark.parametrize("T,bias", [(64, False), (4096, False), (1, True), (4, True),
                                    (16, True), (64, True), (100, True), (2048, False),
                                    (2048, True), (6000, False)])
def test_fused_layer_matches_oracle(dsk, full_layer, tiled_layer, T, bias, layout):
    """Configs 0/1 (near-uniform routing) and 2 (Zipf-biased router), bf16, with
    the expert weights row-major or fragment-tiled. T = 2048, 4096 and 6000 deal
    the large-group GEMMs' tiles one routed group (1, 2, 3 M tiles) per chunk;
    with the Zipf router the groups are far from that size, so chunks straddle
    groups."""
    from ds_kernels import synthetic as syn
    W, w1, w2, nsh, Wn = full_layer
    if layout == "tiled":
        w1, w2 = tiled_layer
    x = syn.tokens(T).to(torch.bfloat16)
    xd = x.to(DEV)
    logits = F.linear(xd.float(), W.wg.to(torch.bfloat16).float().to(DEV))
    if bias:
        logits = logits + syn.zipf_router_bias().to(DEV)
    logits = logits.contiguous()
    out, (idx, w, off) = dsk.moe_fused_forward_logits(logits, xd, w1, w2, 6, nsh, 64,
                                                      return_routing=True)
    lg = logits.cpu().numpy()
    ridx, rw, rcounts = om.route(lg, 6)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(off.cpu().numpy(), om.scan(rcounts))
    np.testing.assert_allclose(np32(w), rw, rtol=F32_TOL, atol=1e-7)
    ref = _oracle_layer(Wn, x, lg, 6)
    err = max_rel_err(np32(out), ref)
    assert err <= BF16_TOL, err
    out2 = dsk.moe_fused_forward_logits(logits, xd, w1, w2, 6, nsh, 64)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("layout", ["row_major", "tiled"])
@pytest.mark.parametrize("T,bias", [(1, True), (16, True), (64, True), (100, False),
                                    (4096, False)])
def test_layer_forward_with_gate_matches_oracle(dsk, full_layer, tiled_layer, T, bias, layout):
    """Gate included (fp32 K-slice sums of bf16 products, added by the router).

    The reference's logits are F.linear(x.float(), W.float()) (moe_fused.py:131),
    whose fp32 summation order is the BLAS's; this library sums in another
    order. Both are within gate_logit_error_bound of the exact (fp64) logits,
    so routing is pinned against the exact logits:
      * tokens whose exact top-7 logits are more than twice the bound apart at
        every gap must get the exact top-6 bit for bit (indices and order);
      * the others (at T=4096 the smallest gap is 2e-6 against a bound near
        5e-4) must get a choice that some fp32 evaluation inside the bound makes.
    Offsets are bit-exact against the oracle's when every token's selection
    equals the exact one, and always equal the scan of the returned indices.
    Weights are the softmax at the chosen experts (1e-5); the layer output is
    within the bf16 bar on every token whose selection equals the oracle's."""
    from ds_kernels import synthetic as syn
    from gpu_util import assert_routing_admissible, gate_logit_error_bound, routing_safe_tokens
    W, w1, w2, nsh, Wn = full_layer
    wg = W.wg.to(torch.bfloat16)
    if layout == "tiled":
        w1, w2 = tiled_layer
        wgd = dsk.tile_weights(wg[None])[0].to(DEV)
    else:
        wgd = wg.to(DEV)
    x = syn.tokens(T).to(torch.bfloat16)
    b = syn.zipf_router_bias() if bias else None
    out, (idx, w, off) = dsk.moe_layer_forward(x.to(DEV), wgd, w1, w2, 6, nsh,
                                               gate_bias=b.to(DEV) if bias else None,
                                               return_routing=True)
    lg = x.double().numpy() @ wg.double().numpy().T
    if bias:
        lg = lg + b.double().numpy()
    bound = gate_logit_error_bound(x.double().numpy(), wg.double().numpy(),
                                   b.numpy() if bias else None)
    safe, margin = routing_safe_tokens(lg, bound, 6)
    ridx, _, rcounts = om.route(lg.astype(np.float32), 6)
    gidx = idx.cpu().numpy()
    np.testing.assert_array_equal(gidx[safe], ridx[safe])
    assert_routing_admissible(gidx, lg, bound)
    same = (gidx == ridx).all(axis=1)
    print(f"T={T}: {int((~safe).sum())} of {T} tokens within the fp32 bound "
          f"(min gap {margin.min():.3g}); {int((~same).sum())} selections differ from fp64")
    gcounts = np.bincount(gidx.ravel(), minlength=64)
    np.testing.assert_array_equal(off.cpu().numpy(), om.scan(gcounts))
    if same.all():
        np.testing.assert_array_equal(off.cpu().numpy(), om.scan(rcounts))
    p = om.softmax(lg.astype(np.float32))
    np.testing.assert_allclose(np32(w), np.take_along_axis(p, gidx.astype(np.int64), axis=1),
                               rtol=1e-5, atol=1e-7)
    ref = _oracle_layer(Wn, x, lg.astype(np.float32), 6)
    assert max_rel_err(np32(out)[same], ref[same]) <= BF16_TOL
    out2 = dsk.moe_layer_forward(x.to(DEV), wgd, w1, w2, 6, nsh,
                                 gate_bias=b.to(DEV) if bias else None)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("case", ["random", "zipf", "all_tied", "neg_inf"])
def test_single_token_routing_in_gemm_matches_route_kernel(dsk, full_layer, tiled_layer, case):
    """At T = 1 the fused layer routes inside GEMM1's prologue (no route launch).
    Its routing outputs must be the route kernel's (moe_routing on the same
    logits) bit for bit: expert indices and order, weights, offsets (the scan of
    the counts); ties go to the lower index and -inf experts are never picked
    while finite ones remain."""
    from ds_kernels import synthetic as syn
    W, w1, w2, nsh, Wn = full_layer
    w1, w2 = tiled_layer
    g = torch.Generator().manual_seed(7)
    if case == "all_tied":
        logits = torch.zeros(1, 64)
    else:
        logits = torch.randn(1, 64, generator=g)
        if case == "zipf":
            logits = logits + syn.zipf_router_bias()
        if case == "neg_inf":
            logits[0, ::3] = -float("inf")
    logits = logits.float().contiguous().to(DEV)
    x = syn.tokens(1).to(torch.bfloat16).to(DEV)
    out, (idx, w, off) = dsk.moe_fused_forward_logits(logits, x, w1, w2, 6, nsh, 64,
                                                      return_routing=True)
    ridx, rw, rcounts = dsk.moe_routing(logits, 6)
    assert torch.equal(idx, ridx)
    assert torch.equal(w, rw)
    assert torch.equal(off, dsk.moe_scan(rcounts))
    if case == "all_tied":
        assert idx.cpu().tolist() == [[0, 1, 2, 3, 4, 5]]
    if case == "neg_inf":
        assert all(int(e) % 3 != 0 for e in idx.cpu().ravel())
    lg = logits.cpu().numpy()
    ref = _oracle_layer(Wn, x.cpu(), lg, 6)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("T", [16, 300])
def test_layer_forward_graph_replay_matches_eager(dsk, full_layer, tiled_layer, T):
    """The layer captured in a HIP graph (T=16: single routing launch and the
    small-group GEMMs; T=300: scan and permutation kernels and the large-group
    GEMMs) gives the eager result bit for bit on every replay, with eager layer
    calls on other inputs between the replays."""
    from ds_kernels import synthetic as syn
    W, _, _, nsh, _ = full_layer
    w1, w2 = tiled_layer
    wgd = dsk.tile_weights(W.wg.to(torch.bfloat16)[None])[0].to(DEV)
    bias = syn.zipf_router_bias().to(DEV)
    x = syn.tokens(T).to(torch.bfloat16).to(DEV)
    x_other = syn.tokens(T + 7).to(torch.bfloat16).to(DEV)
    ref = dsk.moe_layer_forward(x, wgd, w1, w2, 6, nsh, gate_bias=bias)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = dsk.moe_layer_forward(x, wgd, w1, w2, 6, nsh, gate_bias=bias)
    for _ in range(3):
        out.zero_()
        dsk.moe_layer_forward(x_other, wgd, w1, w2, 6, nsh, gate_bias=bias)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    del g


def test_op_pipeline_matches_fused(dsk, full_layer):
    """Reference call sequence (routing->scan->dispatch->gemm1->swiglu->gemm2->combine),
    routed experts only, vs the oracle without shared experts."""
    from ds_kernels import synthetic as syn
    W, w1, w2, nsh, Wn = full_layer
    T = 256
    x = syn.tokens(T).to(torch.bfloat16)
    xd = x.to(DEV)
    wg = W.wg.to(DEV)
    packed_w1 = w1[:64].contiguous()
    packed_w2 = w2[:64].contiguous()
    out = dsk.route_dispatch_combine(xd, wg, packed_w1, packed_w2, 6)
    out_f = dsk.route_dispatch_combine(xd, wg, packed_w1, packed_w2, 6, fuse_swiglu=True)
    fused = dsk.fused_moe_forward(xd, wg, None, 6, packed_w1, packed_w2)
    lg = F.linear(xd.float(), wg.float()).cpu().numpy()
    ref = _oracle_layer(Wn, x, lg, 6, shared=False)
    for o in (out, out_f, fused):
        assert max_rel_err(np32(o), ref) <= BF16_TOL


def test_concurrent_calls_on_two_streams(dsk, full_layer, tiled_layer):
    """The library keeps no per-call global state (thread-local error text and
    per-device caches only), so calls from two host threads, each on its own
    stream, run side by side. Each thread runs the fused layer 4 times (T = 16 and
    T = 4096); every result equals the single-threaded one bit for bit."""
    import threading
    from ds_kernels import synthetic as syn
    W, _, _, nsh, _ = full_layer
    w1, w2 = tiled_layer
    wgd = dsk.tile_weights(W.wg.to(torch.bfloat16)[None])[0].to(DEV)
    xs = [syn.tokens(T, seed=s).to(torch.bfloat16).to(DEV) for T, s in ((16, 1), (4096, 2))]
    ref = [dsk.moe_layer_forward(x, wgd, w1, w2, 6, nsh) for x in xs]
    torch.cuda.synchronize()
    results = [[None] * 4 for _ in xs]
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for r in range(4):
                    results[i][r] = dsk.moe_layer_forward(xs[i], wgd, w1, w2, 6, nsh)
            s.synchronize()
        except Exception as e:  # handed to the main thread
            errors.append(e)

    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=60)
    assert not errors, errors
    for i in range(2):
        for r in range(4):
            assert torch.equal(results[i][r], ref[i]), (i, r)


@pytest.mark.parametrize("T,E,K,nsh", [(65, 8, 1, 0), (100, 16, 2, 2), (300, 64, 6, 2),
                                       (1000, 8, 1, 2), (777, 64, 3, 0), (4097, 16, 6, 2)])
def test_fused_layer_small_shapes_routing_and_output(dsk, T, E, K, nsh):
    """The T > 64 routing of the fused layer (route, then the scan and the
    permutation in one kernel, 32 tokens per workgroup) for other expert counts,
    top-k values, token counts that are not multiples of 32 or 64, and with or
    without shared groups: offsets and indices bit-exact against the oracle,
    the layer output within the bf16 bar."""
    H, I = 256, 128
    g = torch.Generator().manual_seed(T * 7 + E + K)
    gates = (torch.randn(E, I, H, generator=g) * 0.05).to(torch.bfloat16)
    ups = (torch.randn(E, I, H, generator=g) * 0.05).to(torch.bfloat16)
    downs = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    shared = None
    if nsh:
        shared = tuple((torch.randn(*s, generator=g) * 0.05).to(torch.bfloat16)
                       for s in ((nsh * I, H), (nsh * I, H), (H, nsh * I)))
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    w1, w2, n = dsk.pack_tensors(gates, ups, downs, device=torch.device(DEV), shared=shared)
    assert n == nsh
    out, (idx, w, off) = dsk.moe_fused_forward_logits(logits.to(DEV), x.to(DEV), w1, w2, K, n,
                                                      E, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.numpy()
    ridx, rw, rcounts = om.route(lg, K)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    roff = om.scan(rcounts)
    np.testing.assert_array_equal(off.cpu().numpy()[:E + 1], roff)
    f = lambda t: t.float().numpy()  # noqa: E731
    ref = om.moe_layer(f(x), None, f(gates), f(ups), f(downs), K,
                       shared=tuple(f(t) for t in shared) if shared else None, logits=lg)
    assert max_rel_err(np32(out), ref) <= BF16_TOL


# -------------------------------------------- module-level drop-in (a10) --
# A DeepSeekMoE-shaped module (reference moe.py:6-75: gate.weight,
# experts[i].{gate,up,down}_proj as bias-free nn.Linear, shared_experts,
# num_experts_per_tok) built from the seeded synthetic weights, as the
# reference's e2e test builds DeepSeekMoE and hands it to FusedMoELayer
# (tests/test_fused_moe_e2e.py:56-91).
class _ExpertMLP(torch.nn.Module):
    def __init__(self, gate, up, down):
        super().__init__()
        mk = lambda w: torch.nn.Linear(w.shape[1], w.shape[0], bias=False,  # noqa: E731
                                       device=DEV, dtype=torch.bfloat16)
        self.gate_proj, self.up_proj, self.down_proj = mk(gate), mk(up), mk(down)
        with torch.no_grad():
            for lin, w in ((self.gate_proj, gate), (self.up_proj, up), (self.down_proj, down)):
                lin.weight.copy_(w.to(DEV))


class _Gate(torch.nn.Module):
    def __init__(self, weight):
        super().__init__()
        self.weight = torch.nn.Parameter(weight.to(DEV), requires_grad=False)


class _MoEModule(torch.nn.Module):
    def __init__(self, W, gate_dtype, shared=True):
        super().__init__()
        self.num_experts_per_tok = 6
        self.gate = _Gate(W.wg.to(gate_dtype))
        self.experts = torch.nn.ModuleList(
            [_ExpertMLP(W.gates[e], W.ups[e], W.downs[e]) for e in range(W.gates.shape[0])])
        self.shared_experts = _ExpertMLP(*W.shared) if shared else None


@pytest.fixture(scope="module")
def moe_modules(full_layer):
    W = full_layer[0]
    return {"bf16": _MoEModule(W, torch.bfloat16), "fp32": _MoEModule(W, torch.float32),
            "no_shared": _MoEModule(W, torch.bfloat16, shared=False)}


def test_prepack_experts_and_verify(dsk, moe_modules):
    """prepack_experts on the module's experts gives the reference layouts
    (expert_prepack.py:105-130: [E, 2I, H] gate rows then up rows, [E, H, I]),
    verify_prepack agrees, and prepack_with_shared appends the shared expert
    as two width-I groups (tiled and row-major)."""
    m = moe_modules["bf16"]
    experts = list(m.experts)
    w1, w2 = dsk.prepack_experts(experts)
    assert tuple(w1.shape) == (64, 2816, 2048) and tuple(w2.shape) == (64, 2048, 1408)
    assert w1.dtype == torch.bfloat16 and w1.is_cuda
    for e in (0, 17, 63):
        assert torch.equal(w1[e, :1408], experts[e].gate_proj.weight)
        assert torch.equal(w1[e, 1408:], experts[e].up_proj.weight)
        assert torch.equal(w2[e], experts[e].down_proj.weight)
    assert dsk.verify_prepack(experts)
    rw1, rw2, nsh = dsk.prepack_with_shared(experts, m.shared_experts, tiled=False)
    assert nsh == 2 and tuple(rw1.shape) == (66, 2816, 2048)
    assert torch.equal(rw1[:64], w1) and torch.equal(rw2[:64], w2)
    sh = m.shared_experts
    for j in range(2):
        sl = slice(j * 1408, (j + 1) * 1408)
        assert torch.equal(rw1[64 + j, :1408], sh.gate_proj.weight[sl])
        assert torch.equal(rw1[64 + j, 1408:], sh.up_proj.weight[sl])
        assert torch.equal(rw2[64 + j], sh.down_proj.weight[:, sl])
    tw1, tw2, _ = dsk.prepack_with_shared(experts, m.shared_experts)
    assert torch.equal(dsk.untile_weights(tw1), rw1) and torch.equal(dsk.untile_weights(tw2), rw2)
    with pytest.raises(RuntimeError, match="CUDA device"):
        dsk.prepack_experts([_cpu_expert()])
    with pytest.raises(AttributeError, match="missing attribute 'gate_proj'"):
        dsk.prepack_experts([torch.nn.Linear(4, 4)])


def _cpu_expert():
    e = torch.nn.Module()
    for n, shp in (("gate_proj", (8, 16)), ("up_proj", (8, 16)), ("down_proj", (16, 8))):
        setattr(e, n, torch.nn.Linear(shp[1], shp[0], bias=False))
    return e


@pytest.mark.parametrize("gate", ["bf16", "fp32"])
@pytest.mark.parametrize("T", [1, 16, 128, 4096])
def test_fused_moe_layer_module(dsk, full_layer, moe_modules, gate, T):
    """FusedMoELayer(module)(x) against the oracle DeepSeekMoE.forward.

    bf16 gate weight: the layer runs the library's gate (fragment-tiled gate
    weight, one call for the whole layer); routing is pinned against the exact
    logits as in test_layer_forward_with_gate_matches_oracle. fp32 gate weight:
    the layer keeps torch's fp32 linear for the logits (the reference's own
    formula), and the oracle gets the same logits. The output equals the
    lower-level call on the module's own packed weights bit for bit, and is
    within the bf16 bar of the oracle on every token routed as the oracle
    routes it. A 3-D input gives the same rows."""
    from gpu_util import assert_routing_admissible, gate_logit_error_bound, routing_safe_tokens
    from ds_kernels import synthetic as syn
    W, _, _, _, Wn = full_layer
    m = moe_modules[gate]
    layer = dsk.FusedMoELayer(m)
    x = syn.tokens(T, seed=7).to(torch.bfloat16)
    xd = x.to(DEV)
    out = layer(xd)
    assert out.shape == (T, 2048) and out.dtype == torch.bfloat16
    if gate == "bf16":
        assert layer.gate_weight.dim() == 4          # tiled for the gate kernel
        same_call, (idx, _, _) = dsk.moe_layer_forward(xd, layer.gate_weight, layer.w1, layer.w2,
                                                       6, layer.n_shared_groups,
                                                       return_routing=True)
        lg = x.double().numpy() @ W.wg.to(torch.bfloat16).double().numpy().T
        bound = gate_logit_error_bound(x.double().numpy(),
                                       W.wg.to(torch.bfloat16).double().numpy())
        safe, _ = routing_safe_tokens(lg, bound, 6)
        gidx = idx.cpu().numpy()
        ridx, _, _ = om.route(lg.astype(np.float32), 6)
        np.testing.assert_array_equal(gidx[safe], ridx[safe])
        assert_routing_admissible(gidx, lg, bound)
        lg32 = lg.astype(np.float32)
    else:
        assert layer.gate_weight.dtype == torch.float32
        logits = F.linear(xd.float(), layer.gate_weight)
        same_call, (idx, _, _) = dsk.moe_fused_forward_logits(
            logits, xd, layer.w1, layer.w2, 6, layer.n_shared_groups, 64, return_routing=True)
        lg32 = logits.cpu().numpy()
        gidx = idx.cpu().numpy()
        np.testing.assert_array_equal(gidx, om.route(lg32, 6)[0])
    assert torch.equal(out, same_call)
    same = (gidx == om.route(lg32, 6)[0]).all(axis=1)
    ref = _oracle_layer(Wn, x, lg32, 6)
    assert max_rel_err(np32(out)[same], ref[same]) <= BF16_TOL
    if T % 4 == 0:
        out3 = layer(xd.view(4, T // 4, 2048))
        assert out3.shape == (4, T // 4, 2048)
        assert torch.equal(out3.reshape(T, 2048), out)


@pytest.mark.parametrize("T", [1, 16, 128])
def test_fused_moe_module_without_shared_and_functional_api(dsk, full_layer, moe_modules, T):
    """The reference e2e test's two APIs with shared experts disabled
    (test_fused_moe_e2e.py:33,56-91): FusedMoELayer on a module without
    shared_experts, and fused_moe_forward(x, gate_weight, experts) packing the
    experts on first use and reusing the cached pack on the second call. Both
    compute the logits with the library's gate (bf16 weight), so each output is
    compared with the oracle on the tokens whose selection equals the exact
    logits' (all tokens outside the fp32 error bound, see
    test_layer_forward_with_gate_matches_oracle)."""
    from ds_kernels import moe_fused
    from ds_kernels import synthetic as syn
    W, _, _, _, Wn = full_layer
    m = moe_modules["no_shared"]
    layer = dsk.FusedMoELayer(m)
    assert layer.n_shared_groups == 0
    x = syn.tokens(T, seed=9).to(torch.bfloat16)
    xd = x.to(DEV)
    out = layer(xd)
    _, (idx_layer, _, _) = dsk.moe_layer_forward(xd, layer.gate_weight, layer.w1, layer.w2, 6, 0,
                                                 return_routing=True)
    experts = list(m.experts)
    f1 = dsk.fused_moe_forward(xd, m.gate.weight, experts, top_k=6)
    assert id(experts) in moe_fused._WEIGHT_CACHE
    assert moe_fused._WEIGHT_CACHE[id(experts)][0].dim() == 5   # cached fragment-tiled
    f2 = dsk.fused_moe_forward(xd, m.gate.weight, experts, top_k=6)
    assert torch.equal(f1, f2)
    # the reference layout passed explicitly: the row-major kernels, the same bits
    rw1, rw2 = dsk.prepack_experts(experts)
    f3 = dsk.fused_moe_forward(xd, m.gate.weight, None, 6, rw1, rw2)
    assert torch.equal(f1, f3)
    idx_fn = om.route(dsk.moe_gate(xd, m.gate.weight).cpu().numpy(), 6)[0]
    lg32 = (x.double().numpy() @ W.wg.to(torch.bfloat16).double().numpy().T).astype(np.float32)
    ridx = om.route(lg32, 6)[0]
    ref = _oracle_layer(Wn, x, lg32, 6, shared=False)
    for o, gi in ((out, idx_layer.cpu().numpy()), (f1, idx_fn)):
        same = (gi == ridx).all(axis=1)
        assert same.mean() >= 0.9
        assert max_rel_err(np32(o)[same], ref[same]) <= BF16_TOL
    moe_fused._WEIGHT_CACHE.pop(id(experts), None)

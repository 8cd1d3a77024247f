"""Pins the numpy MoE oracle (CPU only) against the reference tests' known
answers, library routines and brute-force definitions."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as om

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


@pytest.mark.parametrize("case", GOLD["scan"], ids=lambda c: c["name"])
def test_scan_kat(case):
    np.testing.assert_array_equal(om.scan(np.array(case["counts"], np.int32)),
                                  np.array(case["offsets"], np.int32))


def test_routing_all_zero_kat():
    kat = GOLD["routing_all_zero"]
    logits = np.zeros((kat["num_tokens"], kat["num_experts"]), np.float32)
    idx, w, counts = om.route(logits, kat["top_k"])
    for r in range(kat["num_tokens"]):
        assert idx[r].tolist() == kat["topk_indices_row"]
    assert np.all(w == np.float32(kat["topk_weight"]))
    assert counts.tolist() == kat["expert_counts"]


def test_routing_matches_torch_topk_without_ties():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(513, 64, generator=g)
    idx, w, counts = om.route(logits.numpy(), 6)
    tw, ti = torch.topk(torch.softmax(logits, -1), 6, dim=-1, sorted=True)
    np.testing.assert_array_equal(idx, ti.numpy())          # same set and descending order
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-6, atol=0)
    assert counts.sum() == 513 * 6
    np.testing.assert_array_equal(counts, np.bincount(ti.numpy().ravel(), minlength=64))


def test_routing_partial_tie_goes_to_lower_index():
    logits = np.full((2, 64), -5.0, np.float32)
    logits[:, [7, 3, 60, 11, 20]] = [4.0, 3.0, 2.0, 1.0, 0.5]
    logits[:, [40, 9]] = 0.25        # two-way tie for the 6th place
    idx, w, _ = om.route(logits, 6)
    assert idx[0].tolist() == [7, 3, 60, 11, 20, 9]
    # weights are softmax probabilities in descending order
    assert np.all(np.diff(w[0]) <= 0)


def test_routing_brute_force_small():
    rng = np.random.default_rng(1)
    logits = rng.integers(-3, 4, size=(40, 8)).astype(np.float32)   # many ties
    idx, w, counts = om.route(logits, 3)
    for t in range(40):
        picked = []
        for _ in range(3):
            best = None
            for e in range(8):
                if e in picked:
                    continue
                if best is None or logits[t, e] > logits[t, best]:
                    best = e
            picked.append(best)
        assert idx[t].tolist() == picked
        ex = np.exp(logits[t] - logits[t].max())
        np.testing.assert_allclose(w[t], (ex / ex.sum())[picked], rtol=1e-6)


def _random_routing(T, E, K, seed):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    counts = np.bincount(idx.ravel(), minlength=E).astype(np.int32)
    return idx, w, counts


def test_permute_brute_force_definition():
    T, E, K = 23, 8, 3
    idx, w, counts = _random_routing(T, E, K, 2)
    off = om.scan(counts)
    token_map, dw, slot_of = om.permute(idx, w, off, E)
    # definition: slot(t,k) = offsets[e] + #{t' < t : e in idx[t']}
    for t in range(T):
        for k in range(K):
            e = idx[t, k]
            rank = sum(1 for t2 in range(t) if e in idx[t2].tolist())
            s = off[e] + rank
            assert slot_of[t, k] == s
            assert token_map[s] == t
            assert dw[s] == w[t, k]


def test_dispatch_invariants():
    """Invariants of the reference dispatch test (test_moe_dispatch_kernel.py:114-210)."""
    T, E, K, H = 64, 64, 6, 16
    idx, w, counts = _random_routing(T, E, K, 3)
    off = om.scan(counts)
    x = np.random.default_rng(4).standard_normal((T, H)).astype(np.float32)
    disp, token_map, dw = om.dispatch(x, idx, w, off, E)
    np.testing.assert_array_equal(np.bincount(token_map, minlength=T), np.full(T, K))
    for e in range(E):
        seg = token_map[off[e]:off[e + 1]]
        assert set(seg.tolist()) == set(np.nonzero((idx == e).any(1))[0].tolist())
        assert np.all(np.diff(seg) > 0)                    # ascending tokens
    np.testing.assert_array_equal(disp, x[token_map])     # exact row copy
    np.testing.assert_array_equal(dw, w[token_map, [list(idx[t]).index(e) for t, e in
                                                    zip(token_map, np.repeat(np.arange(E), counts))]])


def test_grouped_linear_matches_torch_linear():
    rng = np.random.default_rng(5)
    E, N, Kd = 5, 24, 32
    counts = np.array([3, 0, 7, 1, 4], np.int32)
    off = om.scan(counts)
    S = int(off[-1]) + 2                                   # two uncovered rows at the end
    a = rng.standard_normal((S, Kd)).astype(np.float32)
    wt = rng.standard_normal((E, N, Kd)).astype(np.float32)
    out = om.grouped_linear(a, wt, off)
    for e in range(E):
        s0, s1 = off[e], off[e + 1]
        ref = F.linear(torch.from_numpy(a[s0:s1]), torch.from_numpy(wt[e])).numpy()
        np.testing.assert_allclose(out[s0:s1], ref, rtol=1e-5, atol=1e-5)
    assert np.all(out[off[-1]:] == 0)


def test_swiglu_matches_torch_silu():
    x = np.random.default_rng(6).uniform(-8, 8, (17, 2 * 40)).astype(np.float32)
    ref = (F.silu(torch.from_numpy(x[:, :40])) * torch.from_numpy(x[:, 40:])).numpy()
    np.testing.assert_allclose(om.swiglu(x), ref, rtol=1e-5, atol=1e-6)


def test_combine_brute_force_and_zero_weights():
    rng = np.random.default_rng(7)
    S, T, H = 50, 9, 8
    y = rng.standard_normal((S, H)).astype(np.float32)
    tm = rng.integers(0, T, S).astype(np.int32)
    dw = rng.random(S).astype(np.float32)
    out = om.combine(y, tm, dw, T)
    ref = np.zeros((T, H), np.float64)
    for s in range(S):                                     # test_moe_combine_kernel.py:47-64
        ref[tm[s]] += y[s].astype(np.float64) * dw[s]
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    assert np.all(om.combine(y, tm, np.zeros(S, np.float32), T) == 0)


def test_bf16_round_matches_torch():
    x = np.random.default_rng(8).standard_normal(10000).astype(np.float32) * 100
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(om.bf16_round(x), ref)


def test_moe_layer_matches_dense_formulation():
    """Per-expert loop oracle vs every expert on every token, masked by the
    routing weights (torch), shared expert included."""
    g = torch.Generator().manual_seed(9)
    T, E, K, H, I = 37, 8, 3, 32, 16
    wg = torch.randn(E, H, generator=g) * 0.3
    gates = torch.randn(E, I, H, generator=g) * 0.2
    ups = torch.randn(E, I, H, generator=g) * 0.2
    downs = torch.randn(E, H, I, generator=g) * 0.2
    sh = (torch.randn(2 * I, H, generator=g) * 0.2, torch.randn(2 * I, H, generator=g) * 0.2,
          torch.randn(H, 2 * I, generator=g) * 0.2)
    x = torch.randn(T, H, generator=g)
    out = om.moe_layer(x.numpy(), wg.numpy(), gates.numpy(), ups.numpy(), downs.numpy(), K,
                       shared=tuple(t.numpy() for t in sh))
    probs = torch.softmax(x @ wg.T, -1)
    tw, ti = torch.topk(probs, K, -1)
    dense_w = torch.zeros(T, E).scatter_(1, ti, tw)
    all_out = torch.stack([F.linear(F.silu(F.linear(x, gates[e])) * F.linear(x, ups[e]), downs[e])
                           for e in range(E)], 1)                     # [T, E, H]
    ref = (all_out * dense_w[:, :, None]).sum(1)
    ref += F.linear(F.silu(F.linear(x, sh[0])) * F.linear(x, sh[1]), sh[2])
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-4, atol=1e-5)

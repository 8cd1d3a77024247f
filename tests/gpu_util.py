"""Helpers shared by the GPU parity tests."""
import numpy as np
import torch


def np32(t: torch.Tensor) -> np.ndarray:
    """Any torch tensor -> float32 numpy on the CPU (bf16 values are exact in fp32)."""
    return t.detach().float().cpu().numpy()


def bf16_np(a) -> np.ndarray:
    """Round an array to bf16 (as torch does) and return it as float32 numpy."""
    return torch.as_tensor(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def max_rel_err(got, ref) -> float:
    """Tolerance metric: max|got - ref| / max|ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (denom if denom > 0 else 1.0))


BF16_TOL = 2e-2   # bf16 outputs, fp32 accumulation
F32_TOL = 1e-5    # fp32 elementwise outputs


def gate_logit_error_bound(x: np.ndarray, wg: np.ndarray, bias=None) -> np.ndarray:
    """Per-(token, expert) bound on |fp32 router logit - exact logit| for the
    library's gate (bf16 products, exact in fp32; fp32 MFMA accumulation over
    n <= 16 K slices; the route kernel adds the slice planes, then the bias).

    Each product passes through at most d roundings: <= 16 inside its MFMA step
    (a 16-term dot plus the accumulator add, in any order), <= H/(16 n) - 1
    later accumulator adds in its slice, <= n - 1 plane additions and 1 bias
    add, so d <= H/(16 n) + n + 15 <= H/16 + 32 for any n in [1, 16]. For any
    summation order |fl(sum) - sum| <= gamma_d * sum |terms| (Higham, Accuracy
    and Stability of Numerical Algorithms, 2nd ed., eq. 4.4), with
    gamma_d = d u / (1 - d u); u = 2^-23 also covers truncating adds. The fp64
    reference sum adds its own gamma_H (u = 2^-53).
    x [T, H], wg [E, H] (the bf16 values), bias [E] or None -> [T, E]."""
    x = np.asarray(x, np.float64)
    wg = np.asarray(wg, np.float64)
    H = x.shape[1]
    d = H // 16 + 32
    g32 = d * 2.0 ** -23 / (1 - d * 2.0 ** -23)
    g64 = H * 2.0 ** -53 / (1 - H * 2.0 ** -53)
    mag = np.abs(x) @ np.abs(wg).T
    if bias is not None:
        mag = mag + np.abs(np.asarray(bias, np.float64))[None, :]
    return (g32 + g64) * mag


def routing_safe_tokens(lg64: np.ndarray, bound: np.ndarray, top_k: int):
    """Tokens whose exact top-(k+1) logits are separated by more than twice the
    fp32 error bound at every consecutive gap: any fp32 evaluation within the
    bound selects, and orders, the same top-k as the exact logits.
    Returns (safe mask [T], min consecutive gap per token [T])."""
    s = -np.sort(-lg64, axis=1)[:, :top_k + 1]
    gaps = s[:, :top_k] - s[:, 1:top_k + 1]
    b = bound.max(axis=1)
    return (gaps > 2 * b[:, None]).all(axis=1), gaps.min(axis=1)


def assert_routing_admissible(idx: np.ndarray, lg64: np.ndarray, bound: np.ndarray):
    """Every chosen expert's exact logit is within twice the error bound of the
    exact logit at its rank: the choice is one that an fp32 evaluation inside
    the bound can make (used for tokens whose margin is below the bound)."""
    s = -np.sort(-lg64, axis=1)[:, :idx.shape[1]]
    chosen = np.take_along_axis(lg64, idx.astype(np.int64), axis=1)
    b = 2 * bound.max(axis=1, keepdims=True)
    assert np.all(np.abs(chosen - s) <= b), "routing choice outside the fp32 error bound"
    assert all(len(set(r)) == len(r) for r in idx.tolist()), "an expert chosen twice"

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

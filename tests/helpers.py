"""Shared helpers of the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

# tolerances of the MoE output vs the oracle (fp32 and bf16 layer bars):
# max |out - ref| <= TOL * max |ref|
TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def rel_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    if scale == 0:
        return float(np.abs(got).max())
    return float(np.abs(got - ref).max() / scale)


def row_rel_err(got, ref, floor: float) -> float:
    """Largest per-row error: max over rows of max|got - ref| / max(max|ref row|, floor).
    Catches a row that is wrong by much less than the largest row of the tensor."""
    got = np.asarray(got, np.float64).reshape(len(got), -1)
    ref = np.asarray(ref, np.float64).reshape(len(ref), -1)
    scale = np.maximum(np.abs(ref).max(axis=1), floor)
    return float((np.abs(got - ref).max(axis=1) / scale).max())


def to_np(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy (bf16 widened to its exact float32 values)."""
    t = t.detach()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.cpu().numpy()


def banner(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def tie_free(logits: np.ndarray, k: int) -> bool:
    s = -np.sort(-logits, axis=1)
    return not (s[:, : k] == s[:, 1: k + 1]).any()

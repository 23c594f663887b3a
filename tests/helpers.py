"""Shared helpers of the test suite."""
from __future__ import annotations

import numpy as np
import torch

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


def bits(t: torch.Tensor) -> np.ndarray:
    """Host array the C oracle reads: float32 values or raw 16-bit patterns."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def oracle_dtype(dt: torch.dtype) -> int:
    return {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dt]


def rel_err(a, b) -> float:
    """max |a - b| / max |b|: the relative error used for every tolerance."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def load_golden(name: str):
    return np.load(f"{GOLDEN}/{name}.npz", allow_pickle=False)

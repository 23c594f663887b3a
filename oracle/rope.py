"""Rotary position embedding restated in numpy - TEST INFRASTRUCTURE ONLY.

Only tests/ import this module.  Follows ``apply_rotary_emb``
(``dsalt/kernels/window_utils.py:74-89``: half-split rotation, ``q * cos + rotate_half(q) * sin``
with ``rotate_half(x) = [-x2, x1]``) with cos/sin gathered at each token's position in its
sequence and cast to the tensor type (``dsalt/modules/dsalt_attention.py:566-585``).  Every
elementwise operation of that expression rounds to the tensor type (products and the sum
computed in float32, then rounded), so bf16/fp16 results are emulated bit for bit.
"""
from __future__ import annotations

import numpy as np

__all__ = ["round_to", "rope"]


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to bf16 / fp16 (nearest, ties to even), returned as float32."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def rope(x: np.ndarray, cu: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """x [T, H, D] float32 values of the tensor type; cos/sin [max_pos, D] float32."""
    x = np.asarray(x, np.float32)
    T, H, D = x.shape
    half = D // 2
    pos = np.empty(T, np.int64)
    for s in range(len(cu) - 1):
        pos[cu[s]:cu[s + 1]] = np.arange(cu[s + 1] - cu[s])
    c = round_to(cos[pos], dtype)[:, None, :]
    s = round_to(sin[pos], dtype)[:, None, :]
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    a = round_to(x * c, dtype)
    b = round_to(rot * s, dtype)
    return round_to(a + b, dtype)

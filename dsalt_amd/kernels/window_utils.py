"""Window-mask builders and RoPE helpers with the reference's semantics.

``build_local_window_mask`` / ``build_local_window_mask_packed`` mirror
``dsalt/kernels/window_utils.py:19-70`` (row ``i`` attends ``[i - w_i + 1, i]`` within its
sequence).  They materialise ``[T, T]`` masks for the dense masked-attention API; the sparse
operator never builds them.  ``apply_rotary_emb`` / ``build_rope_cache`` follow
``window_utils.py:73-107`` (half-split rotation).
"""
from __future__ import annotations

import torch


def build_local_window_mask(seq_len: int, window_sizes: torch.Tensor, device) -> torch.Tensor:
    rows = torch.arange(seq_len, device=device)
    w = window_sizes.to(device).clamp(min=1, max=seq_len).long()
    lo = (rows - w + 1).clamp(min=0)
    cols = rows.unsqueeze(0)
    return (cols >= lo.unsqueeze(1)) & (cols <= rows.unsqueeze(1))


def build_local_window_mask_packed(cu_seqlens: torch.Tensor, window_sizes: torch.Tensor, total_len: int,
                                   device) -> torch.Tensor:
    cu = cu_seqlens.to(device).long()
    lens = cu[1:] - cu[:-1]
    seq_ids = torch.repeat_interleave(torch.arange(lens.numel(), device=device), lens)
    starts = cu[:-1][seq_ids]
    pos = torch.arange(total_len, device=device)
    lo = starts + (pos - starts - window_sizes.to(device).clamp(min=1).long() + 1).clamp(min=0)
    col = pos.unsqueeze(0)
    same = seq_ids.unsqueeze(1) == seq_ids.unsqueeze(0)
    return same & (col >= lo.unsqueeze(1)) & (col <= pos.unsqueeze(1))


def apply_rotary_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    half = q.shape[-1] // 2

    def rot(x):
        return torch.cat([-x[..., half:], x[..., :half]], dim=-1)

    return q * cos + rot(q) * sin, k * cos + rot(k) * sin


def build_rope_cache(seq_len: int, head_dim: int, device, dtype=torch.float32, base: float = 10000.0,
                     scale: float = 1.0):
    theta = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device, dtype=dtype) / head_dim))
    positions = torch.arange(seq_len, device=device, dtype=dtype) / scale
    emb = torch.cat([torch.outer(positions, theta)] * 2, dim=-1)
    return emb.cos(), emb.sin()

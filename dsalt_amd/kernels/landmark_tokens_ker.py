"""Hybrid landmark score on the GPU.

Mirrors ``hybrid_scores_per_head`` of ``dsalt/kernels/landmark_tokens_ker.py:19-61``:
``s = alpha * z(|x W_V^T|_h) + (1 - alpha) * z(|x|)`` with z-statistics over all rows of
``x``.  Norms, statistics and z run in the HIP selection kernels (canonical fp64
arithmetic); the final mix is re-expressed in torch so ``scores`` stays differentiable in
``alpha`` as in the reference.
"""
from __future__ import annotations

import torch

from .. import ops


def hybrid_scores_per_head(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int):
    """``(scores [T, n_heads], z_x [T], z_v [T, n_heads])`` for hidden states ``x [T, d]``,
    value projection ``W_V [n_kv*dh, d]`` and per-head ``alpha [n_heads]`` in (0, 1)."""
    T = x.shape[0]
    n_kv = W_V.shape[0] // dh
    with torch.no_grad():
        v = (x.detach() @ W_V.detach().T).view(T, n_kv, dh)
        cu = torch.tensor([0, T], dtype=torch.int32, device=x.device)
        w = torch.zeros(T, dtype=torch.int32, device=x.device)
        _, z_x, z_v, _ = ops.select_landmarks(x.detach(), v, alpha.detach(), w, cu, 0, max_seqlen=max(T, 1),
                                              stats_scope=ops.STATS_PACKED, want_scores=True)
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)
    a = alpha.to(torch.float32)
    scores = a * z_v + (1.0 - a) * z_x.unsqueeze(1)
    return scores, z_x, z_v

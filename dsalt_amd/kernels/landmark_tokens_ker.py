"""Hybrid landmark score on the GPU.

Mirrors ``hybrid_scores_per_head`` of ``dsalt/kernels/landmark_tokens_ker.py:19-61``:
``s = alpha * z(|x W_V^T|_h) + (1 - alpha) * z(|x|)`` with z-statistics (mean, unbiased std
clamped at 1e-6) over all rows of ``x``.  Norms, statistics and z run in the HIP selection
kernels (canonical fp64 arithmetic).  The score is differentiable in ``x``, ``W_V`` and
``alpha`` as the reference's torch expression is: the backward applies the closed-form
gradient of the z-score,
    dn_i = (g_i - mean(g) - z_i * sum_j(g_j z_j) / (N - 1)) / s
(the last term vanishes where the std is clamped), then the norm gradients ``n_i / |n_i|``.
"""
from __future__ import annotations

import torch

from .. import ops


def _zscore_grad(g: torch.Tensor, z: torch.Tensor, n: torch.Tensor) -> torch.Tensor:
    """d loss / d n for z = (n - mean n) / max(std n, 1e-6) over dim 0 (fp64)."""
    N = n.shape[0]
    std = n.std(0, keepdim=True) if N > 1 else torch.full_like(n[:1], float("nan"))
    s = std.clamp(min=1e-6)
    clamped = ~(std > 1e-6)
    corr = (g * z).sum(0, keepdim=True) / max(N - 1, 1)
    corr = torch.where(clamped, torch.zeros_like(corr), corr)
    return (g - g.mean(0, keepdim=True) - z * corr) / s


def _norm_grad(dn: torch.Tensor, vec: torch.Tensor, n: torch.Tensor) -> torch.Tensor:
    """d loss / d vec for n = |vec| over the last dim (0 where n is 0, as torch's norm)."""
    safe = torch.where(n > 0, n, torch.ones_like(n))
    return torch.where((n > 0).unsqueeze(-1), vec * (dn / safe).unsqueeze(-1), torch.zeros_like(vec))


class _HybridScore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W_V, alpha, n_heads, dh):
        T = x.shape[0]
        n_kv = W_V.shape[0] // dh
        v = (x @ W_V.T).view(T, n_kv, dh)
        cu = torch.tensor([0, T], dtype=torch.int32, device=x.device)
        w = torch.zeros(T, dtype=torch.int32, device=x.device)
        _, z_x, z_v, _ = ops.select_landmarks(x, v, alpha, w, cu, 0, max_seqlen=max(T, 1),
                                              stats_scope=ops.STATS_PACKED, want_scores=True)
        if n_kv != n_heads:
            z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)
        a = alpha.to(torch.float32)
        scores = a * z_v + (1.0 - a) * z_x.unsqueeze(1)
        ctx.save_for_backward(x, W_V, alpha, v, z_x, z_v)
        ctx.n_heads, ctx.n_kv = n_heads, n_kv
        ctx.mark_non_differentiable(z_x, z_v)
        return scores, z_x, z_v

    @staticmethod
    def backward(ctx, g_scores, g_zx, g_zv):
        x, W_V, alpha, v, z_x, z_v = ctx.saved_tensors
        T, H, G = x.shape[0], ctx.n_heads, ctx.n_kv
        if g_scores is None:
            return None, None, None, None, None
        g = g_scores.double()
        a = alpha.double()
        d_alpha = (g * (z_v.double() - z_x.double().unsqueeze(1))).sum(0) if ctx.needs_input_grad[2] else None
        dx = dW = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            # the norms as the kernels round them (to the input dtype); token-sized vectors in
            # fp64, the [T, d] products in fp32
            xf, vf = x.float(), v.float()
            n_x = xf.norm(dim=-1).to(x.dtype).double()
            n_v = vf.norm(dim=-1).to(x.dtype).double()                               # [T, G]
            g_zx_ = (g * (1.0 - a)).sum(1, keepdim=True)                             # [T, 1]
            g_zv_ = (g * a).view(T, G, H // G).sum(2)                                # [T, G]
            z_v_g = z_v.double().view(T, G, H // G)[:, :, 0]
            dn_x = _zscore_grad(g_zx_, z_x.double().unsqueeze(1), n_x.unsqueeze(1))[:, 0]
            dn_v = _zscore_grad(g_zv_, z_v_g, n_v)
            dvec = _norm_grad(dn_v.float(), vf, n_v.float()).reshape(T, -1)          # [T, G*dh]
            if ctx.needs_input_grad[0]:
                dx = (_norm_grad(dn_x.float(), xf, n_x.float()) + dvec @ W_V.float()).to(x.dtype)
            if ctx.needs_input_grad[1]:
                dW = (dvec.T @ xf).to(W_V.dtype)
        return dx, dW, d_alpha.to(alpha.dtype) if d_alpha is not None else None, None, None


def hybrid_scores_per_head(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int):
    """``(scores [T, n_heads], z_x [T], z_v [T, n_heads])`` for hidden states ``x [T, d]``,
    value projection ``W_V [n_kv*dh, d]`` and per-head ``alpha [n_heads]`` in (0, 1).
    ``scores`` carries gradients to ``x``, ``W_V`` and ``alpha``; ``z_x`` and ``z_v`` are
    returned detached."""
    return _HybridScore.apply(x, W_V, alpha, n_heads, dh)

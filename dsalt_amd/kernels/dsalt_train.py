"""The DSALT training attention (differentiable selectors) as a torch autograd function.

Drop-in for ``dsalt_triton_train_attention`` / ``DSALTTrainFunction`` of
``dsalt/kernels/dsalt_triton_train.py:586-780``: same arguments
``(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win, win_edge, n_max, cu_list)``,
output ``[T, H, D]`` in float32 holding values rounded to the input dtype, gradients for q, k,
v, ``lmk_logw`` (``d_logw``) and ``w_cont`` (``d_w~`` summed over heads).

Per query i with continuous window w~ = w_cont[i] the row attends to
  * band keys j with ``0 <= d = i - j <= w~``, logit bias 0 in the core ``d <= w~ - win_edge``
    and ``log sigmoid((w~ - d) / tau_win)`` outside it (:136-147);
  * landmarks ``p = lmk_pos[h, s, slot] >= 0`` with ``p < i - w~`` (:180-184), logit bias
    ``lmk_logw[h, s, slot]``.
Differences, all deliberate:
  * float32 inputs are computed in float32 (the reference casts them to float16, :608-611);
  * k/v may carry fewer heads than q (grouped-query attention read in place; each key/value
    head's gradient sums its query heads inside the kernels, without a materialised repeat);
  * landmark slots may come in any order (sorted for the kernels, d_logw returned in the
    caller's order);
  * ``n_max`` is accepted and not needed: the key-parallel backward bounds its query scan
    by each sequence's largest window, read from ``w_cont``;
  * the backward is deterministic (no float atomics);
  * ``d_logw`` and ``d_w~`` come back in the dtype of ``lmk_logw`` / ``w_cont`` (the reference
    rounds them to q's dtype, :757-761).
"""
from __future__ import annotations

import math

import torch

from .. import ops
from .autotune import tuned_variant
from .dsalt_attn import pad_head_dim, padded_head_dim


class DSALTTrainFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win, win_edge, n_max=256,
                cu_list=None):
        if lmk_pos.dim() != 3:
            raise ValueError(f"lmk_pos must be [H, S, k], got {tuple(lmk_pos.shape)}")
        idx_s, logw_s, perm = ops.sort_landmarks(lmk_pos.unsqueeze(2), lmk_logw.unsqueeze(2))
        max_seqlen = ops._max_seqlen(cu_seqlens, cu_list)
        cu_i = cu_seqlens.detach().to(torch.int32)
        w_c = w_cont.detach().to(torch.float32).contiguous()
        head_dim = q.shape[-1]
        scale = 1.0 / math.sqrt(head_dim)
        dp = padded_head_dim(head_dim)  # other head_dims run zero-padded (see dsalt_attn)
        q, k, v = (pad_head_dim(t, dp) for t in (q, k, v))
        plan = ops.new_plan(q, k, cu_i, idx_s, max_seqlen=max_seqlen)
        variant = tuned_variant(dp, q.device, q.dtype)  # autotune_blocks' choice, if made
        out, lse = ops.train_forward(q, k, v, w_c, cu_i, idx_s, logw_s, tau_win=float(tau_win),
                                     win_edge=float(win_edge), scale=scale, max_seqlen=max_seqlen, plan=plan,
                                     variant=variant)
        ctx.save_for_backward(q, k, v, out, lse, idx_s, logw_s, perm, w_c, cu_i, plan)
        ctx.max_seqlen, ctx.scale, ctx.variant = max_seqlen, scale, variant
        ctx.tau_win, ctx.win_edge = float(tau_win), float(win_edge)
        ctx.logw_dtype, ctx.w_dtype = lmk_logw.dtype, w_cont.dtype
        ctx.head_dim = head_dim
        return out[..., :head_dim].float().contiguous()

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse, idx_s, logw_s, perm, w_c, cu_i, plan = ctx.saved_tensors
        dq, dk, dv, dlogw, d_w = ops.train_backward(
            pad_head_dim(grad_out.to(q.dtype), q.shape[-1]), q, k, v, out, lse, w_c, cu_i, idx_s, logw_s,
            tau_win=ctx.tau_win,
            win_edge=ctx.win_edge, scale=ctx.scale, max_seqlen=ctx.max_seqlen,
            want_dlogw=ctx.needs_input_grad[4], plan=plan, variant=ctx.variant)
        d_logw = None
        if ctx.needs_input_grad[4] and dlogw is not None:
            d_logw = torch.zeros_like(dlogw).scatter_(-1, perm, dlogw)[:, :, 0].to(ctx.logw_dtype)
        d_wc = d_w.to(ctx.w_dtype) if ctx.needs_input_grad[5] else None
        d = ctx.head_dim
        if d != q.shape[-1]:
            dq, dk, dv = (t[..., :d].contiguous() for t in (dq, dk, dv))
        return dq, dk, dv, None, d_logw, d_wc, None, None, None, None, None


def _dynamo_opaque(fn):
    disable = getattr(getattr(torch, "_dynamo", None), "disable", None)
    return disable(fn) if disable is not None else fn


@_dynamo_opaque
def dsalt_train_attention(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win=1.0, win_edge=4.0, n_max=256,
                          cu_list=None):
    """Differentiable sparse DSALT attention for training; see the module docstring."""
    return DSALTTrainFunction.apply(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win, win_edge, n_max,
                                    cu_list)


# the reference's public name, kept so callers switch without edits
dsalt_triton_train_attention = dsalt_train_attention

"""The DSALT sparse-attention operator as a torch autograd function.

Drop-in for ``dsalt_triton_attention`` / ``DSALTAttentionFunction`` of
``dsalt/kernels/dsalt_triton_attn.py:257-349``: same arguments
``(q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens)``, output ``[T, H, D]`` in float32
holding values rounded to the input dtype (the reference returns ``out.float()``), gradients
for q, k, v and lmk_bias.  Differences, all deliberate:
  * float32 inputs are computed in float32 (the reference silently casts them to float16,
    :266-269);
  * k/v may carry fewer heads than q (grouped-query attention read in place, forward and
    backward: each key/value head's gradient sums its query heads inside the kernels);
  * landmark indices may come in any order: each set is sorted before the kernels, which
    need ascending positions, and d_bias is returned in the caller's order;
  * the backward is deterministic (no float atomics);
  * 4-D ``lmk_indices [H, S, n_blocks, k]`` select the block-causal variant
    (``block_size`` query rows per set); its backward is not implemented.
"""
from __future__ import annotations

import math

import torch

from .. import ops
from .autotune import tuned_variant


def _mode_of(lmk_indices):
    return ops.SELECT_BLOCK if lmk_indices.dim() == 4 else ops.SELECT_GLOBAL


class DSALTAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens, max_seqlen=None, block_size=512):
        mode = _mode_of(lmk_indices)
        idx4 = lmk_indices if mode == ops.SELECT_BLOCK else lmk_indices.unsqueeze(2)
        bias4 = None
        if lmk_bias is not None:
            bias4 = lmk_bias if mode == ops.SELECT_BLOCK else lmk_bias.unsqueeze(2)
        idx_s, bias_s, perm = ops.sort_landmarks(idx4, bias4)
        if max_seqlen is None:
            max_seqlen = ops._max_seqlen(cu_seqlens)
        w_i = w_sizes.detach().clamp(min=1).to(torch.int32)
        cu_i = cu_seqlens.detach().to(torch.int32)
        scale = 1.0 / math.sqrt(q.shape[-1])
        plan = ops.new_plan(q, k, cu_i, idx_s, max_seqlen=max_seqlen, select_mode=mode, block_size=block_size)
        variant = tuned_variant(q.shape[-1], q.device, q.dtype)  # autotune_blocks' choice, if made
        out, lse = ops.attention_forward(q, k, v, w_i, cu_i, idx_s, bias_s, scale=scale, max_seqlen=max_seqlen,
                                         select_mode=mode, block_size=block_size, plan=plan, variant=variant)
        ctx.save_for_backward(q, k, v, out, lse, idx_s, bias_s if bias_s is not None else torch.empty(0),
                              perm, w_i, cu_i, plan)
        ctx.has_bias = bias_s is not None
        ctx.mode, ctx.max_seqlen, ctx.scale, ctx.variant = mode, max_seqlen, scale, variant
        ctx.bias_dtype = lmk_bias.dtype if lmk_bias is not None else None
        return out.float()

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse, idx_s, bias_s, perm, w_i, cu_i, plan = ctx.saved_tensors
        if ctx.mode == ops.SELECT_BLOCK:
            raise NotImplementedError("the backward of the block-causal landmark variant is not implemented")
        dq, dk, dv, db = ops.attention_backward(grad_out.to(q.dtype), q, k, v, out, lse, w_i, cu_i, idx_s,
                                                bias_s if ctx.has_bias else None, scale=ctx.scale,
                                                max_seqlen=ctx.max_seqlen, want_dbias=ctx.needs_input_grad[4],
                                                plan=plan, variant=ctx.variant)
        d_bias = None
        if ctx.needs_input_grad[4] and db is not None:
            d_bias = torch.zeros_like(db).scatter_(-1, perm, db)[:, :, 0].to(ctx.bias_dtype)
        return dq, dk, dv, None, d_bias, None, None, None, None


def _dynamo_opaque(fn):
    disable = getattr(getattr(torch, "_dynamo", None), "disable", None)
    return disable(fn) if disable is not None else fn


@_dynamo_opaque
def dsalt_attention(q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens, *, max_seqlen=None, cu_list=None,
                    block_size=512):
    """Sparse attention over ``A(i) = W(i) U L(i)``; see the module docstring."""
    if max_seqlen is None and cu_list is not None:
        max_seqlen = ops._max_seqlen(cu_seqlens, cu_list)
    return DSALTAttentionFunction.apply(q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens, max_seqlen,
                                        block_size)


# the reference's public name, kept so callers switch without edits
dsalt_triton_attention = dsalt_attention

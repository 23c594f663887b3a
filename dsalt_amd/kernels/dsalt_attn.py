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
A head_dim the kernels are not compiled for (any up to 128) runs on q, k, v zero-padded to
the next compiled size (64 or 128) with the logit scale of the true head_dim, as the
reference pads to the next power of two (``dsalt_triton_attn.py:263``): the padded columns
add nothing to any product, and the output and gradients are sliced back.
"""
from __future__ import annotations

import math

import torch

from .. import ops
from .autotune import tuned_variant


def _mode_of(lmk_indices):
    return ops.SELECT_BLOCK if lmk_indices.dim() == 4 else ops.SELECT_GLOBAL


def padded_head_dim(head_dim: int) -> int:
    """The compiled head_dim (64 or 128) a head_dim runs at."""
    if head_dim < 1 or head_dim > 128:
        raise ValueError(f"head_dim {head_dim} is not supported: the kernels are compiled for head_dim up to 128")
    return 64 if head_dim <= 64 else 128


def pad_head_dim(t: torch.Tensor, dp: int) -> torch.Tensor:
    """[..., D] zero-padded to [..., dp] (the tensor itself when D == dp)."""
    d = t.shape[-1]
    return t if d == dp else torch.nn.functional.pad(t, (0, dp - d))


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
        head_dim = q.shape[-1]
        scale = 1.0 / math.sqrt(head_dim)
        dp = padded_head_dim(head_dim)
        q, k, v = (pad_head_dim(t, dp) for t in (q, k, v))
        plan = ops.new_plan(q, k, cu_i, idx_s, max_seqlen=max_seqlen, select_mode=mode, block_size=block_size)
        variant = tuned_variant(dp, q.device, q.dtype)  # autotune_blocks' choice, if made
        out, lse = ops.attention_forward(q, k, v, w_i, cu_i, idx_s, bias_s, scale=scale, max_seqlen=max_seqlen,
                                         select_mode=mode, block_size=block_size, plan=plan, variant=variant)
        ctx.save_for_backward(q, k, v, out, lse, idx_s, bias_s if bias_s is not None else torch.empty(0),
                              perm, w_i, cu_i, plan)
        ctx.has_bias = bias_s is not None
        ctx.mode, ctx.max_seqlen, ctx.scale, ctx.variant = mode, max_seqlen, scale, variant
        ctx.bias_dtype = lmk_bias.dtype if lmk_bias is not None else None
        ctx.head_dim = head_dim
        return out[..., :head_dim].float().contiguous()

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse, idx_s, bias_s, perm, w_i, cu_i, plan = ctx.saved_tensors
        if ctx.mode == ops.SELECT_BLOCK:
            raise NotImplementedError("the backward of the block-causal landmark variant is not implemented")
        go = pad_head_dim(grad_out.to(q.dtype), q.shape[-1])
        dq, dk, dv, db = ops.attention_backward(go, q, k, v, out, lse, w_i, cu_i, idx_s,
                                                bias_s if ctx.has_bias else None, scale=ctx.scale,
                                                max_seqlen=ctx.max_seqlen, want_dbias=ctx.needs_input_grad[4],
                                                plan=plan, variant=ctx.variant)
        d_bias = None
        if ctx.needs_input_grad[4] and db is not None:
            d_bias = torch.zeros_like(db).scatter_(-1, perm, db)[:, :, 0].to(ctx.bias_dtype)
        d = ctx.head_dim
        if d != q.shape[-1]:
            dq, dk, dv = (t[..., :d].contiguous() for t in (dq, dk, dv))
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

"""Fused linear cross-entropy for large vocabularies (the LM head and its loss).

Drop-in for ``LigerFusedLinearCrossEntropyFunction`` and ``fused_linear_cross_entropy_forward``
/ ``_backward`` of ``dsalt/kernels/cross_entropy.py:351-670``: rows of the hidden states are
taken in chunks; per chunk the logits ``x W^T (+ b)`` come from one GEMM (hipBLASLt through
torch), the HIP row kernel (``dsalt_cross_entropy_rows``) computes the losses and writes the
gradient over the logits in place, and two more GEMMs turn it into ``grad_input`` and the
``grad_weight`` contribution; the full ``[rows, V]`` logits never exist.  The forward
computes the gradients (as the reference does); the backward scales them by the upstream
gradient.

Options: ``ce_weight``, ``ignore_index``, ``lse_square_scale`` (z-loss), ``label_smoothing``,
``reduction`` ("mean", "sum", "none"), ``softcap``, ``return_z_loss``, ``accum_dtype``,
``use_token_scaling``, ``return_token_accuracy``, ``return_predicted_tokens``.
Differences, all deliberate:
  * chunks hold up to 2 GiB of logits (the reference sizes them by ``V / hidden``): fewer,
    larger GEMMs on a 288 GB device;
  * without ``accum_dtype`` the weight gradient accumulates with one ``addmm`` per chunk in
    the weight's dtype (one rounding per chunk where the reference rounds the chunk's product
    and then the sum);
  * the token-scaling factor is the target's probability from the row kernel's float32
    log-sum-exp (the reference takes it from a softmax in the logits' dtype);
  * a per-row upstream gradient (``reduction="none"``) must be uniform: the gradients are
    reduced over rows in the forward (the reference reads only its first element).
"""
from __future__ import annotations

import torch

from .. import ops

_CHUNK_BYTES = 1 << 31


def _chunk_rows(BT: int, V: int, elem: int) -> int:
    rows = max(256, (_CHUNK_BYTES // max(1, V * elem)) // 256 * 256)
    return max(1, min(BT, rows))


def fused_linear_cross_entropy_forward(_input, weight, target, ce_weight=None, bias=None, ignore_index=-100,
                                       lse_square_scale=0.0, label_smoothing=0.0, reduction="mean", softcap=None,
                                       return_z_loss=False, accum_dtype=None, use_token_scaling=False,
                                       return_token_accuracy=False, return_predicted_tokens=False):
    """(loss, z_loss, token_accuracy, predicted_tokens, grad_input, grad_weight, grad_bias)."""
    BT, H = _input.shape
    V = weight.shape[0]
    dev = _input.device
    tgt = target.to(torch.int64)
    keep = tgt != ignore_index
    bad = keep & ((tgt < 0) | (tgt >= V))
    n_non_ignore, n_bad = (int(v) for v in torch.stack([keep.sum(), bad.sum()]).tolist())
    if n_bad:
        raise ValueError(f"{n_bad} target(s) outside [0, {V}) that are not ignore_index")
    sum_w, w_sum = float(n_non_ignore), 0.0
    if ce_weight is not None:
        if ce_weight.shape[0] != V or not torch.is_floating_point(ce_weight):
            raise ValueError(f"ce_weight must be a floating tensor of size V={V}")
        sum_w = float(ce_weight[tgt[keep]].sum().item())
        w_sum = float(ce_weight.sum().item())
    need_grad = _input.requires_grad
    grad_input = torch.zeros_like(_input) if need_grad else None
    grad_weight = grad_bias = None
    if need_grad:
        wd = accum_dtype if accum_dtype is not None else weight.dtype
        if weight.requires_grad:
            grad_weight = torch.zeros(weight.shape, dtype=wd, device=dev)
        if bias is not None:
            grad_bias = torch.zeros(bias.shape, dtype=wd, device=dev)
    loss_1d = torch.zeros(BT, dtype=torch.float32, device=dev)
    z_1d = torch.zeros(BT, dtype=_input.dtype, device=dev) if return_z_loss else None
    acc_1d = torch.zeros(BT, dtype=torch.float32, device=dev) if return_token_accuracy else None
    pred_1d = torch.full((BT,), -1, dtype=torch.int64, device=dev) if return_predicted_tokens else None
    x = _input.detach()
    wt = weight.detach()
    chunk = _chunk_rows(BT, V, _input.element_size())
    for s0 in range(0, BT, chunk):
        s1 = min(BT, s0 + chunk)
        xc = x[s0:s1]
        logits = torch.nn.functional.linear(xc, wt, bias.detach() if bias is not None else None).contiguous()
        l, z, a, p = ops.cross_entropy_rows(
            logits, tgt[s0:s1], ce_weight=ce_weight, ignore_index=ignore_index, n_non_ignore=float(n_non_ignore),
            sum_non_ignore_weight=sum_w, weight_sum=w_sum, lse_square_scale=lse_square_scale,
            label_smoothing=label_smoothing, softcap=softcap, reduction=reduction, want_grad=need_grad,
            token_scaling=use_token_scaling, want_z=return_z_loss, want_accuracy=return_token_accuracy,
            want_predicted=return_predicted_tokens)
        loss_1d[s0:s1] = l
        if z_1d is not None:
            z_1d[s0:s1] = z
        if acc_1d is not None:
            acc_1d[s0:s1] = a
        if pred_1d is not None:
            pred_1d[s0:s1] = p
        if need_grad:  # logits now hold d loss / d logits
            torch.mm(logits, wt, out=grad_input[s0:s1])
            if grad_weight is not None:
                if grad_weight.dtype == logits.dtype:
                    grad_weight.addmm_(logits.t(), xc)
                else:
                    grad_weight += torch.mm(logits.t(), xc).to(grad_weight.dtype)
            if grad_bias is not None:
                grad_bias += logits.sum(dim=0).to(grad_bias.dtype)
    if reduction == "none":
        loss, z_loss = loss_1d, z_1d
        token_accuracy = acc_1d
    else:
        loss = loss_1d.sum()
        z_loss = z_1d.sum() if z_1d is not None else None
        token_accuracy = acc_1d.sum() / n_non_ignore if acc_1d is not None else None
    if grad_weight is not None:
        grad_weight = grad_weight.to(weight.dtype)
    if grad_bias is not None:
        grad_bias = grad_bias.to(bias.dtype)
    return loss, z_loss, token_accuracy, pred_1d, grad_input, grad_weight, grad_bias


def fused_linear_cross_entropy_backward(grad_output, grad_input, grad_weight, grad_bias):
    """The forward's gradients times the (uniform) upstream gradient."""
    if grad_output.numel() != 1:
        g0 = grad_output.reshape(-1)[0]
        if not torch.all(grad_output == g0):
            raise NotImplementedError("per-row upstream gradients of reduction='none' are not supported: the "
                                      "gradients are reduced over rows in the forward")
        grad_output = g0
    if torch.equal(grad_output, torch.ones((), dtype=grad_output.dtype, device=grad_output.device)):
        return grad_input, grad_weight, grad_bias
    scale = grad_output.to(torch.float32)
    out = []
    for g in (grad_input, grad_weight, grad_bias):
        out.append(None if g is None else (g.float() * scale).to(g.dtype))
    return tuple(out)


class LigerFusedLinearCrossEntropyFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, _input, weight, target, bias=None, ce_weight=None, ignore_index=-100, lse_square_scale=0.0,
                label_smoothing=0.0, reduction="mean", softcap=None, return_z_loss: bool = False, accum_dtype=None,
                use_token_scaling: bool = False, return_token_accuracy: bool = False,
                return_predicted_tokens: bool = False):
        loss, z_loss, acc, pred, gi, gw, gb = fused_linear_cross_entropy_forward(
            _input, weight, target, ce_weight=ce_weight, bias=bias, ignore_index=ignore_index,
            lse_square_scale=lse_square_scale, label_smoothing=label_smoothing, reduction=reduction, softcap=softcap,
            return_z_loss=return_z_loss, accum_dtype=accum_dtype, use_token_scaling=use_token_scaling,
            return_token_accuracy=return_token_accuracy, return_predicted_tokens=return_predicted_tokens)
        ctx.save_for_backward(gi, gw, gb)
        if acc is not None:
            ctx.mark_non_differentiable(acc)  # a count ratio: no gradient flows through it
        return loss, z_loss, acc, pred

    @staticmethod
    def backward(ctx, grad_output, grad_output2, grad_output3, grad_output4):
        gi, gw, gb = ctx.saved_tensors
        gi, gw, gb = fused_linear_cross_entropy_backward(grad_output, gi, gw, gb)
        return (gi, gw, None, gb) + (None,) * 11


def fused_linear_cross_entropy(x, weight, target, **kw):
    """Loss (first output of the autograd function) of the fused linear cross-entropy."""
    return LigerFusedLinearCrossEntropyFunction.apply(x, weight, target, *_pos(kw))[0]


def _pos(kw):
    names = ("bias", "ce_weight", "ignore_index", "lse_square_scale", "label_smoothing", "reduction", "softcap",
             "return_z_loss", "accum_dtype", "use_token_scaling", "return_token_accuracy", "return_predicted_tokens")
    defaults = (None, None, -100, 0.0, 0.0, "mean", None, False, None, False, False, False)
    unknown = set(kw) - set(names)
    if unknown:
        raise TypeError(f"unknown arguments {sorted(unknown)}")
    return tuple(kw.get(n, d) for n, d in zip(names, defaults))

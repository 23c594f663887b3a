"""Row cross-entropy of the fused linear cross-entropy, restated in numpy - TEST INFRASTRUCTURE ONLY.

Only tests/ import this module.  Follows ``liger_cross_entropy_kernel``
(``dsalt/kernels/cross_entropy.py:133-310``) and its driver
``fused_linear_cross_entropy_forward`` (:351-545) for one batch of logits, in float64:
  * x <- softcap * tanh(x / softcap) when softcap is set; lse = log sum exp(x);
  * loss_i = w_y (lse - x_y); with label smoothing eps = ls / V:
    loss_i = (1 - ls) loss_i + eps * sum_c w_c (lse - x_c)   (w = 1 without class weights);
  * z_i = lse_square_scale * lse^2;
  * reduction "mean": loss / sum of w_y over non-ignored rows, z / n_non_ignored;
  * gradient wrt the (softcapped) logits:
      no class weights: (softmax (1 + 2 zs lse) - eps - (1 - ls) onehot) [/ n_non_ignored],
      class weights:    (1 - ls) w_y (softmax - onehot) [/ sum w_y]
                        + eps (softmax sum_c w_c - w) [/ sum w_y] + 2 zs lse softmax [/ n],
    times (1 - tanh^2) for the softcap; ignored rows get zero loss and gradient;
  * token scaling multiplies loss, z and gradient by the row's (detached) probability of its
    target; argmax = first index of the largest logit.
"""
from __future__ import annotations

import numpy as np

__all__ = ["ce_rows"]


def ce_rows(x, target, ce_weight=None, ignore_index=-100, lse_square_scale=0.0, label_smoothing=0.0,
            reduction="mean", softcap=None, use_token_scaling=False):
    """(loss [N], z_loss [N], grad [N, V], argmax [N], lse [N]) in float64."""
    x = np.asarray(x, np.float64)
    N, V = x.shape
    target = np.asarray(target, np.int64)
    keep = target != ignore_index
    n_non_ignore = int(keep.sum())
    w = np.ones(V) if ce_weight is None else np.asarray(ce_weight, np.float64)
    sum_w_y = float(w[target[keep]].sum()) if ce_weight is not None else float(n_non_ignore)
    w_sum = float(w.sum())
    xs = softcap * np.tanh(x / softcap) if softcap is not None else x
    m = xs.max(1, keepdims=True)
    lse = (m + np.log(np.exp(xs - m).sum(1, keepdims=True)))[:, 0]
    sm = np.exp(xs - lse[:, None])
    eps = label_smoothing / V
    loss = np.zeros(N)
    z = np.zeros(N)
    grad = np.zeros_like(x)
    argmax = np.full(N, -1)
    for i in range(N):
        if not keep[i]:
            continue
        y = target[i]
        argmax[i] = int(np.argmax(xs[i]))
        wy = w[y] if ce_weight is not None else 1.0
        li = wy * (lse[i] - xs[i, y])
        if label_smoothing > 0:
            li = li * (1 - label_smoothing) + eps * float((w * (lse[i] - xs[i])).sum())
        zi = lse_square_scale * lse[i] ** 2
        if ce_weight is None:
            g = sm[i] * (1 + 2 * lse_square_scale * lse[i]) - eps
            g[y] -= 1 - label_smoothing
            if reduction == "mean":
                g = g / n_non_ignore
        else:
            go = (1 - label_smoothing) * sm[i]
            go[y] -= 1 - label_smoothing
            go *= wy
            gs = eps * (-w + sm[i] * w_sum)
            gz = 2 * lse_square_scale * lse[i] * sm[i]
            if reduction == "mean":
                go, gs, gz = go / sum_w_y, gs / sum_w_y, gz / n_non_ignore
            g = go + gs + gz
        if softcap is not None:
            g = g * (1 - np.tanh(x[i] / softcap) ** 2)
        if reduction == "mean":
            li = li / sum_w_y
            zi = zi / n_non_ignore
        if use_token_scaling:
            s = sm[i, y]
            li, zi, g = li * s, zi * s, g * s
        loss[i] = li + zi
        z[i] = zi
        grad[i] = g
    return loss, z, grad, argmax, lse

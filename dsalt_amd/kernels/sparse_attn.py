"""Dense masked attention with an explicit boolean mask (the reference's CPU-path API).

``sparse_attention_forward`` / ``sparse_attention_forward_packed`` keep the signatures of
``dsalt/kernels/sparse_attn.py:5-57``: boolean mask (True = attend) -> additive ``-inf``
mask in the query dtype -> scaled dot-product attention.  They cost O(T^2) and exist for
callers that build explicit masks; the DSALT operator itself is
``dsalt_attention``.  GPU tensors only: the CPU restatement of this path is the test oracle.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _gpu_only(*ts):
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError("dsalt_amd runs on the GPU only; got a tensor on " + str(t.device))


def sparse_attention_forward(q, k, v, attn_mask, dropout_p: float = 0.0, training: bool = False):
    """Masked SDPA for ``[B, H, T, D]`` tensors."""
    _gpu_only(q, k, v, attn_mask)
    additive = torch.zeros(attn_mask.shape, dtype=q.dtype, device=q.device)
    additive.masked_fill_(~attn_mask, float("-inf"))
    if additive.dim() == 3:
        additive = additive.unsqueeze(0)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=additive, dropout_p=dropout_p if training else 0.0)


def sparse_attention_forward_packed(q, k, v, attn_mask, dropout_p: float = 0.0, training: bool = False):
    """Masked SDPA for packed ``[T, H, D]`` tensors and a ``[T, T]`` mask."""
    _gpu_only(q, k, v, attn_mask)
    q_, k_, v_ = (t.transpose(0, 1).unsqueeze(0) for t in (q, k, v))
    additive = attn_mask.to(dtype=q.dtype).masked_fill(~attn_mask, float("-inf")).unsqueeze(0).unsqueeze(0)
    out = F.scaled_dot_product_attention(q_, k_, v_, attn_mask=additive, dropout_p=dropout_p if training else 0.0)
    return out.squeeze(0).transpose(0, 1).contiguous()

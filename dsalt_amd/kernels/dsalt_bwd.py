"""Standalone backward with the reference's signature.

Drop-in for ``dsalt_triton_backward`` (``dsalt/kernels/dsalt_triton_bwd.py:219-324``):
returns ``(dq, dk, dv, d_bias)`` in float32.  ``lmk_K`` / ``lmk_V`` (the gathered
landmark rows) are accepted for signature compatibility; the kernels read the landmark rows
of ``k`` / ``v`` at ``lmk_pos`` directly, which are the same values.  The block map, tile
sizes, warps and stages belong to the Triton launch and are ignored: the HIP kernels fix
their own tiles (see ``autotune.get_tuned_config``).  A head_dim other than 64 or 128 (up to
128) runs zero-padded to the next compiled size, as in ``dsalt_attn``.
"""
from __future__ import annotations

import torch

from .. import ops
from .dsalt_attn import pad_head_dim, padded_head_dim


def dsalt_backward(grad_out, q, k, v, out, lse, lmk_K, lmk_V, lmk_pos, lmk_bias, w_sizes, cu_seqlens, scale,
                   seq_block_map=None, total_blk=None, BLOCK_M=None, BLOCK_N=None, HEAD_DIM_C=None,
                   num_warps=None, num_stages=None, *, max_seqlen=None):
    del lmk_K, lmk_V, seq_block_map, total_blk, BLOCK_M, BLOCK_N, HEAD_DIM_C, num_warps, num_stages
    dt = q.dtype if q.dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
    idx4 = lmk_pos.unsqueeze(2) if lmk_pos.dim() == 3 else lmk_pos
    bias4 = None if lmk_bias is None else (lmk_bias.unsqueeze(2) if lmk_bias.dim() == 3 else lmk_bias)
    idx_s, bias_s, perm = ops.sort_landmarks(idx4, bias4)
    w_i = w_sizes.detach().clamp(min=1).to(torch.int32)
    d = q.shape[-1]
    dp = padded_head_dim(d)
    go, qp, kp, vp, op = (pad_head_dim(t.to(dt), dp) for t in (grad_out, q, k, v, out))
    dq, dk, dv, db = ops.attention_backward(go, qp, kp, vp, op, lse.float(), w_i, cu_seqlens, idx_s, bias_s,
                                            scale=scale, max_seqlen=max_seqlen)
    if d != dp:
        dq, dk, dv = (t[..., :d].contiguous() for t in (dq, dk, dv))
    d_bias = torch.zeros_like(db).scatter_(-1, perm, db)
    if lmk_pos.dim() == 3:
        d_bias = d_bias[:, :, 0]
    return dq.float(), dk.float(), dv.float(), d_bias


dsalt_triton_backward = dsalt_backward

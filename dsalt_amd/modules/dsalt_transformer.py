"""Pre-norm decoder block around the DSALT attention layer.

Mirrors ``SwiGLUFFN`` and ``DSALTTransformerBlock`` of
``dsalt/modules/dsalt_transformer.py:10-85`` (RMSNorm -> DSALTAttention -> residual, RMSNorm
-> SwiGLU FFN -> residual; optional activation checkpointing), with the attention layer's
landmark variant exposed (``select_mode``, ``block_size``, ``stats_scope``).  Without
autograd the FFN runs its gate and up projections as one GEMM over the concatenated
weights and the gated activation as one HIP kernel over that buffer (same per-element
arithmetic as silu(g) * u).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

from .. import ops
from ..kernels.RMSENorm import RMSENorm
from .dsalt_attention import DSALTAttention


class SwiGLUFFN(nn.Module):
    """``down(silu(gate(x)) * up(x))``."""

    def __init__(self, d_model: int, d_ff: int, dropout: float = 0.0):
        super().__init__()
        self.gate_proj = nn.Linear(d_model, d_ff, bias=False)
        self.up_proj = nn.Linear(d_model, d_ff, bias=False)
        self.down_proj = nn.Linear(d_ff, d_model, bias=False)
        self.drop = nn.Dropout(dropout)
        self._gu_cache = None
        self.gemm_events = None  # a list to collect (start, end) events of the gate/up GEMM

    def _gate_up_weight(self):
        ws = (self.gate_proj.weight, self.up_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        if self._gu_cache is None or self._gu_cache[0] != key:
            with torch.no_grad():
                self._gu_cache = (key, torch.cat(ws))
        return self._gu_cache[1]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() or self.training:
            return self.drop(self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x)))
        d_ff = self.gate_proj.weight.shape[0]
        w = self._gate_up_weight()
        if self.gemm_events is not None:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
            gu = F.linear(x, w)
            ev[1].record()
            self.gemm_events.append(ev)
        else:
            gu = F.linear(x, w)
        g2 = gu.reshape(-1, 2 * d_ff)
        h = ops.silu_mul(g2[:, :d_ff], g2[:, d_ff:]).view(*gu.shape[:-1], d_ff)
        return self.down_proj(h)


class DSALTTransformerBlock(nn.Module):
    def __init__(self, d_model: int, n_heads: int, n_min: int, n_max: int, k_lmk: int, max_seq_len: int, d_ff: int,
                 dropout: float = 0.0, yarn_scale: float = 1.0, layer_idx: int = 0, n_kv_heads: int | None = None,
                 qkv_bias: bool = False, rope_base: float = 10000.0, select_mode: str = "global",
                 block_size: int = 512, stats_scope: str = "packed"):
        super().__init__()
        self.layer_idx = layer_idx
        self.attn_norm = RMSENorm(d_model)
        self.ffn_norm = RMSENorm(d_model)
        self.attn = DSALTAttention(d_model=d_model, n_heads=n_heads, n_min=n_min, n_max=n_max, k_lmk=k_lmk,
                                   max_seq_len=max_seq_len, dropout=dropout, yarn_scale=yarn_scale,
                                   layer_idx=layer_idx, n_kv_heads=n_kv_heads, qkv_bias=qkv_bias,
                                   rope_base=rope_base, select_mode=select_mode, block_size=block_size,
                                   stats_scope=stats_scope)
        self.ffn = SwiGLUFFN(d_model=d_model, d_ff=d_ff, dropout=dropout)

    def forward(self, x, cu_seqlens=None, max_seqlen=None, gradient_checkpointing: bool = False, rope_cs=None,
                cu_list=None):
        if gradient_checkpointing and self.training:
            aux = torch.zeros((), device=x.device, dtype=x.dtype)

            def attn_part(h):
                nonlocal aux
                out, aux = self.attn(h, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, rope_cs=rope_cs,
                                     cu_list=cu_list)
                return out

            x = x + torch.utils.checkpoint.checkpoint(attn_part, self.attn_norm(x), use_reentrant=False)
            x = x + torch.utils.checkpoint.checkpoint(self.ffn, self.ffn_norm(x), use_reentrant=False)
            return x, aux
        x_attn, aux = self.attn(self.attn_norm(x), cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, rope_cs=rope_cs,
                                cu_list=cu_list)
        x = x + x_attn
        x = x + self.ffn(self.ffn_norm(x))
        return x, aux

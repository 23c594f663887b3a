"""Causal language model on DSALT attention.

Mirrors ``DSALTLMHeadModel`` of ``dsalt/model/dsalt_lm.py:64-284``: token embedding, a stack
of ``DSALTTransformerBlock``, final RMSNorm and an LM head (tied to the embedding by
default); packed input (``cu_seqlens``) or batched ``[B, T]``; with ``labels`` the loss
(chunked cross-entropy, :19-39, or the fused linear cross-entropy), without them the logits of every position (:280).
Initialisation as :164-172.  Per forward the RoPE rows are gathered once for all layers
and ``cu_seqlens`` is copied to the host once (:220-235).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.RMSENorm import RMSENorm
from ..modules.dsalt_transformer import DSALTTransformerBlock
from .config import DSALTConfig


def _chunked_cross_entropy(x, weight, labels, chunk_size: int = 512):
    """Mean token cross-entropy of ``x @ weight^T`` against ``labels`` (-100 ignored), over
    row chunks so the full logits never exist at once (dsalt/model/dsalt_lm.py:19-39)."""
    loss_acc = torch.zeros((), device=x.device, dtype=torch.float32)
    valid_acc = torch.zeros((), device=x.device, dtype=torch.float32)
    for start in range(0, x.shape[0], chunk_size):
        end = min(start + chunk_size, x.shape[0])
        y = labels[start:end]
        logits = F.linear(x[start:end], weight)
        loss_acc = loss_acc + F.cross_entropy(logits, y, ignore_index=-100, reduction="sum")
        valid_acc = valid_acc + (y != -100).sum()
    return loss_acc / valid_acc.clamp(min=1.0)


class DSALTLMHeadModel(nn.Module):
    def __init__(self, vocab_size: int, d_model: int, n_layers: int, n_heads: int, n_min: int, n_max: int,
                 k_lmk: int, max_seq_len: int, d_ff: int | None = None, dropout: float = 0.0,
                 yarn_scale: float = 1.0, tie_weights: bool = True, padding_idx: int | None = None,
                 lm_head_chunk_size: int = 2048, loss_fn: str = "chunked", aux_loss_weight: float = 0.0,
                 n_kv_heads: int | None = None, qkv_bias: bool = False, rope_base: float = 10000.0,
                 select_mode: str = "global", block_size: int = 512, stats_scope: str = "packed"):
        super().__init__()
        if loss_fn not in ("auto", "chunked", "liger"):
            raise ValueError(f"unknown loss_fn {loss_fn!r} (one of 'auto', 'chunked', 'liger')")
        self.d_model, self.n_layers, self.vocab_size = d_model, n_layers, vocab_size
        self.lm_head_chunk_size, self.loss_fn, self.aux_loss_weight = lm_head_chunk_size, loss_fn, aux_loss_weight
        if d_ff is None:
            d_ff = ((int(8 / 3 * d_model) + 127) // 128) * 128
        self.embed_tokens = nn.Embedding(vocab_size, d_model, padding_idx=padding_idx)
        self.embed_dropout = nn.Dropout(dropout)
        self.layers = nn.ModuleList([
            DSALTTransformerBlock(d_model=d_model, n_heads=n_heads, n_min=n_min, n_max=n_max, k_lmk=k_lmk,
                                  max_seq_len=max_seq_len, d_ff=d_ff, dropout=dropout, yarn_scale=yarn_scale,
                                  layer_idx=i, n_kv_heads=n_kv_heads, qkv_bias=qkv_bias, rope_base=rope_base,
                                  select_mode=select_mode, block_size=block_size, stats_scope=stats_scope)
            for i in range(n_layers)])
        self.final_norm = RMSENorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        if tie_weights:
            self.lm_head.weight = self.embed_tokens.weight
        self._init_weights()

    @classmethod
    def from_config(cls, config: DSALTConfig) -> "DSALTLMHeadModel":
        return cls(**config.to_dict())

    def _init_weights(self):
        nn.init.normal_(self.embed_tokens.weight, std=0.02)
        residual_std = 0.02 / math.sqrt(2 * self.n_layers)
        for name, module in self.named_modules():
            if isinstance(module, nn.Linear):
                std = residual_std if any(k in name for k in ("out_proj", "down_proj")) else 0.02
                nn.init.normal_(module.weight, std=std)
                if module.bias is not None:
                    nn.init.zeros_(module.bias)

    def _compute_loss(self, x, labels):
        """"chunked": torch logits per row chunk + F.cross_entropy (:19-39); "liger" and "auto":
        the fused linear cross-entropy (HIP row kernel between the chunk GEMMs, :42-51; the
        reference's "auto" measures both once, here the fused path is taken)."""
        flat_x = x.view(-1, self.d_model)
        flat_labels = labels.view(-1).long()
        if self.loss_fn in ("liger", "auto"):
            from ..kernels.cross_entropy import LigerFusedLinearCrossEntropyFunction
            return LigerFusedLinearCrossEntropyFunction.apply(flat_x.contiguous(), self.lm_head.weight,
                                                              flat_labels.contiguous())[0]
        return _chunked_cross_entropy(flat_x, self.lm_head.weight, flat_labels, self.lm_head_chunk_size)

    @staticmethod
    def _to_autocast_dtype(x):
        dev = x.device.type
        enabled = torch.is_autocast_enabled(dev)
        dtype = torch.get_autocast_dtype(dev)
        return x.to(dtype) if enabled and x.dtype != dtype else x

    @staticmethod
    def _packed_rope_meta(cu_seqlens, total_len, attn0):
        """RoPE rows of every token (float32, gathered once for all layers) and a host copy
        of cu_seqlens."""
        dev = cu_seqlens.device
        cu = cu_seqlens.long()
        lens = cu[1:] - cu[:-1]
        seq_ids = torch.repeat_interleave(torch.arange(lens.numel(), device=dev), lens)
        pos_ids = torch.arange(total_len, device=dev) - cu[:-1][seq_ids]
        cos, sin = attn0._rope_tables32()
        return (cos[pos_ids], sin[pos_ids]), cu_seqlens.detach().to("cpu").tolist()

    def forward(self, input_ids, cu_seqlens=None, max_seqlen=None, labels=None, gradient_checkpointing: bool = False,
                padding_mask=None):
        del padding_mask
        if max_seqlen is None:
            max_seqlen = input_ids.shape[-1]
        x = self._to_autocast_dtype(self.embed_dropout(self.embed_tokens(input_ids)))
        aux_loss = torch.zeros((), device=input_ids.device, dtype=x.dtype)
        rope_cs = cu_list = None
        if cu_seqlens is not None:
            rope_cs, cu_list = self._packed_rope_meta(cu_seqlens, input_ids.shape[0], self.layers[0].attn)
        for layer in self.layers:
            x, layer_aux = layer(x, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen,
                                 gradient_checkpointing=gradient_checkpointing, rope_cs=rope_cs, cu_list=cu_list)
            aux_loss = aux_loss + layer_aux
        x = self.final_norm(x)
        if labels is not None:
            loss = self._compute_loss(x, labels) + self.aux_loss_weight * aux_loss
            return {"loss": loss, "logits": None, "aux_loss": aux_loss.detach()}
        return {"loss": None, "logits": self.lm_head(x), "aux_loss": None}

    def num_parameters(self, trainable_only: bool = True) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad or not trainable_only)

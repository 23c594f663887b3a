"""Landmark selection and packed-sequence metadata with the reference's signatures.

Mirrors ``dsalt/kernels/selectors.py``:
  ``_seq_meta`` (:15-34) and ``_build_seq_block_map`` (:37-67): host metadata, here cached
  on the full ``cu_seqlens`` contents (the reference keys its caches on
  ``(total_len, num_seqs)`` only, so two raggings with equal totals collide);
  ``_compute_landmark_indices`` (:75-134): one HIP selection call (norms, z statistics,
  exclusion ``j_rel < w_j``, top-k with lowest-index ties, ``-1`` padding);
  ``_build_landmark_kv`` (:137-159): one HIP gather.
New keyword arguments select the block-causal variant (``select_mode="block"``, one set per
``block_size`` query rows from earlier positions only, the semantics of
``results/causal_landmark_check.py:95-113``) and the scope of the z statistics
(``"packed"``, the reference's whole-batch statistics, or ``"sequence"``).
"""
from __future__ import annotations

import torch

from .. import ops

_SEQ_META_CACHE: dict = {}
_SEQ_BLOCK_MAP_CACHE: dict = {}
_MODES = {"global": ops.SELECT_GLOBAL, "block": ops.SELECT_BLOCK}
_SCOPES = {"packed": ops.STATS_PACKED, "sequence": ops.STATS_SEQUENCE}


def _cu_key(cu_seqlens: torch.Tensor, cu_list):
    if cu_list is not None:
        return tuple(int(c) for c in cu_list)
    return tuple(int(c) for c in cu_seqlens.detach().to("cpu").tolist())


def _seq_meta(cu_seqlens: torch.Tensor, total: int, device, cu_list: list | None = None):
    """``(num_seqs, lens, starts, seq_ids, seq_off, max_len)`` of a packed batch."""
    key = (_cu_key(cu_seqlens, cu_list), str(device))
    if key in _SEQ_META_CACHE:
        return _SEQ_META_CACHE[key]
    cu = torch.tensor(key[0], dtype=torch.long, device=device)
    num_seqs = cu.numel() - 1
    lens = cu[1:] - cu[:-1]
    starts = cu[:-1]
    seq_ids = torch.repeat_interleave(torch.arange(num_seqs, device=device), lens)
    seq_off = torch.arange(total, device=device) - starts[seq_ids]
    max_len = max(key[0][i + 1] - key[0][i] for i in range(num_seqs)) if num_seqs else 0
    val = (num_seqs, lens, starts, seq_ids, seq_off, max_len)
    _SEQ_META_CACHE[key] = val
    return val


def _build_seq_block_map(cu_seqlens: torch.Tensor, block_m: int, device, cu_list: list | None = None):
    """``([total_blocks, 2] int32 (sequence, block-in-sequence), total_blocks)``."""
    cuk = _cu_key(cu_seqlens, cu_list)
    key = (cuk, int(block_m), str(device))
    if key in _SEQ_BLOCK_MAP_CACHE:
        return _SEQ_BLOCK_MAP_CACHE[key]
    cu = torch.tensor(cuk, dtype=torch.long)
    lens = cu[1:] - cu[:-1]
    blocks_per = (lens + block_m - 1) // block_m
    total = int(blocks_per.sum())
    seq_col = torch.repeat_interleave(torch.arange(lens.numel(), dtype=torch.int32), blocks_per)
    blk_col = (torch.arange(total, dtype=torch.int32)
               - torch.repeat_interleave(blocks_per.cumsum(0) - blocks_per, blocks_per).int())
    result = torch.stack([seq_col, blk_col], dim=1).contiguous().to(device)
    _SEQ_BLOCK_MAP_CACHE[key] = (result, total)
    return result, total


def _max_seqlen(cu_seqlens, cu_list):
    if cu_list is not None:
        return max(1, max(int(cu_list[i + 1]) - int(cu_list[i]) for i in range(len(cu_list) - 1)))
    return max(1, int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item()))


def _compute_landmark_indices(x, W_V, alpha, w_sizes, cu_seqlens, k_lmk, n_min, total_len, cu_list=None,
                              head_dim=None, *, select_mode: str = "global", block_size: int = 512,
                              stats_scope: str = "packed"):
    """Hard top-k landmark indices per (head, sequence[, query block]).

    Returns ``(idx, z_x, z_v)``: ``idx`` int64 ``[H, S, k]`` (global) or ``[H, S, n_blocks, k]``
    (block-causal), ascending within each set with ``-1`` padding; ``z_x [T]`` and
    ``z_v [T, H]`` are the standardized signals (global variant; ``None`` for block-causal).
    ``n_min`` is accepted for signature compatibility and unused, as in the reference.
    """
    del n_min, total_len
    n_heads = alpha.shape[0]
    dh = head_dim if head_dim is not None else W_V.shape[0] // n_heads
    T = x.shape[0]
    n_kv = W_V.shape[0] // dh
    mode = _MODES[select_mode]
    with torch.no_grad():
        v = (x.detach() @ W_V.detach().T).view(T, n_kv, dh)
        w = w_sizes.detach().long().to(torch.int32)
        res = ops.select_landmarks(x.detach(), v, alpha.detach(), w, cu_seqlens, k_lmk,
                                   max_seqlen=_max_seqlen(cu_seqlens, cu_list), select_mode=mode,
                                   block_size=block_size, stats_scope=_SCOPES[stats_scope],
                                   want_scores=mode == ops.SELECT_GLOBAL)
    if mode == ops.SELECT_BLOCK:
        return res.long(), None, None
    idx, z_x, z_v, _ = res
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)
    return idx[:, :, 0].long(), z_x, z_v


def _build_landmark_kv(K, V, lmk_indices, cu_seqlens, k_lmk, n_heads, head_dim, *, block_size=None,
                       max_seqlen=None):
    """Gather landmark keys/values ``[H, S, k, D]`` (or ``[H, S, n_blocks, k, D]``); rows of
    ``-1`` slots are zero."""
    block = lmk_indices.dim() == 4
    idx = lmk_indices if block else lmk_indices.unsqueeze(2)
    mode = ops.SELECT_BLOCK if block else ops.SELECT_GLOBAL
    if max_seqlen is None:
        max_seqlen = _max_seqlen(cu_seqlens, None)
    if block and block_size is None:
        block_size = -(-max_seqlen // idx.shape[2])
        block_size = -(-block_size // 64) * 64
    lk, lv = ops.gather_landmarks(K, V, cu_seqlens, idx, max_seqlen=max_seqlen, select_mode=mode,
                                  block_size=block_size or 512, n_heads=n_heads)
    if not block:
        lk, lv = lk[:, :, 0], lv[:, :, 0]
    return lk, lv

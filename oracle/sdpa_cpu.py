"""The reference library's CPU attention path, timed as the CPU baseline - TEST INFRASTRUCTURE ONLY.

Restates the masked-SDPA fallback that ``DSALTAttention._packed`` takes without Triton
(``dsalt/modules/dsalt_attention.py:626-634``): landmark scores and top-k
(``oracle/select_oracle.c``), the boolean ``[T, T]`` mask of ``_build_mask_packed``
(``dsalt_attention.py:95-144``: window band OR the per-sequence union of landmarks), the
additive ``-inf`` mask in the input dtype and ``F.scaled_dot_product_attention``
(``dsalt/kernels/sparse_attn.py:29-57``), with autograd for the backward.

Training workloads time the reference's dense training path instead (``_packed_train``,
``dsalt_attention.py:489-563``): the per-head log-bias rows (soft window edge, landmark
log-weights ``log sigmoid(s / tau_lmk)`` from the selection's scores) built with autograd
through ``w~`` and the log-weights, SDPA, and the backward into q, k, v, ``w~`` and the
log-weights.

A dense masked SDPA costs O(T) per query row whatever the sparsity, so the timing runs the
full-length selection and a bounded sample of query rows (all heads, all keys); the
per-token time is ``t_select / T + t_attention / rows``; rows run in chunks of 256 query rows.  Only bench.py's ``cpu_baseline``
leg calls this.
"""
from __future__ import annotations

import os
import time

import numpy as np
import torch
import torch.nn.functional as F

from . import select as OS


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _odt(dt: torch.dtype) -> int:
    return {torch.float32: OS.DTYPE_F32, torch.bfloat16: OS.DTYPE_BF16, torch.float16: OS.DTYPE_F16}[dt]


def literal_mask_rows(w: torch.Tensor, cu: torch.Tensor, idx: np.ndarray, rows: torch.Tensor) -> torch.Tensor:
    """Rows ``rows`` of the reference fallback's [T, T] mask (one mask for all heads)."""
    T = int(cu[-1])
    seq = torch.searchsorted(cu[1:].long(), rows.long(), right=True)
    st = cu[seq].long()
    rel = rows.long() - st
    lo = (rel - w[rows].long().clamp(min=1) + 1).clamp(min=0) + st
    col = torch.arange(T).unsqueeze(0)
    m = (col >= lo.unsqueeze(1)) & (col <= rows.long().unsqueeze(1))
    for s in torch.unique(seq).tolist():
        pos = idx[:, s].reshape(-1)
        L = int(cu[s + 1] - cu[s])
        pos = np.unique(pos[(pos >= 0) & (pos < L)])
        if len(pos):
            r = (seq == s).nonzero()[:, 0]
            m[r.unsqueeze(1), torch.as_tensor(pos + int(cu[s])).unsqueeze(0)] = True
    return m


def train_bias_rows(w_cont, cu, pos, logw, rows, tau_win, win_edge):
    """Rows ``rows`` of the dense training log-bias, ``[H, R, T]``, differentiable in
    ``w_cont`` (``[T]``) and ``logw`` (``[H, S, k]``); ``pos`` ``[H, S, k]`` int."""
    T = int(cu[-1])
    H = pos.shape[0]
    seq = torch.searchsorted(cu[1:].long(), rows.long(), right=True)
    st = cu[seq].long()
    col = torch.arange(T)
    d = (rows.long()[:, None] - col[None, :]).to(w_cont.dtype)
    wi = w_cont[rows][:, None]
    lb = torch.log(torch.sigmoid((wi - d) / tau_win).clamp(min=1e-20))
    lb = torch.where(d <= wi - win_edge, torch.zeros_like(lb), lb)
    band = (d >= 0) & (d <= wi) & (col[None, :] >= st[:, None])
    lb = lb.masked_fill(~band, float("-inf"))
    out = []
    for h in range(H):
        b = lb
        for s in torch.unique(seq).tolist():
            ps = pos[h, s].long()
            ok = ps >= 0
            ps, lw = ps[ok], logw[h, s][ok]
            if ps.numel() == 0:
                continue
            rel = (rows.long() - int(cu[s]))[:, None].to(w_cont.dtype)
            vis = (seq == s)[:, None] & (ps[None, :] <= rel) & (ps[None, :].to(w_cont.dtype) < rel - wi)
            term = torch.full((rows.numel(), T), float("-inf"), dtype=lb.dtype)
            term = term.index_put((torch.arange(rows.numel())[:, None].expand_as(vis), (ps + int(cu[s]))[None, :]
                                   .expand_as(vis)), torch.where(vis, lw[None, :].expand_as(vis),
                                                                 torch.full_like(vis, float("-inf"), dtype=lb.dtype)))
            b = torch.maximum(b, term)
        out.append(b)
    return torch.stack(out)


def _train_attention_rows(q, k, v, dout, w_cont, logw, cu, pos, rows, tau_win, win_edge):
    qs = q.detach().clone().requires_grad_(True)
    kk = k.detach().clone().requires_grad_(True)
    vv = v.detach().clone().requires_grad_(True)
    wc = w_cont.detach().clone().requires_grad_(True)
    lw = logw.detach().clone().requires_grad_(True)
    bias = train_bias_rows(wc, cu, pos, lw, rows, tau_win, win_edge)
    out = F.scaled_dot_product_attention(qs.transpose(0, 1)[None], kk.transpose(0, 1)[None],
                                         vv.transpose(0, 1)[None], attn_mask=bias.to(q.dtype)[None])
    out = out[0].transpose(0, 1)
    out.backward(dout)
    return out


def _attention_rows(q, k, v, dout, mask):
    qs = q.detach().clone().requires_grad_(True)
    kk = k.detach().clone().requires_grad_(True)
    vv = v.detach().clone().requires_grad_(True)
    additive = torch.zeros(mask.shape, dtype=q.dtype).masked_fill(~mask, float("-inf"))[None, None]
    out = F.scaled_dot_product_attention(qs.transpose(0, 1)[None], kk.transpose(0, 1)[None],
                                         vv.transpose(0, 1)[None], attn_mask=additive)
    out = out[0].transpose(0, 1)
    out.backward(dout)
    return out


def time_baseline(x: dict, k_lmk: int, stats_scope: int, target_s: float = 12.0, backward: bool = True,
                  train=None):
    """Times the CPU path on the inputs ``x`` (CPU tensors from dsalt_amd.workloads).
    ``train = (tau_win, win_edge, tau_lmk)`` times the dense training path.

    Returns a dict with tokens_per_s, threads, rows and the timing split.
    """
    threads = torch.get_num_threads()
    T, H = x["q"].shape[:2]
    rep = H // x["k"].shape[1]
    # grouped K/V heads are repeated per query head, as the reference's fallback does
    # (dsalt/modules/dsalt_attention.py:254-268)
    kx = x["k"].repeat_interleave(rep, dim=1) if rep > 1 else x["k"]
    vx = x["v"].repeat_interleave(rep, dim=1) if rep > 1 else x["v"]
    t0 = time.perf_counter()
    res = OS.select(_bits(x["h"]), _bits(x["v"]), x["alpha"].numpy(), x["w"].numpy(), x["cu"].numpy(), k_lmk,
                    _odt(x["h"].dtype), stats_scope=stats_scope, want_scores=train is not None)
    if train is not None:
        idx, _, _, sc = res
        pos = torch.as_tensor(idx[:, :, 0]).long()
        starts = x["cu"][:-1].long()
        s_sel = torch.as_tensor(sc)[starts[None, :, None] + pos.clamp(min=0),
                                    torch.arange(pos.shape[0])[:, None, None]]
        logw = torch.log(torch.sigmoid(s_sel / train[2]).clamp(min=1e-20))
        logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    else:
        idx = res
    t_sel = time.perf_counter() - t0

    def attn(nrows):
        t1 = time.perf_counter()
        chunk = min(64 if train is not None else 256, nrows)
        for r0 in range(T - nrows, T, chunk):
            rows = torch.arange(r0, min(T, r0 + chunk))
            if train is not None:
                _train_attention_rows(x["q"][rows], kx, vx, x["dout"][rows], x["w_cont"], logw, x["cu"],
                                      pos, rows, train[0], train[1])
                continue
            m = literal_mask_rows(x["w"], x["cu"], idx, rows)
            if backward:
                _attention_rows(x["q"][rows], kx, vx, x["dout"][rows], m)
            else:
                with torch.no_grad():
                    additive = torch.zeros(m.shape, dtype=x["q"].dtype).masked_fill(~m, float("-inf"))[None, None]
                    F.scaled_dot_product_attention(x["q"][rows].transpose(0, 1)[None], kx.transpose(0, 1)[None],
                                                   vx.transpose(0, 1)[None], attn_mask=additive)
        return time.perf_counter() - t1

    probe = min(T, 256)
    if train is not None:
        probe = min(T, 64)
    attn(probe)  # first call pays one-time setup
    t_probe = attn(probe)
    rows = int(min(T, max(probe, (target_s / max(t_probe, 1e-3)) * probe)))
    rows = max(probe, (rows // probe) * probe)
    t_att = attn(rows)
    per_token = t_sel / T + t_att / rows
    return dict(tokens_per_s=1.0 / per_token, threads=threads, rows=rows, t_select=t_sel, t_attention=t_att,
                cpu_count=os.cpu_count())

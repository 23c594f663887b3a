"""fp64 restatement of the DSALT training variant - TEST INFRASTRUCTURE ONLY.

Only tests/ import this module; the product never does.

Semantics (the dense reference the training kernel is checked against,
``dsalt/modules/dsalt_attention.py:520-563``, fed to SDPA as in ``_packed_train`` :488-518):
  * band: keys ``j`` with ``0 <= d = i - j <= w~(i)``; logit bias 0 in the core
    ``d <= w~ - win_edge``, else ``log sigmoid((w~ - d) / tau_win)`` (:537-544);
  * landmarks: slot ``p`` (``p >= 0``) of the row's set where ``p <= i`` and ``p < i - w~``
    (:549-553), logit bias ``lmk_logw`` (-inf for empty slots);
  * union by elementwise max (landmark columns lie left of the band, so the two never meet);
  * ``O = softmax(q k^T scale + bias) V``, ``LSE`` in natural log.
Gradients (``dsalt/kernels/dsalt_triton_train.py:312-379``): ``P = exp(logit - LSE)``,
``dS = P (dO V^T - delta)``, ``dQ = scale dS K``, ``dK = scale dS^T Q``, ``dV = P^T dO``,
``d lmk_logw = sum_i dS`` over the rows that see the slot (:329-333), and
``d w~(i) = sum_h sum_j dS_ij (1 - sigmoid(z_ij)) / tau`` over band keys outside the core,
``z = (w~ - d) / tau`` (:372-375); the band's hard cut carries no gradient.

Dense ``[L, L]`` blocks per (head, sequence): for the small shapes of the parity tests.
"""
from __future__ import annotations

import numpy as np

__all__ = ["train_bias", "train_fwd", "train_bwd"]


def _sigmoid(x):
    return np.exp(-np.logaddexp(0.0, -x))


def train_bias(w_seq, lmk_pos_hs, lmk_logw_hs, tau_win, win_edge):
    """[L, L] fp64 logit bias of one (head, sequence); also the d bias / d w~ factor."""
    w = np.asarray(w_seq, np.float64)
    L = w.shape[0]
    i = np.arange(L)[:, None].astype(np.float64)
    j = np.arange(L)[None, :].astype(np.float64)
    d = i - j
    wi = w[:, None]
    z = (wi - d) / tau_win
    in_band = (d >= 0) & (d <= wi)
    core = d <= wi - win_edge
    win = np.where(core, 0.0, np.log(np.maximum(_sigmoid(z), 1e-20)))
    bias = np.where(in_band, win, -np.inf)
    dbias_dw = np.where(in_band & ~core, (1.0 - _sigmoid(z)) / tau_win, 0.0)
    for p, lw in zip(np.asarray(lmk_pos_hs).tolist(), np.asarray(lmk_logw_hs, np.float64).tolist()):
        if p < 0 or p >= L:
            continue
        rows = (p <= np.arange(L)) & (p < np.arange(L) - w)
        bias[rows, p] = np.maximum(bias[rows, p], lw)
    return bias, dbias_dw


def _blocks(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge):
    T, H, D = q.shape
    for h in range(H):
        for s in range(len(cu) - 1):
            st, en = int(cu[s]), int(cu[s + 1])
            if en == st:  # an empty sequence has no rows
                continue
            bias, dbw = train_bias(w_cont[st:en], lmk_pos[h, s], lmk_logw[h, s], tau_win, win_edge)
            logits = (q[st:en, h] @ k[st:en, h].T) * scale + bias
            yield h, s, st, en, logits, dbw


def train_fwd(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge):
    """O [T,H,D] and LSE [T,H] in float64."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    out = np.zeros_like(q)
    lse = np.full(q.shape[:2], -np.inf)
    for h, s, st, en, lg, _ in _blocks(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge):
        m = lg.max(1, keepdims=True)
        p = np.exp(lg - m)
        l = p.sum(1, keepdims=True)
        out[st:en, h] = (p / l) @ v[st:en, h]
        lse[st:en, h] = (m + np.log(l))[:, 0]
    return out, lse


def train_bwd(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge, dout, out=None):
    """(dq, dk, dv, d_w [T], d_logw [H,S,K]) in float64; ``out`` feeds delta (exact when None)."""
    q, k, v, dout = (np.asarray(t, np.float64) for t in (q, k, v, dout))
    o_ref, lse = train_fwd(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge)
    o = o_ref if out is None else np.asarray(out, np.float64)
    delta = (o * dout).sum(-1)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dw = np.zeros(q.shape[0])
    dlogw = np.zeros(np.asarray(lmk_logw).shape)
    for h, s, st, en, lg, dbw in _blocks(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge):
        p = np.exp(lg - lse[st:en, h][:, None])
        ds = p * (dout[st:en, h] @ v[st:en, h].T - delta[st:en, h][:, None])
        dq[st:en, h] = scale * ds @ k[st:en, h]
        dk[st:en, h] = scale * ds.T @ q[st:en, h]
        dv[st:en, h] = p.T @ dout[st:en, h]
        dw[st:en] += (ds * dbw).sum(1)
        L = en - st
        wv = np.asarray(w_cont[st:en], np.float64)
        for slot, pos in enumerate(np.asarray(lmk_pos[h, s]).tolist()):
            if 0 <= pos < L:
                rows = (pos <= np.arange(L)) & (pos < np.arange(L) - wv)
                dlogw[h, s, slot] = ds[rows, pos].sum()
    return dq, dk, dv, dw, dlogw


def _banded(q, k, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge, rb):
    """Row blocks of at most ``rb`` rows with the logits over their band keys [kr0, i1) and
    over the landmark slots (the same semantics as ``train_bias``, with each slot a key of
    its own; the sets of the workloads hold distinct positions, where the two agree)."""
    T, H, D = q.shape
    for h in range(H):
        for s in range(len(cu) - 1):
            st, en = int(cu[s]), int(cu[s + 1])
            L = en - st
            wv = np.asarray(w_cont[st:en], np.float64)
            pos = np.asarray(lmk_pos[h, s]).astype(np.int64)
            lw = np.asarray(lmk_logw[h, s], np.float64)
            okp = (pos >= 0) & (pos < L)
            pz = np.where(okp, pos, 0)
            for i0 in range(0, L, rb):
                i1 = min(L, i0 + rb)
                rows = np.arange(i0, i1)
                wr = wv[i0:i1]
                kr0 = int(max(0, np.floor((rows - np.maximum(wr, 0.0)).min())))
                d = (rows[:, None] - np.arange(kr0, i1)[None, :]).astype(np.float64)
                z = (wr[:, None] - d) / tau_win
                in_band = (d >= 0) & (d <= wr[:, None])
                core = d <= wr[:, None] - win_edge
                sig = _sigmoid(z)
                win = np.where(core, 0.0, np.log(np.maximum(sig, 1e-20)))
                sb = (q[st + i0:st + i1, h] @ k[st + kr0:st + i1, h].T) * scale + np.where(in_band, win, -np.inf)
                dbw = np.where(in_band & ~core, (1.0 - sig) / tau_win, 0.0)
                vis = okp[None, :] & (pos[None, :] <= rows[:, None]) & (pos[None, :] < rows[:, None] - wr[:, None])
                sl = (q[st + i0:st + i1, h] @ k[st + pz, h].T) * scale + np.where(vis, lw[None, :], -np.inf)
                yield h, s, st, i0, i1, kr0, pz, okp, sb, sl, dbw


def train_fwd_banded(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge, rb=512):
    """``train_fwd`` over banded row blocks: the same values for full-length sequences."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    out = np.zeros_like(q)
    lse = np.full(q.shape[:2], -np.inf)
    for h, s, st, i0, i1, kr0, pz, okp, sb, sl, _ in _banded(q, k, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win,
                                                              win_edge, rb):
        m = np.maximum(sb.max(1), sl.max(1) if sl.shape[1] else -np.inf)[:, None]
        pb, pl = np.exp(sb - m), np.exp(sl - m)
        l = pb.sum(1, keepdims=True) + pl.sum(1, keepdims=True)
        out[st + i0:st + i1, h] = (pb @ v[st + kr0:st + i1, h] + pl @ v[st + pz, h]) / l
        lse[st + i0:st + i1, h] = (m + np.log(l))[:, 0]
    return out, lse


def train_bwd_banded(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge, dout, out=None, rb=512):
    """``train_bwd`` over banded row blocks (dq, dk, dv, d_w, d_logw)."""
    q, k, v, dout = (np.asarray(t, np.float64) for t in (q, k, v, dout))
    o_ref, lse = train_fwd_banded(q, k, v, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win, win_edge, rb)
    o = o_ref if out is None else np.asarray(out, np.float64)
    delta = (o * dout).sum(-1)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dw = np.zeros(q.shape[0])
    dlogw = np.zeros(np.asarray(lmk_logw).shape)
    for h, s, st, i0, i1, kr0, pz, okp, sb, sl, dbw in _banded(q, k, w_cont, cu, lmk_pos, lmk_logw, scale, tau_win,
                                                                win_edge, rb):
        r = slice(st + i0, st + i1)
        ls = lse[r, h][:, None]
        pb, pl = np.exp(sb - ls), np.exp(sl - ls)
        dl = delta[r, h][:, None]
        dsb = pb * (dout[r, h] @ v[st + kr0:st + i1, h].T - dl)
        dsl = pl * (dout[r, h] @ v[st + pz, h].T - dl)
        dq[r, h] += scale * (dsb @ k[st + kr0:st + i1, h] + dsl @ k[st + pz, h])
        dk[st + kr0:st + i1, h] += scale * (dsb.T @ q[r, h])
        dv[st + kr0:st + i1, h] += pb.T @ dout[r, h]
        np.add.at(dk[:, h], st + pz[okp], scale * (dsl.T @ q[r, h])[okp])
        np.add.at(dv[:, h], st + pz[okp], (pl.T @ dout[r, h])[okp])
        dw[r] += (dsb * dbw).sum(1)
        dlogw[h, s] += dsl.sum(0)
    return dq, dk, dv, dw, dlogw

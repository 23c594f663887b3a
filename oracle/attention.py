"""fp64 restatement of the DSALT attention operator - TEST INFRASTRUCTURE ONLY.

Only tests/, the smoke check and bench.py's CPU-baseline leg import this module; the
product never does.

Kernel semantics (the operator the GPU implements), restated from
``dsalt/kernels/dsalt_triton_attn.py``:
  * window keys ``j`` with ``i - w_i + 1 <= j <= i`` (:102-106), ``w_i`` clamped at 1 (:70);
  * landmark keys at positions ``p`` with ``0 <= p < seq_len``, ``p <= i`` and
    ``p < i - w_i + 1`` (:132-135), logit ``q.k * scale + bias`` (:140), so a landmark
    inside the window is never counted twice;
  * ``O = softmax(logits) V`` and ``LSE = log sum exp(logits)`` in natural log (:150-164);
  * the same mask written as exact torch code in ``results/causal_landmark_check.py:119-147``.
Backward (``dsalt/kernels/dsalt_triton_bwd.py:141-199``): ``P = exp(logit - LSE)``,
``dP = dO V^T``, ``dS = P (dP - delta)`` with ``delta = rowsum(O dO)`` (:44),
``dQ = scale dS K``, ``dK = scale dS^T Q``, ``dV = P^T dO``, ``d_bias = sum_i dS`` (:153).

Literal fallback (``dsalt/modules/dsalt_attention.py:95-144`` with
``dsalt/kernels/sparse_attn.py:29-57``): one ``[T, T]`` mask shared by all heads, the
window band OR-ed with the union over heads of each sequence's landmarks applied to every
row of the sequence without a causal cut.

Everything here is float64 numpy; banded blocks turn the sparse pattern into small dense
GEMMs so full-length sequences finish in seconds.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "attention_fwd",
    "attention_probs",
    "attention_bwd",
    "dense_mask_kernel",
    "dense_attention",
    "literal_mask",
    "valid_landmarks",
]


def _rows_lo(w: np.ndarray, st: int, rows: np.ndarray) -> np.ndarray:
    wi = np.maximum(w[st + rows].astype(np.int64), 1)
    return np.maximum(rows - wi + 1, 0)


def valid_landmarks(lmk_row: np.ndarray, seq_len: int) -> np.ndarray:
    """Slots of one landmark set that hold a position inside the sequence."""
    return np.nonzero((lmk_row >= 0) & (lmk_row < seq_len))[0]


def _set_of_row(i: int, block_size: int | None) -> int:
    return 0 if block_size is None else i // block_size


def _row_blocks(seq_len: int, block_size: int | None, rb: int = 512):
    """Row blocks that never straddle two landmark sets."""
    step = rb if block_size is None else min(rb, block_size)
    if block_size is not None and block_size % step:
        step = block_size
    for i0 in range(0, seq_len, step):
        yield i0, min(seq_len, i0 + step)


def _block_logits(q, k, w, st, i0, i1, lmk_row, bias_row, scale):
    """Logits of rows [i0, i1) over the band [kr0, i1) and the landmark slots."""
    rows = np.arange(i0, i1)
    lo = _rows_lo(w, st, rows)
    kr0 = int(lo.min())
    cols = np.arange(kr0, i1)
    sb = (q[st + i0:st + i1] @ k[st + kr0:st + i1].T) * scale
    band = (cols[None, :] >= lo[:, None]) & (cols[None, :] <= rows[:, None])
    sb = np.where(band, sb, -np.inf)
    pos = lmk_row
    kl = k[st + np.maximum(pos, 0)]
    sl = (q[st + i0:st + i1] @ kl.T) * scale
    if bias_row is not None:
        sl = sl + bias_row[None, :]
    lmk_ok = (pos[None, :] >= 0) & (pos[None, :] < lo[:, None])
    sl = np.where(lmk_ok, sl, -np.inf)
    return kr0, sb, sl, band, lmk_ok


def attention_fwd(q, k, v, w, cu, lmk_idx, scale, lmk_bias=None, block_size=None):
    """O [T,H,D] and LSE [T,H] (float64) of the kernel semantics.

    q [T,H,D]; k, v [T,Hkv,D]; w [T] int; cu [S+1]; lmk_idx [H,S,n_sets,K] with
    sequence-relative positions (-1 = empty, any order); lmk_bias same shape or None.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, H, D = q.shape
    rep = H // k.shape[1]
    out = np.zeros((T, H, D))
    lse = np.full((T, H), -np.inf)
    for h in range(H):
        g = h // rep
        qh, kh, vh = q[:, h], k[:, g], v[:, g]
        for s in range(len(cu) - 1):
            st, L = int(cu[s]), int(cu[s + 1] - cu[s])
            for i0, i1 in _row_blocks(L, block_size):
                b = _set_of_row(i0, block_size)
                pos = lmk_idx[h, s, b].astype(np.int64)
                pos = np.where(pos < L, pos, -1)
                bias = None if lmk_bias is None else lmk_bias[h, s, b].astype(np.float64)
                kr0, sb, sl, _, _ = _block_logits(qh, kh, w, st, i0, i1, pos, bias, scale)
                m = np.maximum(sb.max(1), sl.max(1) if sl.shape[1] else -np.inf)
                pb = np.exp(sb - m[:, None])
                pl = np.exp(sl - m[:, None])
                l = pb.sum(1) + pl.sum(1)
                o = pb @ vh[st + kr0:st + i1] + pl @ vh[st + np.maximum(pos, 0)]
                out[st + i0:st + i1, h] = o / l[:, None]
                lse[st + i0:st + i1, h] = m + np.log(l)
    return out, lse


def attention_probs(q, k, w, cu, lmk_idx, scale, seq=0, lmk_bias=None, block_size=None):
    """Dense [H, L, L] float64 attention probabilities of sequence ``seq`` (the matrix the
    reference rebuilds as ``_last_P``, dsalt/modules/dsalt_attention.py:636-702, here with
    the kernel semantics above: window band and the landmarks left of it)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    T, H, D = q.shape
    rep = H // k.shape[1]
    st, L = int(cu[seq]), int(cu[seq + 1] - cu[seq])
    P = np.zeros((H, L, L))
    for h in range(H):
        qh, kh = q[:, h], k[:, h // rep]
        for i0, i1 in _row_blocks(L, block_size):
            b = _set_of_row(i0, block_size)
            pos = lmk_idx[h, seq, b].astype(np.int64)
            pos = np.where(pos < L, pos, -1)
            bias = None if lmk_bias is None else lmk_bias[h, seq, b].astype(np.float64)
            kr0, sb, sl, _, _ = _block_logits(qh, kh, w, st, i0, i1, pos, bias, scale)
            m = np.maximum(sb.max(1), sl.max(1) if sl.shape[1] else -np.inf)
            pb = np.exp(sb - m[:, None])
            pl = np.exp(sl - m[:, None])
            l = (pb.sum(1) + pl.sum(1))[:, None]
            P[h, i0:i1, kr0:i1] = pb / l
            for slot, p in enumerate(pos.tolist()):
                if p >= 0:
                    P[h, i0:i1, p] += pl[:, slot] / l[:, 0]
    return P


def attention_bwd(q, k, v, w, cu, lmk_idx, scale, dout, lmk_bias=None, block_size=None, out=None,
                  operand_round=None):
    """(dq, dk, dv, d_bias) in float64 for the kernel semantics.

    ``out`` is the forward output used for ``delta``; when None the exact fp64
    forward is used.  ``operand_round`` (tests of the gradient checker only) is applied
    to P and dS before the products that consume them, as 16-bit kernels round those
    operands to the input dtype (the reference casts P to the input dtype before its
    products, ``dsalt_triton_bwd.py:148,196-199``); None keeps everything in fp64.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    dout = np.asarray(dout, np.float64)
    T, H, D = q.shape
    rep = H // k.shape[1]
    o_ref, lse = attention_fwd(q, k, v, w, cu, lmk_idx, scale, lmk_bias, block_size)
    o = o_ref if out is None else np.asarray(out, np.float64)
    delta = (o * dout).sum(-1)
    dq = np.zeros_like(q)
    dk = np.zeros((T, H, D))
    dv = np.zeros((T, H, D))
    dbias = np.zeros(lmk_idx.shape)
    for h in range(H):
        g = h // rep
        qh, kh, vh, doh = q[:, h], k[:, g], v[:, g], dout[:, h]
        for s in range(len(cu) - 1):
            st, L = int(cu[s]), int(cu[s + 1] - cu[s])
            for i0, i1 in _row_blocks(L, block_size):
                b = _set_of_row(i0, block_size)
                pos = lmk_idx[h, s, b].astype(np.int64)
                pos = np.where(pos < L, pos, -1)
                bias = None if lmk_bias is None else lmk_bias[h, s, b].astype(np.float64)
                kr0, sb, sl, _, _ = _block_logits(qh, kh, w, st, i0, i1, pos, bias, scale)
                ls = lse[st + i0:st + i1, h][:, None]
                pb = np.exp(sb - ls)
                pl = np.exp(sl - ls)
                dl = delta[st + i0:st + i1, h][:, None]
                vb = vh[st + kr0:st + i1]
                vl = vh[st + np.maximum(pos, 0)]
                dsb = pb * (doh[st + i0:st + i1] @ vb.T - dl)
                dsl = pl * (doh[st + i0:st + i1] @ vl.T - dl)
                db_row = dsl.sum(0)
                if operand_round is not None:
                    pb, pl, dsb, dsl = (operand_round(a) for a in (pb, pl, dsb, dsl))
                kb = kh[st + kr0:st + i1]
                kl = kh[st + np.maximum(pos, 0)]
                dq[st + i0:st + i1, h] += scale * (dsb @ kb + dsl @ kl)
                dk[st + kr0:st + i1, h] += scale * (dsb.T @ qh[st + i0:st + i1])
                dv[st + kr0:st + i1, h] += pb.T @ doh[st + i0:st + i1]
                ok = pos >= 0
                np.add.at(dk[:, h], st + pos[ok], scale * (dsl.T @ qh[st + i0:st + i1])[ok])
                np.add.at(dv[:, h], st + pos[ok], (pl.T @ doh[st + i0:st + i1])[ok])
                dbias[h, s, b] += db_row
    if rep > 1:
        dk = dk.reshape(T, H // rep, rep, D).sum(2)
        dv = dv.reshape(T, H // rep, rep, D).sum(2)
    return dq, dk, dv, dbias


# ----------------------------------------------------------------------------------
# brute-force forms (tiny sizes): the mask written entry by entry from its definition
# ----------------------------------------------------------------------------------
def dense_mask_kernel(w, cu, lmk_idx, block_size=None):
    """[H, T, T] bool mask of the kernel semantics, built by explicit loops."""
    H = lmk_idx.shape[0]
    T = int(cu[-1])
    m = np.zeros((H, T, T), bool)
    for h in range(H):
        for s in range(len(cu) - 1):
            st, en = int(cu[s]), int(cu[s + 1])
            for i in range(en - st):
                wi = max(int(w[st + i]), 1)
                lo = max(i - wi + 1, 0)
                for j in range(lo, i + 1):
                    m[h, st + i, st + j] = True
                b = _set_of_row(i, block_size)
                for p in lmk_idx[h, s, b]:
                    p = int(p)
                    if 0 <= p < en - st and p <= i and p < lo:
                        m[h, st + i, st + p] = True
    return m


def dense_attention(q, k, v, mask, scale):
    """softmax(q k^T scale + (-inf where ~mask)) v per head; mask [H|1, T, T]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, H, D = q.shape
    rep = H // k.shape[1]
    out = np.zeros((T, H, D))
    lse = np.zeros((T, H))
    for h in range(H):
        mh = mask[h if mask.shape[0] > 1 else 0]
        s = (q[:, h] @ k[:, h // rep].T) * scale
        s = np.where(mh, s, -np.inf)
        mx = s.max(1, keepdims=True)
        p = np.exp(s - mx)
        l = p.sum(1, keepdims=True)
        out[:, h] = (p / l) @ v[:, h // rep]
        lse[:, h] = (mx + np.log(l))[:, 0]
    return out, lse


def literal_mask(w, cu, lmk_idx):
    """[1, T, T] mask of the reference's CPU fallback (dsalt_attention.py:95-144).

    Window band of ``build_local_window_mask_packed`` (window_utils.py:40-70), then for
    each sequence the union over heads of the valid landmarks is switched on for every row
    of that sequence (:133-142), with no causal cut.
    """
    T = int(cu[-1])
    m = np.zeros((T, T), bool)
    for s in range(len(cu) - 1):
        st, en = int(cu[s]), int(cu[s + 1])
        for i in range(en - st):
            wi = max(int(w[st + i]), 1)
            lo = max(i - wi + 1, 0)
            m[st + i, st + lo:st + i + 1] = True
        cols = set()
        for h in range(lmk_idx.shape[0]):
            for p in lmk_idx[h, s].reshape(-1):
                p = int(p)
                if 0 <= p < en - st:
                    cols.add(st + p)
        if cols:
            c = np.array(sorted(cols))
            m[st:en][:, c] = True
    return m[None]

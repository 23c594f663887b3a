"""Shared helpers of the test suite."""
from __future__ import annotations

import numpy as np
import torch

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


def bits(t: torch.Tensor) -> np.ndarray:
    """Host array the C oracle reads: float32 values or raw 16-bit patterns."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def oracle_dtype(dt: torch.dtype) -> int:
    return {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dt]


def rel_err(a, b) -> float:
    """max |a - b| / max |b|: the relative error used for every tolerance."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if b.size == 0:  # nothing to compare (no landmark slots, no rows)
        assert a.size == 0, (a.shape, b.shape)
        return 0.0
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def load_golden(name: str):
    return np.load(f"{GOLDEN}/{name}.npz", allow_pickle=False)


def _pool_map(fn, items):
    """Map over items in threads (the oracle's numpy and C calls release the GIL), each
    thread's BLAS calls single-threaded so the threads do not oversubscribe the cores."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits
    items = list(items)
    with threadpool_limits(1), ThreadPoolExecutor(max(1, min(len(items), os.cpu_count() or 1, 16))) as ex:
        return list(ex.map(fn, items))


def oracle_select_by_group(h, v, alpha, w, cu, k_lmk, mode, block_size, scope):
    """C-oracle landmark indices [H, S, n_sets, k], one call per key/value head in parallel.

    A head's set depends on the shared hidden-state statistics, its own value head's
    statistics and its alpha only, so each call takes one value head with its query heads."""
    from oracle import select as OS
    H, G = alpha.shape[0], v.shape[1]
    rep = H // G
    hb, wn, cun, an = bits(h), w.numpy(), cu.numpy(), alpha.numpy()
    od = oracle_dtype(h.dtype)

    def one(g):
        return OS.select(hb, bits(v[:, g:g + 1]), an[g * rep:(g + 1) * rep], wn, cun, k_lmk, od, mode=mode,
                         block_size=block_size, stats_scope=scope)

    return np.concatenate(_pool_map(one, range(G)), axis=0)


def oracle_fwd_heads(q, k, v, w, cu, idx, scale, heads, block_size=None):
    """float64 oracle (O, LSE) of the listed query heads, one head per thread."""
    from oracle import attention as OA
    H, G = q.shape[1], k.shape[1]
    rep = H // G
    wn, cun = w.numpy(), cu.numpy()

    def one(hh):
        g = hh // rep
        return OA.attention_fwd(f64(q[:, hh:hh + 1]), f64(k[:, g:g + 1]), f64(v[:, g:g + 1]), wn, cun,
                                idx[hh:hh + 1], scale, block_size=block_size)

    return _pool_map(one, heads)


def oracle_bwd_heads(q, k, v, w, cu, idx, scale, dout, heads, out=None):
    """float64 oracle (dq, dk, dv, d_bias) of the listed heads (one key/value head per query
    head), one head per thread; ``out`` [T, H, D] (the stored forward output) feeds delta."""
    from oracle import attention as OA
    wn, cun = w.numpy(), cu.numpy()
    o = None if out is None else f64(out)

    def one(hh):
        return OA.attention_bwd(f64(q[:, hh:hh + 1]), f64(k[:, hh:hh + 1]), f64(v[:, hh:hh + 1]), wn, cun,
                                idx[hh:hh + 1], scale, f64(dout[:, hh:hh + 1]),
                                out=None if o is None else o[:, hh:hh + 1])

    return _pool_map(one, heads)


# bf16 selection fixtures: inputs regenerated from their recipe (torch's CPU generator),
# checked against the stored SHA-256 of their bits before use
BF16_SELECT_SPECS = {
    # name: (seed, lens, H, dh, extra hidden columns, k, w_max, heavy tails)
    "b4_h8": (700, [1024, 1024, 1024, 1024], 8, 64, 256, 64, 256, False),
    "h16": (701, [4096], 16, 64, 256, 128, 512, True),
}


def bf16_select_inputs(name: str):
    """(x [T, H*dh + extra] bf16, alpha [H], w [T] float, cu [S+1] int32) of a bf16 selection
    fixture: x = [v | h] with the value vectors v [T, H, dh] first, so x @ [I | 0]^T = v."""
    seed, lens, H, dh, extra, k, wmax, heavy = BF16_SELECT_SPECS[name]
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    v = torch.randn(T, H, dh, generator=g)
    hx = torch.randn(T, extra, generator=g)
    if heavy:  # heavy tails from powers of two (exact on every CPU, unlike exp)
        v = v * torch.exp2(torch.round(torch.randn(T, H, 1, generator=g) * 1.4427))
        hx = hx * torch.exp2(torch.round(0.5 * torch.randn(T, 1, generator=g) * 1.4427))
    x = torch.cat([v.reshape(T, H * dh), hx], 1).to(torch.bfloat16)
    alpha = torch.full((H,), 0.5)
    w = torch.round(torch.sigmoid(torch.randn(T, generator=g)) * wmax).clamp(16, wmax)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return x, alpha, w, cu


def sha256_of(t: torch.Tensor) -> str:
    import hashlib
    return hashlib.sha256(t.contiguous().view(torch.int16).numpy().tobytes()).hexdigest()


def topk_violations(idx, scores, w, cu, k):
    """Checks that each set of ``idx`` [H, S, k] (ascending, -1 padded) is a top-k of
    ``scores`` [T, H] over the set's candidates (tokens j with j - start >= w_j): returns
    (number of sets with a violation, largest score gap max(unselected) - min(selected))."""
    idx = np.asarray(idx)
    scores = np.asarray(scores, np.float64)
    w = np.asarray(w).astype(np.int64)
    cu = np.asarray(cu).astype(np.int64)
    bad, gap = 0, -np.inf
    for h in range(idx.shape[0]):
        for s in range(len(cu) - 1):
            st, en = int(cu[s]), int(cu[s + 1])
            rel = np.arange(en - st)
            cand = rel[rel >= w[st:en]]
            sel = idx[h, s][idx[h, s] >= 0]
            if len(cand) <= k:
                if not np.array_equal(np.sort(sel), cand):
                    bad += 1
                continue
            if len(sel) != k or not np.isin(sel, cand).all():
                bad += 1
                continue
            rest = np.setdiff1d(cand, sel)
            g = scores[st + rest, h].max() - scores[st + sel, h].min()
            gap = max(gap, g)
            if g > 0:
                bad += 1
    return bad, gap


# ---------------------------------------------------------------- gradient checker
# A gradient is compared per head in two ways, so that a large landmark row cannot hide the
# error of the ordinary rows (a landmark row sums contributions of up to every query of its
# sequence, so its entries can be tens of times larger than any other row's):
#   * class bound: rows are split into landmark rows (a position that some set of the head
#     holds) and all others; in each class max |a - b| / max |b| < tol;
#   * row bound: every row whose norm is at least ROW_FLOOR times the median row norm of its
#     class satisfies ||a_i - b_i|| / ||b_i|| < tol.
# Rows below the floor (gradients that cancel to almost nothing, such as the first row's dq)
# are held by the class bound only.
ROW_FLOOR = 0.25
# fp32 gradients: class bound FP32_TOL, row bound FP32_ROW_TOL.  dS = P (dP - delta) cancels in
# rows that see few keys with |delta| far above |dq| / (scale |k|) (up to 25-fold at head_dim 128:
# a query one token into its sequence, one of its two keys dominant), and such a row's dq then
# carries that factor times the rounding of its fp32 dot products dP = dO . v (128 terms: 1.5e-5
# absolute at the 99.99th percentile, in the kernels' order as in plain sequential order).  The
# worst row over 368 random fp32 configurations of the sweep was 1.8e-5 off; a float32
# computation on the CPU lands in the same range on other rows of the same cases.
FP32_TOL = 1e-5
FP32_ROW_TOL = 4e-5


def landmark_rows(idx, cu, T: int) -> np.ndarray:
    """bool [T, H]: row t holds a position of one of head h's landmark sets.

    idx [H, S, n_sets, k] (or [H, S, k]) sequence-relative positions, -1 for empty slots."""
    idx = np.asarray(idx)
    if idx.ndim == 3:
        idx = idx[:, :, None, :]
    cu = np.asarray(cu).astype(np.int64)
    H, S = idx.shape[:2]
    m = np.zeros((T, H), bool)
    for h in range(H):
        for s in range(S):
            st, L = int(cu[s]), int(cu[s + 1] - cu[s])
            p = idx[h, s].reshape(-1).astype(np.int64)
            p = p[(p >= 0) & (p < L)]
            m[st + p, h] = True
    return m


def grad_errors(a, b, lmk=None, floor: float = ROW_FLOOR) -> dict:
    """Class and row errors of one head's gradient a against b ([T, D]); lmk [T] bool marks
    the landmark rows (None: one class)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    T = b.shape[0]
    lmk = np.zeros(T, bool) if lmk is None else np.asarray(lmk, bool)
    rn = np.linalg.norm(b, axis=1)
    en = np.linalg.norm(a - b, axis=1)
    out = {}
    for cls, m in (("landmark", lmk), ("other", ~lmk)):
        if not m.any():
            continue
        den = np.abs(b[m]).max()
        out[f"{cls}_class"] = float(np.abs(a[m] - b[m]).max() / (den if den > 0 else 1.0))
        sel = m & (rn >= floor * np.median(rn[m])) & (rn > 0)
        if sel.any():
            r = en[sel] / rn[sel]
            j = int(np.argmax(r))
            out[f"{cls}_row"] = float(r[j])
            out[f"{cls}_row_at"] = int(np.nonzero(sel)[0][j])
            out[f"{cls}_rows_checked"] = int(sel.sum())
    return out


def assert_grad_close(what, a, b, tol: float, lmk=None, floor: float = ROW_FLOOR, row_tol: float | None = None) -> dict:
    """Raises AssertionError (with every figure) unless both bounds above hold: the class bound
    within tol, the row bound within row_tol (default tol)."""
    e = grad_errors(a, b, lmk, floor)
    rt = tol if row_tol is None else row_tol
    bad = {k: v for k, v in e.items() if (k.endswith("_class") and not v < tol) or (k.endswith("_row") and not v < rt)}
    assert not bad, (what, tol, rt, e)
    return e


def check_grads(what, got, ref, idx, cu, tol: float) -> None:
    """dq [T, H, D] per query head and dk, dv [T, G, D] per key/value head (each group's
    landmark rows: the union of its query heads' sets) through ``assert_grad_close``.
    The reference's backward takes delta = rowsum(O dO) from the stored output
    (dsalt/kernels/dsalt_triton_bwd.py:17-49), so ``ref`` is the oracle fed the output the
    kernels stored: rows whose dP - delta nearly cancels then compare like for like.  With the
    fp32 tolerance (tol <= FP32_TOL) the row bound is FP32_ROW_TOL.

    got: tensors or arrays (dq, dk, dv); ref: float64 arrays of the same shapes."""
    got = [f64(t) if isinstance(t, torch.Tensor) else np.asarray(t, np.float64) for t in got]
    ref = [np.asarray(t, np.float64) for t in ref]
    idx = idx.cpu().numpy() if isinstance(idx, torch.Tensor) else np.asarray(idx)
    cu = cu.cpu().numpy() if isinstance(cu, torch.Tensor) else np.asarray(cu)
    T, H = got[0].shape[:2]
    G = got[1].shape[1]
    rep = H // G
    lm = landmark_rows(idx, cu, T)
    rt = FP32_ROW_TOL if tol <= FP32_TOL else tol
    for h in range(H):
        assert_grad_close((what, "dq", h), got[0][:, h], ref[0][:, h], tol, row_tol=rt)
    for g in range(G):
        lg = lm[:, g * rep:(g + 1) * rep].any(1)
        for name, a, b in (("dk", got[1], ref[1]), ("dv", got[2], ref[2])):
            assert_grad_close((what, name, g), a[:, g], b[:, g], tol, lg, row_tol=rt)

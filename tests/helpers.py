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


def oracle_bwd_heads(q, k, v, w, cu, idx, scale, dout, heads):
    """float64 oracle (dq, dk, dv, d_bias) of the listed heads (one key/value head per query
    head), one head per thread."""
    from oracle import attention as OA
    wn, cun = w.numpy(), cu.numpy()

    def one(hh):
        return OA.attention_bwd(f64(q[:, hh:hh + 1]), f64(k[:, hh:hh + 1]), f64(v[:, hh:hh + 1]), wn, cun,
                                idx[hh:hh + 1], scale, f64(dout[:, hh:hh + 1]))

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

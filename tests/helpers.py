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

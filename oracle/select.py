"""Landmark-selection oracle - TEST INFRASTRUCTURE ONLY.

Wraps the C restatement ``oracle/select_oracle.c`` (canonical arithmetic, see its
header) and adds an independent pure-numpy brute force used to pin it on small inputs.
Only tests/, the smoke check and bench.py's CPU-baseline leg import this module.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import oracle_lib_path

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
SELECT_GLOBAL, SELECT_BLOCK = 0, 1
STATS_PACKED, STATS_SEQUENCE = 0, 1

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = oracle_lib_path()
        if not os.path.exists(path):
            from .build import build_oracle
            build_oracle()
        L = ctypes.CDLL(path)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_select_flat.argtypes = [i32] * 12 + [vp, i64, vp, i64, i64] + [vp] * 7
        L.oracle_select_flat.restype = i32
        L.oracle_norms_flat.argtypes = [i32] * 5 + [vp, i64, vp, i64, i64, vp, vp]
        L.oracle_norms_flat.restype = None
        L.oracle_canon_sqrt64.argtypes = [ctypes.c_double]
        L.oracle_canon_sqrt64.restype = ctypes.c_double
        L.oracle_range_sums.argtypes = [vp, i64, i64, vp, vp]
        L.oracle_range_sums.restype = None
        _LIB = L
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _bits(x: np.ndarray, dtype: int) -> np.ndarray:
    """Host array holding the raw element bits the C code reads."""
    if dtype == DTYPE_F32:
        return np.ascontiguousarray(x, dtype=np.float32)
    assert x.dtype in (np.uint16, np.int16), "16-bit inputs are passed as raw bits"
    return np.ascontiguousarray(x.view(np.uint16))


def select(h, v, alpha, w, cu, k_lmk, dtype, mode=SELECT_GLOBAL, block_size=512,
           stats_scope=STATS_PACKED, want_scores=False):
    """Landmark indices [H, S, n_sets, k] (int32) and, in the global variant, z_x [T],
    z_v [T, n_kv], scores [T, H].

    h [T, hidden] and v [T, n_kv, D] are float32 arrays (dtype F32) or uint16 arrays of
    bf16/fp16 bits.
    """
    hb, vb = _bits(h, dtype), _bits(v, dtype)
    T, hidden = hb.shape
    _, G, D = vb.shape
    alpha = np.ascontiguousarray(alpha, np.float32)
    H = alpha.shape[0]
    w = np.ascontiguousarray(w, np.int32)
    cu = np.ascontiguousarray(cu, np.int32)
    S = cu.shape[0] - 1
    maxlen = int(max(1, (cu[1:] - cu[:-1]).max())) if S else 1
    nsets = 1 if mode == SELECT_GLOBAL else -(-maxlen // block_size)
    idx = np.empty((H, S, nsets, k_lmk), np.int32)
    zx = np.empty(T, np.float32) if want_scores else None
    zv = np.empty((T, G), np.float32) if want_scores else None
    sc = np.empty((T, H), np.float32) if want_scores else None
    rc = lib().oracle_select_flat(T, S, maxlen, H, G, D, k_lmk, mode, block_size, dtype, hidden,
                                  stats_scope, _ptr(hb), hidden, _ptr(vb), G * D, D,
                                  _ptr(alpha), _ptr(w), _ptr(cu), _ptr(idx), _ptr(zx), _ptr(zv),
                                  _ptr(sc))
    assert rc == 0
    if want_scores:
        return idx, zx, zv, sc
    return idx


def norms(h, v, dtype):
    """Row norms (nx [T], nv [n_kv, T]) with the canonical arithmetic."""
    hb, vb = _bits(h, dtype), _bits(v, dtype)
    T, hidden = hb.shape
    _, G, D = vb.shape
    nx = np.empty(T, np.float32)
    nv = np.empty((G, T), np.float32)
    lib().oracle_norms_flat(T, G, D, dtype, hidden, _ptr(hb), hidden, _ptr(vb), G * D, D,
                            _ptr(nx), _ptr(nv))
    return nx, nv


def canon_sqrt64(x: float) -> float:
    return lib().oracle_canon_sqrt64(float(x))


def range_sums(x: np.ndarray, r0: int, r1: int):
    x = np.ascontiguousarray(x, np.float32)
    s1, s2 = ctypes.c_double(), ctypes.c_double()
    lib().oracle_range_sums(_ptr(x), r0, r1, ctypes.byref(s1), ctypes.byref(s2))
    return s1.value, s2.value


# ----------------------------------------------------------------------------------
# independent brute force (numpy, float64 statistics, tiny inputs only)
# ----------------------------------------------------------------------------------
def brute_topk(scores: np.ndarray, cand: np.ndarray, k: int) -> np.ndarray:
    """Top-k of ``scores`` over candidate positions by (score desc, index asc),
    ascending output padded with -1: an argsort over (-score, index) pairs."""
    idx = np.nonzero(cand)[0]
    order = np.lexsort((idx, -scores[idx].astype(np.float64)))
    sel = np.sort(idx[order[:k]])
    out = np.full(k, -1, np.int64)
    out[:len(sel)] = sel
    return out


def brute_scores(nx: np.ndarray, nv: np.ndarray, alpha: np.ndarray, r: slice):
    """Hybrid score [n, H] over a range, statistics in float64 numpy."""
    x = nx[r].astype(np.float64)
    zx = ((x - x.mean()) / max(x.std(ddof=1) if len(x) > 1 else 0.0, 1e-6)).astype(np.float32)
    G = nv.shape[0]
    H = alpha.shape[0]
    out = np.empty((len(x), H), np.float32)
    for h in range(H):
        y = nv[h // (H // G), r].astype(np.float64)
        zv = ((y - y.mean()) / max(y.std(ddof=1) if len(y) > 1 else 0.0, 1e-6)).astype(np.float32)
        a = np.float32(alpha[h])
        out[:, h] = (a * zv) + (np.float32(1.0) - a) * zx
    return out

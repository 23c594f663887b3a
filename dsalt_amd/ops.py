"""Torch-tensor wrappers over the C ABI: one function per library entry point.

Tensors must live on a ROCm device; every call is enqueued on torch's current stream and
allocates its outputs and workspace through torch's caching allocator.  There is no CPU
path: CPU tensors or a missing library raise.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, SELECT_BLOCK, SELECT_GLOBAL, STATS_PACKED,
                   STATS_SEQUENCE, VARIANT_DEFAULT, VARIANT_DQ_BN64, VARIANT_FWD_BN32, VARIANT_FWD_RG2,
                   VARIANT_LMK_SHORT, BwdArgs, CeArgs, FwdArgs, GatherArgs, Problem, ProbsArgs, RopeArgs, SelectArgs,
                   SiluMulArgs,
                   TrainBwdArgs,
                   TrainFwdArgs)

_DT = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}
MAX_LANDMARKS = 2048  # landmarks per set (the training variant: at most 512)
# select_landmarks(border_cap=...): full capacity with the block-causal candidate pruning
# forced at any sequence length (it runs by itself from 65536 tokens on)
SELECT_FORCE_PRUNE = 0x3FFFFFFF


def dtype_code(dt: torch.dtype) -> int:
    if dt not in _DT:
        raise TypeError(f"dsalt_amd supports float32, bfloat16 and float16 tensors, got {dt}")
    return _DT[dt]


def _gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("dsalt_amd runs on the GPU only; got a tensor on " + str(t.device))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _rows3(t: torch.Tensor, name: str) -> torch.Tensor:
    """[T, H, D] with unit stride along D (other strides free)."""
    if t.dim() != 3:
        raise ValueError(f"{name} must be [T, H, D], got shape {tuple(t.shape)}")
    if t.stride(2) != 1:
        t = t.contiguous()
    return t


def _check_tokens(q, k, v, w, cu_seqlens):
    T, H, D = q.shape
    if k.shape[0] != T or v.shape != k.shape or k.shape[2] != D:
        raise ValueError(f"k and v must be [T, n_kv, D] matching q {tuple(q.shape)}, got {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    if H % k.shape[1]:
        raise ValueError("n_heads must be a multiple of n_kv_heads")
    if w.dim() != 1 or w.shape[0] != T:
        raise ValueError("w must be [T]")
    if cu_seqlens.dim() != 1 or cu_seqlens.shape[0] < 2:
        raise ValueError("cu_seqlens must be [S+1] with S >= 1")


def _max_seqlen(cu_seqlens: torch.Tensor, cu_list=None) -> int:
    if cu_list is not None:
        return max(1, max(int(cu_list[i + 1]) - int(cu_list[i]) for i in range(len(cu_list) - 1)))
    lens = (cu_seqlens[1:] - cu_seqlens[:-1])
    return max(1, int(lens.max().item()))  # one device-to-host sync, as the reference's .tolist()


def n_sets(select_mode: int, max_seqlen: int, block_size: int) -> int:
    return 1 if select_mode == SELECT_GLOBAL else -(-max_seqlen // block_size)


def _problem(T, S, maxlen, H, G, D, K, mode, block_size, dtype) -> Problem:
    return Problem(T, S, maxlen, H, G, D, K, mode, block_size if mode == SELECT_BLOCK else 0, dtype)


def _workspace(nbytes: int, dev) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


def _set_workspace(args, nbytes: int, dev):
    """A workspace of nbytes in args (none when nbytes is 0: a caller-given plan replaces the
    forward's only workspace); returns the tensor to keep alive."""
    if nbytes == 0:
        args.workspace, args.workspace_bytes = None, 0
        return None
    ws = _workspace(nbytes, dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    return ws


# --------------------------------------------------------------------- selection
def select_landmarks(h: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, w: torch.Tensor,
                     cu_seqlens: torch.Tensor, k_lmk: int, *, max_seqlen: int | None = None,
                     select_mode: int = SELECT_GLOBAL, block_size: int = 512,
                     stats_scope: int = STATS_PACKED, want_scores: bool = False,
                     border_cap: int | None = None, plan: torch.Tensor | None = None):
    """Landmark indices [H, S, n_sets, k] (int32, ascending, -1 padded).

    h [T, hidden], v [T, n_kv, D] (value vectors x W_V^T without bias), alpha [H] in (0,1),
    w [T] integer windows, cu_seqlens [S+1].  With ``want_scores`` (global variant) also
    returns z_x [T], z_v [T, n_kv] and scores [T, H] in fp32.  ``plan`` (ops.new_plan)
    receives the forward's row plan of these windows, computed in the norms launch; pass it
    to attention_forward with ``plan_ready=True``.
    """
    dev = _gpu(h, v, alpha, w, cu_seqlens)
    if h.dim() != 2 or h.stride(1) != 1:
        h = h.contiguous()
    v = _rows3(v, "v")
    dt = dtype_code(h.dtype)
    if v.dtype != h.dtype:
        raise TypeError("h and v must share a dtype")
    # the kernels read rows in 16-byte vectors: other widths are zero-padded (zero columns
    # leave every row norm, and so every score, unchanged)
    vec = 16 // h.element_size()
    if h.shape[1] % vec:
        h = torch.nn.functional.pad(h, (0, (-h.shape[1]) % vec))
    if v.shape[2] % vec:
        v = torch.nn.functional.pad(v, (0, (-v.shape[2]) % vec))
    T, hidden = h.shape
    _, G, D = v.shape
    H = alpha.shape[0]
    S = cu_seqlens.shape[0] - 1
    if v.shape[0] != T or w.shape[0] != T:
        raise ValueError("h, v and w must have the same number of rows")
    if not 0 <= k_lmk <= MAX_LANDMARKS:
        raise ValueError(f"k_lmk must be in [0, {MAX_LANDMARKS}]")
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    nset = n_sets(select_mode, maxlen, block_size)
    alpha_c = alpha.detach().to(torch.float32).contiguous()
    w_c = w.detach().to(torch.int32).contiguous()
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    idx = torch.empty((H, S, nset, k_lmk), dtype=torch.int32, device=dev)
    zx = zv = sc = None
    if want_scores:
        zx = torch.empty(T, dtype=torch.float32, device=dev)
        zv = torch.empty((T, G), dtype=torch.float32, device=dev)
        sc = torch.empty((T, H), dtype=torch.float32, device=dev)
    a = SelectArgs()
    a.p = _problem(T, S, maxlen, H, G, D, k_lmk, select_mode, block_size, dt)
    a.hidden, a.stats_scope = hidden, stats_scope
    a.h, a.h_stride_t = h.data_ptr(), h.stride(0)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.alpha, a.w, a.cu_seqlens = alpha_c.data_ptr(), w_c.data_ptr(), cu_c.data_ptr()
    a.lmk_idx = idx.data_ptr() if idx.numel() else None
    a.z_x = zx.data_ptr() if zx is not None else None
    a.z_v = zv.data_ptr() if zv is not None else None
    a.scores = sc.data_ptr() if sc is not None else None
    a.plan = _check_plan(plan, a) or None
    L = _lib.load()
    if border_cap is None:
        need = L.dsalt_select_workspace_bytes(ctypes.byref(a))
    else:
        need = L.dsalt_select_workspace_bytes_cap(ctypes.byref(a), int(border_cap))
    if need == 0:
        _lib.check("dsalt_select", L.dsalt_select(ctypes.byref(a), None))
    ws = _workspace(need, dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    if border_cap is None:
        rc = L.dsalt_select(ctypes.byref(a), _stream(dev))
    else:
        rc = L.dsalt_select_with_border_cap(ctypes.byref(a), _stream(dev), int(border_cap))
    _lib.check("dsalt_select", rc)
    if want_scores:
        return idx, zx, zv, sc
    return idx


# ------------------------------------------------------------------------ forward
def _fwd_args(q, k, v, w, cu_seqlens, lmk_idx, lmk_bias, scale, max_seqlen, select_mode, block_size,
              need_w=True):
    """Checked FwdArgs with fresh outputs; returns (args, out, lse, tensors to keep alive)."""
    dev = _gpu(q, k, v, w, cu_seqlens, lmk_idx, lmk_bias)
    q, k, v = _rows3(q, "q"), _rows3(k, "k"), _rows3(v, "v")
    dt = dtype_code(q.dtype)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k and v must share a dtype")
    T, H, D = q.shape
    G = k.shape[1]
    S = cu_seqlens.shape[0] - 1
    _check_tokens(q, k, v, w, cu_seqlens)
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    K = lmk_idx.shape[-1]
    if lmk_bias is not None and tuple(lmk_bias.shape) != tuple(lmk_idx.shape):
        raise ValueError("lmk_bias must have the shape of lmk_idx")
    if lmk_idx.shape[:2] != (H, S) or lmk_idx.dim() != 4:
        raise ValueError(f"lmk_idx must be [H, S, n_sets, K], got {tuple(lmk_idx.shape)}")
    if lmk_idx.shape[2] != n_sets(select_mode, maxlen, block_size):
        raise ValueError("lmk_idx n_sets does not match select_mode / block_size / max_seqlen")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    w_c = w.detach().to(torch.int32).contiguous() if need_w else None
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    li = lmk_idx.to(torch.int32).contiguous()
    lb = lmk_bias.detach().to(torch.float32).contiguous() if lmk_bias is not None else None
    out = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    a = FwdArgs()
    a.p = _problem(T, S, maxlen, H, G, D, K, select_mode, block_size, dt)
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.w = w_c.data_ptr() if w_c is not None else None
    a.cu_seqlens = cu_c.data_ptr()
    a.lmk_idx = li.data_ptr() if li.numel() else None
    a.lmk_bias = lb.data_ptr() if lb is not None and lb.numel() else None
    a.out, a.o_stride_t, a.o_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse, a.scale = lse.data_ptr(), scale
    return a, out, lse, (q, k, v, w_c, cu_c, li, lb)


def new_plan(q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor, lmk_idx: torch.Tensor, *,
             max_seqlen=None, select_mode=SELECT_GLOBAL, block_size=512) -> torch.Tensor:
    """An empty row-plan buffer (uint8) for attention_forward(plan=...) / attention_backward(plan=...)."""
    T, H, D = q.shape
    S = cu_seqlens.shape[0] - 1
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    prob = _problem(T, S, maxlen, H, k.shape[1], D, lmk_idx.shape[-1], select_mode, block_size,
                    dtype_code(q.dtype))
    n = _lib.load().dsalt_plan_bytes(ctypes.byref(prob))
    return torch.empty(max(n, 1), dtype=torch.uint8, device=q.device)


def _check_plan(plan, a) -> int:
    if plan is None:
        return 0
    need = _lib.load().dsalt_plan_bytes(ctypes.byref(a.p))
    if plan.dtype != torch.uint8 or not plan.is_contiguous() or plan.numel() < need or plan.device.type != "cuda":
        raise ValueError(f"plan must be a contiguous uint8 device tensor of at least {need} bytes (ops.new_plan)")
    return plan.data_ptr()


def attention_forward(q, k, v, w, cu_seqlens, lmk_idx, lmk_bias=None, *, scale=None,
                      max_seqlen=None, select_mode=SELECT_GLOBAL, block_size=512, plan=None,
                      variant=VARIANT_DEFAULT, plan_ready=False):
    """(out [T,H,D] in q.dtype, lse [T,H] fp32).  lmk_idx [H,S,n_sets,K] int32 ascending with
    -1 padding at the end of each set (as select_landmarks returns; a position may repeat, each
    copy counts).  ``plan`` (ops.new_plan) receives the row plan for attention_backward of the
    same rows; ``variant`` picks a tiling (VARIANT_* bits, kernels.autotune); ``plan_ready``:
    ``plan`` already holds the row plan of these windows (select_landmarks(plan=...)), so the
    forward reads it instead of recomputing it."""
    a, out, lse, keep = _fwd_args(q, k, v, w, cu_seqlens, lmk_idx, lmk_bias, scale, max_seqlen, select_mode,
                                  block_size)
    a.plan = _check_plan(plan, a) or None
    a.variant = int(variant)
    a.plan_ready = 1 if (plan_ready and plan is not None) else 0
    if q.shape[0] == 0:
        return out, lse
    dev = out.device
    L = _lib.load()
    ws = _set_workspace(a, L.dsalt_fwd_workspace_bytes(ctypes.byref(a)), dev)  # noqa: F841 (kept alive)
    _lib.check("dsalt_fwd", L.dsalt_fwd(ctypes.byref(a), _stream(dev)))
    return out, lse


def _w_cont(w_cont: torch.Tensor, T: int) -> torch.Tensor:
    if w_cont.dim() != 1 or w_cont.shape[0] != T:
        raise ValueError("w_cont must be [T]")
    return w_cont.detach().to(torch.float32).contiguous()


def train_forward(q, k, v, w_cont, cu_seqlens, lmk_idx, lmk_logw, *, tau_win=1.0, win_edge=4.0, scale=None,
                  max_seqlen=None, plan=None, variant=VARIANT_DEFAULT):
    """Training variant: (out [T,H,D] in q.dtype, lse [T,H] fp32).  w_cont [T] continuous
    windows; lmk_idx [H,S,1,K] ascending with -1 last; lmk_logw [H,S,1,K] landmark log-weights
    (-inf or any value in -1 slots)."""
    a, out, lse, keep = _fwd_args(q, k, v, w_cont, cu_seqlens, lmk_idx, lmk_logw, scale, max_seqlen,
                                  SELECT_GLOBAL, 0, need_w=False)
    a.plan = _check_plan(plan, a) or None
    a.variant = int(variant)
    if q.shape[0] == 0:
        return out, lse
    dev = out.device
    wc = _w_cont(w_cont, q.shape[0])
    t = TrainFwdArgs()
    t.base, t.w_cont, t.tau_win, t.win_edge = a, wc.data_ptr(), float(tau_win), float(win_edge)
    L = _lib.load()
    ws = _workspace(L.dsalt_train_fwd_workspace_bytes(ctypes.byref(t)), dev)
    t.base.workspace, t.base.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check("dsalt_train_fwd", L.dsalt_train_fwd(ctypes.byref(t), _stream(dev)))
    return out, lse


# ----------------------------------------------------------------------- backward
def _bwd_args(dout, q, k, v, out, lse, w, cu_seqlens, lmk_idx, lmk_bias, scale, max_seqlen, want_dbias,
              need_w=True):
    """Checked BwdArgs with fresh gradients; returns (args, dq, dk, dv, d_bias, keep-alive)."""
    dev = _gpu(dout, q, k, v, out, lse, w, cu_seqlens, lmk_idx, lmk_bias)
    q, k, v, out, dout = (_rows3(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out"),
                                                   (dout, "dout")))
    dt = dtype_code(q.dtype)
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    T, H, D = q.shape
    G = k.shape[1]
    S = cu_seqlens.shape[0] - 1
    _check_tokens(q, k, v, w, cu_seqlens)
    if tuple(out.shape) != (T, H, D) or tuple(dout.shape) != (T, H, D) or tuple(lse.shape) != (T, H):
        raise ValueError("out / dout must be [T, H, D] and lse [T, H]")
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    K = lmk_idx.shape[-1]
    if lmk_idx.dim() != 4 or lmk_idx.shape[:3] != (H, S, 1):
        raise ValueError(f"lmk_idx must be [H, S, 1, K] (global variant), got {tuple(lmk_idx.shape)}")
    if lmk_bias is not None and tuple(lmk_bias.shape) != tuple(lmk_idx.shape):
        raise ValueError("lmk_bias must have the shape of lmk_idx")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    w_c = w.detach().to(torch.int32).contiguous() if need_w else None
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    li = lmk_idx.to(torch.int32).contiguous()
    lb = lmk_bias.detach().to(torch.float32).contiguous() if lmk_bias is not None else None
    lse = lse.detach().to(torch.float32).contiguous()
    dq = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    dk = torch.empty((T, G, D), dtype=q.dtype, device=dev)
    dv = torch.empty((T, G, D), dtype=q.dtype, device=dev)
    db = torch.empty(tuple(lmk_idx.shape), dtype=torch.float32, device=dev) if want_dbias else None
    a = BwdArgs()
    a.p = _problem(T, S, maxlen, H, G, D, K, SELECT_GLOBAL, 0, dt)
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.out, a.o_stride_t, a.o_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.dout, a.do_stride_t, a.do_stride_h = dout.data_ptr(), dout.stride(0), dout.stride(1)
    a.lse, a.cu_seqlens = lse.data_ptr(), cu_c.data_ptr()
    a.w = w_c.data_ptr() if w_c is not None else None
    a.lmk_idx = li.data_ptr() if li.numel() else None
    a.lmk_bias = lb.data_ptr() if lb is not None and lb.numel() else None
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.d_bias = db.data_ptr() if db is not None and db.numel() else None
    a.scale = scale
    return a, dq, dk, dv, db, (q, k, v, out, dout, w_c, cu_c, li, lb, lse)


def attention_backward(dout, q, k, v, out, lse, w, cu_seqlens, lmk_idx, lmk_bias=None, *,
                       scale=None, max_seqlen=None, want_dbias=True, plan=None, variant=VARIANT_DEFAULT):
    """(dq [T,H,D], dk, dv [T,n_kv,D]) in q.dtype and d_bias [H,S,1,K] fp32 (or None).
    Global selection variant; grouped key/value heads are read in place and their gradients
    summed over the group inside the kernels.  ``plan``: the buffer attention_forward filled
    for the same rows (skips recomputing the row plan)."""
    a, dq, dk, dv, db, keep = _bwd_args(dout, q, k, v, out, lse, w, cu_seqlens, lmk_idx, lmk_bias, scale,
                                        max_seqlen, want_dbias)
    a.plan = _check_plan(plan, a) or None
    a.variant = int(variant)
    if q.shape[0] == 0:
        return dq.zero_(), dk.zero_(), dv.zero_(), db
    dev = dq.device
    L = _lib.load()
    need = L.dsalt_bwd_workspace_bytes(ctypes.byref(a))
    if need == 0:
        _lib.check("dsalt_bwd", L.dsalt_bwd(ctypes.byref(a), None))
    ws = _workspace(need, dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check("dsalt_bwd", L.dsalt_bwd(ctypes.byref(a), _stream(dev)))
    return dq, dk, dv, db


def train_backward(dout, q, k, v, out, lse, w_cont, cu_seqlens, lmk_idx, lmk_logw, *, tau_win=1.0,
                   win_edge=4.0, scale=None, max_seqlen=None, want_dlogw=True, plan=None, variant=VARIANT_DEFAULT):
    """Training variant: (dq [T,H,D], dk, dv [T,n_kv,D]) in q.dtype, d_logw [H,S,1,K] fp32 (or
    None) and d_w [T] fp32, the window gradient summed over heads."""
    a, dq, dk, dv, db, keep = _bwd_args(dout, q, k, v, out, lse, w_cont, cu_seqlens, lmk_idx, lmk_logw, scale,
                                        max_seqlen, want_dlogw, need_w=False)
    a.plan = _check_plan(plan, a) or None
    a.variant = int(variant)
    T = q.shape[0]
    d_w = torch.zeros(T, dtype=torch.float32, device=dq.device)
    if T == 0:
        return dq.zero_(), dk.zero_(), dv.zero_(), db, d_w
    dev = dq.device
    wc = _w_cont(w_cont, T)
    t = TrainBwdArgs()
    t.base, t.w_cont, t.tau_win, t.win_edge, t.d_w = a, wc.data_ptr(), float(tau_win), float(win_edge), \
        d_w.data_ptr()
    L = _lib.load()
    need = L.dsalt_train_bwd_workspace_bytes(ctypes.byref(t))
    if need == 0:
        _lib.check("dsalt_train_bwd", L.dsalt_train_bwd(ctypes.byref(t), None))
    ws = _workspace(need, dev)
    t.base.workspace, t.base.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check("dsalt_train_bwd", L.dsalt_train_bwd(ctypes.byref(t), _stream(dev)))
    return dq, dk, dv, db, d_w


# ------------------------------------------------------------------------- gather
def gather_landmarks(k, v, cu_seqlens, lmk_idx, *, max_seqlen=None, select_mode=SELECT_GLOBAL,
                     block_size=512, n_heads=None):
    """(lmk_k, lmk_v) [H, S, n_sets, K, D]; rows of -1 slots are zero."""
    dev = _gpu(k, v, cu_seqlens, lmk_idx)
    k, v = _rows3(k, "k"), _rows3(v, "v")
    dt = dtype_code(k.dtype)
    T, G, D = k.shape
    H = lmk_idx.shape[0] if n_heads is None else n_heads
    S = cu_seqlens.shape[0] - 1
    K = lmk_idx.shape[-1]
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    if lmk_idx.dim() != 4 or lmk_idx.shape[1] != S or lmk_idx.shape[2] != n_sets(select_mode, maxlen, block_size):
        raise ValueError(f"lmk_idx must be [H, S, n_sets, K] matching select_mode/block_size, got "
                         f"{tuple(lmk_idx.shape)}")
    li = lmk_idx.to(torch.int32).contiguous()
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    shape = tuple(lmk_idx.shape) + (D,)
    lk = torch.empty(shape, dtype=k.dtype, device=dev)
    lv = torch.empty(shape, dtype=k.dtype, device=dev)
    a = GatherArgs()
    a.p = _problem(T, S, maxlen, H, G, D, K, select_mode, block_size, dt)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.cu_seqlens, a.lmk_idx = cu_c.data_ptr(), li.data_ptr()
    a.lmk_k, a.lmk_v = lk.data_ptr(), lv.data_ptr()
    if lk.numel() == 0:
        return lk, lv
    L = _lib.load()
    _lib.check("dsalt_gather_landmarks", L.dsalt_gather_landmarks(ctypes.byref(a), _stream(dev)))
    return lk, lv


def rope_qk_(q, k, cu_seqlens, cos, sin, *, max_seqlen=None):
    """Rotary embedding of q [T, Hq, D] and k [T, Hk, D] in place (either may be None);
    cos/sin [max_pos, D] fp32 tables indexed by each token's position in its sequence.
    q and k may be strided views of one fused projection output."""
    dev = _gpu(q, k, cu_seqlens, cos, sin)
    ref = q if q is not None else k
    if ref is None:
        return q, k
    for t, n in ((q, "q"), (k, "k")):
        if t is not None and (t.dim() != 3 or t.stride(2) != 1):
            raise ValueError(f"{n} must be [T, H, D] with unit stride along D")
    T, _, D = ref.shape
    if k is not None and q is not None and (k.shape[0] != T or k.shape[2] != D or k.dtype != q.dtype):
        raise ValueError("q and k must share T, D and dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2 \
            or cos.shape[1] != D:
        raise ValueError("cos/sin must be float32 [max_pos, head_dim]")
    cos, sin = cos.contiguous(), sin.contiguous()
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    a = RopeArgs()
    a.total_len, a.num_seqs, a.max_seqlen = T, cu_c.shape[0] - 1, maxlen
    a.n_q_heads = q.shape[1] if q is not None else 0
    a.n_k_heads = k.shape[1] if k is not None else 0
    a.head_dim, a.dtype = D, dtype_code(ref.dtype)
    if q is not None:
        a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    if k is not None:
        a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.cu_seqlens, a.cos, a.sin, a.max_pos = cu_c.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0]
    L = _lib.load()
    _lib.check("dsalt_rope_qk", L.dsalt_rope_qk(ctypes.byref(a), _stream(dev)))
    return q, k


def export_probs(q, k, w, cu_seqlens, lmk_idx, lse, lmk_bias=None, *, seq=0, rows=None, w_cap=None, scale=None,
                 max_seqlen=None, select_mode=SELECT_GLOBAL, block_size=512, want_lmk=True, seq_len=None):
    """(p_win [H, rows, w_cap], p_lmk [H, rows, K] or None), fp32: the probabilities the
    forward used for sequence ``seq`` (``lse`` from attention_forward on the same inputs),
    window keys as p_win[h, i, c] = P(i, i - c), landmark slots as p_lmk[h, i, slot].
    ``seq_len`` (the sequence's length, when the caller knows it) lets the outputs skip their
    zero fill."""
    dev = _gpu(q, k, w, cu_seqlens, lmk_idx, lse, lmk_bias)
    q, k = _rows3(q, "q"), _rows3(k, "k")
    T, H, D = q.shape
    S = cu_seqlens.shape[0] - 1
    maxlen = max_seqlen if max_seqlen is not None else _max_seqlen(cu_seqlens)
    if rows is None or w_cap is None:
        cu_h = cu_seqlens.detach().to("cpu").tolist()
        n = cu_h[seq + 1] - cu_h[seq]
        seq_len = n
        rows = n if rows is None else rows
        if w_cap is None:
            w_cap = int(w[cu_h[seq]:cu_h[seq + 1]].max().item()) if n else 1
            w_cap = max(1, min(w_cap, n))
    K = lmk_idx.shape[-1]
    if lmk_idx.dim() != 4 or lmk_idx.shape[:2] != (H, S) or lmk_idx.shape[2] != n_sets(select_mode, maxlen, block_size):
        raise ValueError(f"lmk_idx must be [H, S, n_sets, K], got {tuple(lmk_idx.shape)}")
    w_c = w.detach().to(torch.int32).contiguous()
    cu_c = cu_seqlens.detach().to(torch.int32).contiguous()
    li = lmk_idx.to(torch.int32).contiguous()
    lb = lmk_bias.detach().to(torch.float32).contiguous() if lmk_bias is not None else None
    lse_c = lse.detach().to(torch.float32).contiguous()
    alloc = torch.empty if rows == seq_len else torch.zeros  # the kernel writes every row of the sequence
    p_win = alloc((H, rows, w_cap), dtype=torch.float32, device=dev)
    p_lmk = alloc((H, rows, K), dtype=torch.float32, device=dev) if want_lmk and K else None
    a = ProbsArgs()
    a.p = _problem(T, S, maxlen, H, k.shape[1], D, K, select_mode, block_size, dtype_code(q.dtype))
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.w, a.cu_seqlens = w_c.data_ptr(), cu_c.data_ptr()
    a.lmk_idx = li.data_ptr() if li.numel() else None
    a.lmk_bias = lb.data_ptr() if lb is not None and lb.numel() else None
    a.lse = lse_c.data_ptr()
    a.scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    a.seq, a.rows, a.w_cap = seq, rows, w_cap
    a.p_win = p_win.data_ptr()
    a.p_lmk = p_lmk.data_ptr() if p_lmk is not None else None
    L = _lib.load()
    _lib.check("dsalt_export_probs", L.dsalt_export_probs(ctypes.byref(a), _stream(dev)))
    return p_win, p_lmk


_REDUCTIONS = {"none": 0, "mean": 1, "sum": 2}


def _aligned_rows(t: torch.Tensor) -> bool:
    """Rows of the 2-D tensor start on 16-byte boundaries (what the kernels' vector loads need)."""
    return t.data_ptr() % 16 == 0 and (t.shape[0] <= 1 or (t.stride(0) * t.element_size()) % 16 == 0)


def _padded_rows(t: torch.Tensor) -> torch.Tensor:
    """A copy of the 2-D tensor whose rows start on 16-byte boundaries (row stride rounded up)."""
    vec = 16 // t.element_size()
    buf = torch.empty((t.shape[0], -(-t.shape[1] // vec) * vec), dtype=t.dtype, device=t.device)
    buf[:, :t.shape[1]].copy_(t)
    return buf[:, :t.shape[1]]


def cross_entropy_rows(logits, target, *, ce_weight=None, ignore_index=-100, n_non_ignore=None,
                       sum_non_ignore_weight=None, weight_sum=None, lse_square_scale=0.0, label_smoothing=0.0,
                       softcap=None, reduction="mean", want_grad=True, token_scaling=False, want_z=False,
                       want_accuracy=False, want_predicted=False):
    """Row losses of ``logits`` [rows, V] against ``target`` [rows] (int64), and with
    ``want_grad`` the gradient wrt the logits written over them.  The batch totals of the
    "mean" reduction default to this call's rows.  Returns (loss [rows] fp32, z [rows] in the
    logits' type or None, accuracy [rows] or None, predicted [rows] int64 or None)."""
    dev = _gpu(logits, target, ce_weight)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, V] with unit column stride")
    if not _aligned_rows(logits):  # e.g. an odd vocabulary: run on a padded copy, gradient copied back
        buf = _padded_rows(logits)
        res = cross_entropy_rows(buf, target, ce_weight=ce_weight, ignore_index=ignore_index,
                                 n_non_ignore=n_non_ignore, sum_non_ignore_weight=sum_non_ignore_weight,
                                 weight_sum=weight_sum, lse_square_scale=lse_square_scale,
                                 label_smoothing=label_smoothing, softcap=softcap, reduction=reduction,
                                 want_grad=want_grad, token_scaling=token_scaling, want_z=want_z,
                                 want_accuracy=want_accuracy, want_predicted=want_predicted)
        if want_grad:
            logits.copy_(buf)
        return res
    rows, V = logits.shape
    tgt = target.detach().to(torch.int64).contiguous()
    cw = ce_weight.detach().to(torch.float32).contiguous() if ce_weight is not None else None
    keep = tgt != ignore_index
    if n_non_ignore is None:
        n_non_ignore = float(keep.sum().item())
    if sum_non_ignore_weight is None:
        sum_non_ignore_weight = float(cw[tgt[keep]].sum().item()) if cw is not None else n_non_ignore
    if weight_sum is None:
        weight_sum = float(cw.sum().item()) if cw is not None else 0.0
    loss = torch.empty(rows, dtype=torch.float32, device=dev)
    z = torch.empty(rows, dtype=logits.dtype, device=dev) if want_z else None
    acc = torch.empty(rows, dtype=torch.float32, device=dev) if want_accuracy else None
    pred = torch.empty(rows, dtype=torch.int64, device=dev) if want_predicted else None
    a = CeArgs()
    a.rows, a.n_cols, a.dtype = rows, V, dtype_code(logits.dtype)
    a.logits, a.logits_stride = logits.data_ptr(), logits.stride(0)
    a.target = tgt.data_ptr()
    a.ce_weight = cw.data_ptr() if cw is not None else None
    a.loss = loss.data_ptr()
    a.z_loss = z.data_ptr() if z is not None else None
    a.accuracy = acc.data_ptr() if acc is not None else None
    a.predicted = pred.data_ptr() if pred is not None else None
    a.ignore_index = int(ignore_index)
    a.n_non_ignore, a.sum_non_ignore_weight, a.weight_sum = n_non_ignore, sum_non_ignore_weight, weight_sum
    a.lse_square_scale, a.label_smoothing = float(lse_square_scale), float(label_smoothing)
    a.softcap = float(softcap) if softcap is not None else 0.0
    if reduction not in _REDUCTIONS:
        raise ValueError(f"reduction must be one of {list(_REDUCTIONS)}")
    a.reduction, a.want_grad, a.token_scaling = _REDUCTIONS[reduction], int(want_grad), int(token_scaling)
    L = _lib.load()
    _lib.check("dsalt_cross_entropy_rows", L.dsalt_cross_entropy_rows(ctypes.byref(a), _stream(dev)))
    return loss, z, acc, pred


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up for 2-D [rows, cols] tensors with unit column stride (gate and up may
    be column ranges of one buffer); a new contiguous output unless ``out`` is given."""
    dev = _gpu(gate, up, out)
    if gate.dim() != 2 or gate.shape != up.shape or gate.stride(1) != 1 or up.stride(1) != 1 or gate.dtype != up.dtype:
        raise ValueError("gate and up must be [rows, cols] of one dtype with unit column stride")
    if out is None:
        out = torch.empty(gate.shape, dtype=gate.dtype, device=dev)
    if gate.shape[0] and not (_aligned_rows(gate) and _aligned_rows(up) and _aligned_rows(out)):
        o = silu_mul(_padded_rows(gate), _padded_rows(up), _padded_rows(out))  # rows off 16-byte boundaries
        return out.copy_(o)
    a = SiluMulArgs(gate.shape[0], gate.shape[1], dtype_code(gate.dtype), gate.data_ptr(), gate.stride(0),
                    up.data_ptr(), up.stride(0), out.data_ptr(), out.stride(0))
    L = _lib.load()
    _lib.check("dsalt_silu_mul", L.dsalt_silu_mul(ctypes.byref(a), _stream(dev)))
    return out


def sort_landmarks(idx: torch.Tensor, bias: torch.Tensor | None = None):
    """Sort each set ascending with -1 last (the order the kernels require); returns
    (sorted int32 indices, bias permuted the same way or None, permutation)."""
    big = torch.iinfo(torch.int32).max
    key = torch.where(idx < 0, torch.full_like(idx, big), idx).to(torch.int64)
    srt, perm = key.sort(dim=-1)
    out = torch.where(srt == big, torch.full_like(srt, -1), srt).to(torch.int32)
    b = bias.gather(-1, perm) if bias is not None else None
    return out, b, perm

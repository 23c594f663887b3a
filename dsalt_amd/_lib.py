"""ctypes binding of ``libdsalt_amd.so`` (the C ABI in ``include/dsalt_amd.h``).

The structures below mirror the header field by field; ``tests/test_abi.py`` checks their
sizes and offsets against the C compiler's.  Loading imports torch first so the library
binds to the HIP runtime torch already uses (both carry the SONAME libamdhip64.so.7).
There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdsalt_amd.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
SELECT_GLOBAL, SELECT_BLOCK = 0, 1
STATS_PACKED, STATS_SEQUENCE = 0, 1
ERR_NAMES = {1: "invalid argument", 2: "unsupported", 3: "workspace", 4: "HIP error"}
ABI_VERSION = 3
FWD_NOALLOC_MAX_PLAN_BYTES = 4 << 20  # DSALT_FWD_NOALLOC_MAX_PLAN_BYTES
# tile variants of the attention kernels (DSALT_VARIANT_*)
VARIANT_DEFAULT, VARIANT_FWD_BN32, VARIANT_FWD_RG2, VARIANT_DQ_BN64, VARIANT_LMK_SHORT = 0, 1, 2, 4, 8
VARIANT_FWD_BN64 = 16
VARIANT_FWD_8W = 32

_i32, _i64, _vp, _sz, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float


class DsaltError(RuntimeError):
    """A call into the HIP library returned an error code."""

    def __init__(self, func: str, code: int, msg: str):
        super().__init__(f"{func} failed ({ERR_NAMES.get(code, code)}): {msg}")
        self.code = code


class Problem(ctypes.Structure):
    _fields_ = [("total_len", _i32), ("num_seqs", _i32), ("max_seqlen", _i32), ("n_heads", _i32),
                ("n_kv_heads", _i32), ("head_dim", _i32), ("k_lmk", _i32), ("select_mode", _i32),
                ("block_size", _i32), ("dtype", _i32)]


class SelectArgs(ctypes.Structure):
    _fields_ = [("p", Problem), ("hidden", _i32), ("stats_scope", _i32),
                ("h", _vp), ("h_stride_t", _i64),
                ("v", _vp), ("v_stride_t", _i64), ("v_stride_h", _i64),
                ("alpha", _vp), ("w", _vp), ("cu_seqlens", _vp), ("lmk_idx", _vp),
                ("z_x", _vp), ("z_v", _vp), ("scores", _vp),
                ("workspace", _vp), ("workspace_bytes", _sz), ("plan", _vp)]


class FwdArgs(ctypes.Structure):
    _fields_ = [("p", Problem),
                ("q", _vp), ("q_stride_t", _i64), ("q_stride_h", _i64),
                ("k", _vp), ("k_stride_t", _i64), ("k_stride_h", _i64),
                ("v", _vp), ("v_stride_t", _i64), ("v_stride_h", _i64),
                ("w", _vp), ("cu_seqlens", _vp), ("lmk_idx", _vp), ("lmk_bias", _vp),
                ("out", _vp), ("o_stride_t", _i64), ("o_stride_h", _i64),
                ("lse", _vp), ("scale", _f32),
                ("workspace", _vp), ("workspace_bytes", _sz), ("plan", _vp), ("variant", _i32),
                ("plan_ready", _i32)]


class BwdArgs(ctypes.Structure):
    _fields_ = [("p", Problem),
                ("q", _vp), ("q_stride_t", _i64), ("q_stride_h", _i64),
                ("k", _vp), ("k_stride_t", _i64), ("k_stride_h", _i64),
                ("v", _vp), ("v_stride_t", _i64), ("v_stride_h", _i64),
                ("out", _vp), ("o_stride_t", _i64), ("o_stride_h", _i64),
                ("dout", _vp), ("do_stride_t", _i64), ("do_stride_h", _i64),
                ("lse", _vp), ("w", _vp), ("cu_seqlens", _vp), ("lmk_idx", _vp), ("lmk_bias", _vp),
                ("dq", _vp), ("dk", _vp), ("dv", _vp), ("d_bias", _vp), ("scale", _f32),
                ("workspace", _vp), ("workspace_bytes", _sz), ("plan", _vp), ("variant", _i32)]


class TrainFwdArgs(ctypes.Structure):
    _fields_ = [("base", FwdArgs), ("w_cont", _vp), ("tau_win", _f32), ("win_edge", _f32)]


class TrainBwdArgs(ctypes.Structure):
    _fields_ = [("base", BwdArgs), ("w_cont", _vp), ("tau_win", _f32), ("win_edge", _f32), ("d_w", _vp)]


class RopeArgs(ctypes.Structure):
    _fields_ = [("total_len", _i32), ("num_seqs", _i32), ("max_seqlen", _i32), ("n_q_heads", _i32),
                ("n_k_heads", _i32), ("head_dim", _i32), ("dtype", _i32),
                ("q", _vp), ("q_stride_t", _i64), ("q_stride_h", _i64),
                ("k", _vp), ("k_stride_t", _i64), ("k_stride_h", _i64),
                ("cu_seqlens", _vp), ("cos", _vp), ("sin", _vp), ("max_pos", _i32)]


class ProbsArgs(ctypes.Structure):
    _fields_ = [("p", Problem),
                ("q", _vp), ("q_stride_t", _i64), ("q_stride_h", _i64),
                ("k", _vp), ("k_stride_t", _i64), ("k_stride_h", _i64),
                ("w", _vp), ("cu_seqlens", _vp), ("lmk_idx", _vp), ("lmk_bias", _vp), ("lse", _vp),
                ("scale", _f32), ("seq", _i32), ("rows", _i32), ("w_cap", _i32), ("p_win", _vp), ("p_lmk", _vp)]


class CeArgs(ctypes.Structure):
    _fields_ = [("rows", _i32), ("n_cols", _i32), ("dtype", _i32), ("logits", _vp), ("logits_stride", _i64),
                ("target", _vp), ("ce_weight", _vp), ("loss", _vp), ("z_loss", _vp), ("accuracy", _vp),
                ("predicted", _vp), ("ignore_index", _i64), ("n_non_ignore", _f32), ("sum_non_ignore_weight", _f32),
                ("weight_sum", _f32), ("lse_square_scale", _f32), ("label_smoothing", _f32), ("softcap", _f32),
                ("reduction", _i32), ("want_grad", _i32), ("token_scaling", _i32)]


class SiluMulArgs(ctypes.Structure):
    _fields_ = [("rows", _i32), ("cols", _i32), ("dtype", _i32), ("gate", _vp), ("gate_stride", _i64),
                ("up", _vp), ("up_stride", _i64), ("out", _vp), ("out_stride", _i64)]


class GatherArgs(ctypes.Structure):
    _fields_ = [("p", Problem),
                ("k", _vp), ("k_stride_t", _i64), ("k_stride_h", _i64),
                ("v", _vp), ("v_stride_t", _i64), ("v_stride_h", _i64),
                ("cu_seqlens", _vp), ("lmk_idx", _vp), ("lmk_k", _vp), ("lmk_v", _vp)]


# name -> (argtypes, restype); every function declared in include/dsalt_amd.h
SIGNATURES = {
    "dsalt_abi_version": ([], ctypes.c_int),
    "dsalt_last_error": ([], ctypes.c_char_p),
    "dsalt_select_workspace_bytes": ([ctypes.POINTER(SelectArgs)], _sz),
    "dsalt_select": ([ctypes.POINTER(SelectArgs), _vp], ctypes.c_int),
    "dsalt_select_with_border_cap": ([ctypes.POINTER(SelectArgs), _vp, ctypes.c_int], ctypes.c_int),
    "dsalt_select_workspace_bytes_cap": ([ctypes.POINTER(SelectArgs), ctypes.c_int], _sz),
    "dsalt_plan_bytes": ([ctypes.POINTER(Problem)], _sz),
    "dsalt_fwd_workspace_bytes": ([ctypes.POINTER(FwdArgs)], _sz),
    "dsalt_fwd": ([ctypes.POINTER(FwdArgs), _vp], ctypes.c_int),
    "dsalt_fwd_noalloc": ([ctypes.POINTER(FwdArgs), _vp], ctypes.c_int),
    "dsalt_bwd_workspace_bytes": ([ctypes.POINTER(BwdArgs)], _sz),
    "dsalt_bwd": ([ctypes.POINTER(BwdArgs), _vp], ctypes.c_int),
    "dsalt_gather_landmarks": ([ctypes.POINTER(GatherArgs), _vp], ctypes.c_int),
    "dsalt_train_fwd_workspace_bytes": ([ctypes.POINTER(TrainFwdArgs)], _sz),
    "dsalt_train_fwd": ([ctypes.POINTER(TrainFwdArgs), _vp], ctypes.c_int),
    "dsalt_train_bwd_workspace_bytes": ([ctypes.POINTER(TrainBwdArgs)], _sz),
    "dsalt_train_bwd": ([ctypes.POINTER(TrainBwdArgs), _vp], ctypes.c_int),
    "dsalt_rope_qk": ([ctypes.POINTER(RopeArgs), _vp], ctypes.c_int),
    "dsalt_silu_mul": ([ctypes.POINTER(SiluMulArgs), _vp], ctypes.c_int),
    "dsalt_export_probs": ([ctypes.POINTER(ProbsArgs), _vp], ctypes.c_int),
    "dsalt_cross_entropy_rows": ([ctypes.POINTER(CeArgs), _vp], ctypes.c_int),
    "dsalt_timing_enable": ([ctypes.c_int], ctypes.c_int),
    "dsalt_timing_report": ([ctypes.c_char_p, _sz], ctypes.c_int),
}

_LIB = None


def load(path: str | None = None):
    """Load the HIP library (once).  Raises if it has not been built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    import torch  # noqa: F401  -- bind to torch's HIP runtime first

    p = path or LIB_PATH
    if not os.path.exists(p):
        raise ImportError(f"{p} is missing: build it with `python -m dsalt_amd.build` "
                          "(dsalt_amd has no CPU fallback)")
    lib = ctypes.CDLL(p)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.dsalt_abi_version() != ABI_VERSION:
        raise ImportError(f"{p}: unexpected ABI version {lib.dsalt_abi_version()}")
    if path is None:
        _LIB = lib
    return lib


def check(func: str, rc: int) -> None:
    if rc != 0:
        msg = load().dsalt_last_error()
        raise DsaltError(func, rc, msg.decode() if msg else "")

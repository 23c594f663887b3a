"""The C-ABI library (CPU only: no kernel launches).

* every function declared in include/*.h is exported by libdsalt_amd.so;
* the ctypes mirrors of the argument structs have the C compiler's sizes and offsets;
* argument validation rejects bad problems with the documented error codes.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess

import pytest

from dsalt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HEADERS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(dsalt_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(_lib.SIGNATURES) == names
    assert lib.dsalt_abi_version() == _lib.ABI_VERSION == 3


STRUCTS = {
    "dsalt_problem": _lib.Problem,
    "dsalt_select_args": _lib.SelectArgs,
    "dsalt_fwd_args": _lib.FwdArgs,
    "dsalt_bwd_args": _lib.BwdArgs,
    "dsalt_gather_args": _lib.GatherArgs,
    "dsalt_train_fwd_args": _lib.TrainFwdArgs,
    "dsalt_train_bwd_args": _lib.TrainBwdArgs,
    "dsalt_rope_args": _lib.RopeArgs,
    "dsalt_silu_mul_args": _lib.SiluMulArgs,
    "dsalt_probs_args": _lib.ProbsArgs,
    "dsalt_ce_args": _lib.CeArgs,
}


def test_struct_layouts_match_c(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADERS[0]}"', "int main(void){"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                          check=True).stdout.splitlines())
    for cname, cls in STRUCTS.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, (cname, f)


def _valid_fwd():
    a = _lib.FwdArgs()
    a.p = _lib.Problem(128, 1, 128, 2, 2, 64, 8, 0, 0, _lib.DTYPE_BF16)
    fake = 1 << 20  # never dereferenced: validation fails before any launch
    a.q = a.k = a.v = a.out = fake
    a.q_stride_t = a.k_stride_t = a.v_stride_t = a.o_stride_t = 128
    a.q_stride_h = a.k_stride_h = a.v_stride_h = a.o_stride_h = 64
    a.w = a.cu_seqlens = a.lmk_idx = a.lse = fake
    a.scale = 0.125
    return a


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 96, 2), ("k_lmk", 2049, 1), ("n_kv_heads", 3, 1), ("dtype", 7, 1),
    ("select_mode", 1, 1), ("max_seqlen", 0, 1)])
def test_fwd_validation(field, value, code):
    lib = _lib.load()
    a = _valid_fwd()
    setattr(a.p, field, value)
    assert lib.dsalt_fwd(ctypes.byref(a), None) == code
    assert lib.dsalt_last_error()


def test_block_sizes_and_the_sets_of_a_tile():
    """Any block_size >= 1; when it is not a multiple of 64 the forward stages every set a
    64-row tile's rows use: at most 2048 slots (sets x k_lmk)."""
    lib = _lib.load()
    a = _valid_fwd()
    a.p.select_mode = _lib.SELECT_BLOCK
    for bs in (100, 64, 7):
        a.p.block_size = bs
        assert lib.dsalt_fwd(ctypes.byref(a), None) == 3  # accepted up to the missing workspace
    a.p.block_size, a.p.k_lmk = 16, 512  # 64-row tiles in 16-row blocks: 4 sets x 512
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 3
    a.p.k_lmk = 513
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 2
    assert b"sets" in lib.dsalt_last_error()
    a.p.block_size = 0
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 1


def test_misaligned_and_null_pointers_rejected():
    lib = _lib.load()
    a = _valid_fwd()
    a.q = (1 << 20) + 2
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 1
    a = _valid_fwd()
    a.q_stride_t = 100  # 200 bytes: not a multiple of 16
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 1
    assert lib.dsalt_fwd(None, None) == 1


def test_backward_rejects_unsupported_variants():
    lib = _lib.load()
    a = _lib.BwdArgs()
    a.p = _lib.Problem(256, 1, 256, 4, 2, 64, 8, 0, 0, _lib.DTYPE_BF16)
    assert lib.dsalt_bwd(ctypes.byref(a), None) == 1  # GQA is accepted; the null tensors are not
    a.p = _lib.Problem(256, 1, 256, 4, 4, 64, 8, 1, 128, _lib.DTYPE_BF16)
    assert lib.dsalt_bwd(ctypes.byref(a), None) == 2  # block-causal backward
    assert b"block" in lib.dsalt_last_error()


def test_unknown_variant_bits_and_plan_size():
    lib = _lib.load()
    a = _valid_fwd()
    a.variant = _lib.VARIANT_FWD_BN32 | _lib.VARIANT_FWD_RG2
    a.workspace, a.workspace_bytes = 0, 0
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 3  # variant accepted, workspace missing
    a.variant = 64
    assert lib.dsalt_fwd(ctypes.byref(a), None) == 1
    assert b"variant" in lib.dsalt_last_error()
    p = _lib.Problem(1000, 2, 600, 4, 2, 64, 16, 0, 0, _lib.DTYPE_BF16)
    tiles = 2 * 10  # sequences x 64-row tiles of the longest
    assert lib.dsalt_plan_bytes(ctypes.byref(p)) >= tiles * (64 + 16 * 4 + 4)
    p.head_dim = 96
    assert lib.dsalt_plan_bytes(ctypes.byref(p)) == 0


def test_workspaces_drop_the_plan_when_a_plan_is_given():
    """The row plan is the forward's only workspace: with a caller-given plan buffer dsalt_fwd
    needs none, and the backward's workspace shrinks by the plan's bytes."""
    lib = _lib.load()
    a = _valid_fwd()
    a.plan = None
    plan_b = lib.dsalt_plan_bytes(ctypes.byref(a.p))
    assert plan_b > 0 and lib.dsalt_fwd_workspace_bytes(ctypes.byref(a)) == plan_b
    a.plan = 1 << 20  # any non-null address: only the query runs
    assert lib.dsalt_fwd_workspace_bytes(ctypes.byref(a)) == 0
    b = _lib.BwdArgs()
    b.p = _lib.Problem(256, 1, 256, 4, 4, 64, 8, 0, 0, _lib.DTYPE_BF16)
    fake = 1 << 20
    b.q = b.k = b.v = b.out = b.dout = b.dq = b.dk = b.dv = b.w = b.cu_seqlens = b.lse = b.lmk_idx = fake
    b.q_stride_t = b.k_stride_t = b.v_stride_t = b.o_stride_t = b.do_stride_t = 4 * 64
    b.q_stride_h = b.k_stride_h = b.v_stride_h = b.o_stride_h = b.do_stride_h = 64
    b.scale = 0.125
    full = lib.dsalt_bwd_workspace_bytes(ctypes.byref(b))
    assert full > 0
    b.plan = fake
    assert lib.dsalt_bwd_workspace_bytes(ctypes.byref(b)) == full - lib.dsalt_plan_bytes(ctypes.byref(b.p))


def test_workspace_sizes_and_small_workspace():
    lib = _lib.load()
    s = _lib.SelectArgs()
    s.p = _lib.Problem(1024, 2, 512, 4, 4, 64, 16, 0, 0, _lib.DTYPE_BF16)
    s.hidden, s.stats_scope = 256, _lib.STATS_SEQUENCE
    fake = 1 << 20
    s.h = s.v = s.alpha = s.w = s.cu_seqlens = s.lmk_idx = fake
    s.h_stride_t, s.v_stride_t, s.v_stride_h = 256, 256, 64
    need = lib.dsalt_select_workspace_bytes(ctypes.byref(s))
    assert need >= 1024 * 5 * 4
    s.workspace, s.workspace_bytes = fake, need - 1
    assert lib.dsalt_select(ctypes.byref(s), None) == 3
    s.p.select_mode, s.p.block_size = 1, 128
    assert lib.dsalt_select_workspace_bytes(ctypes.byref(s)) > 0


def _valid_train_fwd():
    t = _lib.TrainFwdArgs()
    t.base = _valid_fwd()
    t.base.w = None  # the training variant reads w_cont, not w
    t.w_cont, t.tau_win, t.win_edge = 1 << 20, 1.0, 4.0
    return t


@pytest.mark.parametrize("field,value,code", [
    ("tau_win", 0.0, 1), ("tau_win", -1.0, 1), ("win_edge", -0.5, 1), ("win_edge", float("nan"), 1),
    ("w_cont", None, 1)])
def test_train_validation(field, value, code):
    lib = _lib.load()
    t = _valid_train_fwd()
    setattr(t, field, value)
    assert lib.dsalt_train_fwd(ctypes.byref(t), None) == code
    assert lib.dsalt_last_error()


def test_train_rejects_block_sets_and_small_workspace():
    lib = _lib.load()
    t = _valid_train_fwd()
    need = lib.dsalt_train_fwd_workspace_bytes(ctypes.byref(t))
    assert need >= 128 * 4
    t.base.workspace, t.base.workspace_bytes = 1 << 20, need - 1
    assert lib.dsalt_train_fwd(ctypes.byref(t), None) == 3
    t.base.p.select_mode, t.base.p.block_size = 1, 64
    assert lib.dsalt_train_fwd(ctypes.byref(t), None) == 2
    b = _lib.TrainBwdArgs()
    b.base.p = _lib.Problem(128, 1, 128, 2, 2, 64, 8, 0, 0, _lib.DTYPE_BF16)
    fake = 1 << 20
    b.base.q = b.base.k = b.base.v = b.base.out = b.base.dout = fake
    b.base.dq = b.base.dk = b.base.dv = fake
    for f in ("q", "k", "v", "o", "do"):
        setattr(b.base, f + "_stride_t", 128)
        setattr(b.base, f + "_stride_h", 64)
    b.base.cu_seqlens = b.base.lmk_idx = b.base.lse = fake
    b.base.scale = 0.125
    b.w_cont, b.tau_win, b.win_edge = fake, 1.0, 4.0
    assert lib.dsalt_train_bwd(ctypes.byref(b), None) == 1  # d_w missing
    b.d_w = fake
    need = lib.dsalt_train_bwd_workspace_bytes(ctypes.byref(b))
    assert need >= 128 * 4 + 128 * 2 * 4
    b.base.workspace, b.base.workspace_bytes = fake, need - 16
    assert lib.dsalt_train_bwd(ctypes.byref(b), None) == 3
    # sets of more than 512 landmarks: the inference operator only
    b.base.p.k_lmk = 513
    assert lib.dsalt_train_bwd(ctypes.byref(b), None) == 2
    t = _valid_train_fwd()
    t.base.p.k_lmk = 513
    assert lib.dsalt_train_fwd(ctypes.byref(t), None) == 2
    assert b"512" in lib.dsalt_last_error()


def _valid_rope():
    a = _lib.RopeArgs()
    a.total_len, a.num_seqs, a.max_seqlen, a.n_q_heads, a.n_k_heads, a.head_dim, a.dtype = 128, 1, 128, 4, 2, 64, 1
    fake = 1 << 20
    a.q = a.k = a.cu_seqlens = a.cos = a.sin = fake
    a.q_stride_t, a.q_stride_h = 512, 64
    a.k_stride_t, a.k_stride_h = 512, 64
    a.max_pos = 128
    return a


@pytest.mark.parametrize("field,value", [("head_dim", 72), ("head_dim", 512), ("dtype", 5), ("max_pos", 100),
                                         ("num_seqs", 0), ("q_stride_h", 63), ("cos", None), ("sin", (1 << 20) + 4)])
def test_rope_validation(field, value):
    lib = _lib.load()
    a = _valid_rope()
    setattr(a, field, value)
    assert lib.dsalt_rope_qk(ctypes.byref(a), None) == 1
    assert lib.dsalt_last_error()


@pytest.mark.parametrize("field,value", [("cols", -1), ("cols", 40), ("dtype", 3), ("up", None),
                                         ("out", (1 << 20) + 2), ("gate_stride", 8), ("out_stride", 36)])
def test_silu_mul_validation(field, value):
    lib = _lib.load()
    a = _lib.SiluMulArgs(64, 32, 1, 1 << 20, 64, (1 << 20) + 64, 64, 1 << 21, 32)
    setattr(a, field, value)
    assert lib.dsalt_silu_mul(ctypes.byref(a), None) == 1


@pytest.mark.parametrize("field,value", [("seq", 1), ("seq", -1), ("rows", 129), ("w_cap", 0), ("p_win", None),
                                         ("lse", None), ("scale", 0.0)])
def test_export_probs_validation(field, value):
    lib = _lib.load()
    a = _lib.ProbsArgs()
    a.p = _lib.Problem(128, 1, 128, 2, 2, 64, 8, 0, 0, _lib.DTYPE_BF16)
    fake = 1 << 20
    a.q = a.k = a.w = a.cu_seqlens = a.lmk_idx = a.lse = a.p_win = a.p_lmk = fake
    a.q_stride_t = a.k_stride_t = 128
    a.q_stride_h = a.k_stride_h = 64
    a.scale, a.seq, a.rows, a.w_cap = 0.125, 0, 128, 64
    setattr(a, field, value)
    assert lib.dsalt_export_probs(ctypes.byref(a), None) == 1


@pytest.mark.parametrize("field,value", [("n_cols", 0), ("n_cols", 130), ("dtype", 4), ("reduction", 3),
                                         ("logits", (1 << 20) + 8), ("logits_stride", 64), ("logits_stride", 100),
                                         ("target", None), ("label_smoothing", 1.5), ("softcap", -1.0)])
def test_cross_entropy_validation(field, value):
    lib = _lib.load()
    a = _lib.CeArgs()
    a.rows, a.n_cols, a.dtype, a.logits, a.logits_stride = 16, 128, 1, 1 << 20, 128
    a.target = a.loss = 1 << 21
    a.ignore_index, a.n_non_ignore, a.reduction, a.want_grad = -100, 16.0, 1, 1
    setattr(a, field, value)
    assert lib.dsalt_cross_entropy_rows(ctypes.byref(a), None) == 1

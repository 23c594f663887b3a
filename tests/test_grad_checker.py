"""The gradient checker of the GPU tests must be able to fail (CPU only).

The headline workload's landmark rows collect gradient from up to every query of the
sequence, so one bound over all rows (max |a - b| / max |b|) lets an error of tens of
percent on every other row pass.  ``tests.helpers.assert_grad_close`` bounds landmark rows
and the other rows separately and adds a per-row bound.  Here it is fed float64 oracle
gradients of one head of the benchmark workloads at their full length:
  * the oracle's own gradients rounded to bf16, and gradients computed with P and dS rounded
    to bf16 before their products (the operand rounding of the 16-bit kernels), must pass
    (both with delta from the output rounded to bf16, as the GPU tests feed the oracle the
    output the kernels stored);
  * planted mistakes must fail: every non-landmark dK row 5 % too large, every dQ row 5 % too
    large, every landmark dV row 5 % too large, one ordinary dK row of median norm 50 % too
    large (which the single all-rows bound accepts).
The fp32 bounds (class 1e-5, row FP32_ROW_TOL) likewise: gradients computed in float32 pass,
one ordinary dq row 1e-4 off fails.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate
from oracle import attention as OA
from tests.helpers import (FP32_ROW_TOL, FP32_TOL, assert_grad_close, f64, landmark_rows, oracle_select_by_group,
                           rel_err)

TOL = 2e-2


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(torch.float64).numpy()


@pytest.fixture(scope="module", params=["fwdbwd_bf16_h16_l32768", "fwdbwd_bf16_b4_h8_l8192"])
def grads(request):
    """One head of the workload at full length: exact and bf16-operand gradients, landmark rows."""
    wl = WORKLOADS[request.param]
    x = generate(wl, heads=1)
    idx = oracle_select_by_group(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, ops.SELECT_GLOBAL,
                                 wl.block_size, ops.STATS_SEQUENCE)
    args = (f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(), idx,
            1.0 / math.sqrt(wl.head_dim), f64(x["dout"]))
    o, _ = OA.attention_fwd(*args[:7])
    exact = OA.attention_bwd(*args, out=_bf16(o))[:3]
    emul = OA.attention_bwd(*args, out=_bf16(o), operand_round=_bf16)[:3]
    lmk = landmark_rows(idx, x["cu"].numpy(), x["q"].shape[0])[:, 0]
    assert lmk.sum() > 0 and (~lmk).sum() > 0
    return request.param, [g[:, 0] for g in exact], [_bf16(g[:, 0]) for g in emul], lmk


def _check_all(got, ref, lmk):
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_grad_close(name, a, b, TOL, lmk if name != "dq" else None)


def test_rounded_oracle_passes(grads):
    _, exact, _, lmk = grads
    _check_all([_bf16(g) for g in exact], exact, lmk)


def test_bf16_operand_arithmetic_passes(grads):
    _, exact, emul, lmk = grads
    _check_all(emul, exact, lmk)


def test_non_landmark_dk_rows_scaled_fail(grads):
    _, exact, emul, lmk = grads
    dk = emul[1].copy()
    dk[~lmk] *= 1.05
    with pytest.raises(AssertionError):
        assert_grad_close("dk", dk, exact[1], TOL, lmk)


def test_every_dq_row_scaled_fails(grads):
    _, exact, emul, lmk = grads
    with pytest.raises(AssertionError):
        assert_grad_close("dq", emul[0] * 1.05, exact[0], TOL)


def test_landmark_dv_rows_scaled_fail(grads):
    _, exact, emul, lmk = grads
    dv = emul[2].copy()
    dv[lmk] *= 1.05
    with pytest.raises(AssertionError):
        assert_grad_close("dv", dv, exact[2], TOL, lmk)


def test_one_ordinary_row_wrong_fails_where_the_single_bound_passes(grads):
    name, exact, emul, lmk = grads
    b = exact[1]
    rn = np.linalg.norm(b, axis=1)
    other = np.nonzero(~lmk)[0]
    j = other[np.argsort(rn[other])[len(other) // 2]]  # an ordinary row of median norm
    dk = emul[1].copy()
    dk[j] *= 1.5
    with pytest.raises(AssertionError):
        assert_grad_close("dk", dk, b, TOL, lmk)
    if name == "fwdbwd_bf16_h16_l32768":
        # the single bound over all rows does not see it at the headline shape
        assert rel_err(dk, b) < TOL


# ------------------------------------------------------------------ fp32 bounds
@pytest.fixture(scope="module")
def fp32_case():
    """Three ragged sequences, one head of head_dim 128, windows up to 441, three landmarks per
    sequence: float64 gradients and gradients computed in float32 (dense masked softmax in torch,
    delta from the float32 output, as the GPU tests feed the oracle the stored output)."""
    g = torch.Generator().manual_seed(935)
    lens = [279, 589, 151]
    T, D = sum(lens), 128
    q, k, v, do = (torch.randn(T, 1, D, generator=g) for _ in range(4))
    w = torch.randint(1, 442, (T,), generator=g, dtype=torch.int32).numpy()
    cu = np.array([0] + list(np.cumsum(lens)))
    idx = np.stack([np.sort(torch.randperm(n, generator=g)[:3].numpy()) for n in lens])[None, :, None, :]
    mask = torch.from_numpy(OA.dense_mask_kernel(w, cu, idx))[0]
    scale = 1.0 / math.sqrt(D)
    q2, k2, v2, do2 = q[:, 0], k[:, 0], v[:, 0], do[:, 0]
    p = torch.softmax(torch.where(mask, q2 @ k2.T * scale, torch.tensor(-math.inf)), dim=1)
    out = p @ v2
    ds = p * (do2 @ v2.T - (out * do2).sum(1, keepdim=True))
    f32 = [(ds @ k2 * scale).double().numpy(), (ds.T @ q2 * scale).double().numpy(), (p.T @ do2).double().numpy()]
    exact = OA.attention_bwd(f64(q), f64(k), f64(v), w, cu, idx, scale, f64(do), out=f64(out)[:, None])[:3]
    lmk = landmark_rows(idx, cu, T)[:, 0]
    return f32, [e[:, 0] for e in exact], lmk


def test_fp32_arithmetic_passes_the_fp32_bounds(fp32_case):
    f32, exact, lmk = fp32_case
    for name, a, b in zip(("dq", "dk", "dv"), f32, exact):
        assert_grad_close(name, a, b, FP32_TOL, lmk if name != "dq" else None, row_tol=FP32_ROW_TOL)


def test_fp32_one_ordinary_row_wrong_fails(fp32_case):
    f32, exact, lmk = fp32_case
    rn = np.linalg.norm(exact[0], axis=1)
    j = np.argsort(rn)[len(rn) // 2]  # a row of median norm, 1e-4 off
    dq = f32[0].copy()
    dq[j] *= 1 + 1e-4
    with pytest.raises(AssertionError):
        assert_grad_close("dq", dq, exact[0], FP32_TOL, row_tol=FP32_ROW_TOL)

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
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate
from oracle import attention as OA
from tests.helpers import assert_grad_close, f64, landmark_rows, oracle_select_by_group, rel_err

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

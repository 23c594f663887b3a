"""Training variant (soft-edge band, weighted landmarks) on the GPU against the float64 oracle.

Tolerances (relative, max|a-b| / max|b|): 1e-5 for fp32, 2e-2 for bf16 and fp16, for the
output and every gradient (q, k, v, landmark log-weights, continuous windows).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.kernels import dsalt_triton_train_attention
from oracle import train as OT
from tests.helpers import f64, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _inputs(lens, H, D, K, wlo, whi, dt, seed, integer_every=0):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(dt)
    k = torch.randn(T, H, D, generator=g).to(dt)
    v = torch.randn(T, H, D, generator=g).to(dt)
    w = wlo + torch.rand(T, generator=g) * (whi - wlo)
    if integer_every:
        w[::integer_every] = w[::integer_every].floor()  # the band end and the landmark cut at d = w~
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    pos = torch.full((H, len(lens), K), -1, dtype=torch.int32)
    for hh in range(H):
        for s, L in enumerate(lens):
            n = min(K - (hh % 2), L)  # leave a -1 slot in every other head
            pos[hh, s, :n] = torch.randperm(L, generator=g)[:n].sort().values.to(torch.int32)
    logw = torch.nn.functional.logsigmoid(torch.randn(pos.shape, generator=g))
    logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    do = torch.randn(T, H, D, generator=g).to(dt)
    return q, k, v, w, cu, pos, logw, do, max(lens)


def _oracle(q, k, v, w, cu, pos, logw, do, scale, tau, edge):
    return (OT.train_fwd(f64(q), f64(k), f64(v), w.double().numpy(), cu.numpy(), pos.numpy(), logw.double().numpy(),
                         scale, tau, edge),
            OT.train_bwd(f64(q), f64(k), f64(v), w.double().numpy(), cu.numpy(), pos.numpy(), logw.double().numpy(),
                         scale, tau, edge, f64(do)))


def _check(lens, H, D, K, wlo, whi, dt, seed, tau=1.0, edge=4.0, integer_every=0):
    q, k, v, w, cu, pos, logw, do, maxlen = _inputs(lens, H, D, K, wlo, whi, dt, seed, integer_every)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, wd, cud = (t.to(DEV) for t in (q, k, v, w, cu))
    idx = pos.unsqueeze(2).to(DEV)
    lw = logw.unsqueeze(2).to(DEV)
    out, lse = ops.train_forward(qd, kd, vd, wd, cud, idx, lw, tau_win=tau, win_edge=edge, scale=scale,
                                 max_seqlen=maxlen)
    dq, dk, dv, dlw, dw = ops.train_backward(do.to(DEV), qd, kd, vd, out, lse, wd, cud, idx, lw, tau_win=tau,
                                             win_edge=edge, scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    (ro, rl), (rdq, rdk, rdv, rdw, rdlw) = _oracle(q, k, v, w, cu, pos, logw, do, scale, tau, edge)
    tol = TOL[dt]
    assert rel_err(f64(out), ro) < tol
    assert rel_err(f64(lse), rl) < (1e-6 if dt == torch.float32 else 2e-3)
    for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv), ("d_w", dw, rdw),
                       ("d_logw", dlw[:, :, 0], rdlw)):
        e = rel_err(f64(a), b)
        assert e < tol, (name, e)
    fin = torch.isfinite(logw)
    assert torch.all(dlw[:, :, 0].cpu()[~fin] == 0)  # empty slots get no gradient
    return out, lse, dq, dk, dv, dlw, dw


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
def test_train_d64(dt):
    _check([300, 181, 64], 4, 64, 24, 0.5, 90.0, dt, seed=41, integer_every=5)


def test_train_d128_bf16():
    _check([333, 200], 2, 128, 40, 1.0, 120.0, torch.bfloat16, seed=42, tau=0.7, edge=6.0)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_train_edge_wider_than_windows(dt):
    # win_edge above every window: the whole band carries the soft-edge bias (no core)
    _check([257, 99], 2, 64, 16, 0.0, 7.5, dt, seed=43, tau=2.0, edge=9.0, integer_every=3)


def test_train_long_windows():
    # windows up to the whole sequence: the key-parallel sweep takes several compacted segments
    _check([2300, 700], 2, 64, 16, 1.0, 2300.0, torch.bfloat16, seed=44, integer_every=7)


def test_train_without_edge_matches_operator():
    """win_edge 0 puts the whole band in the core: the training kernels reduce to the operator
    with window floor(w~) + 1 and the log-weights as landmark bias."""
    q, k, v, w, cu, pos, logw, do, maxlen = _inputs([400, 150], 4, 64, 24, 0.0, 80.0, torch.bfloat16, seed=45,
                                                     integer_every=4)
    qd, kd, vd, wd, cud = (t.to(DEV) for t in (q, k, v, w, cu))
    idx, lw = pos.unsqueeze(2).to(DEV), logw.unsqueeze(2).to(DEV)
    out, lse = ops.train_forward(qd, kd, vd, wd, cud, idx, lw, tau_win=1.0, win_edge=0.0, max_seqlen=maxlen)
    wi = (w.floor() + 1).to(torch.int32).to(DEV)
    out2, lse2 = ops.attention_forward(qd, kd, vd, wi, cud, idx, lw, max_seqlen=maxlen)
    assert rel_err(f64(out), f64(out2)) < 1e-6
    assert rel_err(f64(lse), f64(lse2)) < 1e-6
    g1 = ops.train_backward(do.to(DEV), qd, kd, vd, out, lse, wd, cud, idx, lw, tau_win=1.0, win_edge=0.0,
                            max_seqlen=maxlen)
    g2 = ops.attention_backward(do.to(DEV), qd, kd, vd, out2, lse2, wi, cud, idx, lw, max_seqlen=maxlen)
    for a, b in zip(g1[:4], g2):
        assert rel_err(f64(a), f64(b)) < 1e-6
    assert torch.all(g1[4] == 0)  # no soft edge: no window gradient


def test_train_deterministic():
    q, k, v, w, cu, pos, logw, do, maxlen = _inputs([1024], 4, 64, 32, 1.0, 200.0, torch.bfloat16, seed=46)
    qd, kd, vd, wd, cud = (t.to(DEV) for t in (q, k, v, w, cu))
    idx, lw = pos.unsqueeze(2).to(DEV), logw.unsqueeze(2).to(DEV)
    out, lse = ops.train_forward(qd, kd, vd, wd, cud, idx, lw, max_seqlen=maxlen)
    r1 = ops.train_backward(do.to(DEV), qd, kd, vd, out, lse, wd, cud, idx, lw, max_seqlen=maxlen)
    r2 = ops.train_backward(do.to(DEV), qd, kd, vd, out, lse, wd, cud, idx, lw, max_seqlen=maxlen)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_autograd_function_gqa_unsorted_slots():
    """The reference's call: unsorted landmark slots, grouped k/v heads, float32 output, and
    gradients for q, k, v, lmk_logw and w_cont through autograd."""
    H, G, D, K = 8, 2, 64, 12
    lens = [260, 141]
    g = torch.Generator().manual_seed(47)
    T = sum(lens)
    dt = torch.bfloat16
    q = torch.randn(T, H, D, generator=g).to(dt)
    k = torch.randn(T, G, D, generator=g).to(dt)
    v = torch.randn(T, G, D, generator=g).to(dt)
    w = 2.0 + torch.rand(T, generator=g) * 60.0
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    pos = torch.full((H, 2, K), -1, dtype=torch.int64)
    for hh in range(H):
        for s, L in enumerate(lens):
            n = K - (hh % 3)
            pos[hh, s, :n] = torch.randperm(L, generator=g)[:n]  # unsorted, -1 last
            pos[hh, s] = pos[hh, s][torch.randperm(K, generator=g)]  # and -1 anywhere
    logw = torch.nn.functional.logsigmoid(torch.randn(pos.shape, generator=g))
    logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    do = torch.randn(T, H, D, generator=g)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    lwd = logw.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    out = dsalt_triton_train_attention(qd, kd, vd, pos.to(DEV), lwd, wd, cu.to(DEV), tau_win=1.3, win_edge=5.0,
                                       n_max=64, cu_list=cu.tolist())
    assert out.dtype == torch.float32 and out.shape == (T, H, D)
    out.backward(do.to(DEV))
    kr = np.repeat(f64(k), H // G, axis=1)
    vr = np.repeat(f64(v), H // G, axis=1)
    scale = 1.0 / math.sqrt(D)
    ro, _ = OT.train_fwd(f64(q), kr, vr, w.double().numpy(), cu.numpy(), pos.numpy(), logw.double().numpy(),
                         scale, 1.3, 5.0)
    rdq, rdk, rdv, rdw, rdlw = OT.train_bwd(f64(q), kr, vr, w.double().numpy(), cu.numpy(), pos.numpy(),
                                            logw.double().numpy(), scale, 1.3, 5.0,
                                            do.to(dt).double().numpy())
    rdk = rdk.reshape(T, G, H // G, D).sum(2)
    rdv = rdv.reshape(T, G, H // G, D).sum(2)
    assert rel_err(f64(out), ro) < 2e-2
    for name, a, b in (("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv), ("d_w", wd.grad, rdw),
                       ("d_logw", lwd.grad, rdlw)):
        e = rel_err(f64(a), b)
        assert e < 2e-2, (name, e)
    assert lwd.grad.dtype == torch.float32 and wd.grad.dtype == torch.float32
    assert torch.all(lwd.grad.cpu()[pos < 0] == 0)

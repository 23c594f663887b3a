"""Training variant (soft-edge band, weighted landmarks) on the GPU against the float64 oracle.

Tolerances (relative, max|a-b| / max|b|): 1e-5 for fp32, 2e-2 for bf16 and fp16, for the
output and every gradient (q, k, v, landmark log-weights, continuous windows); the gradients of
q, k and v per head through ``tests.helpers.check_grads`` (landmark rows and the other rows
each against their own largest entry, and a per-row bound).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.kernels import dsalt_triton_train_attention
from oracle import train as OT
from tests.helpers import check_grads, f64, rel_err

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
            n = max(0, min(K - (hh % 2), L))  # leave a -1 slot in every other head
            pos[hh, s, :n] = torch.randperm(L, generator=g)[:n].sort().values.to(torch.int32)
    logw = torch.nn.functional.logsigmoid(torch.randn(pos.shape, generator=g))
    logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    do = torch.randn(T, H, D, generator=g).to(dt)
    return q, k, v, w, cu, pos, logw, do, max(lens)


def _oracle(q, k, v, w, cu, pos, logw, do, scale, tau, edge, out=None):
    """(forward, backward) of the oracle; ``out``: the stored output that feeds delta."""
    return (OT.train_fwd(f64(q), f64(k), f64(v), w.double().numpy(), cu.numpy(), pos.numpy(), logw.double().numpy(),
                         scale, tau, edge),
            OT.train_bwd(f64(q), f64(k), f64(v), w.double().numpy(), cu.numpy(), pos.numpy(), logw.double().numpy(),
                         scale, tau, edge, f64(do), out=None if out is None else f64(out)))


def _check(lens, H, D, K, wlo, whi, dt, seed, tau=1.0, edge=4.0, integer_every=0, variant=0):
    q, k, v, w, cu, pos, logw, do, maxlen = _inputs(lens, H, D, K, wlo, whi, dt, seed, integer_every)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, wd, cud = (t.to(DEV) for t in (q, k, v, w, cu))
    idx = pos.unsqueeze(2).to(DEV)
    lw = logw.unsqueeze(2).to(DEV)
    out, lse = ops.train_forward(qd, kd, vd, wd, cud, idx, lw, tau_win=tau, win_edge=edge, scale=scale,
                                 max_seqlen=maxlen, variant=variant)
    dq, dk, dv, dlw, dw = ops.train_backward(do.to(DEV), qd, kd, vd, out, lse, wd, cud, idx, lw, tau_win=tau,
                                             win_edge=edge, scale=scale, max_seqlen=maxlen, variant=variant)
    torch.cuda.synchronize()
    (ro, rl), (rdq, rdk, rdv, rdw, rdlw) = _oracle(q, k, v, w, cu, pos, logw, do, scale, tau, edge, out=out)
    tol = TOL[dt]
    assert rel_err(f64(out), ro) < tol
    assert rel_err(f64(lse), rl) < (1e-6 if dt == torch.float32 else 2e-3)
    check_grads("train", (dq, dk, dv), (rdq, rdk, rdv), pos, cu, tol)
    for name, a, b in (("d_w", dw, rdw), ("d_logw", dlw[:, :, 0], rdlw)):
        e = rel_err(f64(a), b)
        assert e < tol, (name, e)
    fin = torch.isfinite(logw)
    assert torch.all(dlw[:, :, 0].cpu()[~fin] == 0)  # empty slots get no gradient
    return out, lse, dq, dk, dv, dlw, dw


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
def test_train_d64(dt):
    _check([300, 181, 64], 4, 64, 24, 0.5, 90.0, dt, seed=41, integer_every=5)


def _train_variants():
    from dsalt_amd.kernels import autotune as AT
    return [c["variant"] for c in AT._candidate_configs(64, None, 2)]


@pytest.mark.parametrize("variant", _train_variants())
def test_train_d64_every_tiling(variant):
    """Every tiling the autotune may choose for 16-bit head_dim 64: the training operator runs the
    tuned variant's instantiations of the soft-edge kernels."""
    _check([700, 181], 4, 64, 24, 0.5, 300.0, torch.bfloat16, seed=51, integer_every=5, variant=variant)


def test_train_d128_bf16():
    _check([333, 200], 2, 128, 40, 1.0, 120.0, torch.bfloat16, seed=42, tau=0.7, edge=6.0)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_train_edge_wider_than_windows(dt):
    # win_edge above every window: the whole band carries the soft-edge bias (no core)
    _check([257, 99], 2, 64, 16, 0.0, 7.5, dt, seed=43, tau=2.0, edge=9.0, integer_every=3)


@pytest.mark.parametrize("dt,edge", [(torch.float32, 4.0), (torch.float32, 10.0), (torch.bfloat16, 4.0)])
def test_train_windows_longer_than_sequences(dt, edge):
    # w~ up to 3x the longest sequence (integer and fractional): every band key of such a row
    # lies in the core; the kernels clamp w~ keeping floor and fraction of one value (clamping
    # the floor alone once moved the edge onto core keys of the rows near the sequence ends)
    _check([150, 64, 1], 3, 64, 20, 5.0, 450.0, dt, seed=45, edge=edge, integer_every=3)


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
                                            do.to(dt).double().numpy(), out=f64(out.detach()))
    rdk = rdk.reshape(T, G, H // G, D).sum(2)
    rdv = rdv.reshape(T, G, H // G, D).sum(2)
    assert rel_err(f64(out), ro) < 2e-2
    check_grads("train_autograd", (qd.grad, kd.grad, vd.grad), (rdq, rdk, rdv), pos, cu, 2e-2)
    for name, a, b in (("d_w", wd.grad, rdw), ("d_logw", lwd.grad, rdlw)):
        e = rel_err(f64(a), b)
        assert e < 2e-2, (name, e)
    assert lwd.grad.dtype == torch.float32 and wd.grad.dtype == torch.float32
    assert torch.all(lwd.grad.cpu()[pos < 0] == 0)


# ------------------------------------------------------------- the layer's training branch
def _hybrid_ref(x, W, alpha, H, dh):
    """float64 torch restatement of the hybrid score (dsalt/kernels/landmark_tokens_ker.py:19-61)."""
    T = x.shape[0]
    n = x.norm(dim=-1)
    zx = (n - n.mean()) / n.std().clamp(min=1e-6)
    G = W.shape[0] // dh
    nv = (x @ W.T).view(T, G, dh).norm(dim=-1)
    zv = (nv - nv.mean(0, keepdim=True)) / nv.std(0, keepdim=True).clamp(min=1e-6)
    zv = zv.repeat_interleave(H // G, dim=1)
    return alpha * zv + (1.0 - alpha) * zx[:, None]


def _dense_bias_ref(w_seq, pos, logw, tau, edge):
    """Differentiable [H, L, L] training log-bias of one sequence, out of place (the dense form
    of dsalt/modules/dsalt_attention.py:520-563); checked against the oracle's train_bias."""
    L = w_seq.shape[0]
    i = torch.arange(L, dtype=torch.float64)
    d = i[:, None] - i[None, :]
    wi = w_seq[:, None]
    lb = torch.log(torch.sigmoid((wi - d) / tau).clamp(min=1e-20))
    lb = torch.where(d <= wi - edge, torch.zeros_like(lb), lb)
    lb = lb.masked_fill(~((d >= 0) & (d <= wi)), float("-inf"))
    out = []
    for h in range(pos.shape[0]):
        b = lb
        for s in range(pos.shape[1]):
            p = int(pos[h, s])
            if p < 0:
                continue
            rows = (p <= i) & (p < i - w_seq)
            hit = rows[:, None] & (torch.arange(L)[None, :] == p)
            b = torch.maximum(b, torch.where(hit, logw[h, s], torch.full_like(b, float("-inf"))))
        out.append(b)
    return torch.stack(out)


def test_hybrid_score_gradients_match_torch_float64():
    from dsalt_amd.kernels import hybrid_scores_per_head
    g = torch.Generator().manual_seed(50)
    T, d, H, G, dh = 333, 128, 4, 2, 32
    x = torch.randn(T, d, generator=g)
    W = torch.randn(G * dh, d, generator=g) / math.sqrt(d)
    alpha = torch.sigmoid(torch.randn(H, generator=g))
    up = torch.randn(T, H, generator=g)
    xd, Wd, ad = (t.to(DEV).requires_grad_(True) for t in (x, W, alpha))
    s, _, _ = hybrid_scores_per_head(xd, Wd, ad, H, dh)
    (s * up.to(DEV)).sum().backward()
    xr, Wr, ar = (t.double().requires_grad_(True) for t in (x, W, alpha))
    sr = _hybrid_ref(xr, Wr, ar, H, dh)
    (sr * up.double()).sum().backward()
    assert rel_err(f64(s), f64(sr)) < 1e-6
    for name, a, b in (("x", xd.grad, xr.grad), ("W_V", Wd.grad, Wr.grad), ("alpha", ad.grad, ar.grad)):
        e = rel_err(f64(a), f64(b))
        assert e < 1e-5, (name, e)


def test_layer_training_branch_against_float64_dense():
    """DSALTAttention in training mode (fp32): output and the gradients of every parameter
    (win_gate through the soft window edge, alpha_w through the landmark log-weights) and of
    x, against the dense float64 composition of the same selectors."""
    import copy

    from dsalt_amd.kernels import window_utils as WU
    from dsalt_amd.modules import DSALTAttention
    torch.manual_seed(51)
    d, H, G, L, S = 256, 4, 2, 192, 2
    T, dh = L * S, 64
    m = DSALTAttention(d, H, 4, 48, 16, 1024, n_kv_heads=G, qkv_bias=True).to(DEV).train()
    with torch.no_grad():
        m.win_gate.weight.mul_(8.0)  # spread the windows over [n_min, n_max]
    mr = copy.deepcopy(m).cpu().double()
    x = torch.randn(T, d)
    cot = torch.randn(T, d)
    cu_list = [0, L, T]
    cu = torch.tensor(cu_list, dtype=torch.int32)
    xd = x.to(DEV).requires_grad_(True)
    out, _ = m(xd, cu.to(DEV), cu_list=cu_list)
    (out * cot.to(DEV)).sum().backward()
    with torch.no_grad():
        w_gpu, pos, _ = m._train_selectors(xd.detach(), cu.to(DEV), T, torch.device(DEV), cu_list)
    pos = pos.cpu()

    xr = x.double().requires_grad_(True)
    q = mr.q_proj(xr).view(T, H, dh)
    k = mr.k_proj(xr).view(T, G, dh)
    v = mr.v_proj(xr).view(T, G, dh)
    p_ids = torch.cat([torch.arange(L)] * S)
    q, k = WU.apply_rotary_emb(q, k, mr.rope_cos[p_ids].unsqueeze(1), mr.rope_sin[p_ids].unsqueeze(1))
    k, v = k.repeat_interleave(H // G, 1), v.repeat_interleave(H // G, 1)
    w_ref = mr._window_continuous(xr)
    w_c = w_ref + (w_gpu.cpu().double() - w_ref).detach()  # the GPU's fp32 windows, gradient of w_ref
    sc = _hybrid_ref(xr, mr.v_proj.weight, mr._alpha(), H, dh)
    outs = []
    for s in range(S):
        st = s * L
        ps = pos[:, s]
        s_sel = sc[st + ps.clamp(min=0), torch.arange(H)[:, None]]
        lw = torch.log(torch.sigmoid(s_sel / mr.tau_lmk).clamp(min=1e-20))
        lw = torch.where(ps >= 0, lw, torch.full_like(lw, float("-inf")))
        bias = _dense_bias_ref(w_c[st:st + L], ps, lw, mr.tau_win, float(mr.win_edge))
        for h in range(H):
            ob, _ = OT.train_bias(w_c[st:st + L].detach().numpy(), ps[h].numpy(), lw[h].detach().numpy(),
                                  mr.tau_win, float(mr.win_edge))
            fin = np.isfinite(ob)
            assert np.array_equal(fin, torch.isfinite(bias[h]).numpy())
            assert np.abs(ob[fin] - bias[h].detach().numpy()[fin]).max() < 1e-12
        qs, ks, vs = (t[st:st + L].transpose(0, 1) for t in (q, k, v))
        a = torch.softmax(qs @ ks.transpose(1, 2) / math.sqrt(dh) + bias, -1)
        outs.append((a @ vs).transpose(0, 1).reshape(L, d))
    ref = mr.out_proj(torch.cat(outs))
    (ref * cot.double()).sum().backward()
    assert rel_err(f64(out), f64(ref)) < 2e-5
    named = dict(m.named_parameters())
    for n, pr in mr.named_parameters():
        e = rel_err(f64(named[n].grad), f64(pr.grad))
        assert e < 1e-4, (n, e)
    assert float(named["win_gate.weight"].grad.abs().max()) > 0
    assert float(named["alpha_w"].grad.abs().max()) > 0
    assert rel_err(f64(xd.grad), f64(xr.grad)) < 1e-4


# ------------------------------------------------------------- the benchmark's training workload
def _workload_logw(x, idx, sc, tau_lmk):
    pos = idx[:, :, 0].long()
    H = pos.shape[0]
    starts = x["cu"][:-1].long()
    s_sel = sc[starts[None, :, None] + pos.clamp(min=0), torch.arange(H, device=sc.device)[:, None, None]]
    logw = torch.log(torch.sigmoid(s_sel / tau_lmk).clamp(min=1e-20))
    return torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))


def test_train_workload_shortened_against_oracle():
    from dsalt_amd.workloads import WORKLOADS, generate
    wl = WORKLOADS["train_bf16_h16_l32768"]
    x = {k: v.to(DEV) for k, v in generate(wl, seqlen=2048, heads=2).items()}
    maxlen = 2048
    idx, _, _, sc = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=maxlen,
                                         stats_scope=ops.STATS_SEQUENCE, want_scores=True)
    logw = _workload_logw(x, idx, sc, wl.tau_lmk)
    out, lse = ops.train_forward(x["q"], x["k"], x["v"], x["w_cont"], x["cu"], idx, logw.unsqueeze(2),
                                 tau_win=wl.tau_win, win_edge=wl.win_edge, max_seqlen=maxlen)
    dq, dk, dv, dlw, dw = ops.train_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w_cont"], x["cu"], idx,
                                             logw.unsqueeze(2), tau_win=wl.tau_win, win_edge=wl.win_edge,
                                             max_seqlen=maxlen)
    torch.cuda.synchronize()
    c = {k: v.cpu() for k, v in x.items()}
    pos = idx[:, :, 0].cpu()
    (ro, _), (rdq, rdk, rdv, rdw, rdlw) = _oracle(c["q"], c["k"], c["v"], c["w_cont"], c["cu"], pos, logw.cpu(),
                                                  c["dout"], 1.0 / 8.0, wl.tau_win, wl.win_edge, out=out)
    check_grads("train_workload", (dq, dk, dv), (rdq, rdk, rdv), pos, c["cu"], 2e-2)
    for name, a, b in (("out", out, ro), ("d_w", dw, rdw), ("d_logw", dlw[:, :, 0], rdlw)):
        e = rel_err(f64(a), b)
        assert e < 2e-2, (name, e)


def test_train_workload_full_size_without_edge_is_the_operator():
    """At the benchmark's full shape (T=32768, H=16): with win_edge 0 the training kernels
    give the operator's output and gradients (window floor(w~)+1, log-weights as bias)."""
    from dsalt_amd.workloads import WORKLOADS, generate
    wl = WORKLOADS["train_bf16_h16_l32768"]
    x = {k: v.to(DEV) for k, v in generate(wl).items()}
    maxlen = wl.seqlen
    idx, _, _, sc = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=maxlen,
                                         stats_scope=ops.STATS_SEQUENCE, want_scores=True)
    lw = _workload_logw(x, idx, sc, wl.tau_lmk).unsqueeze(2)
    out, lse = ops.train_forward(x["q"], x["k"], x["v"], x["w_cont"], x["cu"], idx, lw, tau_win=1.0, win_edge=0.0,
                                 max_seqlen=maxlen)
    wi = x["w"] + 1
    out2, lse2 = ops.attention_forward(x["q"], x["k"], x["v"], wi, x["cu"], idx, lw, max_seqlen=maxlen)
    assert rel_err(f64(out), f64(out2)) < 1e-6
    g1 = ops.train_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w_cont"], x["cu"], idx, lw, tau_win=1.0,
                            win_edge=0.0, max_seqlen=maxlen)
    g2 = ops.attention_backward(x["dout"], x["q"], x["k"], x["v"], out2, lse2, wi, x["cu"], idx, lw,
                                max_seqlen=maxlen)
    for a, b in zip(g1[:4], g2):
        assert rel_err(f64(a), f64(b)) < 1e-6

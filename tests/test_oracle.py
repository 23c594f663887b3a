"""Pins the CPU oracle before anything is compared against it.

Parity status of each oracle function (how it is pinned):
  select_oracle.c norms          math: fp64 norm within 1 ulp of the dtype; canon_sqrt64 vs sqrt
  select_oracle.c range_sums     math: math.fsum
  select_oracle.c z / scores     golden (reference hybrid_scores_per_head) + mean 0 / unbiased std 1
                                 + alpha in {0,1} reduces to a single signal
  select_oracle.c global top-k   golden (reference _compute_landmark_indices, uniform / ragged /
                                 GQA / padding) + numpy brute force with ties + exclusion invariants
  select_oracle.c block top-k    golden (reference causal_landmark_check._select, MHA and GQA)
                                 + first block empty + candidates before the block only
  attention.attention_fwd        golden (reference _block_attention) + dense brute force +
                                 causal-SDPA and O=V special cases + no-double-count
  attention.attention_bwd        central finite differences + torch autograd of the dense form
  attention.literal_mask         golden (reference _build_mask_packed + masked SDPA)
  attention.attention_probs      P @ V reproduces attention_fwd's output for random V; rows sum
                                 to 1; zero off the dense kernel mask
  train.train_bias / train_fwd   golden (reference _dense_logbias_from_kernel + SDPA, float64)
                                 + win_edge 0 reduces to attention_fwd with window floor(w~)+1
  cross_entropy.ce_rows          torch F.cross_entropy + autograd (ignore_index, class weights, label
                                 smoothing, mean/sum/none), softcap and z-loss and token scaling
                                 through torch autograd of their definitions
  rope.rope                      torch's evaluation of the reference expression (CPU, bf16/fp16/fp32)
                                 + rotation of 2-vectors preserves norms (fp32)
  train.train_bwd                golden (float64 autograd of the reference dense form)
                                 + central finite differences in w~ and lmk_logw
  train.train_fwd_banded /       train_fwd / train_bwd (dense, pinned above) on ragged sequences
  train.train_bwd_banded         with several row blocks, edges wider than windows, empty slots
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import select as OS
from oracle import cross_entropy as OCE
from oracle import rope as OR
from oracle import train as OT
from tests.helpers import bits, load_golden, rel_err


# ----------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("name", ["uniform", "ragged", "gqa", "pad"])
def test_select_matches_reference_golden(name):
    z = load_golden(f"select_{name}")
    idx, zx, zv, sc = OS.select(z["x"], z["v"], z["alpha"], z["w"].astype(np.int64), z["cu"], int(z["k"]),
                                OS.DTYPE_F32, want_scores=True)
    np.testing.assert_array_equal(idx[:, :, 0], z["idx"])
    np.testing.assert_allclose(zx, z["z_x"], atol=3e-6)
    rep = z["z_v"].shape[1] // zv.shape[1]
    np.testing.assert_allclose(np.repeat(zv, rep, axis=1), z["z_v"], atol=3e-6)
    np.testing.assert_allclose(sc, z["scores"], atol=3e-6)


@pytest.mark.parametrize("name", ["mha", "gqa", "b64"])
def test_block_causal_matches_reference_golden(name):
    z = load_golden(f"block_causal_{name}")
    T, B, k = z["x"].shape[0], int(z["block"]), int(z["k"])
    cu = np.array([0, T])
    idx = OS.select(z["x"], z["v"], z["alpha"], z["w"].astype(np.int64), cu, k, OS.DTYPE_F32,
                    mode=OS.SELECT_BLOCK, block_size=B)
    np.testing.assert_array_equal(idx[:, 0], z["sets"])
    scale = 1.0 / math.sqrt(z["q"].shape[-1])
    o, _ = OA.attention_fwd(z["q"], z["kk"], z["vv"], z["w"].astype(np.int64), cu, idx, scale, block_size=B)
    assert np.abs(o - z["out"]).max() < 1e-5


def test_literal_fallback_matches_reference_golden():
    z = load_golden("literal_fallback")
    T = z["x"].shape[0]
    idx = OS.select(z["x"], z["v"], z["alpha"], z["w"].astype(np.int64), z["cu"], int(z["k"]), OS.DTYPE_F32)
    np.testing.assert_array_equal(idx[:, :, 0], z["idx"])
    m = OA.literal_mask(z["w"].astype(np.int64), z["cu"], idx)
    mref = np.unpackbits(z["mask"], axis=-1)[:, :T].astype(bool)
    np.testing.assert_array_equal(m[0], mref)
    o, _ = OA.dense_attention(z["q"], z["kk"], z["vv"], m, 1.0 / math.sqrt(z["q"].shape[-1]))
    assert np.abs(o - z["out"]).max() < 1e-5


def test_window_masks_match_reference_golden():
    z = load_golden("window_masks")
    L = z["m1"].shape[0]
    m = OA.dense_mask_kernel(z["w1"].astype(np.int64), np.array([0, L]), np.full((1, 1, 1, 0), -1))
    np.testing.assert_array_equal(m[0], z["m1"])
    m2 = OA.dense_mask_kernel(z["w2"].astype(np.int64), z["cu"], np.full((1, len(z["cu"]) - 1, 1, 0), -1))
    np.testing.assert_array_equal(m2[0], z["m2"])


# ------------------------------------------------------------- selection by math
def test_canon_sqrt_close_to_sqrt():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(0, 1, 2000), 10.0 ** rng.uniform(-200, 200, 2000), [4.0, 1e-300, 2.0]])
    for x in xs:
        y = OS.canon_sqrt64(x)
        assert abs(y - math.sqrt(x)) <= 2 * np.spacing(math.sqrt(x)), x
    assert OS.canon_sqrt64(0.0) == 0.0


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [64, 128, 256, 1024, 96, 98, 100, 13])
def test_norms_match_fp64_norm(dt, n):
    # widths that are not whole 16-byte vectors (98, 100, 13) too: summed as the zero-padded row
    g = torch.Generator().manual_seed(n)
    h = (torch.randn(50, n, generator=g) * 3).to(dt)
    v = torch.randn(50, 2, 64, generator=g).to(dt)
    from tests.helpers import bits, oracle_dtype
    nx, nv = OS.norms(bits(h), bits(v), oracle_dtype(dt))
    hp = torch.nn.functional.pad(h, (0, (-n) % (16 // h.element_size())))
    assert np.array_equal(OS.norms(bits(hp), bits(v), oracle_dtype(dt))[0], nx)
    exact = np.linalg.norm(h.double().numpy(), axis=1)
    ref = torch.tensor(exact).to(torch.float32).to(dt).to(torch.float64).numpy()
    ulp = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dt]
    assert np.all(np.abs(nx - ref) <= ulp * ref * 1.01)
    exv = np.linalg.norm(v.double().numpy(), axis=2).T
    refv = torch.tensor(exv).to(torch.float32).to(dt).to(torch.float64).numpy()
    assert np.all(np.abs(nv - refv) <= ulp * refv * 1.01)


def test_range_sums_match_fsum():
    rng = np.random.default_rng(1)
    x = (rng.lognormal(0, 1, 5000)).astype(np.float32)
    s1, s2 = OS.range_sums(x, 17, 4999)
    xs = x[17:4999].astype(np.float64)
    assert abs(s1 - math.fsum(xs)) <= 1e-13 * abs(s1)
    assert abs(s2 - math.fsum(xs * xs)) <= 1e-13 * abs(s2)


def _rand_case(seed, T=96, hidden=32, G=2, D=64, H=4, dt=np.float32):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((T, hidden)).astype(np.float32)
    v = rng.standard_normal((T, G, D)).astype(np.float32)
    alpha = rng.uniform(0.1, 0.9, H).astype(np.float32)
    w = rng.integers(1, 24, T)
    return h, v, alpha, w


def test_z_has_mean_zero_and_unbiased_unit_std():
    h, v, alpha, w = _rand_case(2, T=64)
    _, zx, zv, _ = OS.select(h, v, alpha, w, np.array([0, 64]), 4, OS.DTYPE_F32, want_scores=True)
    assert abs(zx.astype(np.float64).mean()) < 1e-6
    assert abs(zx.astype(np.float64).std(ddof=1) - 1.0) < 1e-6   # biased std would give 0.992
    assert np.all(np.abs(zv.astype(np.float64).std(axis=0, ddof=1) - 1.0) < 1e-6)


@pytest.mark.parametrize("a", [0.0, 1.0])
def test_alpha_extremes_rank_by_one_signal(a):
    h, v, _, w = _rand_case(3, T=80, H=2, G=2)
    w[:] = 1
    alpha = np.full(2, a, np.float32)
    idx = OS.select(h, v, alpha, w, np.array([0, 80]), 8, OS.DTYPE_F32)
    nx, nv = OS.norms(h, v, OS.DTYPE_F32)
    for hh in range(2):
        sig = nv[hh] if a == 1.0 else nx
        cand = np.arange(80) >= 1
        expect = np.sort(np.nonzero(cand)[0][np.argsort(-sig[cand], kind="stable")[:8]])
        np.testing.assert_array_equal(idx[hh, 0, 0], expect)


@pytest.mark.parametrize("seed", range(6))
def test_topk_matches_brute_force_with_ties(seed):
    rng = np.random.default_rng(10 + seed)
    T, H = 70, 3
    # integer-valued vectors create many exactly equal norms, i.e. score ties
    h = rng.integers(-2, 3, (T, 16)).astype(np.float32)
    v = rng.integers(-2, 3, (T, 1, 64)).astype(np.float32)
    alpha = np.array([0.5, 0.25, 1.0], np.float32)
    w = rng.integers(1, 30, T)
    cu = np.array([0, 40, 70])
    idx, zx, zv, sc = OS.select(h, v, alpha, w, cu, 9, OS.DTYPE_F32, want_scores=True)
    for s in range(2):
        st, en = cu[s], cu[s + 1]
        cand = np.arange(en - st) >= w[st:en]
        for hh in range(H):
            ref = OS.brute_topk(sc[st:en, hh], cand, 9)
            np.testing.assert_array_equal(idx[hh, s, 0], ref)
            sel = idx[hh, s, 0][idx[hh, s, 0] >= 0]
            assert np.all(sel >= w[st + sel])  # never a token covered by its own window
            assert len(sel) == min(9, cand.sum())


def test_scores_match_float64_brute_force():
    h, v, alpha, w = _rand_case(4, T=120, H=4, G=2)
    _, _, _, sc = OS.select(h, v, alpha, w, np.array([0, 120]), 4, OS.DTYPE_F32, want_scores=True)
    nx, nv = OS.norms(h, v, OS.DTYPE_F32)
    ref = OS.brute_scores(nx, nv, alpha, slice(0, 120))
    np.testing.assert_allclose(sc, ref, atol=2e-6)


def test_block_mode_structure():
    h, v, alpha, w = _rand_case(5, T=200, H=2, G=2)
    w = np.minimum(w, 8)
    idx = OS.select(h, v, alpha, w, np.array([0, 200]), 16, OS.DTYPE_F32, mode=OS.SELECT_BLOCK, block_size=64)
    assert idx.shape == (2, 1, 4, 16)
    assert np.all(idx[:, 0, 0] == -1)  # the first block has no earlier tokens
    for b in range(1, 4):
        sel = idx[:, 0, b][idx[:, 0, b] >= 0]
        assert np.all(sel < 64 * b)
    # block statistics over the prefix: the last block equals a global selection on the prefix
    pre = OS.select(h[:192], v[:192], alpha, w[:192], np.array([0, 192]), 16, OS.DTYPE_F32)
    np.testing.assert_array_equal(pre[:, 0, 0], idx[:, 0, 3])


# ------------------------------------------------------------- attention by math
def _attn_case(seed, lens=(40, 27), H=2, G=2, D=8, K=6, wmax=12):
    rng = np.random.default_rng(seed)
    T = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)])
    q = rng.standard_normal((T, H, D))
    k = rng.standard_normal((T, G, D))
    v = rng.standard_normal((T, G, D))
    w = rng.integers(1, wmax, T)
    idx = np.full((H, len(lens), 1, K), -1)
    for hh in range(H):
        for s, L in enumerate(lens):
            c = np.sort(rng.choice(L, size=min(K - 1, L), replace=False))
            idx[hh, s, 0, :len(c)] = c
    return q, k, v, w, cu, idx


@pytest.mark.parametrize("seed", range(3))
def test_fwd_matches_dense_brute_force(seed):
    q, k, v, w, cu, idx = _attn_case(seed, G=1 if seed == 2 else 2)
    bias = np.random.default_rng(seed).standard_normal(idx.shape)
    o, lse = OA.attention_fwd(q, k, v, w, cu, idx, 0.35, lmk_bias=bias)
    m = OA.dense_mask_kernel(w, cu, idx)
    # bias enters as an additive logit: fold it into a brute-force loop
    T, H, D = q.shape
    rep = H // k.shape[1]
    for hh in range(H):
        for s in range(len(cu) - 1):
            st, en = cu[s], cu[s + 1]
            for i in range(st, en):
                cols = np.nonzero(m[hh, i])[0]
                lg = q[i, hh] @ k[cols, hh // rep].T * 0.35
                for t, c in enumerate(cols):
                    slots = np.nonzero(idx[hh, s, 0] == c - st)[0]
                    if len(slots) and not (i - st - max(w[i], 1) + 1 <= c - st <= i - st):
                        lg[t] += bias[hh, s, 0, slots[0]]
                pmx = lg.max()
                p = np.exp(lg - pmx)
                ref = (p / p.sum()) @ v[cols, hh // rep]
                assert np.abs(o[i, hh] - ref).max() < 1e-12
                assert abs(lse[i, hh] - (pmx + np.log(p.sum()))) < 1e-12


def test_fwd_special_cases():
    rng = np.random.default_rng(7)
    T, H, D = 50, 2, 8
    q, k, v = (rng.standard_normal((T, H, D)) for _ in range(3))
    cu = np.array([0, T])
    empty = np.full((H, 1, 1, 0), -1)
    # w = 1 and no landmarks: every row attends only to itself
    o, _ = OA.attention_fwd(q, k, v, np.ones(T, int), cu, empty, 0.3)
    np.testing.assert_allclose(o, v, atol=1e-14)
    # w >= i+1 and no landmarks: causal softmax attention
    o, _ = OA.attention_fwd(q, k, v, np.full(T, T), cu, empty, 0.3)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.tensor(q).transpose(0, 1), torch.tensor(k).transpose(0, 1), torch.tensor(v).transpose(0, 1),
        is_causal=True, scale=0.3).transpose(0, 1).numpy()
    np.testing.assert_allclose(o, ref, atol=1e-12)
    # landmarks that sit inside every window they could reach add nothing
    w = np.full(T, 10)
    idx = np.full((H, 1, 1, 3), -1)
    idx[:, 0, 0] = [T - 3, T - 2, T - 1]
    o1, _ = OA.attention_fwd(q, k, v, w, cu, idx, 0.3)
    o0, _ = OA.attention_fwd(q, k, v, w, cu, empty, 0.3)
    np.testing.assert_allclose(o1, o0, atol=1e-14)


def test_bwd_matches_finite_differences():
    q, k, v, w, cu, idx = _attn_case(11, lens=(20, 13), H=2, G=2, D=4, K=4, wmax=7)
    rng = np.random.default_rng(12)
    do = rng.standard_normal(q.shape)
    bias = rng.standard_normal(idx.shape) * 0.5
    scale = 0.6
    dq, dk, dv, db = OA.attention_bwd(q, k, v, w, cu, idx, scale, do, lmk_bias=bias)

    def loss(q_, k_, v_, b_):
        o, _ = OA.attention_fwd(q_, k_, v_, w, cu, idx, scale, lmk_bias=b_)
        return float((o * do).sum())

    eps = 1e-6
    for arr, grad, name in ((q, dq, "q"), (k, dk, "k"), (v, dv, "v"), (bias, db, "bias")):
        flat = arr.reshape(-1)
        picks = rng.choice(flat.size, size=min(25, flat.size), replace=False)
        for pidx in picks:
            old = flat[pidx]
            flat[pidx] = old + eps
            lp = loss(q, k, v, bias)
            flat[pidx] = old - eps
            lm = loss(q, k, v, bias)
            flat[pidx] = old
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad.reshape(-1)[pidx]) < 1e-6 + 1e-5 * abs(fd), (name, pidx)


def test_bwd_gqa_sums_groups_and_matches_autograd():
    q, k, v, w, cu, idx = _attn_case(13, lens=(30,), H=4, G=2, D=8, K=5, wmax=9)
    do = np.random.default_rng(14).standard_normal(q.shape)
    dq, dk, dv, _ = OA.attention_bwd(q, k, v, w, cu, idx, 0.4, do)
    m = torch.tensor(OA.dense_mask_kernel(w, cu, idx))
    qt, kt, vt = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    kr = kt.repeat_interleave(2, dim=1)
    vr = vt.repeat_interleave(2, dim=1)
    s = torch.einsum("thd,shd->hts", qt, kr) * 0.4
    s = s.masked_fill(~m, float("-inf"))
    o = torch.einsum("hts,shd->thd", torch.softmax(s, -1), vr)
    (o * torch.tensor(do)).sum().backward()
    assert rel_err(dq, qt.grad.numpy()) < 1e-12
    assert rel_err(dk, kt.grad.numpy()) < 1e-12
    assert rel_err(dv, vt.grad.numpy()) < 1e-12


# ------------------------------------------------------------- training variant
def _train_args(g):
    return (g["q"], g["k"], g["v"], g["w_cont"], g["cu"], g["lmk_pos"], g["lmk_logw"],
            1.0 / math.sqrt(g["q"].shape[-1]), float(g["tau_win"]), float(g["win_edge"]))


def test_train_bias_matches_reference_golden():
    g = load_golden("train_dense")
    L = int(g["cu"][1])
    for h in range(g["q"].shape[1]):
        for s in range(len(g["cu"]) - 1):
            b, _ = OT.train_bias(g["w_cont"][s * L:(s + 1) * L], g["lmk_pos"][h, s], g["lmk_logw"][h, s],
                                 float(g["tau_win"]), float(g["win_edge"]))
            ref = g["bias"][s, h]
            np.testing.assert_array_equal(np.isinf(b), np.isinf(ref))
            fin = np.isfinite(ref)
            assert np.abs(b[fin] - ref[fin]).max() < 1e-12


def test_train_fwd_bwd_match_reference_golden():
    g = load_golden("train_dense")
    a = _train_args(g)
    o, _ = OT.train_fwd(*a)
    assert rel_err(o, g["out"]) < 1e-12
    dq, dk, dv, dw, dlogw = OT.train_bwd(*a, g["cot"])
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dw, "dw")):
        assert rel_err(got, g[key]) < 1e-10, key
    fin = np.isfinite(g["lmk_logw"])
    assert np.abs(dlogw[fin] - g["dlogw"][fin]).max() < 1e-10
    assert np.all(dlogw[~fin] == 0)
    assert np.abs(dw).max() > 1e-3  # the soft edge carries gradient in this case


def test_train_without_soft_edge_is_the_inference_operator():
    """win_edge 0 puts the whole band in the core: attention over [i - floor(w~), i] plus the
    landmarks left of it, each with its log weight as an additive logit."""
    rng = np.random.default_rng(21)
    lens, H, D, K = (37, 29), 2, 8, 5
    T = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v = (rng.standard_normal((T, H, D)) for _ in range(3))
    w_cont = rng.uniform(0.0, 14.0, T)
    w_cont[::7] = np.floor(w_cont[::7])          # integer windows hit the strict landmark cut
    pos = np.full((H, 2, K), -1)
    for h in range(H):
        for s, L in enumerate(lens):
            pos[h, s, :K - 1] = np.sort(rng.choice(L, K - 1, replace=False))
    logw = np.where(pos >= 0, np.log(rng.uniform(0.05, 1.0, pos.shape)), -np.inf)
    o, lse = OT.train_fwd(q, k, v, w_cont, cu, pos, logw, 0.4, 1.3, 0.0)
    bias = np.where(pos >= 0, logw, 0.0)[:, :, None, :]
    o2, lse2 = OA.attention_fwd(q, k, v, np.floor(w_cont).astype(int) + 1, cu, pos[:, :, None, :], 0.4,
                                lmk_bias=bias)
    assert np.abs(o - o2).max() < 1e-12
    assert np.abs(lse - lse2).max() < 1e-12


def test_train_bwd_matches_finite_differences_in_selectors():
    rng = np.random.default_rng(31)
    lens, H, D, K = (26, 19), 2, 4, 4
    T = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, do = (rng.standard_normal((T, H, D)) for _ in range(4))
    w_cont = rng.uniform(1.0, 12.0, T)
    pos = np.full((H, 2, K), -1)
    for h in range(H):
        for s, L in enumerate(lens):
            pos[h, s, :K - 1] = rng.choice(L, K - 1, replace=False)
    logw = np.where(pos >= 0, np.log(rng.uniform(0.05, 1.0, pos.shape)), -np.inf)
    scale, tau, edge = 0.5, 0.8, 3.0
    _, _, _, dw, dlogw = OT.train_bwd(q, k, v, w_cont, cu, pos, logw, scale, tau, edge, do)

    def loss(w_, lw_):
        o, _ = OT.train_fwd(q, k, v, w_, cu, pos, lw_, scale, tau, edge)
        return float((o * do).sum())

    eps = 1e-6
    for t in range(T):
        wp, wm = w_cont.copy(), w_cont.copy()
        wp[t] += eps
        wm[t] -= eps
        fd = (loss(wp, logw) - loss(wm, logw)) / (2 * eps)
        assert abs(fd - dw[t]) < 1e-6 + 1e-5 * abs(fd), t
    for ix in zip(*np.nonzero(pos >= 0)):
        lp, lm = logw.copy(), logw.copy()
        lp[ix] += eps
        lm[ix] -= eps
        fd = (loss(w_cont, lp) - loss(w_cont, lm)) / (2 * eps)
        assert abs(fd - dlogw[ix]) < 1e-6 + 1e-5 * abs(fd), ix


def test_cpu_baseline_training_bias_rows_match_oracle():
    from oracle.sdpa_cpu import train_bias_rows
    rng = np.random.default_rng(61)
    lens, H, K = (50, 41), 3, 5
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    w = torch.tensor(rng.uniform(0.0, 20.0, T))
    w[::5] = w[::5].floor()
    pos = torch.full((H, 2, K), -1, dtype=torch.int64)
    for h in range(H):
        for s, L in enumerate(lens):
            pos[h, s, :K - 1] = torch.tensor(rng.choice(L, K - 1, replace=False))
    logw = torch.where(pos >= 0, torch.tensor(np.log(rng.uniform(0.05, 1, pos.shape))),
                       torch.tensor(float("-inf"), dtype=torch.float64))
    rows = torch.arange(30, T)
    b = train_bias_rows(w, cu, pos, logw, rows, 1.3, 4.0).numpy()
    for h in range(H):
        for s, L in enumerate(lens):
            st = int(cu[s])
            ref, _ = OT.train_bias(w[st:st + L].numpy(), pos[h, s].numpy(), logw[h, s].numpy(), 1.3, 4.0)
            full = np.full((L, T), -np.inf)
            full[:, st:st + L] = ref
            sel = (rows >= st) & (rows < st + L)
            got = b[h][sel.numpy()]
            want = full[(rows[sel] - st).numpy()]
            np.testing.assert_array_equal(np.isinf(got), np.isinf(want))
            fin = np.isfinite(want)
            assert np.abs(got[fin] - want[fin]).max() < 1e-12


@pytest.mark.parametrize("dt,name", [(torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")])
def test_rope_matches_reference_expression(dt, name):
    from dsalt_amd.kernels.window_utils import apply_rotary_emb, build_rope_cache
    g = torch.Generator().manual_seed(70)
    lens = [37, 64, 5]
    T, H, D = sum(lens), 3, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cos, sin = build_rope_cache(80, D, torch.device("cpu"), base=1e6)
    x = (torch.randn(T, H, D, generator=g) * 3).to(dt)
    pos = torch.cat([torch.arange(n) for n in lens])
    ref, _ = apply_rotary_emb(x, x, cos[pos].to(dt).unsqueeze(1), sin[pos].to(dt).unsqueeze(1))
    got = OR.rope(x.float().numpy(), cu, cos.numpy(), sin.numpy(), name)
    np.testing.assert_array_equal(got, ref.float().numpy())
    if name == "f32":  # a rotation keeps the length of every (x_j, x_j+D/2) pair
        n0 = x[..., :32] ** 2 + x[..., 32:] ** 2
        n1 = torch.tensor(got[..., :32] ** 2 + got[..., 32:] ** 2)
        assert torch.allclose(n0, n1, rtol=1e-5)


@pytest.mark.parametrize("block", [None, 16])
def test_attention_probs_reproduce_forward(block):
    q, k, v, w, cu, idx = _attn_case(41, lens=(40, 27), H=2, G=1, K=5)
    if block:
        idx = np.repeat(idx, 3, axis=2)
        idx[:, :, 0] = -1  # the first block sees no landmark
    bias = np.random.default_rng(42).standard_normal(idx.shape)
    o, _ = OA.attention_fwd(q, k, v, w, cu, idx, 0.37, lmk_bias=bias, block_size=block)
    m = OA.dense_mask_kernel(w, cu, idx, block_size=block)
    for s in range(2):
        st, en = cu[s], cu[s + 1]
        P = OA.attention_probs(q, k, w, cu, idx, 0.37, seq=s, lmk_bias=bias, block_size=block)
        np.testing.assert_allclose(P.sum(-1), 1.0, atol=1e-12)
        assert np.all(P[~m[:, st:en, st:en]] == 0)
        got = np.einsum("hij,jhd->ihd", P, v[st:en, :1].repeat(2, axis=1))
        np.testing.assert_allclose(got, o[st:en], atol=1e-12)


def _ce_torch(x, t, w, ii, ls, red, softcap=None, zs=0.0, scaling=False):
    xt = torch.tensor(x, requires_grad=True)
    xc = softcap * torch.tanh(xt / softcap) if softcap is not None else xt
    wt = torch.tensor(w) if w is not None else None
    rows = torch.nn.functional.cross_entropy(xc, torch.tensor(t), weight=wt, ignore_index=ii, reduction="none",
                                             label_smoothing=ls)
    keep = torch.tensor(t) != ii
    lse = torch.logsumexp(xc, -1)
    z = zs * lse ** 2 * keep
    denom_l = (wt[torch.tensor(t)[keep]].sum() if wt is not None else keep.sum()).double()
    if red == "mean":
        rows, z = rows / denom_l, z / keep.sum()
    if scaling:
        p = torch.softmax(xc, -1).gather(1, torch.tensor(t).clamp(min=0)[:, None])[:, 0].detach() * keep
        rows, z = rows * p, z * p
    tot = rows + z
    (tot.sum() if red != "none" else tot.sum()).backward()
    return tot.detach().numpy(), xt.grad.numpy()


@pytest.mark.parametrize("cw,ls,red,softcap,zs,scaling", [
    (False, 0.0, "mean", None, 0.0, False), (True, 0.0, "mean", None, 0.0, False),
    (False, 0.1, "mean", None, 0.0, False), (True, 0.2, "sum", None, 0.0, False),
    (False, 0.0, "none", None, 0.0, False), (False, 0.0, "mean", 7.0, 0.0, False),
    (True, 0.1, "mean", None, 1e-3, False), (False, 0.1, "mean", 5.0, 1e-2, True)])
def test_ce_rows_match_torch(cw, ls, red, softcap, zs, scaling):
    rng = np.random.default_rng(80)
    N, V = 40, 97
    x = rng.standard_normal((N, V)) * 3
    t = rng.integers(0, V, N)
    t[::5] = -100
    w = rng.uniform(0.2, 2.0, V) if cw else None
    loss, z, g, am, _ = OCE.ce_rows(x, t, w, -100, zs, ls, red, softcap, scaling)
    ref_l, ref_g = _ce_torch(x, t, w, -100, ls, red, softcap, zs, scaling)
    np.testing.assert_allclose(loss, ref_l, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(g, ref_g, rtol=1e-9, atol=1e-13)
    keep = t != -100
    xs = softcap * np.tanh(x / softcap) if softcap else x
    assert np.all(am[keep] == xs[keep].argmax(1)) and np.all(am[~keep] == -1)


# ---------------------------------------------------------------- bf16 selection pin
# The reference's own bf16 path (bf16 norms, float32 statistics over the packed batch,
# torch.topk) on workload-like shapes (tests/golden/select_bf16_*.npz): the oracle's canonical
# arithmetic must choose a top-k of the reference's scores in every set.  Where the sets
# differ, the differing tokens tie with the k-th score (bf16 norms collide often; torch.topk
# breaks ties in its own order, the library by the lower index).
@pytest.mark.parametrize("name", ["b4_h8", "h16"])
def test_oracle_bf16_selection_is_a_top_k_of_the_reference_scores(name):
    from tests.helpers import BF16_SELECT_SPECS, bf16_select_inputs, sha256_of, topk_violations
    z = load_golden(f"select_bf16_{name}")
    x, alpha, _, cu = bf16_select_inputs(name)
    assert sha256_of(x) == str(z["x_sha256"]), "input recipe no longer reproduces the fixture's bits"
    w = torch.from_numpy(z["w"])
    _, _, H, dh, _, k, _, _ = BF16_SELECT_SPECS[name]
    T = x.shape[0]
    v = x[:, :H * dh].reshape(T, H, dh)
    ridx = OS.select(bits(x), bits(v), alpha.numpy(), w.int().numpy(), cu.numpy(), k, OS.DTYPE_BF16,
                     stats_scope=OS.STATS_PACKED)[:, :, 0]
    bad, _ = topk_violations(ridx, z["scores"], w, cu, k)
    assert bad == 0
    sc = z["scores"]
    cun = cu.numpy()
    for hh in range(H):
        for s in range(len(cun) - 1):
            a, b = set(ridx[hh, s][ridx[hh, s] >= 0]), set(z["idx"][hh, s][z["idx"][hh, s] >= 0])
            if a == b:
                continue
            st = int(cun[s])
            kth = min(sc[st + j, hh] for j in b)
            assert all(sc[st + j, hh] == kth for j in a ^ b), (hh, s)


@pytest.mark.parametrize("rb", [64, 512])
def test_train_banded_matches_dense(rb):
    """The banded training oracle (full-length workloads) against the dense one."""
    g = np.random.default_rng(91)
    lens = [300, 181, 64]
    T, H, D, K = sum(lens), 3, 16, 12
    q, k, v, do = (g.standard_normal((T, H, D)) for _ in range(4))
    w_cont = g.uniform(0.0, 90.0, T)
    w_cont[::7] = np.floor(w_cont[::7])  # integer windows: the band end and the landmark cut at d = w~
    cu = np.array([0] + list(np.cumsum(lens)), np.int64)
    pos = np.full((H, len(lens), K), -1, np.int64)
    for h in range(H):
        for s, L in enumerate(lens):
            n = min(K - (h % 2), L)
            pos[h, s, :n] = np.sort(g.permutation(L)[:n])
    logw = np.where(pos >= 0, np.log(1.0 / (1.0 + np.exp(-g.standard_normal(pos.shape)))), -np.inf)
    for tau, edge in ((1.0, 4.0), (2.0, 120.0)):
        a = (q, k, v, w_cont, cu, pos, logw, 0.25, tau, edge)
        o1, l1 = OT.train_fwd(*a)
        o2, l2 = OT.train_fwd_banded(*a, rb=rb)
        np.testing.assert_allclose(o2, o1, rtol=0, atol=1e-12)
        np.testing.assert_allclose(l2, l1, rtol=0, atol=1e-12)
        for x, y in zip(OT.train_bwd_banded(*a, do, rb=rb), OT.train_bwd(*a, do)):
            np.testing.assert_allclose(x, y, rtol=0, atol=1e-11)

"""A seeded sweep of random operator configurations on the GPU against the oracle.

Each case draws a packed batch of ragged sequences (empty and one-token sequences included),
grouped key/value heads read in place, head_dim 64 or 128, fp32 / bf16 / fp16, global or
block-causal selection (block sizes that are and are not multiples of 64), landmark counts from
none to more than the sequences hold, landmark biases, and a tiling variant (bits the shape does
not compile are ignored by the library).  Landmark indices must be bit-exact; outputs relative
max|a-b| / max|b| within 1e-5 (fp32) or 2e-2 (16-bit); log-sum-exps within 1e-4 / 2e-2; the
gradients of global sets through the landmark-row / other-row class and per-row bounds of the
other gradient tests.  A second sweep draws configurations of the training operator (soft window
edge, landmark log-weights, continuous windows up to past the sequence ends) and checks them
as tests/test_gpu_train.py does; a third draws selection-only configurations (indices, z and
scores bit-exact), a fourth the autograd operator over head_dims 16-128, and two more the
probability export (against the oracle's dense matrix), plan reuse (bit for bit) and the landmark
gather (exact), over given landmark sets of any block size.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from oracle import attention as OA
from oracle import select as OS
from tests.helpers import bits, check_grads, f64, oracle_dtype, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
LSE_TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}
N_CASES = 24
SET_SLOTS = 2048  # landmark slots the forward stages for one 64-row tile, over all its sets


def draw(seed: int) -> dict:
    """Configuration of case `seed` (numpy's generator, so the draw is fixed across platforms)."""
    r = np.random.default_rng(10_000 + seed)
    S = int(r.integers(1, 5))
    lens = []
    for _ in range(S):
        u = r.random()
        lens.append(0 if u < 0.12 else 1 if u < 0.2 else int(r.integers(2, 700)))
    if max(lens) < 2:  # a batch of one-token sequences only has dq = dk = 0 (test_gpu_edges covers it)
        lens[0] = int(r.integers(64, 400))
    G = int(r.choice([1, 2, 4]))
    H = G * int(r.choice([1, 2, 4]))
    D = int(r.choice([64, 128]))
    dt = [torch.float32, torch.bfloat16, torch.float16][int(r.choice(3, p=[0.3, 0.5, 0.2]))]
    block = r.random() < 0.4
    bs = int(r.choice([17, 50, 64, 100, 128, 256, 512])) if block else 64
    u = r.random()
    K = 0 if u < 0.1 else int(r.integers(1, 64)) if u < 0.45 else int(r.integers(64, 513)) if u < 0.9 \
        else int(r.integers(513, 1200))
    if block:  # a 64-row tile stages every set it spans
        K = min(K, SET_SLOTS // (1 if bs % 64 == 0 else 63 // bs + 2))
    wmax = int(r.integers(1, 700))
    bias = bool(r.random() < 0.3)
    if D == 64:
        variant = int(r.choice([0, 1, 2, 3])) | int(r.choice([0, 4])) | int(r.choice([0, 8]))
    else:
        variant = int(r.choice([0, 2, 16, 32])) | int(r.choice([0, 8]))
    backward = not block and bool(r.random() < 0.7)
    return dict(lens=lens, H=H, G=G, D=D, dt=dt, mode=ops.SELECT_BLOCK if block else ops.SELECT_GLOBAL,
                block=bs, K=K, wmax=wmax, bias=bias, variant=variant, backward=backward, seed=seed)


def inputs(c: dict, hidden: int = 96) -> dict:
    g = torch.Generator().manual_seed(20_000 + c["seed"])
    T, H, G, D, dt = sum(c["lens"]), c["H"], c["G"], c["D"], c["dt"]
    return {"q": torch.randn(T, H, D, generator=g).to(dt), "k": torch.randn(T, G, D, generator=g).to(dt),
            "v": torch.randn(T, G, D, generator=g).to(dt), "h": torch.randn(T, hidden, generator=g).to(dt),
            "w": torch.randint(1, c["wmax"] + 1, (T,), generator=g, dtype=torch.int32),
            "do": torch.randn(T, H, D, generator=g).to(dt),
            "cu": torch.tensor([0] + list(np.cumsum(c["lens"])), dtype=torch.int32),
            "alpha": torch.rand(H, generator=g)}


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_configuration(seed):
    c = draw(seed)
    print("case", {k: (str(v) if k == "dt" else v) for k, v in c.items()}, flush=True)
    x = inputs(c)
    dt, K, mode, bs = c["dt"], c["K"], c["mode"], c["block"]
    maxlen = max(1, max(c["lens"]))
    d = {k: v.to(DEV) for k, v in x.items()}
    idx = ops.select_landmarks(d["h"], d["v"], d["alpha"], d["w"], d["cu"], K, max_seqlen=maxlen, select_mode=mode,
                               block_size=bs, stats_scope=ops.STATS_SEQUENCE)
    ridx = OS.select(bits(x["h"]), bits(x["v"]), x["alpha"].numpy(), x["w"].numpy(), x["cu"].numpy(), K,
                     oracle_dtype(dt), mode=mode, block_size=bs, stats_scope=OS.STATS_SEQUENCE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    bias = None
    if c["bias"] and K > 0:
        bias = torch.randn(idx.shape, generator=torch.Generator().manual_seed(30_000 + seed)) * 0.5
    scale = 1.0 / math.sqrt(c["D"])
    out, lse = ops.attention_forward(d["q"], d["k"], d["v"], d["w"], d["cu"], idx,
                                     None if bias is None else bias.to(DEV), scale=scale, max_seqlen=maxlen,
                                     select_mode=mode, block_size=bs, variant=c["variant"])
    torch.cuda.synchronize()
    ro, rl = OA.attention_fwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(), ridx, scale,
                              lmk_bias=None if bias is None else bias.double().numpy(),
                              block_size=bs if mode == ops.SELECT_BLOCK else None)
    assert rel_err(f64(out), ro) < TOL[dt], "out"
    fin = np.isfinite(rl)
    assert np.all(np.isfinite(lse.cpu().numpy()[fin]))
    assert np.abs(f64(lse)[fin] - rl[fin]).max(initial=0.0) < LSE_TOL[dt], "lse"
    if not c["backward"]:
        return
    dq, dk, dv, db = ops.attention_backward(d["do"], d["q"], d["k"], d["v"], out, lse, d["w"], d["cu"], idx,
                                            None if bias is None else bias.to(DEV), scale=scale, max_seqlen=maxlen,
                                            want_dbias=bias is not None, variant=c["variant"])
    torch.cuda.synchronize()
    rdq, rdk, rdv, rdb = OA.attention_bwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(),
                                          ridx, scale, f64(x["do"]),
                                          lmk_bias=None if bias is None else bias.double().numpy(), out=f64(out))
    check_grads(("sweep", seed), (dq, dk, dv), (rdq, rdk, rdv), ridx, x["cu"], TOL[dt])
    if bias is not None:
        assert rel_err(db.cpu().double().numpy(), rdb) < TOL[dt], "d_bias"


def draw_train(seed: int) -> dict:
    """Training-operator configuration of case `seed` (global sets, one sequence of at least 16
    tokens, so no head's gradients are all the exact zeros of one-token sequences)."""
    r = np.random.default_rng(50_000 + seed)
    S = int(r.integers(1, 4))
    lens = [0 if r.random() < 0.1 else 1 if r.random() < 0.1 else int(r.integers(2, 600)) for _ in range(S)]
    lens[0] = max(lens[0], 16)
    D = int(r.choice([64, 128]))
    dt = [torch.float32, torch.bfloat16, torch.float16][int(r.choice(3, p=[0.3, 0.5, 0.2]))]
    wlo = float(r.uniform(0.3, 50))
    cfg = dict(lens=lens, H=int(r.integers(1, 7)), D=D, dt=dt, K=0 if r.random() < 0.08 else int(r.integers(1, 513)),
               wlo=wlo, whi=float(wlo + r.uniform(0.5, 650)), tau=float(r.uniform(0.3, 2.0)),
               edge=float(r.choice([0.5, 1.0, 4.0, 6.0, 10.0])), integer_every=int(r.choice([0, 3, 5])))
    cfg["variant"] = (int(r.choice([0, 1, 2, 3])) | int(r.choice([0, 4])) | int(r.choice([0, 8]))) if D == 64 else 0
    return cfg


@pytest.mark.parametrize("seed", range(16))
def test_random_training_configuration(seed):
    """The training operator (soft window edge, landmark log-weights, continuous windows that
    may pass the sequence ends) against the float64 oracle, as in tests/test_gpu_train.py."""
    from tests import test_gpu_train as TT
    c = draw_train(seed)
    print("case", {k: (str(v) if k == "dt" else v) for k, v in c.items()}, flush=True)
    TT._check(c["lens"], c["H"], c["D"], c["K"], c["wlo"], c["whi"], c["dt"], seed=60_000 + seed, tau=c["tau"],
              edge=c["edge"], integer_every=c["integer_every"], variant=c["variant"])


def draw_select(seed: int) -> dict:
    """Selection-only configuration of case `seed`: widths that are not whole 16-byte vectors,
    duplicated rows (exact score ties), heavy-tailed norms, alpha at 0 and 1, both statistics
    scopes, block sizes from 1 row."""
    r = np.random.default_rng(110_000 + seed)
    S = int(r.integers(1, 5))
    lens = [0 if r.random() < 0.1 else 1 if r.random() < 0.1 else int(r.integers(2, 3000)) for _ in range(S)]
    lens[0] = max(lens[0], 2)
    G = int(r.choice([1, 2, 4, 8]))
    return dict(lens=lens, G=G, H=G * int(r.choice([1, 2, 3])), D=int(r.choice([32, 64, 80, 128])),
                hidden=int(r.choice([64, 96, 100, 256, 1000, 2048])),
                dt=[torch.float32, torch.bfloat16, torch.float16][int(r.choice(3, p=[0.3, 0.5, 0.2]))],
                mode=int(r.random() < 0.5), bs=int(r.choice([1, 17, 37, 64, 100, 128, 256, 512, 1024])),
                K=int(r.choice([int(r.integers(1, 64)), int(r.integers(64, 600)), int(r.integers(600, 2049))],
                               p=[0.45, 0.4, 0.15])),
                wmax=int(r.integers(1, 1500)), scope=int(r.integers(0, 2)), ties=bool(r.random() < 0.3),
                heavy=bool(r.random() < 0.3), alphas=r.random(8))


@pytest.mark.parametrize("seed", range(16))
def test_random_selection_configuration(seed):
    """Landmark indices (and, for global sets, z and scores) bit-exact with the oracle."""
    c = draw_select(seed)
    print("case", {k: (str(v) if k in ("dt", "alphas") else v) for k, v in c.items()}, flush=True)
    g = torch.Generator().manual_seed(111_000 + seed)
    T, G, H = sum(c["lens"]), c["G"], c["H"]
    h = torch.randn(T, c["hidden"], generator=g)
    v = torch.randn(T, G, c["D"], generator=g)
    if c["heavy"]:
        h = h * torch.exp(0.5 * torch.randn(T, 1, generator=g))
        v = v * torch.exp(torch.randn(T, G, 1, generator=g))
    if c["ties"]:
        src, dst = torch.randint(0, T, (T // 4,), generator=g), torch.randint(0, T, (T // 4,), generator=g)
        h[dst], v[dst] = h[src], v[src]
    h, v = h.to(c["dt"]), v.to(c["dt"])
    alpha = torch.rand(H, generator=g)
    for j in range(H):
        u = c["alphas"][j % 8]
        alpha[j] = 0.0 if u < 0.1 else 1.0 if u < 0.2 else alpha[j]
    w = torch.randint(1, c["wmax"] + 1, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(c["lens"])), dtype=torch.int32)
    mode, want = c["mode"], c["mode"] == 0
    res = ops.select_landmarks(*(t.to(DEV) for t in (h, v, alpha, w, cu)), c["K"], max_seqlen=max(c["lens"]),
                               select_mode=mode, block_size=c["bs"], stats_scope=c["scope"], want_scores=want)
    ref = OS.select(bits(h), bits(v), alpha.numpy(), w.numpy(), cu.numpy(), c["K"], oracle_dtype(c["dt"]),
                    mode=mode, block_size=c["bs"], stats_scope=c["scope"], want_scores=want)
    for a, b in zip(res if want else (res,), ref if want else (ref,)):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


@pytest.mark.parametrize("seed", range(12))
def test_random_autograd_operator_configuration(seed):
    """The autograd operator (unsorted caller sets, landmark bias, head_dims 16-128 run
    zero-padded to the compiled 64 / 128): output and the gradients of q, k, v and the bias
    against the oracle."""
    from dsalt_amd import kernels as KK
    r = np.random.default_rng(70_000 + seed)
    g = torch.Generator().manual_seed(71_000 + seed)
    S = int(r.integers(1, 5))
    lens = [0 if r.random() < 0.1 else 1 if r.random() < 0.1 else int(r.integers(2, 600)) for _ in range(S)]
    lens[0] = max(lens[0], 16)
    G = int(r.choice([1, 2, 4]))
    H = G * int(r.choice([1, 2]))
    D = int(r.choice([16, 32, 48, 64, 72, 80, 96, 100, 112, 128]))
    dt = [torch.float32, torch.bfloat16, torch.float16][int(r.choice(3, p=[0.3, 0.5, 0.2]))]
    K = int(r.integers(0, 80))
    wmax = int(r.integers(1, 400))
    print("case", dict(lens=lens, H=H, G=G, D=D, dt=str(dt), K=K, wmax=wmax), flush=True)
    T = sum(lens)
    q, k, v = (torch.randn(T, n, D, generator=g).to(dt) for n in (H, G, G))
    w = torch.randint(1, wmax + 1, (T,), generator=g).float()
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    idx = torch.full((H, S, K), -1, dtype=torch.int64)
    for hh in range(H):
        for s, L in enumerate(lens):
            c = torch.randperm(L, generator=g)[:max(K - int(r.integers(0, 3)), 0)]
            idx[hh, s, :len(c)] = c
    bias = torch.randn(idx.shape, generator=g) * 0.3
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    bd = bias.to(DEV).requires_grad_(True)
    out = KK.dsalt_triton_attention(qd, kd, vd, idx.to(DEV), bd, w.to(DEV), cu.to(DEV))
    do = torch.randn(out.shape, generator=g)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    idx4, b4 = idx.numpy()[:, :, None], bias.double().numpy()[:, :, None]
    wi = w.clamp(min=1).long().numpy()
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale, lmk_bias=b4)
    assert rel_err(f64(out), ro) < TOL[dt], "out"
    rg = OA.attention_bwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale, f64(do.to(dt)), lmk_bias=b4,
                          out=f64(out.to(dt)))
    check_grads(("autograd", seed), (qd.grad, kd.grad, vd.grad), rg[:3], idx, cu, TOL[dt])
    if K:
        assert rel_err(f64(bd.grad), rg[3][:, :, 0]) < TOL[dt], "d_bias"


def random_sets(g: torch.Generator, H: int, lens: list, mode: int, bs: int, K: int) -> torch.Tensor:
    """[H, S, n_sets, K] int32 landmark sets: each set up to K distinct positions of its sequence
    (block-causal: below the set's first row), ascending, some sets a slot or two short, -1 padded."""
    ns = ops.n_sets(mode, max(max(lens), 1), bs)
    idx = torch.full((H, len(lens), ns, K), -1, dtype=torch.int32)
    for h in range(H):
        for s, L in enumerate(lens):
            for b in range(ns):
                hi = L if mode == ops.SELECT_GLOBAL else min(L, b * bs)
                n = min(max(K - int(torch.randint(0, 3, (1,), generator=g)), 0), hi)
                if n > 0:
                    idx[h, s, b, :n] = torch.randperm(hi, generator=g)[:n].sort().values.to(torch.int32)
    return idx


def draw_api(seed: int) -> dict:
    """Configuration of the operator's other entry points (probability export, plan reuse,
    landmark gather, the allocation-free forward): global or block-causal sets of any block
    size, 0 to 300 landmarks, any tiling variant bits, given landmark sets and biases."""
    r = np.random.default_rng(90_000 + seed)
    S = int(r.integers(1, 5))
    lens = [0 if r.random() < 0.1 else 1 if r.random() < 0.1 else int(r.integers(2, 700)) for _ in range(S)]
    lens[0] = max(lens[0], 16)
    G = int(r.choice([1, 2, 4]))
    mode = seed % 2  # global and block-causal sets alternate
    bs = int(r.choice([17, 64, 100, 128, 256, 512])) if mode else 512
    K = int(r.integers(0, 300))
    if mode and bs % 64:
        K = min(K, SET_SLOTS // (63 // bs + 2))
    return dict(lens=lens, G=G, H=G * int(r.choice([1, 2, 4])), D=int(r.choice([64, 128])),
                dt=[torch.float32, torch.bfloat16, torch.float16][int(r.integers(0, 3))], mode=mode, bs=bs, K=K,
                wmax=int(r.integers(1, 600)), variant=int(r.integers(0, 64)), seed=seed)


def api_inputs(c: dict) -> dict:
    g = torch.Generator().manual_seed(91_000 + c["seed"])
    T, H, G, D, dt = sum(c["lens"]), c["H"], c["G"], c["D"], c["dt"]
    x = {"q": torch.randn(T, H, D, generator=g).to(dt), "k": torch.randn(T, G, D, generator=g).to(dt),
         "v": torch.randn(T, G, D, generator=g).to(dt), "do": torch.randn(T, H, D, generator=g).to(dt),
         "w": torch.randint(1, c["wmax"] + 1, (T,), generator=g, dtype=torch.int32),
         "cu": torch.tensor([0] + list(np.cumsum(c["lens"])), dtype=torch.int32)}
    x["idx"] = random_sets(g, H, c["lens"], c["mode"], c["bs"], c["K"])
    x["bias"] = torch.randn(x["idx"].shape, generator=g) * 0.5
    return x


@pytest.mark.parametrize("seed", range(8))
def test_random_probability_export_configuration(seed):
    """The exported probabilities of every sequence, densified, against the oracle's dense
    attention matrix (relative max|a-b| / max|b|, 1e-5 fp32 / 2e-2 16-bit)."""
    from dsalt_amd.kernels.attention_probs import SparseAttentionProbs
    c = draw_api(seed)
    print("case", {k: (str(v) if k == "dt" else v) for k, v in c.items()}, flush=True)
    x = api_inputs(c)
    mode, bs, maxlen = c["mode"], c["bs"], max(c["lens"])
    scale = 1.0 / math.sqrt(c["D"])
    d = {k: v.to(DEV) for k, v in x.items()}
    _, lse = ops.attention_forward(d["q"], d["k"], d["v"], d["w"], d["cu"], d["idx"], d["bias"], scale=scale,
                                   max_seqlen=maxlen, select_mode=mode, block_size=bs, variant=c["variant"])
    for s, L in enumerate(c["lens"]):
        if L == 0:
            continue
        p_win, p_lmk = ops.export_probs(d["q"], d["k"], d["w"], d["cu"], d["idx"], lse, d["bias"], seq=s, scale=scale,
                                        max_seqlen=maxlen, select_mode=mode, block_size=bs)
        sp = SparseAttentionProbs(p_win, p_lmk, d["idx"][:, s].long() if c["K"] else None, bs if mode else 0)
        ref = OA.attention_probs(f64(x["q"]), f64(x["k"]), x["w"].numpy(), x["cu"].numpy(), x["idx"].numpy(), scale,
                                 seq=s, lmk_bias=x["bias"].double().numpy(), block_size=bs if mode else None)
        assert rel_err(f64(sp.to_dense()), ref) < TOL[c["dt"]], ("sequence", s)


@pytest.mark.parametrize("seed", range(8))
def test_random_plan_and_gather_configuration(seed):
    """A row plan made once and passed in gives the forward (and, for global sets, the backward)
    bit for bit; gathered landmark rows equal the rows at the sets' positions (zero for -1)."""
    c = draw_api(seed)
    print("case", {k: (str(v) if k == "dt" else v) for k, v in c.items()}, flush=True)
    x = api_inputs(c)
    mode, bs, maxlen, var = c["mode"], c["bs"], max(c["lens"]), c["variant"]
    d = {k: v.to(DEV) for k, v in x.items()}
    fa = (d["q"], d["k"], d["v"], d["w"], d["cu"], d["idx"], None)
    out, lse = ops.attention_forward(*fa, max_seqlen=maxlen, select_mode=mode, block_size=bs, variant=var)
    plan = ops.new_plan(d["q"], d["k"], d["cu"], d["idx"], max_seqlen=maxlen, select_mode=mode, block_size=bs)
    o2, l2 = ops.attention_forward(*fa, max_seqlen=maxlen, select_mode=mode, block_size=bs, plan=plan, variant=var)
    assert torch.equal(o2, out) and torch.equal(l2, lse)
    if mode == ops.SELECT_GLOBAL:
        ba = (d["do"], d["q"], d["k"], d["v"], out, lse, d["w"], d["cu"], d["idx"])
        a = ops.attention_backward(*ba, max_seqlen=maxlen, want_dbias=False, variant=var)
        b = ops.attention_backward(*ba, max_seqlen=maxlen, want_dbias=False, plan=plan, variant=var)
        for u, w_ in zip(a[:3], b[:3]):
            assert torch.equal(u, w_)
    lk, lv = ops.gather_landmarks(d["k"], d["v"], d["cu"], d["idx"], max_seqlen=maxlen, select_mode=mode,
                                  block_size=bs, n_heads=c["H"])
    rep = c["H"] // c["G"]
    cu = x["cu"].numpy()
    for name, got, src in (("k", lk, x["k"]), ("v", lv, x["v"])):
        got = got.cpu()
        for h in range(c["H"]):
            for s, L in enumerate(c["lens"]):
                pos = x["idx"][h, s].long()
                ok = (pos >= 0) & (pos < L)
                rows = src[int(cu[s]) + pos.clamp(0, max(L - 1, 0)), h // rep] if L else torch.zeros(
                    pos.shape + (c["D"],), dtype=src.dtype)
                ref = torch.where(ok[..., None], rows, torch.zeros((), dtype=src.dtype))
                assert torch.equal(got[h, s], ref), (name, h, s)

"""Edge cases of the operator on the GPU against the oracle: empty and one-token sequences in a
packed batch (also with block-causal blocks that are not multiples of 64 rows), a batch of
one-token sequences only (whose dq and dk vanish: bounded absolutely), no landmarks,
the largest landmark sets (512 slots and the wide kernels' 2048), every landmark slot empty,
the GQA ratio of the 3B decoder, windows covering whole sequences, and rows more than 2 GiB past
the tensors' base.  Indices bit-exact; outputs and gradients relative max|a-b| / max|b| within 1e-5
(fp32) or 2e-2 (bf16)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from oracle import attention as OA
from oracle import select as OS
from tests.helpers import bits, f64, oracle_dtype, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _case(lens, H, G, D, K, wmax, dt, seed, hidden=128):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    x = {"q": torch.randn(T, H, D, generator=g).to(dt), "k": torch.randn(T, G, D, generator=g).to(dt),
         "v": torch.randn(T, G, D, generator=g).to(dt), "h": torch.randn(T, hidden, generator=g).to(dt),
         "w": torch.randint(1, wmax + 1, (T,), generator=g, dtype=torch.int32),
         "do": torch.randn(T, H, D, generator=g).to(dt),
         "cu": torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32),
         "alpha": torch.rand(H, generator=g)}
    return x


def _run(x, K, mode=ops.SELECT_GLOBAL, block=64, backward=True):
    dt = x["q"].dtype
    H, G = x["q"].shape[1], x["k"].shape[1]
    maxlen = max(1, int((x["cu"][1:] - x["cu"][:-1]).max()))
    d = {k: v.to(DEV) for k, v in x.items()}
    idx = ops.select_landmarks(d["h"], d["v"], d["alpha"], d["w"], d["cu"], K, max_seqlen=maxlen, select_mode=mode,
                               block_size=block, stats_scope=ops.STATS_SEQUENCE)
    ridx = OS.select(bits(x["h"]), bits(x["v"]), x["alpha"].numpy(), x["w"].numpy(), x["cu"].numpy(), K,
                     oracle_dtype(dt), mode=mode, block_size=block, stats_scope=OS.STATS_SEQUENCE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    scale = 1.0 / math.sqrt(x["q"].shape[-1])
    out, lse = ops.attention_forward(d["q"], d["k"], d["v"], d["w"], d["cu"], idx, None, scale=scale,
                                     max_seqlen=maxlen, select_mode=mode, block_size=block)
    bs = block if mode == ops.SELECT_BLOCK else None
    ro, rl = OA.attention_fwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(), ridx, scale,
                              block_size=bs)
    assert rel_err(f64(out), ro) < TOL[dt]
    if not backward:
        return
    kk, vv = d["k"], d["v"]
    if G != H:
        kk, vv = kk.repeat_interleave(H // G, 1), vv.repeat_interleave(H // G, 1)
    dq, dk, dv, _ = ops.attention_backward(d["do"], d["q"], kk, vv, out, lse, d["w"], d["cu"], idx, max_seqlen=maxlen)
    rdq, rdk, rdv, _ = OA.attention_bwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(),
                                        ridx, scale, f64(x["do"]))
    if G != H:
        dk = dk.view(dk.shape[0], G, H // G, -1).float().sum(2)
        dv = dv.view(dv.shape[0], G, H // G, -1).float().sum(2)
    for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert rel_err(f64(a), b) < TOL[dt], name


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_empty_and_single_token_sequences(dt):
    _run(_case([100, 0, 1, 0, 130], 2, 2, 64, 8, 40, dt, seed=200), 8)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_only_one_token_sequences(dt):
    """A batch of one-token and empty sequences only: each query sees its own key alone (P = 1,
    no landmark candidates), so out = v, dv = dO summed over the group's query heads, and dq = dk
    = 0 exactly.  The kernels' dq and dk hold the rounding of dP - delta only: bounded absolutely
    by tol x scale x max|dO . v| x max|k| (a relative bound against the oracle's zeros means
    nothing)."""
    x = _case([1, 1, 0, 1], 4, 2, 64, 8, 30, dt, seed=211)
    d = {k: v.to(DEV) for k, v in x.items()}
    idx = ops.select_landmarks(d["h"], d["v"], d["alpha"], d["w"], d["cu"], 8, max_seqlen=1,
                               stats_scope=ops.STATS_SEQUENCE)
    assert torch.all(idx == -1)
    scale = 1.0 / 8.0
    out, lse = ops.attention_forward(d["q"], d["k"], d["v"], d["w"], d["cu"], idx, None, scale=scale, max_seqlen=1)
    ro, rl = OA.attention_fwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(),
                              idx.cpu().numpy(), scale)
    rep = 2
    assert np.array_equal(ro, np.repeat(f64(x["v"]), rep, axis=1))
    assert rel_err(f64(out), ro) < TOL[dt]
    assert np.abs(f64(lse) - rl).max() < TOL[dt] * np.abs(rl).max()
    dq, dk, dv, _ = ops.attention_backward(d["do"], d["q"], d["k"], d["v"], out, lse, d["w"], d["cu"], idx,
                                           scale=scale, max_seqlen=1, want_dbias=False)
    do, v, k = f64(x["do"]), f64(x["v"]), f64(x["k"])
    rdv = do.reshape(do.shape[0], 2, rep, -1).sum(2)
    assert rel_err(f64(dv), rdv) < TOL[dt]
    dp = np.abs(np.einsum("thd,thd->th", do, np.repeat(v, rep, axis=1))).max()
    bound = TOL[dt] * scale * dp * np.abs(k).max()
    assert np.abs(f64(dq)).max() <= bound and np.abs(f64(dk)).max() <= bound, (np.abs(f64(dq)).max(), bound)


def test_empty_sequences_block_causal():
    _run(_case([0, 300, 0, 1, 70], 2, 2, 64, 8, 40, torch.bfloat16, seed=201), 8, mode=ops.SELECT_BLOCK,
         block=64, backward=False)


def test_empty_sequences_block_causal_any_block_size():
    # blocks of 50 rows: 64-row tiles over two sets, next to empty and one-token sequences
    _run(_case([0, 300, 0, 1, 70], 2, 2, 64, 8, 40, torch.bfloat16, seed=207), 8, mode=ops.SELECT_BLOCK,
         block=50, backward=False)


@pytest.mark.parametrize("D,dt", [(128, torch.bfloat16), (64, torch.float32)])
def test_block_causal_tiles_whose_sets_are_all_empty(D, dt):
    # 17-row blocks: a 64-row tile spans four sets; the first 200 tokens' windows reach the
    # sequence start, so they are never candidates and the first tiles' sets are all empty
    # while later tiles hold landmarks (such tiles once staged a chunk that was never fetched)
    x = _case([400, 60], 4, 2, D, 29, 600, dt, seed=210)
    x["w"][:200] = 600
    _run(x, 29, mode=ops.SELECT_BLOCK, block=17, backward=False)


def test_many_sequences_landmark_sums():
    """64 sequences x 8 heads x 128 slots x head_dim 64: 16384 blocks of landmark partial sums,
    40 % of the slots empty; 512 (head, sequence) pairs in the forward's per-XCD pair order."""
    r = np.random.default_rng(212)
    lens = [int(n) for n in r.integers(40, 400, 64)]
    _run(_case(lens, 8, 8, 64, 128, 300, torch.bfloat16, seed=212), 128)


@pytest.mark.parametrize("D,block", [(128, 50), (64, 64)])
def test_many_sequences_block_causal(D, block):
    """32 sequences x 8 heads (256 (head, sequence) pairs: each XCD walks its pairs' tiles in
    turn), block-causal sets, one of them with tiles over several sets."""
    r = np.random.default_rng(213)
    lens = [int(n) for n in r.integers(40, 500, 32)]
    _run(_case(lens, 8, 8, D, 24, 200, torch.bfloat16, seed=213), 24, mode=ops.SELECT_BLOCK, block=block,
         backward=False)


def test_no_landmarks():
    _run(_case([257, 190], 4, 4, 64, 0, 90, torch.bfloat16, seed=202), 0)


def test_no_landmarks_block_causal_any_block_size():
    _run(_case([257, 190], 4, 4, 64, 0, 90, torch.bfloat16, seed=208), 0, mode=ops.SELECT_BLOCK, block=37,
         backward=False)


def test_largest_landmark_sets():
    _run(_case([1200, 700], 2, 2, 128, 512, 300, torch.bfloat16, seed=203), 512)


def test_largest_landmark_sets_of_the_wide_kernels():
    # 2048 slots: more than the sequences' candidates (every set ends in -1 padding)
    _run(_case([2500, 700], 2, 2, 64, 2048, 300, torch.bfloat16, seed=209), 2048)


def test_gqa_ratio_of_the_3b_decoder():
    _run(_case([640, 333], 16, 2, 128, 32, 200, torch.bfloat16, seed=204), 32)


def test_windows_covering_whole_sequences():
    _run(_case([300, 77], 2, 2, 64, 16, 5000, torch.float32, seed=205), 16)


def test_all_landmark_slots_empty():
    x = _case([200, 130], 2, 2, 64, 8, 30, torch.float32, seed=206)
    d = {k: v.to(DEV) for k, v in x.items()}
    idx = torch.full((2, 2, 1, 8), -1, dtype=torch.int32, device=DEV)
    out, lse = ops.attention_forward(d["q"], d["k"], d["v"], d["w"], d["cu"], idx, None, max_seqlen=200)
    ro, _ = OA.attention_fwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(),
                             idx.cpu().numpy(), 1 / 8.0)
    assert rel_err(f64(out), ro) < 1e-5
    dq, dk, dv, db = ops.attention_backward(d["do"], d["q"], d["k"], d["v"], out, lse, d["w"], d["cu"], idx,
                                            torch.zeros(2, 2, 1, 8, device=DEV), max_seqlen=200)
    assert torch.all(db == 0)
    rdq, _, _, _ = OA.attention_bwd(f64(x["q"]), f64(x["k"]), f64(x["v"]), x["w"].numpy(), x["cu"].numpy(),
                                    idx.cpu().numpy(), 1 / 8.0, f64(x["do"]))
    assert rel_err(f64(dq), rdq) < 1e-5


def test_rows_past_2gib_offsets():
    """A packed batch whose second sequence starts 600000 tokens in (its q, k, v rows 2.3 GiB
    past the tensors' base) against the same sequence alone: indices, outputs, LSE and dQ
    bit-identical, dK / dV bit-identical on every row that is no landmark; landmark rows sum
    their fp32 row-chunk partials over as many chunks as the longest sequence needs, so
    they may differ in the last bits (within 2e-3).  The block-causal forward likewise."""
    H, D, dt, L1, L2, K = 16, 128, torch.bfloat16, 600_000, 2048, 64
    g = torch.Generator(device=DEV).manual_seed(5)
    T = L1 + L2

    def rnd(*s):
        return torch.randn(*s, generator=g, device=DEV).to(dt)

    q, k, v, do, h = rnd(T, H, D), rnd(T, H, D), rnd(T, H, D), rnd(T, H, D), rnd(T, 256)
    w = torch.randint(1, 257, (T,), generator=g, device=DEV, dtype=torch.int32)
    alpha = torch.rand(H, generator=g, device=DEV)
    cu = torch.tensor([0, L1, T], dtype=torch.int32, device=DEV)
    cu2 = torch.tensor([0, L2], dtype=torch.int32, device=DEV)
    assert L1 * H * D * q.element_size() > 2 ** 31

    def run(sl, cu_, maxlen, mode):
        idx = ops.select_landmarks(h[sl], v[sl], alpha, w[sl], cu_, K, max_seqlen=maxlen, select_mode=mode,
                                   block_size=512, stats_scope=ops.STATS_SEQUENCE)
        out, lse = ops.attention_forward(q[sl], k[sl], v[sl], w[sl], cu_, idx, None, max_seqlen=maxlen,
                                         select_mode=mode, block_size=512)
        if mode == ops.SELECT_BLOCK:
            return idx, out, lse
        return (idx, out, lse) + ops.attention_backward(do[sl], q[sl], k[sl], v[sl], out, lse, w[sl], cu_, idx,
                                                        max_seqlen=maxlen, want_dbias=False)[:3]

    for mode in (ops.SELECT_GLOBAL, ops.SELECT_BLOCK):
        a = run(slice(0, T), cu, L1, mode)
        b = run(slice(L1, T), cu2, L2, mode)
        torch.cuda.synchronize()
        assert torch.equal(a[0][:, 1, :b[0].shape[2]], b[0][:, 0]), "indices"
        for name, x, y in zip(("out", "lse", "dq"), a[1:4], b[1:4]):
            assert torch.equal(x[L1:], y), name
        if mode == ops.SELECT_BLOCK:
            continue
        lm = torch.zeros(L2, dtype=torch.bool, device=DEV)
        ix = b[0][:, 0].reshape(-1)
        lm[ix[ix >= 0].long()] = True
        for name, x, y in (("dk", a[4][L1:], b[4]), ("dv", a[5][L1:], b[5])):
            assert torch.equal(x[~lm], y[~lm]), name
            assert float((x[lm].float() - y[lm].float()).abs().max() / y.float().abs().max()) < 2e-3, name

"""Attention forward/backward on the GPU against the float64 oracle.

Tolerances (relative, max|a-b| / max|b|): 1e-5 for fp32, 2e-2 for bf16 and fp16.  Gradients
of q, k and v are held to them per head by ``tests.helpers.check_grads``: landmark rows and
the other rows each against their own largest entry, and every row above a quarter of its
class's median norm against its own norm.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from oracle import attention as OA
from tests.helpers import check_grads, f64, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _inputs(lens, H, G, D, K, wmax, dt, seed, mode=ops.SELECT_GLOBAL, block=128, bias=False):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(dt)
    k = torch.randn(T, G, D, generator=g).to(dt)
    v = torch.randn(T, G, D, generator=g).to(dt)
    w = torch.randint(1, wmax + 1, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    maxlen = max(lens)
    ns = ops.n_sets(mode, maxlen, block)
    idx = torch.full((H, len(lens), ns, K), -1, dtype=torch.int32)
    for hh in range(H):
        for s, L in enumerate(lens):
            for b in range(ns):
                hi = L if mode == ops.SELECT_GLOBAL else min(L, b * block)
                if hi <= 0:
                    continue
                n = min(K - (hh % 2), hi)  # leave some -1 padding
                c = torch.randperm(hi, generator=g)[:n].sort().values
                idx[hh, s, b, :n] = c.to(torch.int32)
    lb = torch.randn(idx.shape, generator=g) * 0.5 if bias else None
    return q, k, v, w, cu, idx, lb, maxlen


def _fwd_check(q, k, v, w, cu, idx, lb, maxlen, mode=ops.SELECT_GLOBAL, block=128):
    dt = q.dtype
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    out, lse = ops.attention_forward(*(t.to(DEV) for t in (q, k, v, w, cu, idx)),
                                     lb.to(DEV) if lb is not None else None, scale=scale, max_seqlen=maxlen,
                                     select_mode=mode, block_size=block)
    torch.cuda.synchronize()
    ro, rl = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale,
                              lmk_bias=None if lb is None else lb.double().numpy(),
                              block_size=None if mode == ops.SELECT_GLOBAL else block)
    e_o = rel_err(f64(out), ro)
    e_l = rel_err(f64(lse), rl)
    assert e_o < TOL[dt], e_o
    assert e_l < (1e-6 if dt == torch.float32 else 2e-3), e_l
    return out, lse


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_fwd_global(dt, D):
    args = _inputs([300, 181, 64], 4, 4, D, 24, 90, dt, seed=D)
    _fwd_check(*args)


def test_fwd_bias_gqa_ragged():
    args = _inputs([257, 130], 8, 2, 64, 40, 70, torch.bfloat16, seed=5, bias=True)
    _fwd_check(*args)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_fwd_block_causal(dt):
    q, k, v, w, cu, idx, lb, maxlen = _inputs([700, 512], 4, 4, 128, 32, 150, dt, seed=6,
                                              mode=ops.SELECT_BLOCK, block=128)
    _fwd_check(q, k, v, w, cu, idx, lb, maxlen, mode=ops.SELECT_BLOCK, block=128)


@pytest.mark.parametrize("dt,D,block,K", [(torch.bfloat16, 64, 100, 32), (torch.bfloat16, 128, 200, 48),
                                          (torch.float32, 64, 48, 40), (torch.float16, 64, 30, 16),
                                          (torch.float32, 128, 7, 24), (torch.bfloat16, 64, 1, 8)])
def test_fwd_block_causal_any_block_size(dt, D, block, K):
    """Block sizes that are not multiples of 64: the rows of a 64-row tile belong to up to
    ceil(63 / block) + 1 sets, staged together (GQA, landmark bias, ragged sequences)."""
    q, k, v, w, cu, idx, lb, maxlen = _inputs([520, 333], 4, 2, D, K, 150, dt, seed=block + D,
                                              mode=ops.SELECT_BLOCK, block=block, bias=True)
    _fwd_check(q, k, v, w, cu, idx, lb, maxlen, mode=ops.SELECT_BLOCK, block=block)


def test_fwd_special_cases():
    T, H, D = 200, 2, 64
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(T, H, D, generator=g).to(torch.float32) for _ in range(3))
    cu = torch.tensor([0, T], dtype=torch.int32)
    idx = torch.full((H, 1, 1, 8), -1, dtype=torch.int32)
    out, _ = ops.attention_forward(q.to(DEV), k.to(DEV), v.to(DEV), torch.ones(T, dtype=torch.int32, device=DEV),
                                   cu.to(DEV), idx.to(DEV), max_seqlen=T)
    assert rel_err(f64(out), f64(v)) < 1e-6  # w = 1, no landmarks: O = V
    out, _ = ops.attention_forward(q.to(DEV), k.to(DEV), v.to(DEV), torch.full((T,), T, dtype=torch.int32,
                                   device=DEV), cu.to(DEV), idx.to(DEV), max_seqlen=T)
    ref = torch.nn.functional.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1),
                                                           v.transpose(0, 1), is_causal=True).transpose(0, 1)
    assert rel_err(f64(out), f64(ref)) < 1e-5  # full windows, no landmarks: causal attention


def _bwd_check(dt, lens, H, D, K, wmax, seed, bias=False):
    q, k, v, w, cu, idx, lb, maxlen = _inputs(lens, H, H, D, K, wmax, dt, seed, bias=bias)
    scale = 1.0 / math.sqrt(D)
    g = torch.Generator().manual_seed(seed + 100)
    do = torch.randn(q.shape, generator=g).to(dt)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx)]
    lbd = lb.to(DEV) if lb is not None else None
    out, lse = ops.attention_forward(*dev, lbd, scale=scale, max_seqlen=maxlen)
    dq, dk, dv, db = ops.attention_backward(do.to(DEV), dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5],
                                            lbd, scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    rdq, rdk, rdv, rdb = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale,
                                          f64(do), lmk_bias=None if lb is None else lb.double().numpy(),
                                          out=f64(out))
    check_grads("bwd", (dq, dk, dv), (rdq, rdk, rdv), idx, cu, TOL[dt])
    assert rel_err(f64(db), rdb) < TOL[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
def test_bwd_global(dt):
    _bwd_check(dt, [300, 181, 64], 4, 64, 24, 90, seed=11)


def test_bwd_bias_d128():
    _bwd_check(torch.bfloat16, [333, 200], 2, 128, 40, 120, seed=12, bias=True)


def test_bwd_deterministic():
    q, k, v, w, cu, idx, lb, maxlen = _inputs([1024], 4, 4, 64, 64, 200, torch.bfloat16, seed=13)
    do = torch.randn(q.shape).to(torch.bfloat16)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx)]
    out, lse = ops.attention_forward(*dev, None, max_seqlen=maxlen)
    r1 = ops.attention_backward(do.to(DEV), dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5],
                                max_seqlen=maxlen)
    r2 = ops.attention_backward(do.to(DEV), dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5],
                                max_seqlen=maxlen)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_bwd_long_windows(dt):
    # windows up to the whole sequence: the key-parallel sweep takes the rows after
    # each key block in several compacted segments
    _bwd_check(dt, [2300, 700], 2, 64, 16, 2300, seed=14)


def test_bwd_long_windows_d128():
    _bwd_check(torch.bfloat16, [1500, 90], 2, 128, 8, 1500, seed=15, bias=True)


@pytest.mark.parametrize("T", [2000, 2100])
def test_landmark_rows_far_apart_in_memory(T):
    """K and V rows 1 MiB apart (strided views of wide buffers; the largest token stride
    the boundary accepts): 2000 rows span just under 2 GiB, so landmark rows are reached
    through 32-bit offsets close to their limit; 2100 rows span more and take 64-bit row
    addresses.  Forward and backward must equal the
    contiguous layout bit for bit."""
    H, D, K = 2, 64, 32
    dt = torch.bfloat16
    q, k, v, w, cu, idx, _, maxlen = _inputs([T], H, H, D, K, 300, dt, seed=31)
    g = torch.Generator().manual_seed(32)
    dout = torch.randn(T, H, D, generator=g).to(dt)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, dout)]
    q_d, k_d, v_d, w_d, cu_d, idx_d, do_d = dev
    row = 1 << 19  # elements per row of the wide buffers (1 MiB in bf16)
    kw = torch.zeros(T, row, dtype=dt, device=DEV)
    vw = torch.zeros(T, row, dtype=dt, device=DEV)
    k_s = kw[:, :H * D].view(T, H, D)
    v_s = vw[:, :H * D].view(T, H, D)
    k_s.copy_(k_d)
    v_s.copy_(v_d)
    assert k_s.stride(0) == row and ((T - 1) * row * 2 < 2 ** 31) == (T == 2000)
    res = []
    for kk, vv in ((k_d, v_d), (k_s, v_s)):
        out, lse = ops.attention_forward(q_d, kk, vv, w_d, cu_d, idx_d, None, max_seqlen=maxlen)
        dq, dk, dv, _ = ops.attention_backward(do_d, q_d, kk, vv, out, lse, w_d, cu_d, idx_d, None,
                                               max_seqlen=maxlen, want_dbias=False)
        torch.cuda.synchronize()
        res.append([t.cpu() for t in (out, lse, dq, dk, dv)])
    del kw, vw, k_s, v_s
    torch.cuda.empty_cache()
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), *res):
        assert torch.equal(a, b), name
    # and the contiguous result is the operator's (oracle at the bf16 tolerance)
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), 1.0 / math.sqrt(D))
    assert rel_err(f64(res[0][0]), ro) < TOL[dt]


# ------------------------------------------------ grouped heads, plan reuse, repeats
def _bwd_gqa_case(H, G, D, dt, seed, lens=(700, 333), K=32, wmax=260):
    q, k, v, w, cu, idx, lb, maxlen = _inputs(list(lens), H, G, D, K, wmax, dt, seed, bias=True)
    g = torch.Generator().manual_seed(seed + 7)
    do = torch.randn(q.shape, generator=g).to(dt)
    return q, k, v, w, cu, idx, lb, maxlen, do


@pytest.mark.parametrize("H,G,D,dt", [(16, 2, 64, torch.bfloat16), (8, 2, 128, torch.bfloat16),
                                      (8, 2, 64, torch.float32), (6, 3, 64, torch.float16)])
def test_bwd_grouped_heads_native(H, G, D, dt):
    """dK/dV of each key/value head sum its query heads inside the kernels (no repeat)."""
    q, k, v, w, cu, idx, lb, maxlen, do = _bwd_gqa_case(H, G, D, dt, seed=40 + H + D)
    scale = 1.0 / math.sqrt(D)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, lb, do)]
    out, lse = ops.attention_forward(*dev[:6], dev[6], scale=scale, max_seqlen=maxlen)
    res = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                 scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    assert res[1].shape == (q.shape[0], G, D) and res[2].shape == (q.shape[0], G, D)
    ref = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do),
                           lmk_bias=lb.double().numpy(), out=f64(out))
    check_grads("gqa", res[:3], ref[:3], idx, cu, TOL[dt])
    assert rel_err(f64(res[3]), ref[3]) < TOL[dt]
    res2 = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                  scale=scale, max_seqlen=maxlen)
    for a, b in zip(res, res2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("H,G,D,dt,K", [(4, 2, 64, torch.bfloat16, 1000), (4, 2, 64, torch.bfloat16, 2048),
                                        (4, 4, 128, torch.float32, 600), (4, 2, 128, torch.float16, 1500)])
def test_large_landmark_sets(H, G, D, dt, K):
    """Sets of more than 512 landmarks (up to 2048): the wide instantiations of the forward,
    the dQ pass and the landmark backward; GQA, landmark bias, a sequence with fewer
    candidates than slots (-1 padding).  Forward against the oracle, every gradient through
    the class and row bounds, bit-identical rerun."""
    q, k, v, w, cu, idx, lb, maxlen, do = _bwd_gqa_case(H, G, D, dt, seed=K + D, lens=(2600, 1300, 400), K=K,
                                                        wmax=300)
    scale = 1.0 / math.sqrt(D)
    out, lse = _fwd_check(q, k, v, w, cu, idx, lb, maxlen)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, lb, do)]
    res = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                 scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    ref = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do),
                           lmk_bias=lb.double().numpy(), out=f64(out))
    check_grads(("large sets", K), res[:3], ref[:3], idx, cu, TOL[dt])
    assert rel_err(f64(res[3]), ref[3]) < TOL[dt]
    res2 = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                  scale=scale, max_seqlen=maxlen)
    for a, b in zip(res, res2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("block,K", [(512, 700), (100, 600), (1024, 2048)])
def test_large_landmark_sets_block_causal(block, K):
    """Block-causal sets of more than 512 landmarks, alone per tile (block 512, 1024) or
    three per tile (block 100: 3 x 600 slots)."""
    q, k, v, w, cu, idx, lb, maxlen = _inputs([3000, 1100], 4, 2, 64, K, 200, torch.bfloat16, seed=block + K,
                                              mode=ops.SELECT_BLOCK, block=block, bias=True)
    _fwd_check(q, k, v, w, cu, idx, lb, maxlen, mode=ops.SELECT_BLOCK, block=block)


def test_bwd_grouped_heads_shared_landmarks():
    """Heads of one group selecting the same positions: each landmark row's gradient is the
    sum over the group's heads (one writer per row)."""
    q, k, v, w, cu, idx, lb, maxlen, do = _bwd_gqa_case(8, 2, 64, torch.bfloat16, seed=47)
    idx[1::2] = idx[0::2]  # heads 2i and 2i+1 (same group) share their sets
    scale = 0.125
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, lb, do)]
    out, lse = ops.attention_forward(*dev[:6], dev[6], scale=scale, max_seqlen=maxlen)
    res = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                 scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    ref = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do),
                           lmk_bias=lb.double().numpy(), out=f64(out))
    check_grads("shared", res[:3], ref[:3], idx, cu, 2e-2)
    assert rel_err(f64(res[3]), ref[3]) < 2e-2


def test_repeated_landmark_positions_count_each_copy():
    """A set that repeats a position: the forward counts every copy and the backward sums
    every copy's gradient (the oracle's semantics), deterministically."""
    q, k, v, w, cu, idx, lb, maxlen, do = _bwd_gqa_case(4, 4, 64, torch.float32, seed=48, K=24)
    for hh in range(4):
        for s in range(2):
            row = idx[hh, s, 0]
            n = int((row >= 0).sum())
            if n >= 4:
                row[1] = row[0]
                row[3] = row[2]
    scale = 0.125
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, lb, do)]
    out, lse = ops.attention_forward(*dev[:6], dev[6], scale=scale, max_seqlen=maxlen)
    res = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                                 scale=scale, max_seqlen=maxlen)
    torch.cuda.synchronize()
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale,
                             lmk_bias=lb.double().numpy())
    assert rel_err(f64(out), ro) < 1e-5
    ref = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do),
                           lmk_bias=lb.double().numpy(), out=f64(out))
    check_grads("repeated", res[:3], ref[:3], idx, cu, 1e-5)
    assert rel_err(f64(res[3]), ref[3]) < 1e-5


@pytest.mark.parametrize("G", [4, 2])
def test_backward_reusing_the_forward_plan_is_bit_identical(G):
    q, k, v, w, cu, idx, lb, maxlen, do = _bwd_gqa_case(4, G, 64, torch.bfloat16, seed=49)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, lb, do)]
    plan = ops.new_plan(dev[0], dev[1], dev[4], dev[5], max_seqlen=maxlen)
    out, lse = ops.attention_forward(*dev[:6], dev[6], max_seqlen=maxlen, plan=plan)
    a = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                               max_seqlen=maxlen)
    b = ops.attention_backward(dev[7], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5], dev[6],
                               max_seqlen=maxlen, plan=plan)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("lens,G,mode", [([700, 333, 64], 4, ops.SELECT_GLOBAL), ([4096], 2, ops.SELECT_GLOBAL),
                                         ([900, 1], 4, ops.SELECT_BLOCK)])
def test_plan_from_selection_is_the_forwards_plan(lens, G, mode):
    """The row plan written by the selection's norms launch equals the one the forward computes,
    byte for byte, and a forward that reads it (plan_ready) gives the same bits."""
    H, D, K = 4, 64, 24
    g = torch.Generator().manual_seed(70 + len(lens))
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(T, G, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, G, D, generator=g).to(torch.bfloat16)
    h = torch.randn(T, 128, generator=g).to(torch.bfloat16)
    w = torch.randint(1, 300, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    dev = [t.to(DEV) for t in (q, k, v, h, w, cu)]
    qd, kd, vd, hd, wd, cud = dev
    maxlen = max(lens)
    alpha = torch.full((H,), 0.5, device=DEV)
    plan_sel = ops.new_plan(qd, kd, cud, torch.empty(H, len(lens), 1, K, dtype=torch.int32, device=DEV),
                            max_seqlen=maxlen)
    plan_sel.fill_(0xAB)
    idx = ops.select_landmarks(hd, vd, alpha, wd, cud, K, max_seqlen=maxlen, select_mode=mode, block_size=128,
                               plan=plan_sel)
    idx2 = ops.select_landmarks(hd, vd, alpha, wd, cud, K, max_seqlen=maxlen, select_mode=mode, block_size=128)
    plan_fwd = torch.zeros_like(plan_sel)
    a = ops.attention_forward(qd, kd, vd, wd, cud, idx, None, max_seqlen=maxlen, select_mode=mode, block_size=128,
                              plan=plan_fwd)
    b = ops.attention_forward(qd, kd, vd, wd, cud, idx, None, max_seqlen=maxlen, select_mode=mode, block_size=128,
                              plan=plan_sel, plan_ready=True)
    torch.cuda.synchronize()
    assert torch.equal(idx, idx2)
    # every byte the forward reads: the three plan sections of the tiles in use
    tiles = len(lens) * ((maxlen + 63) // 64)
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    t64 = al(tiles * 64)  # perm: 64 bytes a tile; bounds: 16 ints a tile; then the largest windows
    sec = [(0, tiles * 64), (t64, t64 + tiles * 64), (2 * t64, 2 * t64 + 4 * tiles)]
    for s0, s1 in sec:
        assert torch.equal(plan_sel[s0:s1], plan_fwd[s0:s1])
    for x, y in zip(a, b):
        assert torch.equal(x, y)

"""Tile variants and the autotune (reference dsalt/kernels/autotune.py:55-278).

Every candidate tiling computes the operator (fwd + bwd against the float64 oracle at the
bf16/fp32 tolerances); autotune_blocks times each candidate once, caches the winner per
(head_dim, dtype, device), and a second call returns the cached config without running
anything; the autograd operator then runs with the cached variant.
"""
from __future__ import annotations

import math

import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.kernels import autotune as AT
from oracle import attention as OA
from tests.helpers import check_grads, f64, rel_err
from tests.test_gpu_attention import _inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _case(dt, D, seed=60):
    q, k, v, w, cu, idx, lb, maxlen = _inputs([900, 400], 4, 2, D, 40, 300, dt, seed)
    g = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(q.shape, generator=g).to(dt)
    return q, k, v, w, cu, idx, maxlen, do


@pytest.mark.parametrize("dt,D", [(torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float32, 64)])
def test_every_candidate_matches_the_oracle(dt, D):
    q, k, v, w, cu, idx, maxlen, do = _case(dt, D)
    scale = 1.0 / math.sqrt(D)
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, do)]
    cands = AT._candidate_configs(D, DEV, 4 if dt == torch.float32 else 2)
    assert cands[0]["variant"] == 0 and len({c["variant"] for c in cands}) == len(cands)
    for cfg in cands:
        plan = ops.new_plan(dev[0], dev[1], dev[4], dev[5], max_seqlen=maxlen)
        out, lse = ops.attention_forward(*dev[:6], None, scale=scale, max_seqlen=maxlen, plan=plan,
                                         variant=cfg["variant"])
        dq, dk, dv, _ = ops.attention_backward(dev[6], dev[0], dev[1], dev[2], out, lse, dev[3], dev[4], dev[5],
                                               None, scale=scale, max_seqlen=maxlen, want_dbias=False, plan=plan,
                                               variant=cfg["variant"])
        torch.cuda.synchronize()
        assert rel_err(f64(out), ro) < TOL[dt], cfg
        rg = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do),
                              out=f64(out))
        check_grads(("variant", cfg["variant"]), (dq, dk, dv), rg[:3], idx, cu, TOL[dt])


@pytest.mark.parametrize("D,variant", [(d, c["variant"]) for d in (64, 128)
                                       for c in AT._candidate_configs(d, None, 2)])
def test_every_candidate_block_causal_forward(D, variant):
    """The block-causal operator with every 16-bit tiling (the autograd operator passes the
    tuned variant in block-causal mode too; the head_dim-128 inference shapes are block-causal):
    128-query blocks, GQA, ragged."""
    dt = torch.bfloat16
    q, k, v, w, cu, idx, lb, maxlen = _inputs([900, 400], 4, 2, D, 40, 300, dt, 63, mode=ops.SELECT_BLOCK,
                                              block=128)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx)]
    scale = 1.0 / math.sqrt(D)
    out, lse = ops.attention_forward(*dev, None, scale=scale, max_seqlen=maxlen, select_mode=ops.SELECT_BLOCK,
                                     block_size=128, variant=variant)
    torch.cuda.synchronize()
    ro, rl = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, block_size=128)
    assert rel_err(f64(out), ro) < TOL[dt]
    assert rel_err(f64(lse), rl) < 2e-3


def test_autotune_caches_and_the_operator_uses_the_winner():
    q, k, v, w, cu, idx, maxlen, do = _case(torch.bfloat16, 64, seed=61)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, do)]
    saved = dict(AT._TUNED_CONFIG)
    AT._TUNED_CONFIG.clear()
    try:
        assert AT.get_tuned_config(64, DEV, torch.bfloat16) is None and AT.tuned_variant(64, DEV, torch.bfloat16) == 0
        calls = []
        base = AT.operator_runner(*dev[:6], dev[6], max_seqlen=maxlen)

        def make_runner(cfg):
            calls.append(cfg["variant"])
            return base(cfg)

        best = AT.autotune_blocks(64, DEV, make_runner, verbose=False, dtype=torch.bfloat16)
        cands = AT._candidate_configs(64, DEV, 2)
        assert sorted(calls) == sorted(c["variant"] for c in cands)
        # forward and backward tilings are chosen separately: the winner takes its forward bits
        # from one candidate and its backward bits from another
        fwd_bits = {c["variant"] & AT._FWD_BITS for c in cands}
        bwd_bits = {c["variant"] & AT._BWD_BITS for c in cands}
        assert best["variant"] & AT._FWD_BITS in fwd_bits and best["variant"] & AT._BWD_BITS in bwd_bits
        assert best == AT._config_of(64, 2, best["variant"])
        again = AT.autotune_blocks(64, DEV, make_runner, verbose=False, dtype=torch.bfloat16)
        assert again is best and len(calls) == len(cands)  # cache hit
        assert AT.get_tuned_config(64, DEV, torch.bfloat16) is best
        assert AT.tuned_variant(64, DEV, torch.bfloat16) == best["variant"]
        # the autograd operator runs with the cached variant and still computes the operator
        from dsalt_amd.kernels.dsalt_attn import dsalt_attention
        qq, kk, vv = (t.clone().requires_grad_(True) for t in dev[:3])
        out = dsalt_attention(qq, kk, vv, dev[5][:, :, 0].long(), None, dev[3], dev[4], max_seqlen=maxlen)
        out.backward(dev[6].float())
        torch.cuda.synchronize()
        scale = 0.125
        ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale)
        rg = OA.attention_bwd(f64(q), f64(k), f64(v), w.numpy(), cu.numpy(), idx.numpy(), scale, f64(do))
        assert rel_err(f64(out), ro) < 2e-2
        for a, b in zip((qq.grad, kk.grad, vv.grad), rg[:3]):
            assert rel_err(f64(a), b) < 2e-2
    finally:
        AT._TUNED_CONFIG.clear()
        AT._TUNED_CONFIG.update(saved)


def test_autotune_with_a_plain_runner_times_whole_steps():
    q, k, v, w, cu, idx, maxlen, do = _case(torch.bfloat16, 64, seed=62)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, do)]
    saved = dict(AT._TUNED_CONFIG)
    AT._TUNED_CONFIG.clear()
    try:
        base = AT.operator_runner(*dev[:6], dev[6], max_seqlen=maxlen)

        def make_runner(cfg):
            r = base(cfg)
            return lambda: r()  # no .forward / .backward

        best = AT.autotune_blocks(64, DEV, make_runner, verbose=False, dtype=torch.bfloat16)
        assert best in AT._candidate_configs(64, DEV, 2)
    finally:
        AT._TUNED_CONFIG.clear()
        AT._TUNED_CONFIG.update(saved)

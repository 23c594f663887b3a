"""Every operator workload at its own full shape, HIP path against the oracle.

The workloads of ``dsalt_amd.workloads`` (batch, heads, length, head_dim, w_max, k, dtype and
landmark variant as the benchmark runs them):
  * forward fp32, H4 L2048, k=32 (the size the reference's CPU fallback handles);
  * forward + backward bf16, four packed 8192-token sequences, H8, k=64;
  * forward + backward bf16, H16 L32768, k=128, heavy-tailed norms (the headline);
  * forward bf16, H16 L131072 D128, block-causal k=256 in 512-query blocks;
  * forward bf16 of one Qwen2.5-3B-shaped decoder layer: 16/2 heads (GQA), D128, hidden
    2048, block-causal k=128, w_max 512, L32768;
  * the 36-layer Qwen2.5-3B-shaped prefill at L32768 through properties (finite logits, a
    bit-identical rerun) and its first layer's selection and attention against the oracle.
  * forward + backward bf16 of the training variant (the headline tensors with continuous
    windows, soft edge 4, landmark log-weights) on all 16 heads against the banded fp64
    training oracle.
Landmark indices must equal the C oracle's bit for bit; outputs must be within 1e-5 (fp32) or
2e-2 (bf16) relative error (max |a - b| / max |b|, per head) of the float64 oracle, and the
LSE within 1e-6 (fp32) or 2e-3 (bf16).  Gradients are held to the same tolerance per head by
``tests.helpers.assert_grad_close``: landmark rows and the other rows each against their own
largest entry, and every row above a quarter of its class's median norm against its own norm
(a landmark row of the headline shape is tens of times larger than an ordinary row, so one
bound over all rows would not see errors on the ordinary rows).  The oracle runs one head
per thread.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate
from tests.helpers import (_pool_map, check_grads, f64, oracle_bwd_heads, oracle_fwd_heads,
                           oracle_select_by_group, rel_err)

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
LSE_TOL = {torch.float32: 1e-6, torch.bfloat16: 2e-3}


def _select(x, wl, dev):
    mode = ops.SELECT_GLOBAL if wl.select_mode == "global" else ops.SELECT_BLOCK
    idx = ops.select_landmarks(dev["h"], dev["v"], dev["alpha"], dev["w"], dev["cu"], wl.k_lmk,
                               max_seqlen=wl.seqlen, select_mode=mode, block_size=wl.block_size,
                               stats_scope=ops.STATS_SEQUENCE)
    torch.cuda.synchronize()
    ridx = oracle_select_by_group(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, mode, wl.block_size,
                                  ops.STATS_SEQUENCE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    return idx, mode


def _check_fwd(x, idx, out, lse, wl, heads):
    block = wl.block_size if wl.select_mode == "block" else None
    scale = 1.0 / math.sqrt(wl.head_dim)
    refs = oracle_fwd_heads(x["q"], x["k"], x["v"], x["w"], x["cu"], idx.cpu().numpy(), scale, heads,
                            block_size=block)
    o, l = f64(out), f64(lse)
    for hh, (ro, rl) in zip(heads, refs):
        e_o = rel_err(o[:, hh], ro[:, 0])
        e_l = rel_err(l[:, hh], rl[:, 0])
        assert e_o < TOL[wl.dtype], (wl.name, hh, "out", e_o)
        assert e_l < LSE_TOL[wl.dtype], (wl.name, hh, "lse", e_l)


def _run(name, fwd_heads=None, bwd=False):
    wl = WORKLOADS[name]
    x = generate(wl)
    dev = {k: v.to(DEV) for k, v in x.items()}
    print(f"workload {name}: selection", flush=True)
    idx, mode = _select(x, wl, dev)
    out, lse = ops.attention_forward(dev["q"], dev["k"], dev["v"], dev["w"], dev["cu"], idx, None,
                                     max_seqlen=wl.seqlen, select_mode=mode, block_size=wl.block_size)
    torch.cuda.synchronize()
    heads = list(range(wl.heads)) if fwd_heads is None else fwd_heads
    print(f"workload {name}: forward on heads {heads}", flush=True)
    _check_fwd(x, idx, out, lse, wl, heads)
    if not bwd:
        return
    print(f"workload {name}: backward", flush=True)
    dq, dk, dv, _ = ops.attention_backward(dev["dout"], dev["q"], dev["k"], dev["v"], out, lse, dev["w"],
                                           dev["cu"], idx, None, max_seqlen=wl.seqlen, want_dbias=False)
    torch.cuda.synchronize()
    refs = oracle_bwd_heads(x["q"], x["k"], x["v"], x["w"], x["cu"], idx.cpu().numpy(),
                            1.0 / math.sqrt(wl.head_dim), x["dout"], list(range(wl.heads)), out=out)
    ref = [np.concatenate([r[j] for r in refs], axis=1) for j in range(3)]
    check_grads(name, (dq, dk, dv), ref, idx, x["cu"], TOL[wl.dtype])
    # the backward is deterministic: a second call gives the same bits
    r2 = ops.attention_backward(dev["dout"], dev["q"], dev["k"], dev["v"], out, lse, dev["w"], dev["cu"], idx,
                                None, max_seqlen=wl.seqlen, want_dbias=False)
    for a, b in zip((dq, dk, dv), r2[:3]):
        assert torch.equal(a, b)


def test_fwd_f32_h4_l2048_full():
    _run("fwd_f32_h4_l2048")


def test_fwdbwd_bf16_b4_h8_l8192_full():
    _run("fwdbwd_bf16_b4_h8_l8192", bwd=True)


def test_fwdbwd_bf16_h16_l32768_full():
    _run("fwdbwd_bf16_h16_l32768", bwd=True)


def test_fwd_bf16_h16_l131072_block_full():
    # selection bit-exact and the forward compared on all 16 heads
    _run("fwd_bf16_h16_l131072_block")


def test_train_bf16_h16_l32768_full():
    """The training variant at the benchmark's shape: the layer's hard selection from floor(w~),
    landmark log-weights log sigmoid(s / tau_lmk), soft edge 4; output, LSE and every gradient
    of all 16 heads against the banded float64 training oracle."""
    from oracle import train as OT
    wl = WORKLOADS["train_bf16_h16_l32768"]
    x = generate(wl)
    dev = {k: v.to(DEV) for k, v in x.items()}
    maxlen = wl.seqlen
    idx, _, _, sc = ops.select_landmarks(dev["h"], dev["v"], dev["alpha"], dev["w"], dev["cu"], wl.k_lmk,
                                         max_seqlen=maxlen, stats_scope=ops.STATS_SEQUENCE, want_scores=True)
    pos = idx[:, :, 0].long()
    H = pos.shape[0]
    s_sel = sc[dev["cu"][:-1].long()[None, :, None] + pos.clamp(min=0), torch.arange(H, device=DEV)[:, None, None]]
    logw = torch.log(torch.sigmoid(s_sel / wl.tau_lmk).clamp(min=1e-20))
    logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    print("workload train_bf16_h16_l32768: forward + backward", flush=True)
    out, lse = ops.train_forward(dev["q"], dev["k"], dev["v"], dev["w_cont"], dev["cu"], idx, logw.unsqueeze(2),
                                 tau_win=wl.tau_win, win_edge=wl.win_edge, max_seqlen=maxlen)
    dq, dk, dv, dlw, dw = ops.train_backward(dev["dout"], dev["q"], dev["k"], dev["v"], out, lse, dev["w_cont"],
                                             dev["cu"], idx, logw.unsqueeze(2), tau_win=wl.tau_win,
                                             win_edge=wl.win_edge, max_seqlen=maxlen)
    torch.cuda.synchronize()
    print("workload train_bf16_h16_l32768: banded oracle on all heads", flush=True)
    pos_c, logw_c, wc, cu = idx[:, :, 0].cpu().numpy(), logw.double().cpu().numpy(), x["w_cont"].double().numpy(), \
        x["cu"].numpy()
    args = [f64(x[n]) for n in ("q", "k", "v", "dout")]
    o_st = f64(out)  # delta from the stored output, as the reference's backward

    def one(hh):
        q1, k1, v1, d1 = (a[:, hh:hh + 1] for a in args)
        o1, l1 = OT.train_fwd_banded(q1, k1, v1, wc, cu, pos_c[hh:hh + 1], logw_c[hh:hh + 1], 1.0 / 8.0,
                                     wl.tau_win, wl.win_edge)
        g1 = OT.train_bwd_banded(q1, k1, v1, wc, cu, pos_c[hh:hh + 1], logw_c[hh:hh + 1], 1.0 / 8.0, wl.tau_win,
                                 wl.win_edge, d1, out=o_st[:, hh:hh + 1])
        return o1, l1, g1

    refs = _pool_map(one, range(H))
    o, l = f64(out), f64(lse)
    for hh, (ro, rl, _) in enumerate(refs):
        assert rel_err(o[:, hh], ro[:, 0]) < 2e-2, hh
        assert rel_err(l[:, hh], rl[:, 0]) < 2e-3, hh
    ref = [np.concatenate([r[2][j] for r in refs], axis=1) for j in range(3)]
    check_grads("train", (dq, dk, dv), ref, idx, x["cu"], 2e-2)
    # window gradient: the sum over heads; log-weight gradient per (head, slot)
    rdw = sum(r[2][3] for r in refs)
    assert rel_err(f64(dw), rdw) < 2e-2
    rdlw = np.concatenate([r[2][4] for r in refs], axis=0)
    assert rel_err(f64(dlw[:, :, 0]), rdlw) < 2e-2


def test_fwd_bf16_h16kv2_l32768_block_full():
    # one Qwen2.5-3B-shaped layer: GQA K/V read in place, all 16 query heads compared
    _run("fwd_bf16_h16kv2_l32768_block")


def test_prefill_qwen3b_l32768_full():
    """36 layers at L=32768: finite logits, a bit-identical rerun, and the first layer's
    block-causal selection (on its own activations, GQA value heads) and attention against
    the oracle."""
    from dsalt_amd.workloads import MODEL_WORKLOADS
    from dsalt_amd.model import DSALTLMHeadModel

    wl = MODEL_WORKLOADS["prefill_qwen3b_l32768"]
    cfg = wl.config()
    torch.manual_seed(wl.seed)
    with torch.device(DEV):
        model = DSALTLMHeadModel.from_config(cfg).to(DEV, wl.dtype).eval()
    T = wl.batch * wl.seqlen
    g = torch.Generator().manual_seed(wl.seed)
    ids = torch.randint(0, cfg.vocab_size, (T,), generator=g).to(DEV)
    cu = torch.arange(0, T + 1, wl.seqlen, dtype=torch.int32, device=DEV)

    captured = {}
    real_select, real_fwd = ops.select_landmarks, ops.attention_forward

    def select_hook(h, v, alpha, w, cu_, k_lmk, **kw):
        r = real_select(h, v, alpha, w, cu_, k_lmk, **kw)
        if "select" not in captured:
            captured["select"] = ([t.detach().cpu() for t in (h, v, alpha, w, cu_)], k_lmk, kw, r.cpu())
        return r

    def fwd_hook(q, k, v, w, cu_, idx, bias, **kw):
        r = real_fwd(q, k, v, w, cu_, idx, bias, **kw)
        if "fwd" not in captured:
            captured["fwd"] = ([t.detach().cpu() for t in (q, k, v, w, cu_, idx)], kw, [t.cpu() for t in r])
        return r

    ops.select_landmarks, ops.attention_forward = select_hook, fwd_hook
    try:
        with torch.no_grad():
            print("prefill: first forward", flush=True)
            lg1 = model(ids, cu_seqlens=cu, max_seqlen=wl.seqlen)["logits"]
    finally:
        ops.select_landmarks, ops.attention_forward = real_select, real_fwd
    with torch.no_grad():
        print("prefill: second forward", flush=True)
        lg2 = model(ids, cu_seqlens=cu, max_seqlen=wl.seqlen)["logits"]
    torch.cuda.synchronize()
    assert lg1.shape == (T, cfg.vocab_size)
    assert bool(torch.isfinite(lg1).all())
    assert torch.equal(lg1, lg2)
    del lg1, lg2, model
    torch.cuda.empty_cache()

    (h, v, alpha, w, cu_c), k_lmk, kw, idx = captured["select"]
    assert v.shape[1] == cfg.n_kv_heads and kw["select_mode"] == ops.SELECT_BLOCK
    print("prefill: layer-0 selection vs oracle", flush=True)
    ridx = oracle_select_by_group(h, v, alpha, w, cu_c, k_lmk, kw["select_mode"], kw["block_size"],
                                  kw["stats_scope"])
    np.testing.assert_array_equal(idx.numpy(), ridx)

    (q, k, v2, w2, cu2, idx2), kw2, (out, lse) = captured["fwd"]
    assert torch.equal(idx2, idx.to(idx2.dtype))
    print("prefill: layer-0 attention vs oracle", flush=True)
    refs = oracle_fwd_heads(q, k, v2, w2, cu2, idx2.numpy(), 1.0 / math.sqrt(q.shape[-1]),
                            list(range(q.shape[1])), block_size=kw2["block_size"])
    o, l = f64(out), f64(lse)
    for hh, (ro, rl) in enumerate(refs):
        assert rel_err(o[:, hh], ro[:, 0]) < TOL[torch.bfloat16], hh
        assert rel_err(l[:, hh], rl[:, 0]) < LSE_TOL[torch.bfloat16], hh

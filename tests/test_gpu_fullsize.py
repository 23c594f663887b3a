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
Landmark indices must equal the C oracle's bit for bit; outputs and gradients must be within
1e-5 (fp32) or 2e-2 (bf16) relative error (max |a - b| / max |b|, per head) of the float64
oracle, and the LSE within 1e-6 (fp32) or 2e-3 (bf16).  The oracle runs one head per thread.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate
from tests.helpers import f64, oracle_bwd_heads, oracle_fwd_heads, oracle_select_by_group, rel_err

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
    g = [f64(t) for t in (dq, dk, dv)]
    refs = oracle_bwd_heads(x["q"], x["k"], x["v"], x["w"], x["cu"], idx.cpu().numpy(),
                            1.0 / math.sqrt(wl.head_dim), x["dout"], list(range(wl.heads)))
    for hh, r in enumerate(refs):
        for name_g, a, b in zip(("dq", "dk", "dv"), g, r[:3]):
            e = rel_err(a[:, hh], b[:, 0])
            assert e < TOL[wl.dtype], (name, hh, name_g, e)
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
    # selection bit-exact on all 16 heads, the forward compared on four of them
    _run("fwd_bf16_h16_l131072_block", fwd_heads=[0, 5, 10, 15])


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

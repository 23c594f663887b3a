"""Fused ingress (RoPE in place on a fused QKV projection) and the decoder stack on the GPU.

RoPE: bit-exact against the oracle's emulation of the reference expression.  Layer and
model outputs: the attention part against the float64 oracle, the rest against the same
torch computation; tolerances are relative (max|a-b| / max|b|) and written per test.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from oracle import rope as OR
from tests.helpers import f64, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_in_place_on_fused_qkv_bit_exact(dt, D):
    from dsalt_amd.kernels.window_utils import build_rope_cache
    g = torch.Generator().manual_seed(D)
    lens = [300, 77, 1]
    T, H, G = sum(lens), 4, 2
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    qkv = (torch.randn(T, (H + 2 * G) * D, generator=g) * 2).to(dt)
    cos, sin = build_rope_cache(512, D, torch.device("cpu"), base=1e6)
    buf = qkv.to(DEV)
    q = buf[:, :H * D].view(T, H, D)
    k = buf[:, H * D:(H + G) * D].view(T, G, D)
    ops.rope_qk_(q, k, cu.to(DEV), cos.to(DEV), sin.to(DEV), max_seqlen=max(lens))
    torch.cuda.synchronize()
    out = buf.cpu().float().numpy()
    ref_q = OR.rope(qkv[:, :H * D].view(T, H, D).float().numpy(), cu.numpy(), cos.numpy(), sin.numpy(), NAME[dt])
    ref_k = OR.rope(qkv[:, H * D:(H + G) * D].view(T, G, D).float().numpy(), cu.numpy(), cos.numpy(), sin.numpy(),
                    NAME[dt])
    np.testing.assert_array_equal(out[:, :H * D], ref_q.reshape(T, -1))
    np.testing.assert_array_equal(out[:, H * D:(H + G) * D], ref_k.reshape(T, -1))
    np.testing.assert_array_equal(out[:, (H + G) * D:], qkv[:, (H + G) * D:].float().numpy())  # v untouched


def test_rope_rejects_positions_past_the_table():
    from dsalt_amd.kernels.window_utils import build_rope_cache
    cos, sin = build_rope_cache(64, 64, torch.device(DEV))
    q = torch.zeros(100, 2, 64, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, 100], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="max_pos"):
        ops.rope_qk_(q, None, cu, cos, sin)


def _layer_both_paths(dt, mode, G=2, rope_cs=False):
    from dsalt_amd.modules import DSALTAttention
    torch.manual_seed(3)
    d, H, T = 256, 4, 640
    m = DSALTAttention(d, H, 16, 96, 12, 1024, n_kv_heads=G, qkv_bias=True, select_mode=mode,
                       block_size=128).to(DEV).to(dt).eval()
    x = torch.randn(T, d, device=DEV).to(dt)
    cu = torch.tensor([0, 400, T], dtype=torch.int32, device=DEV)
    cs = None
    if rope_cs:
        pos = torch.cat([torch.arange(400), torch.arange(T - 400)]).to(DEV)
        cs = (m.rope_cos[pos], m.rope_sin[pos])
    with torch.enable_grad():  # the separate-projection path with autograd
        ref, _ = m(x, cu, rope_cs=cs, cu_list=[0, 400, T])
    with torch.no_grad():      # fused QKV GEMM, RoPE kernel in place, strided attention
        out, aux = m(x, cu, rope_cs=cs, cu_list=[0, 400, T])
    return out, ref.detach(), aux


@pytest.mark.parametrize("dt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("mode", ["global", "block"])
def test_layer_fused_inference_path_matches_projection_path(dt, tol, mode):
    out, ref, aux = _layer_both_paths(dt, mode)
    assert out.dtype == dt and float(aux) == 0.0
    assert rel_err(f64(out), f64(ref)) < tol


def test_layer_fused_path_with_gathered_rope_rows():
    out, ref, _ = _layer_both_paths(torch.float32, "global", G=4, rope_cs=True)
    assert rel_err(f64(out), f64(ref)) < 1e-5


def _small_model(mode, dt=torch.float32, tie=True):
    from dsalt_amd.model import DSALTConfig, DSALTLMHeadModel
    cfg = DSALTConfig(vocab_size=1000, d_model=256, n_layers=2, n_heads=4, n_kv_heads=2, n_min=16, n_max=96, k_lmk=12,
                      max_seq_len=1024, d_ff=512, qkv_bias=True, rope_base=1e6, select_mode=mode, block_size=128,
                      tie_weights=tie, lm_head_chunk_size=128)
    torch.manual_seed(5)
    return DSALTLMHeadModel.from_config(cfg).to(DEV).to(dt)


@pytest.mark.parametrize("mode", ["global", "block"])
def test_model_inference_forward_matches_autograd_forward(mode):
    m = _small_model(mode).eval()
    T = 513
    ids = torch.randint(0, 1000, (T,), device=DEV)
    cu = torch.tensor([0, 300, T], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        lg = m(ids, cu_seqlens=cu)["logits"]
    lg_ref = m(ids, cu_seqlens=cu)["logits"].detach()
    assert lg.shape == (T, 1000)
    assert rel_err(f64(lg), f64(lg_ref)) < 1e-5
    # batched input runs as packed sequences of equal length
    with torch.no_grad():
        lb = m(ids[:512].view(2, 256))["logits"]
        lp = m(ids[:512], cu_seqlens=torch.tensor([0, 256, 512], dtype=torch.int32, device=DEV))["logits"]
    assert rel_err(f64(lb.reshape(512, -1)), f64(lp)) < 1e-5


def test_model_loss_is_mean_token_cross_entropy():
    m = _small_model("global").eval()
    T = 400
    ids = torch.randint(0, 1000, (T,), device=DEV)
    labels = torch.randint(0, 1000, (T,), device=DEV)
    labels[::7] = -100
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        loss = m(ids, cu_seqlens=cu, labels=labels)["loss"]
        lg = m(ids, cu_seqlens=cu)["logits"]
    ref = torch.nn.functional.cross_entropy(lg.float(), labels, ignore_index=-100)
    assert abs(float(loss) - float(ref)) < 1e-4 * abs(float(ref))


def test_model_training_step_reaches_every_parameter():
    m = _small_model("global", tie=False).train()
    T = 300
    ids = torch.randint(0, 1000, (T,), device=DEV)
    cu = torch.tensor([0, 180, T], dtype=torch.int32, device=DEV)
    out = m(ids, cu_seqlens=cu, labels=torch.roll(ids, -1))
    out["loss"].backward()
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
        if "win_gate" in n or "alpha_w" in n or "proj" in n:
            assert float(p.grad.abs().max()) > 0, n


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_silu_mul_on_fused_gate_up_matches_torch(dt):
    g = torch.Generator().manual_seed(9)
    T, F_ = 333, 11008
    gu = (torch.randn(T, 2 * F_, generator=g) * 4).to(dt).to(DEV)
    gu[0, :8] = torch.tensor([0.0, -0.0, 30.0, -30.0, 88.0, -88.0, 1e-3, -1e-3], dtype=dt)
    out = ops.silu_mul(gu[:, :F_], gu[:, F_:])
    ref = torch.nn.functional.silu(gu[:, :F_].contiguous()) * gu[:, F_:].contiguous()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), float((out.float() - ref.float()).abs().max())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("F_", [1, 7, 100, 11001])
def test_silu_mul_any_width(dt, F_):
    # widths off the 8-column vectors: rows on 16-byte boundaries run the kernel's tail; the
    # halves of an odd-width fused buffer and odd-width contiguous rows run on padded copies
    g = torch.Generator().manual_seed(F_)
    T = 129
    gu = (torch.randn(T, 2 * F_, generator=g) * 4).to(dt).to(DEV)
    vec = 16 // gu.element_size()
    pad = -(-F_ // vec) * vec
    aligned = [torch.zeros(T, pad, dtype=dt, device=DEV)[:, :F_] for _ in range(3)]
    aligned[0].copy_(gu[:, :F_])
    aligned[1].copy_(gu[:, F_:])
    cases = ((gu[:, :F_], gu[:, F_:], None), (gu[:, :F_].contiguous(), gu[:, F_:].contiguous(), None),
             (aligned[0], aligned[1], aligned[2]))
    for gate, up, out in cases:
        res = ops.silu_mul(gate, up, out)
        ref = torch.nn.functional.silu(gate.contiguous()) * up.contiguous()
        torch.cuda.synchronize()
        assert torch.equal(res, ref), float((res.float() - ref.float()).abs().max())


@pytest.mark.parametrize("V,aligned", [(2, False), (17, True), (1001, False), (50257, True), (50257, False)])
def test_row_kernel_any_vocabulary(V, aligned):
    # vocabularies off the 8-column vectors: aligned rows (row stride rounded up) run the
    # kernel's tail, contiguous odd rows a padded copy with the gradient copied back
    from oracle import cross_entropy as OCE
    g = torch.Generator().manual_seed(V)
    N = 70
    x = torch.randn(N, V, generator=g) * 3
    t = torch.randint(0, V, (N,), generator=g)
    t[::7] = -100
    t[1] = V - 1  # a target in the tail
    cw = torch.rand(V, generator=g) + 0.2
    for w_, opts in ((None, dict(label_smoothing=0.1, lse_square_scale=1e-3)), (cw, dict(label_smoothing=0.05)),
                     (None, dict(softcap=15.0))):
        if aligned:
            logits = torch.zeros(N, -(-V // 4) * 4, device=DEV)[:, :V]
            logits.copy_(x)
        else:
            logits = x.to(DEV)
        loss, z, acc, pred = ops.cross_entropy_rows(logits, t.to(DEV), ce_weight=None if w_ is None else w_.to(DEV),
                                                    want_z=True, want_accuracy=True, want_predicted=True, **opts)
        torch.cuda.synchronize()
        rl, rz, rg, am, _ = OCE.ce_rows(x.double().numpy(), t.numpy(), None if w_ is None else w_.double().numpy(),
                                        -100, opts.get("lse_square_scale", 0.0), opts.get("label_smoothing", 0.0),
                                        "mean", opts.get("softcap"), False)
        assert rel_err(f64(loss), rl) < 1e-5 and rel_err(f64(logits), rg) < 1e-5, (V, aligned, opts)
        keep = (t != -100).numpy()
        assert np.array_equal(pred.cpu().numpy()[keep], am[keep])


# ------------------------------------------------------------------ fused linear cross-entropy
@pytest.mark.parametrize("opts", [dict(), dict(label_smoothing=0.1, lse_square_scale=1e-3), dict(softcap=20.0),
                                  dict(ce_weight=True, label_smoothing=0.05, reduction="sum"),
                                  dict(use_token_scaling=True), dict(reduction="none")])
def test_row_kernel_matches_oracle(opts):
    from oracle import cross_entropy as OCE
    g = torch.Generator().manual_seed(90)
    N, V = 96, 4000
    x = torch.randn(N, V, generator=g) * 3
    t = torch.randint(0, V, (N,), generator=g)
    t[::6] = -100
    opts = dict(opts)
    cw = torch.rand(V, generator=g) + 0.2 if opts.pop("ce_weight", False) else None
    red = opts.pop("reduction", "mean")
    scaling = opts.pop("use_token_scaling", False)
    zs, ls, cap = opts.get("lse_square_scale", 0.0), opts.get("label_smoothing", 0.0), opts.get("softcap")
    logits = x.to(DEV)
    loss, z, acc, pred = ops.cross_entropy_rows(logits, t.to(DEV), ce_weight=cw.to(DEV) if cw is not None else None,
                                                reduction=red, token_scaling=scaling, lse_square_scale=zs,
                                                label_smoothing=ls, softcap=cap, want_z=True, want_accuracy=True,
                                                want_predicted=True)
    torch.cuda.synchronize()
    rl, rz, rg, am, _ = OCE.ce_rows(x.double().numpy(), t.numpy(), None if cw is None else cw.double().numpy(),
                                    -100, zs, ls, red, cap, scaling)
    assert rel_err(f64(loss), rl) < 1e-5
    assert rel_err(f64(logits), rg) < 1e-5
    if zs:
        assert rel_err(f64(z), rz) < 1e-5
    keep = (t != -100).numpy()
    assert np.array_equal(pred.cpu().numpy()[keep], am[keep]) and np.all(pred.cpu().numpy()[~keep] == -1)
    assert np.array_equal(acc.cpu().numpy(), (am == t.numpy()).astype(np.float32) * keep)


def test_row_kernel_token_scaling_matches_oracle():
    from oracle import cross_entropy as OCE
    g = torch.Generator().manual_seed(91)
    N, V = 64, 1024
    x = torch.randn(N, V, generator=g)
    t = torch.randint(0, V, (N,), generator=g)
    logits = x.to(DEV)
    loss, _, _, _ = ops.cross_entropy_rows(logits, t.to(DEV), token_scaling=True, label_smoothing=0.1)
    rl, _, rg, _, _ = OCE.ce_rows(x.double().numpy(), t.numpy(), label_smoothing=0.1, use_token_scaling=True)
    assert rel_err(f64(loss), rl) < 1e-5 and rel_err(f64(logits), rg) < 1e-5


@pytest.mark.parametrize("dt,tol,V", [(torch.float32, 1e-5, 5000), (torch.bfloat16, 2e-2, 5000),
                                      (torch.float32, 1e-5, 5003)])
def test_fused_linear_cross_entropy_matches_autograd(dt, tol, V):
    from dsalt_amd.kernels.cross_entropy import LigerFusedLinearCrossEntropyFunction
    g = torch.Generator().manual_seed(92)
    BT, H = 700, 256
    x = (torch.randn(BT, H, generator=g)).to(dt).to(DEV).requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.05).to(dt).to(DEV).requires_grad_(True)
    b = (torch.randn(V, generator=g) * 0.1).to(dt).to(DEV).requires_grad_(True)
    t = torch.randint(0, V, (BT,), generator=g).to(DEV)
    t[::9] = -100
    loss, z, acc, _ = LigerFusedLinearCrossEntropyFunction.apply(x, w, t, b, None, -100, 1e-4, 0.1, "mean", None,
                                                                 True, None, False, True, False)
    (loss * 2.0).backward()
    xr, wr, br = (a.detach().double().requires_grad_(True) for a in (x, w, b))
    lg = xr @ wr.T + br
    keep = t != -100
    lr = torch.nn.functional.cross_entropy(lg, t, ignore_index=-100, label_smoothing=0.1)
    lr = lr + 1e-4 * (torch.logsumexp(lg, -1) ** 2 * keep).sum() / keep.sum()
    (lr * 2.0).backward()
    assert abs(loss.item() - lr.item()) < tol * abs(lr.item())
    for a, r in ((x.grad, xr.grad), (w.grad, wr.grad), (b.grad, br.grad)):
        assert rel_err(f64(a), f64(r)) < tol
    assert 0.0 <= float(acc) <= 1.0


def test_model_fused_loss_matches_chunked():
    m = _small_model("global").train()
    T = 400
    ids = torch.randint(0, 1000, (T,), device=DEV)
    labels = torch.roll(ids, -1)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    m.loss_fn = "chunked"
    l1 = m(ids, cu_seqlens=cu, labels=labels)["loss"]
    l1.backward()
    g1 = m.embed_tokens.weight.grad.clone()
    m.zero_grad()
    m.loss_fn = "liger"
    l2 = m(ids, cu_seqlens=cu, labels=labels)["loss"]
    l2.backward()
    l1, l2 = float(l1.detach()), float(l2.detach())
    assert abs(l1 - l2) < 1e-5 * abs(l1)
    assert rel_err(f64(m.embed_tokens.weight.grad), f64(g1)) < 1e-4

"""The reference-named API on the GPU: reference golden outputs, autograd against the
float64 oracle, and the DSALTAttention layer."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import kernels as K
from dsalt_amd import ops
from dsalt_amd.modules import DSALTAttention
from oracle import attention as OA
from tests.helpers import f64, load_golden, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a, dt=None):
    t = torch.as_tensor(a).to(DEV)
    return t.to(dt) if dt is not None else t


@pytest.mark.parametrize("name", ["uniform", "ragged", "gqa", "pad"])
def test_compute_landmark_indices_matches_reference(name):
    z = load_golden(f"select_{name}")
    H = z["alpha"].shape[0]
    dh = z["v"].shape[2]
    idx, zx, zv = K._compute_landmark_indices(_t(z["x"]), _t(z["W_V"]), _t(z["alpha"]), _t(z["w"]), _t(z["cu"]),
                                              int(z["k"]), 1, z["x"].shape[0], [int(c) for c in z["cu"]],
                                              head_dim=dh)
    assert idx.shape == (H, len(z["cu"]) - 1, int(z["k"])) and idx.dtype == torch.int64
    np.testing.assert_array_equal(idx.cpu().numpy(), z["idx"])
    np.testing.assert_allclose(zx.cpu().numpy(), z["z_x"], atol=3e-6)
    np.testing.assert_allclose(zv.cpu().numpy(), z["z_v"], atol=3e-6)
    sc, zx2, _ = K.hybrid_scores_per_head(_t(z["x"]), _t(z["W_V"]), _t(z["alpha"]), H, dh)
    np.testing.assert_allclose(sc.cpu().numpy(), z["scores"], atol=3e-6)


@pytest.mark.parametrize("name", ["b64", "mha", "gqa"])
def test_block_causal_selection_matches_reference(name):
    """The reference's block-causal selection and attention (blocks of 64, and of 32 rows at
    head_dim 8: sets change inside a 64-row tile, q/k/v run zero-padded to head_dim 64)."""
    z = load_golden(f"block_causal_{name}")
    T, B, k = z["x"].shape[0], int(z["block"]), int(z["k"])
    dh = z["v"].shape[2]
    cu = np.array([0, T], np.int32)
    idx, _, _ = K._compute_landmark_indices(_t(z["x"]), _t(z["W_V"]), _t(z["alpha"]), _t(z["w"]), _t(cu), k, 1, T,
                                            [0, T], head_dim=dh, select_mode="block", block_size=B)
    np.testing.assert_array_equal(idx[:, 0].cpu().numpy(), z["sets"])
    # the block-causal attention of the same sets: the reference's exact kernel semantics
    out = K.dsalt_attention(_t(z["q"]), _t(z["kk"]), _t(z["vv"]), idx, None, _t(z["w"]), _t(cu), block_size=B)
    assert rel_err(f64(out), z["out"]) < 1e-5


def test_build_landmark_kv_matches_reference():
    z = load_golden("landmark_gather")
    H, S, k = z["idx"].shape
    lk, lv = K._build_landmark_kv(_t(z["K"]), _t(z["V"]), _t(z["idx"]), _t(z["cu"]), k, H, z["K"].shape[2])
    # the reference gathers head_dim 4; pad the check to the library's 64-wide rows
    assert lk.shape == (H, S, k, z["K"].shape[2])
    np.testing.assert_array_equal(lk.cpu().numpy(), z["lk"])
    np.testing.assert_array_equal(lv.cpu().numpy(), z["lv"])


def test_dense_masked_attention_matches_reference():
    z = load_golden("literal_fallback")
    T = z["x"].shape[0]
    mask = np.unpackbits(z["mask"], axis=-1)[:, :T].astype(bool)
    out = K.sparse_attention_forward_packed(_t(z["q"]), _t(z["kk"]), _t(z["vv"]), _t(mask))
    assert np.abs(out.cpu().numpy() - z["out"]).max() < 1e-5


def _op_case(dt, H=4, G=4, lens=(300, 213), D=64, K_=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(dt)
    k = torch.randn(T, G, D, generator=g).to(dt)
    v = torch.randn(T, G, D, generator=g).to(dt)
    w = torch.randint(1, 80, (T,), generator=g).float()
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    idx = torch.full((H, len(lens), K_), -1, dtype=torch.int64)
    for hh in range(H):
        for s, L in enumerate(lens):
            c = torch.randperm(L, generator=g)[:K_ - 3]  # unsorted, as torch.topk(sorted=False) returns
            idx[hh, s, :len(c)] = c
    bias = torch.randn(idx.shape, generator=g) * 0.3
    return q, k, v, w, cu, idx, bias


@pytest.mark.parametrize("dt,G", [(torch.bfloat16, 4), (torch.float32, 4), (torch.bfloat16, 2)])
def test_autograd_operator_against_oracle(dt, G):
    q, k, v, w, cu, idx, bias = _op_case(dt, G=G)
    tol = 1e-5 if dt == torch.float32 else 2e-2
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    bd = bias.to(DEV).requires_grad_(True)
    out = K.dsalt_triton_attention(qd, kd, vd, idx.to(DEV), bd, w.to(DEV), cu.to(DEV))
    assert out.dtype == torch.float32
    g = torch.Generator().manual_seed(5)
    do = torch.randn(out.shape, generator=g)
    out.backward(do.to(DEV))
    scale = 1.0 / math.sqrt(q.shape[-1])
    idx4 = idx.numpy()[:, :, None]
    b4 = bias.double().numpy()[:, :, None]
    wi = w.clamp(min=1).long().numpy()
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale, lmk_bias=b4)
    assert rel_err(f64(out), ro) < tol
    rdq, rdk, rdv, rdb = OA.attention_bwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale,
                                          f64(do.to(dt)), lmk_bias=b4)
    for name, a, b in (("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv),
                       ("dbias", bd.grad, rdb[:, :, 0])):
        assert rel_err(f64(a), b) < tol, name


def test_standalone_backward_signature():
    q, k, v, w, cu, idx, bias = _op_case(torch.bfloat16)
    dev = [t.to(DEV) for t in (q, k, v, w, cu, idx, bias)]
    out, lse = ops.attention_forward(dev[0], dev[1], dev[2], dev[3].clamp(min=1).int(), dev[4],
                                     ops.sort_landmarks(dev[5].unsqueeze(2), dev[6].unsqueeze(2))[0],
                                     ops.sort_landmarks(dev[5].unsqueeze(2), dev[6].unsqueeze(2))[1])
    do = torch.randn_like(dev[0])
    dq, dk, dv, db = K.dsalt_triton_backward(do, dev[0], dev[1], dev[2], out, lse, None, None, dev[5], dev[6],
                                             dev[3], dev[4], 1.0 / 8.0, None, None, 64, 32, 64)
    assert dq.dtype == torch.float32 and db.shape == idx.shape
    scale = 1.0 / 8.0
    rdq, _, _, rdb = OA.attention_bwd(f64(q), f64(k), f64(v), w.clamp(min=1).long().numpy(), cu.numpy(),
                                      idx.numpy()[:, :, None], scale, f64(do), lmk_bias=bias.double().numpy()[:, :, None])
    assert rel_err(f64(dq), rdq) < 2e-2
    assert rel_err(f64(db), rdb[:, :, 0]) < 2e-2


@pytest.mark.parametrize("mode,d,bs", [("global", 256, 128), ("block", 256, 128), ("global", 320, 128),
                                       ("block", 256, 100)])
def test_dsalt_attention_layer(mode, d, bs):
    """The layer's inference branch (fused QKV, RoPE kernel, strided attention) against its
    parts with the float64 oracle; d = 320 gives head_dim 80 (run zero-padded to 128); block
    size 100 puts the rows of some 64-row tiles in two landmark sets."""
    torch.manual_seed(0)
    H, G, T = 4, 2, 640
    D = d // H
    m = DSALTAttention(d, H, 32, 128, 16, 2048, n_kv_heads=G, qkv_bias=True, select_mode=mode,
                       block_size=bs).to(DEV).eval()
    x = torch.randn(T, d, device=DEV)
    cu = torch.tensor([0, 400, T], dtype=torch.int32, device=DEV)
    out, aux = m(x, cu, cu_list=[0, 400, T])
    assert out.shape == (T, d) and float(aux) == 0.0
    # same computation from its parts, with the float64 oracle as the attention
    with torch.no_grad():
        q = m.q_proj(x).view(T, H, D)
        k = m.k_proj(x).view(T, G, D)
        v = m.v_proj(x).view(T, G, D)
        pos = torch.cat([torch.arange(400), torch.arange(T - 400)]).to(DEV)
        q, k = K.apply_rotary_emb(q, k, m.rope_cos[pos].unsqueeze(1), m.rope_sin[pos].unsqueeze(1))
        w = m._window_sizes(x, floor=True)
        lmk, _, _ = K._compute_landmark_indices(x, m.v_proj.weight, m._alpha(), w, cu, 16, 32, T, [0, 400, T],
                                                head_dim=D, select_mode=mode, block_size=bs)
    idx4 = lmk.cpu().numpy() if mode == "block" else lmk.cpu().numpy()[:, :, None]
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), w.long().cpu().numpy(), cu.cpu().numpy(), idx4,
                             1 / math.sqrt(D), block_size=bs if mode == "block" else None)
    ref = m.out_proj(torch.tensor(ro, dtype=torch.float32, device=DEV).view(T, d))
    assert rel_err(f64(out), f64(ref)) < 1e-5
    # batched input runs as packed sequences
    xb = x[:512].view(2, 256, d)
    ob, _ = m(xb)
    assert ob.shape == (2, 256, d)


@pytest.mark.parametrize("D,dt", [(32, torch.bfloat16), (80, torch.bfloat16), (96, torch.float32), (48, torch.float16)])
def test_autograd_operator_other_head_dims(D, dt):
    """head_dims the kernels are not compiled for run zero-padded to 64 / 128 with the scale of
    the true head_dim (the reference pads to the next power of two): output and gradients
    against the oracle at the true head_dim."""
    from tests.helpers import check_grads
    q, k, v, w, cu, idx, bias = _op_case(dt, G=2, D=D, seed=D)
    tol = 1e-5 if dt == torch.float32 else 2e-2
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    bd = bias.to(DEV).requires_grad_(True)
    out = K.dsalt_triton_attention(qd, kd, vd, idx.to(DEV), bd, w.to(DEV), cu.to(DEV))
    assert out.shape == q.shape
    g = torch.Generator().manual_seed(6)
    do = torch.randn(out.shape, generator=g)
    out.backward(do.to(DEV))
    assert qd.grad.shape == q.shape and kd.grad.shape == k.shape
    scale = 1.0 / math.sqrt(D)
    idx4 = idx.numpy()[:, :, None]
    b4 = bias.double().numpy()[:, :, None]
    wi = w.clamp(min=1).long().numpy()
    ro, _ = OA.attention_fwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale, lmk_bias=b4)
    assert rel_err(f64(out), ro) < tol
    rg = OA.attention_bwd(f64(q), f64(k), f64(v), wi, cu.numpy(), idx4, scale, f64(do.to(dt)), lmk_bias=b4,
                          out=f64(out.to(dt)))
    check_grads(("head_dim", D), (qd.grad, kd.grad, vd.grad), rg[:3], idx, cu, tol)
    assert rel_err(f64(bd.grad), rg[3][:, :, 0]) < tol
    # the standalone backward pads the same way (forward outputs from the padded operator)
    from dsalt_amd.kernels.dsalt_attn import pad_head_dim, padded_head_dim
    dp = padded_head_dim(D)
    idx_s, bias_s, _ = ops.sort_landmarks(idx.to(DEV).unsqueeze(2), bd.detach().unsqueeze(2))
    o_p, lse = ops.attention_forward(*(pad_head_dim(t.detach(), dp) for t in (qd, kd, vd)),
                                     w.to(DEV).clamp(min=1).int(), cu.to(DEV), idx_s, bias_s, scale=scale)
    dq2, dk2, dv2, db2 = K.dsalt_triton_backward(do.to(DEV), qd.detach(), kd.detach(), vd.detach(),
                                                 o_p[..., :D].contiguous(), lse, None, None, idx.to(DEV),
                                                 bd.detach(), w.to(DEV), cu.to(DEV), scale)
    assert dq2.shape == q.shape and dk2.shape == k.shape
    check_grads(("standalone head_dim", D), (dq2, dk2, dv2), rg[:3], idx, cu, tol)

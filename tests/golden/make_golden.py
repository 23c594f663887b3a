"""Writes the golden vectors under tests/golden/ from the reference library's CPU code.

Run in the build container only (it reads /root/reference, which is not available where
the tests run):  python tests/golden/make_golden.py [--only-bf16]

Only functions whose behaviour is a convention rather than mathematics are vectored here:
the exclusion rule, -1 padding and the uniform/ragged branches of
``_compute_landmark_indices`` (dsalt/kernels/selectors.py:75-134), the z-score convention of
``hybrid_scores_per_head`` (dsalt/kernels/landmark_tokens_ker.py:19-61), the literal CPU
fallback mask ``_build_mask_packed`` (dsalt/modules/dsalt_attention.py:95-144) with
``sparse_attention_forward_packed`` (dsalt/kernels/sparse_attn.py:29-57), the window-mask
builders (dsalt/kernels/window_utils.py:19-70), the packed block map
(dsalt/kernels/selectors.py:37-67), the landmark gather (selectors.py:137-159), and the
block-causal selection and exact kernel-semantics attention of
results/causal_landmark_check.py:68-147, and the training log-bias of
dsalt/modules/dsalt_attention.py:520-563 with its SDPA gradients, and the bf16 selection
(the reference's own bf16 norms, float32 statistics and topk at workload-like shapes).
Inputs are small and seeded (float32, the training case float64, the bf16 selection bf16).
"""
from __future__ import annotations

import math
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))


def _import_reference():
    sys.path.insert(0, REF)
    import dsalt.kernels.landmark_tokens_ker as LT
    import dsalt.kernels.selectors as SEL
    import dsalt.kernels.sparse_attn as SA
    import dsalt.kernels.window_utils as WU
    import dsalt.modules.dsalt_attention as DA
    import results.causal_landmark_check as CLC
    return LT, SEL, SA, WU, DA, CLC


def _sort_sets(idx: torch.Tensor) -> np.ndarray:
    """Sort each landmark set ascending with the -1 padding last."""
    a = idx.numpy().astype(np.int64)
    big = np.where(a < 0, np.iinfo(np.int64).max, a)
    s = np.sort(big, axis=-1)
    return np.where(s == np.iinfo(np.int64).max, -1, s)


def selection_cases(LT, SEL):
    cases = {}
    specs = [
        # name, lens, d_model, H, n_kv, dh, k, w_hi
        ("uniform", [64, 64], 32, 4, 4, 8, 8, 20),
        ("ragged", [50, 30, 48], 32, 4, 4, 8, 8, 20),
        ("gqa", [96], 32, 4, 2, 8, 6, 24),
        ("pad", [40], 16, 2, 2, 8, 12, 36),
    ]
    for n, (name, lens, d, H, G, dh, k, whi) in enumerate(specs):
        g = torch.Generator().manual_seed(100 + n)
        T = sum(lens)
        x = torch.randn(T, d, generator=g)
        W_V = torch.randn(G * dh, d, generator=g) / math.sqrt(d)
        alpha = torch.rand(H, generator=g) * 0.8 + 0.1
        w = torch.randint(1, whi + 1, (T,), generator=g).float()
        cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
        v = (x @ W_V.T).view(T, G, dh)
        scores, z_x, z_v = LT.hybrid_scores_per_head(x, W_V, alpha, H, dh)
        cu_list = [int(c) for c in cu]
        SEL._SEQ_META_CACHE.clear()
        idx, _, _ = SEL._compute_landmark_indices(x, W_V, alpha, w, cu, k, 1, T, cu_list,
                                                  head_dim=dh)
        cases[name] = dict(x=x.numpy(), W_V=W_V.numpy(), v=v.numpy(), alpha=alpha.numpy(),
                           w=w.numpy(), cu=cu.numpy(), k=np.int64(k), scores=scores.numpy(),
                           z_x=z_x.numpy(), z_v=z_v.numpy(), idx=_sort_sets(idx))
    return cases


def bf16_selection_cases(SEL):
    """bf16 selection at shapes like the benchmark workloads, shortened: the reference's own
    bf16 arithmetic (norms in bf16, z-statistics in float32 over the packed batch, torch.topk)
    on chosen value vectors: x = [v | h] and W_V = [I | 0], so x @ W_V^T reproduces v exactly
    in bf16.  Stored: the windows, the reference's float32 scores and sets, and the SHA-256 of
    the input bits (x is regenerated from its recipe, tests/helpers.py BF16_SELECT_SPECS)."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(OUT)))
    from tests.helpers import BF16_SELECT_SPECS, bf16_select_inputs, sha256_of
    out = {}
    for name, (seed, lens, H, dh, extra, k, wmax, heavy) in BF16_SELECT_SPECS.items():
        x, alpha, w, cu = bf16_select_inputs(name)
        T = x.shape[0]
        W_V = torch.cat([torch.eye(H * dh), torch.zeros(H * dh, extra)], 1).to(torch.bfloat16)
        assert torch.equal((x @ W_V.T), x[:, :H * dh])  # the value vectors, exactly
        SEL._SEQ_META_CACHE.clear()
        idx, z_x, z_v = SEL._compute_landmark_indices(x, W_V, alpha, w, cu, k, 1, T,
                                                      [int(c) for c in cu], head_dim=dh)
        scores = alpha * z_v + (1.0 - alpha) * z_x.unsqueeze(1)
        out[name] = dict(x_sha256=np.array(sha256_of(x)), w=w.numpy(), scores=scores.float().numpy(),
                         idx=_sort_sets(idx))
    return out


def literal_case(LT, SEL, SA, DA):
    g = torch.Generator().manual_seed(200)
    lens = [56, 40]
    T, d, H, dh, k = sum(lens), 16, 2, 8, 5
    x = torch.randn(T, d, generator=g)
    W_V = torch.randn(H * dh, d, generator=g) / 4.0
    alpha = torch.rand(H, generator=g) * 0.8 + 0.1
    w = torch.randint(1, 17, (T,), generator=g).float()
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    q = torch.randn(T, H, dh, generator=g)
    kk = torch.randn(T, H, dh, generator=g)
    vv = torch.randn(T, H, dh, generator=g)
    mask = DA._build_mask_packed(x, w, W_V, alpha, cu, T, k, dh, torch.device("cpu"))
    out = SA.sparse_attention_forward_packed(q, kk, vv, mask)
    SEL._SEQ_META_CACHE.clear()
    idx, _, _ = SEL._compute_landmark_indices(x, W_V, alpha, w, cu, k, 1, T,
                                              [int(c) for c in cu], head_dim=dh)
    return dict(x=x.numpy(), W_V=W_V.numpy(), v=(x @ W_V.T).view(T, H, dh).numpy(),
                alpha=alpha.numpy(), w=w.numpy(), cu=cu.numpy(), k=np.int64(k), q=q.numpy(),
                kk=kk.numpy(), vv=vv.numpy(), mask=np.packbits(mask.numpy(), axis=-1),
                out=out.numpy(), idx=_sort_sets(idx))


def window_cases(WU):
    g = torch.Generator().manual_seed(300)
    L = 40
    w1 = torch.randint(1, 50, (L,), generator=g).float()
    m1 = WU.build_local_window_mask(L, w1, torch.device("cpu"))
    lens = [23, 17, 30]
    T = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    w2 = torch.randint(1, 12, (T,), generator=g).float()
    m2 = WU.build_local_window_mask_packed(cu, w2, T, torch.device("cpu"))
    return dict(w1=w1.numpy(), m1=m1.numpy(), cu=cu.numpy(), w2=w2.numpy(), m2=m2.numpy())


def blockmap_cases(SEL):
    out = {}
    for n, (lens, bm) in enumerate([([100, 64, 1], 32), ([128], 64), ([5, 70, 33], 16)]):
        cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
        SEL._SEQ_BLOCK_MAP_CACHE.clear()
        m, tot = SEL._build_seq_block_map(cu, bm, torch.device("cpu"))
        out[f"cu{n}"] = cu.numpy()
        out[f"bm{n}"] = np.int64(bm)
        out[f"map{n}"] = m.numpy()
        out[f"tot{n}"] = np.int64(tot)
    return out


def gather_case(SEL):
    g = torch.Generator().manual_seed(400)
    lens = [20, 12]
    T, H, D, k = sum(lens), 3, 4, 5
    K = torch.randn(T, H, D, generator=g)
    V = torch.randn(T, H, D, generator=g)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    idx = torch.randint(0, 12, (H, 2, k), generator=g)
    idx[0, 1, 3:] = -1
    idx[2, 0, 0] = -1
    lk, lv = SEL._build_landmark_kv(K, V, idx, cu, k, H, D)
    return dict(K=K.numpy(), V=V.numpy(), cu=cu.numpy(), idx=idx.numpy(), lk=lk.numpy(),
                lv=lv.numpy())


def block_causal_case(CLC, gqa: bool, seed: int, T: int = 160, B: int = 32, dh: int = 8):
    g = torch.Generator().manual_seed(seed)
    d, H, k = 16, 4, 6
    G = 2 if gqa else H
    x = torch.randn(T, d, generator=g)
    W_V = torch.randn(G * dh, d, generator=g) / 4.0
    alpha = torch.rand(H, generator=g) * 0.8 + 0.1
    w = torch.randint(1, 41, (T,), generator=g).float()
    q = torch.randn(T, H, dh, generator=g)
    kk = torch.randn(T, H, dh, generator=g)
    vv = torch.randn(T, H, dh, generator=g)
    attn = types.SimpleNamespace(head_dim=dh, n_heads=H, k_lmk=k,
                                 v_proj=types.SimpleNamespace(weight=W_V))
    x_norm, xwv = CLC._token_signals(attn, x)
    covered = torch.arange(T) < w.long()
    sx, sv = CLC._prefix_stats(x_norm), CLC._prefix_stats(xwv)
    scale = 1.0 / math.sqrt(dh)
    sets, outs = [], []
    for b0 in range(0, T, B):
        b1 = min(T, b0 + B)
        lmk = CLC._select(attn, x_norm, xwv, covered, alpha, b0, sx, sv)
        sets.append(_sort_sets(lmk))
        outs.append(CLC._block_attention(q, kk, vv, w, lmk, b0, b1, scale).numpy())
    return dict(x=x.numpy(), W_V=W_V.numpy(), v=(x @ W_V.T).view(T, G, dh).numpy(),
                alpha=alpha.numpy(), w=w.numpy(), k=np.int64(k), block=np.int64(B),
                q=q.numpy(), kk=kk.numpy(), vv=vv.numpy(), sets=np.stack(sets, 1),
                out=np.concatenate(outs, 0))


def train_case(DA, seed: int = 600):
    """Training semantics: the dense log-bias of ``DSALTAttention._dense_logbias_from_kernel``
    (dsalt/modules/dsalt_attention.py:520-563: hard band ``0 <= d <= w~`` with the soft edge
    ``log sigmoid((w~ - d)/tau_win)`` outside the core ``d <= w~ - win_edge``, landmarks at
    ``lmk_pos`` weighted by ``lmk_logw`` where ``pos <= i`` and ``pos < i - w~``) fed to SDPA
    as in ``_packed_train`` (:488-518); float64 autograd gives the reference gradients of
    q, k, v, w~ and lmk_logw for a random cotangent."""
    g = torch.Generator().manual_seed(seed)
    N, L, H, D, K = 2, 48, 2, 8, 6
    tau_win, win_edge = 1.5, 4.0
    T = N * L
    q = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    kk = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    vv = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    w_cont = 1.0 + torch.rand(T, generator=g, dtype=torch.float64) * 18.0
    pos = torch.full((H, N, K), -1, dtype=torch.int64)
    for h in range(H):
        for s in range(N):
            n = K - (h + s) % 2
            pos[h, s, :n] = torch.randperm(L, generator=g)[:n]
    logw = torch.log(torch.sigmoid(torch.randn(H, N, K, generator=g, dtype=torch.float64)))
    logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf")))
    cot = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    ns = types.SimpleNamespace(n_heads=H, tau_win=tau_win, win_edge=win_edge)
    qr, kr, vr, wr, lr = (t.clone().requires_grad_(True) for t in (q, kk, vv, w_cont, logw))
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)  # the reference builds its -inf fills in the default dtype
    try:
        bias = DA.DSALTAttention._dense_logbias_from_kernel(ns, wr, pos, lr, N, L, torch.device("cpu"))
    finally:
        torch.set_default_dtype(prev)
    qb = qr.view(N, L, H, D).transpose(1, 2)
    kb = kr.view(N, L, H, D).transpose(1, 2)
    vb = vr.view(N, L, H, D).transpose(1, 2)
    ob = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=bias)
    out = ob.transpose(1, 2).reshape(T, H, D)
    (out * cot).sum().backward()
    return dict(q=q.numpy(), k=kk.numpy(), v=vv.numpy(), w_cont=w_cont.numpy(), lmk_pos=pos.numpy(),
                lmk_logw=logw.numpy(), tau_win=np.float64(tau_win), win_edge=np.float64(win_edge),
                cu=np.arange(0, T + 1, L, dtype=np.int32), cot=cot.numpy(), bias=bias.detach().numpy(),
                out=out.detach().numpy(), dq=qr.grad.numpy(), dk=kr.grad.numpy(), dv=vr.grad.numpy(),
                dw=wr.grad.numpy(), dlogw=lr.grad.numpy())


def main():
    LT, SEL, SA, WU, DA, CLC = _import_reference()
    for name, c in bf16_selection_cases(SEL).items():
        np.savez_compressed(os.path.join(OUT, f"select_bf16_{name}.npz"), **c)
    if "--only-bf16" in sys.argv:
        return
    np.savez_compressed(os.path.join(OUT, "train_dense.npz"), **train_case(DA))
    for name, c in selection_cases(LT, SEL).items():
        np.savez_compressed(os.path.join(OUT, f"select_{name}.npz"), **c)
    np.savez_compressed(os.path.join(OUT, "literal_fallback.npz"), **literal_case(LT, SEL, SA, DA))
    np.savez_compressed(os.path.join(OUT, "window_masks.npz"), **window_cases(WU))
    np.savez_compressed(os.path.join(OUT, "seq_block_map.npz"), **blockmap_cases(SEL))
    np.savez_compressed(os.path.join(OUT, "landmark_gather.npz"), **gather_case(SEL))
    np.savez_compressed(os.path.join(OUT, "block_causal_mha.npz"), **block_causal_case(CLC, False, 500))
    np.savez_compressed(os.path.join(OUT, "block_causal_gqa.npz"), **block_causal_case(CLC, True, 501))
    np.savez_compressed(os.path.join(OUT, "block_causal_b64.npz"),
                        **block_causal_case(CLC, True, 502, T=400, B=64, dh=64))
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()

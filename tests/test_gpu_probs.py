"""Sparse export of the attention probabilities (the metrics' _last_P) against the float64
oracle's dense matrix.  Tolerances (relative, max|a-b| / max|b|): 1e-5 fp32, 2e-2 bf16."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.kernels.attention_probs import SparseAttentionProbs
from oracle import attention as OA
from tests.helpers import f64, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _case(dt, mode, seed, lens=(700, 333), H=4, G=2, D=64, K=24, wmax=120, block=128):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(dt)
    k = torch.randn(T, G, D, generator=g).to(dt)
    v = torch.randn(T, G, D, generator=g).to(dt)
    w = torch.randint(1, wmax + 1, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    ns = ops.n_sets(mode, max(lens), block)
    idx = torch.full((H, len(lens), ns, K), -1, dtype=torch.int32)
    for hh in range(H):
        for s, L in enumerate(lens):
            for b in range(ns):
                hi = L if mode == ops.SELECT_GLOBAL else min(L, b * block)
                n = min(K - (hh % 2), hi)
                if n > 0:
                    idx[hh, s, b, :n] = torch.randperm(hi, generator=g)[:n].sort().values.to(torch.int32)
    bias = torch.randn(idx.shape, generator=g) * 0.5
    return q, k, v, w, cu, idx, bias, max(lens)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", [ops.SELECT_GLOBAL, ops.SELECT_BLOCK])
def test_export_matches_oracle_dense(dt, mode):
    q, k, v, w, cu, idx, bias, maxlen = _case(dt, mode, 60 + mode)
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    dv = [t.to(DEV) for t in (q, k, v, w, cu, idx, bias)]
    _, lse = ops.attention_forward(*dv[:6], dv[6], scale=scale, max_seqlen=maxlen, select_mode=mode, block_size=128)
    for seq in (0, 1):
        p_win, p_lmk = ops.export_probs(dv[0], dv[1], dv[3], dv[4], dv[5], lse, dv[6], seq=seq, scale=scale,
                                        max_seqlen=maxlen, select_mode=mode, block_size=128)
        sp = SparseAttentionProbs(p_win, p_lmk, dv[5][:, seq].long(), 128 if mode == ops.SELECT_BLOCK else 0)
        ref = OA.attention_probs(f64(q), f64(k), w.numpy(), cu.numpy(), idx.numpy(), scale, seq=seq,
                                 lmk_bias=bias.double().numpy(), block_size=128 if mode == ops.SELECT_BLOCK else None)
        dense = sp.to_dense()
        assert rel_err(f64(dense), ref) < TOL[dt]
        # metrics from the sparse form equal those of the dense matrix (trainer's formulas)
        rc = np.maximum(ref, 1e-9)
        ent_ref = -(rc * np.log(rc)).sum(-1)
        assert np.abs(f64(sp.row_entropy()) - ent_ref).max() < (1e-4 if dt == torch.float32 else 5e-2)
        assert np.abs(f64(sp.sink()) - ref[:, :, 0]).max() < TOL[dt]
        dd = dense.double().clamp(min=1e-9)
        assert torch.allclose(sp.row_entropy().double(), -(dd * dd.log()).sum(-1), atol=1e-5)


def test_layer_collects_last_P():
    from dsalt_amd.kernels import apply_rotary_emb, _compute_landmark_indices
    from dsalt_amd.modules import DSALTAttention
    torch.manual_seed(1)
    d, H, G, T = 256, 4, 2, 600
    m = DSALTAttention(d, H, 16, 96, 12, 1024, n_kv_heads=G).to(DEV).eval()
    m._collect_last_P = True
    x = torch.randn(T, d, device=DEV)
    cu = torch.tensor([0, 450, T], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        m(x, cu, cu_list=[0, 450, T])
        q = m.q_proj(x).view(T, H, 64)
        k = m.k_proj(x).view(T, G, 64)
        pos = torch.cat([torch.arange(450), torch.arange(T - 450)]).to(DEV)
        q, k = apply_rotary_emb(q, k, m.rope_cos[pos].unsqueeze(1), m.rope_sin[pos].unsqueeze(1))
        w = m._window_sizes(x, floor=True)
        lmk, _, _ = _compute_landmark_indices(x, m.v_proj.weight, m._alpha(), w, cu, 12, 16, T, [0, 450, T],
                                              head_dim=64)
    ref = OA.attention_probs(f64(q), f64(k), w.long().cpu().numpy(), cu.cpu().numpy(),
                             lmk.cpu().numpy()[:, :, None], 1 / 8.0, seq=0)
    assert m._last_P is not None and m._last_P.shape == (H, 450, 450)
    assert rel_err(f64(m._last_P), ref) < 1e-5
    met = m._last_P_sparse.metrics()
    assert 0 < met["eff_rank"] <= 450 and met["entropy"] > 0

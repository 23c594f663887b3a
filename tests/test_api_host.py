"""Host-side parts of the reference-named API (CPU): packed metadata and mask builders
against the reference's golden outputs."""
from __future__ import annotations

import numpy as np
import torch

from dsalt_amd.kernels import selectors as SEL
from dsalt_amd.kernels import window_utils as WU
from tests.helpers import load_golden


def test_seq_block_map_matches_reference():
    z = load_golden("seq_block_map")
    for n in range(3):
        m, tot = SEL._build_seq_block_map(torch.tensor(z[f"cu{n}"]), int(z[f"bm{n}"]), torch.device("cpu"))
        np.testing.assert_array_equal(m.numpy(), z[f"map{n}"])
        assert tot == int(z[f"tot{n}"])


def test_seq_block_map_cache_distinguishes_raggings():
    # the reference keys its cache on (total_len, num_seqs, block_m): these two collide there
    a, _ = SEL._build_seq_block_map(torch.tensor([0, 10, 100]), 16, torch.device("cpu"))
    b, _ = SEL._build_seq_block_map(torch.tensor([0, 90, 100]), 16, torch.device("cpu"))
    assert a.shape != b.shape or not torch.equal(a, b)


def test_seq_meta():
    cu = torch.tensor([0, 3, 8, 8, 12])
    n, lens, starts, seq_ids, seq_off, max_len = SEL._seq_meta(cu, 12, torch.device("cpu"))
    assert n == 4 and max_len == 5
    assert seq_ids.tolist() == [0, 0, 0, 1, 1, 1, 1, 1, 3, 3, 3, 3]
    assert seq_off.tolist() == [0, 1, 2, 0, 1, 2, 3, 4, 0, 1, 2, 3]


def test_window_masks_match_reference():
    z = load_golden("window_masks")
    m1 = WU.build_local_window_mask(z["m1"].shape[0], torch.tensor(z["w1"]), torch.device("cpu"))
    np.testing.assert_array_equal(m1.numpy(), z["m1"])
    T = int(z["cu"][-1])
    m2 = WU.build_local_window_mask_packed(torch.tensor(z["cu"]), torch.tensor(z["w2"]), T, torch.device("cpu"))
    np.testing.assert_array_equal(m2.numpy(), z["m2"])


def test_rope_cache_matches_closed_form():
    cos, sin = WU.build_rope_cache(16, 8, torch.device("cpu"), dtype=torch.float64, base=100.0)
    theta = 100.0 ** (-np.arange(0, 8, 2) / 8)
    ang = np.arange(16)[:, None] * np.concatenate([theta, theta])[None, :]
    np.testing.assert_allclose(cos.numpy(), np.cos(ang), atol=1e-12)
    q = torch.randn(16, 2, 8, dtype=torch.float64)
    qr, _ = WU.apply_rotary_emb(q, q, cos.unsqueeze(1), sin.unsqueeze(1))
    # a rotation keeps every 2-d pair's norm
    np.testing.assert_allclose((qr[..., :4] ** 2 + qr[..., 4:] ** 2).numpy(),
                               (q[..., :4] ** 2 + q[..., 4:] ** 2).numpy(), atol=1e-12)


def _zscore(n):
    return (n - n.mean(0, keepdim=True)) / n.std(0, keepdim=True).clamp(min=1e-6)


def test_zscore_gradient_closed_form_matches_autograd():
    from dsalt_amd.kernels.landmark_tokens_ker import _norm_grad, _zscore_grad
    g = torch.Generator().manual_seed(3)
    for shape, const in (((97, 3), False), ((40, 1), True), ((2, 2), False)):
        n = (torch.rand(shape, generator=g, dtype=torch.float64) * 3 + 1).requires_grad_(True)
        if const:  # std 0: clamped, the std term carries no gradient
            n = torch.full(shape, 2.5, dtype=torch.float64, requires_grad=True)
        up = torch.randn(shape, generator=g, dtype=torch.float64)
        z = _zscore(n)
        (z * up).sum().backward()
        got = _zscore_grad(up, z.detach(), n.detach())
        assert torch.allclose(got, n.grad, rtol=1e-10, atol=1e-12)
    vec = torch.randn(30, 4, 8, generator=g, dtype=torch.float64)
    vec[3, 1] = 0.0
    vr = vec.clone().requires_grad_(True)
    dn = torch.randn(30, 4, generator=g, dtype=torch.float64)
    (vr.norm(dim=-1) * dn).sum().backward()
    got = _norm_grad(dn, vec, vec.norm(dim=-1))
    assert torch.allclose(got, vr.grad, atol=1e-12)


def test_autotune_candidates_describe_the_compiled_tilings():
    from dsalt_amd.kernels import autotune as AT
    c64 = AT._candidate_configs(64, None, 2)
    assert c64[0] == AT._heuristic_config(64, None, 2) and c64[0]["variant"] == 0
    assert len({c["variant"] for c in c64}) == len(c64) >= 5
    by = {c["variant"]: c for c in c64}
    assert by[AT.VARIANT_FWD_BN32]["BLOCK_N"] == 32 and by[0]["BLOCK_N"] == 64
    assert by[AT.VARIANT_FWD_RG2]["BLOCK_M"] == 128 and by[AT.VARIANT_DQ_BN64]["BLOCK_N_BWD"] == 64
    assert by[AT.VARIANT_LMK_SHORT]["LMK_ROWS"] == 512
    # 16-bit head_dim 128: two row groups per wave or 64-key chunks in the forward
    c128 = {c["variant"]: c for c in AT._candidate_configs(128, None, 2)}
    assert list(c128) == [0, AT.VARIANT_FWD_RG2, AT.VARIANT_FWD_BN64, AT.VARIANT_FWD_8W, AT.VARIANT_LMK_SHORT]
    assert c128[AT.VARIANT_FWD_8W]["BLOCK_M"] == 128 and c128[AT.VARIANT_FWD_8W]["BLOCK_N"] == 32
    assert c128[0]["BLOCK_N"] == 32 and c128[AT.VARIANT_FWD_BN64]["BLOCK_N"] == 64
    assert c128[AT.VARIANT_FWD_RG2]["BLOCK_M"] == 128 and c128[AT.VARIANT_FWD_RG2]["BLOCK_N"] == 32
    # fp32 shapes have one compiled tiling: only the landmark-chunk choice
    assert [c["variant"] for c in AT._candidate_configs(128, None, 4)] == [0, AT.VARIANT_LMK_SHORT]
    assert AT.get_tuned_config.__name__ == "get_tuned_config"


def test_head_dim_padding_helpers():
    """head_dims up to 128 map to the compiled 64 / 128 and pad with zero columns."""
    import pytest as _pt
    import torch as _t
    from dsalt_amd.kernels.dsalt_attn import pad_head_dim, padded_head_dim
    assert [padded_head_dim(d) for d in (1, 32, 64, 65, 96, 128)] == [64, 64, 64, 128, 128, 128]
    for bad in (0, 129, 256):
        with _pt.raises(ValueError):
            padded_head_dim(bad)
    x = _t.randn(5, 3, 40)
    y = pad_head_dim(x, 64)
    assert y.shape == (5, 3, 64) and _t.equal(y[..., :40], x) and not y[..., 40:].any()
    assert pad_head_dim(y, 64) is y

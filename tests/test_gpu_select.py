"""Landmark selection on the GPU against the oracle: indices bit-exact, z and scores
bit-exact (same canonical arithmetic)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate
from oracle import select as OS
from tests.helpers import bits, oracle_dtype

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(T_lens, hidden, G, D, H, dt, wmax, seed, scale_tails=False):
    g = torch.Generator().manual_seed(seed)
    T = sum(T_lens)
    h = torch.randn(T, hidden, generator=g)
    v = torch.randn(T, G, D, generator=g)
    if scale_tails:
        v = v * torch.exp(torch.randn(T, G, 1, generator=g))
        h = h * torch.exp(0.5 * torch.randn(T, 1, generator=g))
    alpha = torch.rand(H, generator=g) * 0.8 + 0.1
    w = torch.randint(1, wmax + 1, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(T_lens)), dtype=torch.int32)
    return h.to(dt), v.to(dt), alpha, w, cu


def _run(h, v, alpha, w, cu, k, mode, block, scope, want=True, border_cap=None):
    dev = [t.to(DEV) for t in (h, v, alpha, w, cu)]
    maxlen = int((cu[1:] - cu[:-1]).max())
    res = ops.select_landmarks(*dev, k, max_seqlen=maxlen, select_mode=mode, block_size=block,
                               stats_scope=scope, want_scores=want and mode == ops.SELECT_GLOBAL,
                               border_cap=border_cap)
    torch.cuda.synchronize()
    ref = OS.select(bits(h), bits(v), alpha.numpy(), w.numpy(), cu.numpy(), k, oracle_dtype(h.dtype), mode=mode,
                    block_size=block, stats_scope=scope, want_scores=want and mode == ops.SELECT_GLOBAL)
    return res, ref


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("scope", [ops.STATS_PACKED, ops.STATS_SEQUENCE])
def test_global_select_bit_exact(dt, scope):
    h, v, alpha, w, cu = _case([300, 517, 64], 256, 4, 64, 8, dt, 40, seed=1)
    (idx, zx, zv, sc), (ridx, rzx, rzv, rsc) = _run(h, v, alpha, w, cu, 24, ops.SELECT_GLOBAL, 512, scope)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(zx.cpu().numpy(), rzx)
    np.testing.assert_array_equal(zv.cpu().numpy(), rzv)
    np.testing.assert_array_equal(sc.cpu().numpy(), rsc)


@pytest.mark.parametrize("scope", [ops.STATS_PACKED, ops.STATS_SEQUENCE])
@pytest.mark.parametrize("want", [False, True])
def test_global_select_long_sequences(scope, want):
    """Sequences longer than 32768 tokens take their statistics from one sel_sums pass instead
    of every top-k part (with or without z and scores for the caller): indices, z and scores
    bit-exact, next to a short sequence of the same batch."""
    h, v, alpha, w, cu = _case([70001, 3000], 256, 2, 64, 4, torch.bfloat16, 300, seed=11)
    res, ref = _run(h, v, alpha, w, cu, 128, ops.SELECT_GLOBAL, 512, scope, want=want)
    for a, b in zip(res if want else (res,), ref if want else (ref,)):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_block_select_bit_exact(dt, D):
    h, v, alpha, w, cu = _case([1000, 700], 128, 2, D, 4, dt, 100, seed=2)
    idx, ridx = _run(h, v, alpha, w, cu, 32, ops.SELECT_BLOCK, 128, ops.STATS_PACKED, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("dt,hidden,D", [(torch.bfloat16, 100, 100), (torch.float16, 1000, 20), (torch.float32, 98, 30)])
def test_row_widths_off_the_vector_size(dt, hidden, D):
    # hidden / head_dim widths that are not whole 16-byte vectors: the operator zero-pads the
    # rows (zero columns change no norm), indices, z and scores stay bit-exact with the oracle
    # on the unpadded rows
    h, v, alpha, w, cu = _case([300, 517], hidden, 2, D, 4, dt, 60, seed=8)
    for mode in (ops.SELECT_GLOBAL, ops.SELECT_BLOCK):
        res, ref = _run(h, v, alpha, w, cu, 24, mode, 100, ops.STATS_SEQUENCE)
        if mode == ops.SELECT_GLOBAL:
            for a_, b_ in zip(res, ref):
                np.testing.assert_array_equal(a_.cpu().numpy(), b_)
        else:
            np.testing.assert_array_equal(res.cpu().numpy(), ref)


def test_padding_when_few_candidates():
    h, v, alpha, w, cu = _case([90], 64, 1, 64, 2, torch.bfloat16, 200, seed=3)
    w[:] = 80  # only positions >= 80 are candidates: 10 of them
    idx, ridx = _run(h, v, alpha, w, cu, 16, ops.SELECT_GLOBAL, 512, ops.STATS_PACKED, want=False)
    got = idx.cpu().numpy()
    np.testing.assert_array_equal(got, ridx)
    assert (got[:, 0, 0, 10:] == -1).all() and (got[:, 0, 0, :10] >= 80).all()


def _tie_case():
    # integer-valued inputs: many exactly equal norms, so selections cut through large tie groups
    g = torch.Generator().manual_seed(4)
    T = 2000
    h = torch.randint(-1, 2, (T, 64), generator=g).float().to(torch.bfloat16)
    v = torch.randint(-1, 2, (T, 2, 64), generator=g).float().to(torch.bfloat16)
    alpha = torch.tensor([0.5, 0.5, 1.0, 0.0])
    w = torch.randint(1, 50, (T,), generator=g, dtype=torch.int32)
    cu = torch.tensor([0, 1200, T], dtype=torch.int32)
    return h, v, alpha, w, cu


@pytest.mark.parametrize("cap", [1, 7, 64, None])
def test_ties_global_many_parts_and_merge_levels(cap):
    # global sets: small caps sort 16-candidate parts and merge 2 or 7 parts per block
    # (several merge levels); None is the production plan
    idx, ridx = _run(*_tie_case(), 50, ops.SELECT_GLOBAL, 512, ops.STATS_PACKED, want=False, border_cap=cap)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("cap", [1, 7, 64])
def test_ties_block_small_boundary_capacity(cap):
    # block-causal sets: the radix boundary bin limited to `cap` keys forces extra passes
    idx, ridx = _run(*_tie_case(), 50, ops.SELECT_BLOCK, 256, ops.STATS_PACKED, want=False, border_cap=cap)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_constant_scores_pick_lowest_indices():
    T = 500
    h = torch.ones(T, 64, dtype=torch.bfloat16)
    v = torch.ones(T, 1, 64, dtype=torch.bfloat16)
    alpha = torch.tensor([0.3])
    w = torch.full((T,), 5, dtype=torch.int32)
    cu = torch.tensor([0, T], dtype=torch.int32)
    idx, ridx = _run(h, v, alpha, w, cu, 20, ops.SELECT_GLOBAL, 512, ops.STATS_PACKED, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(idx.cpu().numpy()[0, 0, 0], np.arange(5, 25))


@pytest.mark.parametrize("name", ["fwd_f32_h4_l2048", "fwdbwd_bf16_b4_h8_l8192", "fwdbwd_bf16_h16_l32768",
                                  "train_bf16_h16_l32768"])
def test_workload_selection_bit_exact(name):
    wl = WORKLOADS[name]
    x = generate(wl)
    v = x["v"]
    scope = ops.STATS_SEQUENCE
    idx, ridx = _run(x["h"], v, x["alpha"], x["w"], x["cu"], wl.k_lmk, ops.SELECT_GLOBAL, 512, scope, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_block_workload_selection_bit_exact_shortened():
    wl = WORKLOADS["fwd_bf16_h16_l131072_block"]
    x = generate(wl, seqlen=8192, heads=4)
    idx, ridx = _run(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, ops.SELECT_BLOCK, 512,
                     ops.STATS_SEQUENCE, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_block_workload_selection_bit_exact_long_prefixes():
    # prefixes of up to 64K candidates take the sampled-threshold path
    wl = WORKLOADS["fwd_bf16_h16_l131072_block"]
    x = generate(wl, seqlen=65536, heads=2)
    idx, ridx = _run(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, ops.SELECT_BLOCK, 512,
                     ops.STATS_SEQUENCE, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_block_sampled_path_packed_sequences_gqa():
    # several sequences (one empty) whose later sets hold 8192+ candidates: the sampled
    # threshold, packed norms with their exclusion flags and the order statistics run at
    # nonzero sequence starts, with two query heads per value head
    h, v, alpha, w, cu = _case([20000, 0, 17000], 128, 2, 64, 4, torch.bfloat16, 300, seed=5)
    idx, ridx = _run(h, v, alpha, w, cu, 64, ops.SELECT_BLOCK, 512, ops.STATS_SEQUENCE, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


# Block-causal candidate pruning (a candidate that k earlier candidates dominate in both
# norms is dropped before the sets' scans) forced on short sequences: the selection must
# stay bit-exact against the oracle, which never prunes.
def test_block_pruned_packed_sequences_gqa():
    h, v, alpha, w, cu = _case([20000, 0, 17000], 128, 2, 64, 4, torch.bfloat16, 300, seed=5)
    idx, ridx = _run(h, v, alpha, w, cu, 64, ops.SELECT_BLOCK, 512, ops.STATS_SEQUENCE, want=False,
                     border_cap=ops.SELECT_FORCE_PRUNE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_block_pruned_alpha_outside_unit_interval():
    # heads with alpha outside [0, 1] (a norm weighted negatively) must scan whole prefixes
    h, v, alpha, w, cu = _case([12000, 9000], 128, 2, 64, 4, torch.bfloat16, 300, seed=9, scale_tails=True)
    alpha[0], alpha[1], alpha[2] = 1.5, -0.25, 1.0
    idx, ridx = _run(h, v, alpha, w, cu, 32, ops.SELECT_BLOCK, 512, ops.STATS_SEQUENCE, want=False,
                     border_cap=ops.SELECT_FORCE_PRUNE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


def test_block_pruned_workload_shortened():
    wl = WORKLOADS["fwd_bf16_h16_l131072_block"]
    x = generate(wl, seqlen=16384, heads=4)
    idx, ridx = _run(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, ops.SELECT_BLOCK, 512,
                     ops.STATS_SEQUENCE, want=False, border_cap=ops.SELECT_FORCE_PRUNE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("K,scope", [(600, ops.STATS_SEQUENCE), (2048, ops.STATS_PACKED)])
def test_global_select_large_sets(K, scope):
    # more than 512 landmarks per set: per-part keys of up to 2048, merges of two parts, a
    # sequence with fewer candidates than slots
    h, v, alpha, w, cu = _case([6000, 1500, 900], 128, 2, 64, 4, torch.bfloat16, 300, seed=17)
    (idx, zx, zv, sc), (ridx, rzx, rzv, rsc) = _run(h, v, alpha, w, cu, K, ops.SELECT_GLOBAL, 512, scope)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(sc.cpu().numpy(), rsc)


@pytest.mark.parametrize("K,block,cap", [(700, 1024, None), (1500, 2048, None), (700, 1024, "prune")])
def test_block_select_large_sets(K, block, cap):
    # block-causal sets of more than 512 landmarks: all-in-LDS, sampled-threshold and radix
    # paths, and with forced pruning the survivor lists
    h, v, alpha, w, cu = _case([12000, 3000], 128, 2, 64, 4, torch.bfloat16, 300, seed=19)
    idx, ridx = _run(h, v, alpha, w, cu, K, ops.SELECT_BLOCK, block, ops.STATS_SEQUENCE, want=False,
                     border_cap=ops.SELECT_FORCE_PRUNE if cap else None)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("block", [1, 37, 100, 200])
def test_block_select_any_block_size(block):
    # block sizes that are not multiples of 64 (sets start at any token), an empty sequence
    h, v, alpha, w, cu = _case([700, 0, 413], 96, 2, 64, 4, torch.bfloat16, 120, seed=13)
    idx, ridx = _run(h, v, alpha, w, cu, 16, ops.SELECT_BLOCK, block, ops.STATS_SEQUENCE, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("block", [64, 128, 37, 100])
def test_block_pruned_block_sizes(block):
    # small block sizes (many sets, each reading its survivor count at its start, any token)
    h, v, alpha, w, cu = _case([9000, 6000], 128, 2, 64, 4, torch.bfloat16, 300, seed=11, scale_tails=True)
    idx, ridx = _run(h, v, alpha, w, cu, 32, ops.SELECT_BLOCK, block, ops.STATS_SEQUENCE, want=False,
                     border_cap=ops.SELECT_FORCE_PRUNE)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)


@pytest.mark.parametrize("name", ["b4_h8", "h16"])
def test_bf16_selection_against_the_reference_scores(name):
    """The GPU's bf16 selection on the fixtures of the reference's own bf16 arithmetic:
    bit-exact to the C oracle, and a top-k of the reference's scores in every set."""
    from tests.helpers import BF16_SELECT_SPECS, bf16_select_inputs, load_golden, sha256_of, topk_violations
    z = load_golden(f"select_bf16_{name}")
    x, alpha, _, cu = bf16_select_inputs(name)
    assert sha256_of(x) == str(z["x_sha256"])
    w = torch.from_numpy(z["w"])
    _, lens, H, dh, _, k, _, _ = BF16_SELECT_SPECS[name]
    T = x.shape[0]
    v = x[:, :H * dh].reshape(T, H, dh)
    idx, ridx = _run(x, v, alpha, w.int(), cu, k, ops.SELECT_GLOBAL, 512, ops.STATS_PACKED, want=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    bad, _ = topk_violations(idx.cpu().numpy()[:, :, 0], z["scores"], w, cu, k)
    assert bad == 0

"""dsalt_fwd_noalloc: the forward with its row plan in the library's static device scratch
(no allocation, no workspace), called through the C ABI.  Its outputs must equal
dsalt_fwd's bit for bit (the same kernels), on two calls in a row, the second with a
smaller input, and on random configurations (block-causal sets, biases, tiling variants); sizes
beyond the scratch are rejected before anything runs."""
from __future__ import annotations

import ctypes

import pytest
import torch

from dsalt_amd import _lib, ops
from tests.test_gpu_attention import _inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(q, k, v, w, cu, idx, maxlen):
    a, out, lse, keep = ops._fwd_args(q, k, v, w, cu, idx, None, None, maxlen, ops.SELECT_GLOBAL, 512)
    return a, out, lse, keep


@pytest.mark.parametrize("dt,D", [(torch.bfloat16, 64), (torch.float32, 128)])
def test_noalloc_forward_equals_forward_twice(dt, D):
    L = _lib.load()
    for lens, seed in (([1500, 700, 333], 70), ([300, 120], 71)):  # second call: a smaller input
        q, k, v, w, cu, idx, _, maxlen = _inputs(lens, 4, 2, D, 40, 250, dt, seed)
        dev = [t.to(DEV) for t in (q, k, v, w, cu, idx)]
        ref_out, ref_lse = ops.attention_forward(*dev, None, max_seqlen=maxlen)
        a, out, lse, keep = _args(*dev, maxlen)
        a.workspace, a.workspace_bytes = None, 0
        stream = torch.cuda.current_stream().cuda_stream
        _lib.check("dsalt_fwd_noalloc", L.dsalt_fwd_noalloc(ctypes.byref(a), stream))
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)


def test_noalloc_rejects_plans_beyond_the_scratch():
    L = _lib.load()
    a = _lib.FwdArgs()
    # 32768 sequences of 64 tokens: 32768 plan tiles, more than the scratch holds
    a.p = _lib.Problem(32768 * 64, 32768, 64, 2, 2, 64, 8, 0, 0, _lib.DTYPE_BF16)
    fake = 1 << 20
    a.q = a.k = a.v = a.out = fake
    a.q_stride_t = a.k_stride_t = a.v_stride_t = a.o_stride_t = 128
    a.q_stride_h = a.k_stride_h = a.v_stride_h = a.o_stride_h = 64
    a.w = a.cu_seqlens = a.lmk_idx = a.lse = fake
    a.scale = 0.125
    assert L.dsalt_plan_bytes(ctypes.byref(a.p)) > _lib.FWD_NOALLOC_MAX_PLAN_BYTES
    assert L.dsalt_fwd_noalloc(ctypes.byref(a), None) == 3
    assert b"scratch" in L.dsalt_last_error()


@pytest.mark.parametrize("seed", range(8))
def test_noalloc_random_configurations(seed):
    """Random configurations of the other entry points' sweep (global or block-causal sets of
    any block size, landmark biases, any tiling variant bits): the allocation-free forward equals
    dsalt_fwd bit for bit."""
    from tests.test_gpu_sweep import api_inputs, draw_api
    c = draw_api(seed)
    print("case", {k: (str(v) if k == "dt" else v) for k, v in c.items()}, flush=True)
    x = api_inputs(c)
    mode, bs, maxlen = c["mode"], c["bs"], max(c["lens"])
    d = [x[n].to(DEV) for n in ("q", "k", "v", "w", "cu", "idx", "bias")]
    ref_out, ref_lse = ops.attention_forward(*d, max_seqlen=maxlen, select_mode=mode, block_size=bs,
                                             variant=c["variant"])
    L = _lib.load()
    a, out, lse, keep = ops._fwd_args(*d, None, maxlen, mode, bs)
    a.variant = c["variant"]
    assert L.dsalt_plan_bytes(ctypes.byref(a.p)) <= _lib.FWD_NOALLOC_MAX_PLAN_BYTES
    a.workspace, a.workspace_bytes = None, 0
    _lib.check("dsalt_fwd_noalloc", L.dsalt_fwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)

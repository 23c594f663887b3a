"""Seeded synthetic inputs for the operator workloads used by the benchmark and tests.

Each workload is generated on the CPU with ``torch.Generator().manual_seed(seed)`` in
float32 and then cast, so the bits handed to the GPU and to any CPU check are identical.
Draw order: q, k, v, h, window normals, upstream gradient.
Windows: ``w_i = clamp(round_half_even(sigmoid(z_i) * w_max), 16, w_max)``.
Landmark score: alpha = 0.5 for every head (the same ranking as z(|v|) + z(|h|)) unless the
workload states another value.
Training workloads draw the same tensors and keep the windows continuous,
``w~_i = clamp(sigmoid(z_i) * w_max, 16, w_max)``; their hard selection uses ``floor(w~)``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    heads: int
    seqlen: int
    head_dim: int
    hidden: int
    dtype: torch.dtype
    w_max: int
    k_lmk: int
    backward: bool
    select_mode: str = "global"  # or "block"
    block_size: int = 512
    heavy_tails: bool = False    # v rows x lognormal(0,1), h rows x lognormal(0,0.5)
    seed: int = 1000
    train: bool = False          # training variant: soft window edge, landmark log-weights
    tau_win: float = 1.0
    win_edge: float = 4.0
    tau_lmk: float = 2.0
    kv_heads: int = 0            # key/value heads (0: as many as query heads)
    alpha: float = 0.5           # landmark score weight of every head

    @property
    def n_kv(self) -> int:
        return self.kv_heads or self.heads

    @property
    def total_len(self) -> int:
        return self.batch * self.seqlen


WORKLOADS = {
    w.name: w
    for w in [
        # forward only, fp32, masked-SDPA size the CPU path handles in full
        Workload("fwd_f32_h4_l2048", 1, 4, 2048, 64, 256, torch.float32, 128, 32, False, seed=1000),
        # forward + backward, bf16, 4 packed sequences of 8192 (70M-class layer)
        Workload("fwdbwd_bf16_b4_h8_l8192", 4, 8, 8192, 64, 512, torch.bfloat16, 256, 64, True, seed=1001),
        # forward + backward, bf16, one 32K sequence, heavy-tailed norms
        Workload("fwdbwd_bf16_h16_l32768", 1, 16, 32768, 64, 1024, torch.bfloat16, 512, 128, True,
                 heavy_tails=True, seed=1002),
        # the same tensors through the training variant (differentiable selectors)
        Workload("train_bf16_h16_l32768", 1, 16, 32768, 64, 1024, torch.bfloat16, 512, 128, True,
                 heavy_tails=True, seed=1002, train=True),
        # forward (inference), bf16, 128K tokens, block-causal landmarks (512-query blocks)
        Workload("fwd_bf16_h16_l131072_block", 1, 16, 131072, 128, 2048, torch.bfloat16, 512, 256, False,
                 select_mode="block", block_size=512, seed=1003),
        # forward (inference) of one decoder layer's attention shaped like the Qwen2.5-3B
        # graft: 16 query heads, 2 key/value heads (GQA, read in place), head_dim 128,
        # hidden 2048, block-causal landmarks k=128 in 512-query blocks, alpha 0.6 (the
        # layer's initial value)
        Workload("fwd_bf16_h16kv2_l32768_block", 1, 16, 32768, 128, 2048, torch.bfloat16, 512, 128, False,
                 select_mode="block", block_size=512, seed=1004, kv_heads=2, alpha=0.6),
    ]
}


def make_windows(z: torch.Tensor, w_max: int) -> torch.Tensor:
    w = torch.round(torch.sigmoid(z) * w_max)
    return w.clamp(16, w_max).to(torch.int32)


def generate(wl: Workload, device="cpu", seqlen: int | None = None, heads: int | None = None):
    """Inputs of a workload as a dict of tensors on ``device``.

    ``seqlen`` / ``heads`` shrink the shape for tests while keeping the recipe.
    Keys: q [T,H,D]; k, v [T,n_kv,D]; h [T,hidden]; w [T] int32; cu [S+1] int32; alpha [H] fp32;
    dout [T,H,D] (backward workloads); w_cont [T] fp32 (training workloads, with w = floor).
    """
    L = seqlen or wl.seqlen
    H = heads or wl.heads
    G = max(1, H * wl.n_kv // wl.heads)
    T = wl.batch * L
    g = torch.Generator().manual_seed(wl.seed)
    q = torch.randn(T, H, wl.head_dim, generator=g)
    k = torch.randn(T, G, wl.head_dim, generator=g)
    v = torch.randn(T, G, wl.head_dim, generator=g)
    h = torch.randn(T, wl.hidden, generator=g)
    zw = torch.randn(T, generator=g)
    if wl.heavy_tails:
        v = v * torch.exp(torch.randn(T, G, 1, generator=g))
        h = h * torch.exp(0.5 * torch.randn(T, 1, generator=g))
    out = dict(
        q=q.to(wl.dtype), k=k.to(wl.dtype), v=v.to(wl.dtype), h=h.to(wl.dtype),
        w=make_windows(zw, wl.w_max),
        cu=torch.arange(0, T + 1, L, dtype=torch.int32),
        alpha=torch.full((H,), wl.alpha, dtype=torch.float32),
    )
    if wl.train:
        out["w_cont"] = (torch.sigmoid(zw) * wl.w_max).clamp(16, wl.w_max).to(torch.float32)
        out["w"] = out["w_cont"].floor().to(torch.int32)
    if wl.backward:
        out["dout"] = torch.randn(T, H, wl.head_dim, generator=g).to(wl.dtype)
    return {kk: vv.to(device) for kk, vv in out.items()}


@dataclass(frozen=True)
class ModelWorkload:
    """A whole-model prefill: random-init weights of a named shape, random token ids."""
    name: str
    batch: int
    seqlen: int
    dtype: torch.dtype
    seed: int = 2000

    def config(self):
        from .model import qwen25_3b_config
        return qwen25_3b_config(max_seq_len=self.seqlen)


MODEL_WORKLOADS = {
    w.name: w
    for w in [
        # Qwen2.5-3B-shaped DSALT decoder (36 layers, hidden 2048, 16/2 heads, head_dim 128,
        # SwiGLU 11008, vocab 151936), block-causal landmarks k=128, w_max=512, prefill of 32K
        ModelWorkload("prefill_qwen3b_l32768", 1, 32768, torch.bfloat16),
    ]
}

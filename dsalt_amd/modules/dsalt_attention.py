"""DSALT attention layer on MI355X.

Mirrors ``DSALTAttention`` of ``dsalt/modules/dsalt_attention.py:147-704`` (constructor,
parameters and ``forward(x, cu_seqlens, max_seqlen, rope_cs, cu_list) -> (out, aux)``).
Inference branch of ``_packed`` (:610-634):
  * one fused q/k/v projection GEMM (the three weights concatenated, cached until a
    weight changes) and RoPE applied in place to its q and k columns by a HIP kernel;
    the attention reads q, k and v through strides from that one buffer (no [T, H, D]
    copies, no materialised GQA repeat);
  * windows ``w = floor(n_min + sigmoid(win_gate(x)) (n_max - n_min))``, at least 1
    (:277-284), and ``alpha = sigmoid(alpha_w)`` (:228, :243-244);
  * landmark selection (``_compute_landmark_indices``, on ``x W_V^T`` without the bias as
    in the reference) and the sparse operator with zero landmark bias (:622).
``select_mode="block"`` switches to block-causal landmarks (``block_size`` query rows per
set, statistics of the prefix), the variant of ``results/causal_landmark_check.py:150-189``.
Batched ``[B, T, d]`` input is run as ``B`` packed sequences of length ``T``.

Training branch (``self.training``, :597-603, :440-487): the differentiable selectors --
continuous windows ``w~ = n_min + sigmoid(win_gate(x)) (n_max - n_min)`` (gradient to
``win_gate`` through the soft window edge) and landmark log-weights
``log sigmoid(s / tau_lmk)`` of the hybrid score at the hard-selected positions (gradient to
``alpha_w``, ``x`` and ``v_proj``) -- feed the training attention kernels.  Global landmark
sets only, as in the reference.

Analysis export (:636-702): with ``_collect_last_P`` set (off by default: it costs a kernel
and O(L (w + k)) memory per layer), eval-mode inference stores the first sequence's
attention probabilities as ``_last_P_sparse`` (``kernels.attention_probs``: window band +
landmark slots, the probabilities the forward used) and, for sequences up to
``last_P_dense_max`` tokens, the dense ``[H, L, L]`` matrix as ``_last_P`` for callers that
index it like the reference's.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from ..kernels.dsalt_attn import dsalt_attention, pad_head_dim, padded_head_dim
from ..kernels.dsalt_train import dsalt_train_attention
from ..kernels.landmark_tokens_ker import hybrid_scores_per_head
from ..kernels.selectors import _compute_landmark_indices
from ..kernels.window_utils import apply_rotary_emb, build_rope_cache


class DSALTAttention(nn.Module):
    def __init__(self, d_model: int, n_heads: int, n_min: int, n_max: int, k_lmk: int, max_seq_len: int,
                 dropout: float = 0.0, yarn_scale: float = 1.0, layer_idx: int = 0, n_kv_heads: int | None = None,
                 qkv_bias: bool = False, rope_base: float = 10000.0, select_mode: str = "global",
                 block_size: int = 512, stats_scope: str = "packed"):
        super().__init__()
        assert d_model % n_heads == 0
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.n_kv_heads = n_kv_heads if n_kv_heads is not None else n_heads
        assert n_heads % self.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads"
        self.n_rep = n_heads // self.n_kv_heads
        self.kv_dim = self.n_kv_heads * self.head_dim
        self.n_min, self.n_max, self.k_lmk = n_min, n_max, k_lmk
        self.max_seq_len = max_seq_len
        self.dropout = dropout
        self.yarn_scale = yarn_scale
        self.rope_base = rope_base
        self.layer_idx = layer_idx
        self.select_mode = select_mode
        self.block_size = block_size
        self.stats_scope = stats_scope
        self.q_proj = nn.Linear(d_model, d_model, bias=qkv_bias)
        self.k_proj = nn.Linear(d_model, self.kv_dim, bias=qkv_bias)
        self.v_proj = nn.Linear(d_model, self.kv_dim, bias=qkv_bias)
        self.out_proj = nn.Linear(d_model, d_model, bias=False)
        self.win_gate = nn.Linear(d_model, 1, bias=True)
        self.alpha_w = nn.Parameter(torch.full((n_heads,), math.log(0.6 / 0.4)))
        self.tau_win, self.tau_lmk, self.win_edge = 1.0, 2.0, 4
        self._last_P = None
        self._collect_last_P = False
        self._qkv_cache = None
        self._last_P_sparse = None
        self.last_P_dense_max = 4096
        cos, sin = build_rope_cache(max_seq_len, self.head_dim, torch.device("cpu"), base=rope_base, scale=yarn_scale)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def _alpha(self) -> torch.Tensor:
        return torch.sigmoid(self.alpha_w)

    def _window_continuous(self, x: torch.Tensor) -> torch.Tensor:
        return self.n_min + torch.sigmoid(self.win_gate(x).squeeze(-1)) * (self.n_max - self.n_min)

    @torch.no_grad()
    def _window_sizes(self, x: torch.Tensor, floor: bool) -> torch.Tensor:
        w = self._window_continuous(x)
        return (w.floor() if floor else w.round()).clamp(min=1)

    def _aux_zero(self, device, dtype):
        return torch.zeros((), device=device, dtype=dtype)

    def _apply_out_proj(self, out: torch.Tensor) -> torch.Tensor:
        return self.out_proj(out.to(self.out_proj.weight.dtype))

    @torch.no_grad()
    def warmup(self, device) -> None:
        was = self.training
        self.eval()
        n = max(self.n_min * 2, 64)
        x = torch.randn(n, self.d_model, device=device, dtype=self.q_proj.weight.dtype)
        self._packed(x, torch.tensor([0, n], dtype=torch.int32, device=device), n, device, cu_list=[0, n])
        torch.cuda.synchronize(device)
        self.train(was)

    def forward(self, x, cu_seqlens=None, max_seqlen=None, rope_cs=None, cu_list=None):
        if cu_seqlens is not None:
            return self._packed(x, cu_seqlens, x.shape[0], x.device, rope_cs, cu_list)
        B, T, _ = x.shape
        cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=x.device)
        out, aux = self._packed(x.reshape(B * T, -1), cu, B * T, x.device, None, list(range(0, (B + 1) * T, T)))
        return out.view(B, T, -1), aux

    def _train_selectors(self, x, cu_seqlens, total_len, device, cu_list=None):
        """``(w_cont [T], lmk_pos [H, S, k] int64, lmk_logw [H, S, k])`` of the training branch
        (``dsalt_attention.py:457-487``): hard landmark positions from the floored windows,
        log-weights differentiable in ``alpha_w`` (and in ``x`` / ``v_proj`` through the
        hybrid score), windows differentiable in ``win_gate``."""
        w_cont = self._window_continuous(x)
        alpha = self._alpha()
        with torch.no_grad():
            w_disc = w_cont.floor().clamp(min=1)
            lmk_pos, _, _ = _compute_landmark_indices(x.detach(), self.v_proj.weight.detach(),
                                                      alpha.detach().float(), w_disc, cu_seqlens, self.k_lmk,
                                                      self.n_min, total_len, cu_list, head_dim=self.head_dim,
                                                      stats_scope=self.stats_scope)
        scores, _, _ = hybrid_scores_per_head(x, self.v_proj.weight, alpha, self.n_heads, self.head_dim)
        starts = cu_seqlens[:-1].to(device).long()
        abs_pos = starts[None, :, None] + lmk_pos.clamp(min=0)
        head_ix = torch.arange(self.n_heads, device=device)[:, None, None]
        s_sel = scores[abs_pos, head_ix]
        lmk_logw = torch.log(torch.sigmoid(s_sel / self.tau_lmk).clamp(min=1e-20))
        lmk_logw = torch.where(lmk_pos >= 0, lmk_logw, torch.full_like(lmk_logw, float("-inf")))
        return w_cont, lmk_pos, lmk_logw

    def _packed_train_triton(self, q, k, v, x, cu_seqlens, total_len, device, cu_list=None):
        """Differentiable sparse training attention (``dsalt_attention.py:440-455``)."""
        if self.select_mode != "global":
            raise NotImplementedError("the training branch takes global landmark sets (select_mode='global')")
        w_cont, lmk_pos, lmk_logw = self._train_selectors(x, cu_seqlens, total_len, device, cu_list)
        return dsalt_train_attention(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win=self.tau_win,
                                     win_edge=float(self.win_edge), n_max=self.n_max, cu_list=cu_list)

    def _fused_qkv_weight(self):
        """Concatenated [W_q; W_k; W_v] (and biases), rebuilt when a projection changes."""
        ps = [m.weight for m in (self.q_proj, self.k_proj, self.v_proj)]
        bs = [m.bias for m in (self.q_proj, self.k_proj, self.v_proj)]
        key = tuple((t.data_ptr(), t._version, t.dtype) for t in ps + [b for b in bs if b is not None])
        if self._qkv_cache is None or self._qkv_cache[0] != key:
            with torch.no_grad():
                w = torch.cat(ps)
                b = torch.cat(bs) if bs[0] is not None else None
            self._qkv_cache = (key, w, b)
        return self._qkv_cache[1], self._qkv_cache[2]

    def _rope_tables32(self):
        """The RoPE tables as float32 (the buffers follow the module's dtype; values already
        rounded to a 16-bit type round to themselves again in the kernel)."""
        c, s = self.rope_cos, self.rope_sin
        if c.dtype == torch.float32:
            return c, s
        key = (c.data_ptr(), c._version, s.data_ptr(), s._version)
        if getattr(self, "_rope32", None) is None or self._rope32[0] != key:
            self._rope32 = (key, c.float(), s.float())
        return self._rope32[1], self._rope32[2]

    @torch.no_grad()
    def _packed_inference(self, x, cu_seqlens, total_len, device, rope_cs=None, cu_list=None):
        H, G, D = self.n_heads, self.n_kv_heads, self.head_dim
        w_qkv, b_qkv = self._fused_qkv_weight()
        qkv = F.linear(x, w_qkv, b_qkv)                                            # [T, (H + 2G) D]
        q = qkv[:, :H * D].view(total_len, H, D)
        k = qkv[:, H * D:(H + G) * D].view(total_len, G, D)
        v = qkv[:, (H + G) * D:].view(total_len, G, D)
        maxlen = ops._max_seqlen(cu_seqlens, cu_list)
        if rope_cs is None:
            cos, sin = self._rope_tables32()
            ops.rope_qk_(q, k, cu_seqlens, cos, sin, max_seqlen=maxlen)
        else:  # rows already gathered per token: token t reads row t
            cu1 = torch.tensor([0, total_len], dtype=torch.int32, device=device)
            ops.rope_qk_(q, k, cu1, rope_cs[0].float(), rope_cs[1].float(), max_seqlen=total_len)
        w = self._window_sizes(x, floor=True)
        lmk, _, _ = _compute_landmark_indices(x, self.v_proj.weight, self._alpha().float(), w, cu_seqlens, self.k_lmk,
                                              self.n_min, total_len, cu_list, head_dim=D, select_mode=self.select_mode,
                                              block_size=self.block_size, stats_scope=self.stats_scope)
        idx = lmk.to(torch.int32) if lmk.dim() == 4 else lmk.to(torch.int32).unsqueeze(2)
        mode = ops.SELECT_BLOCK if self.select_mode == "block" else ops.SELECT_GLOBAL
        w32 = w.to(torch.int32)
        # head_dims other than the compiled 64 / 128 run zero-padded, scaled by the true head_dim
        dp = padded_head_dim(D)
        if dp != D:
            q, k, v = (pad_head_dim(t, dp) for t in (q, k, v))
        scale = 1.0 / math.sqrt(D)
        out, lse = ops.attention_forward(q, k, v, w32, cu_seqlens, idx, None, scale=scale, max_seqlen=maxlen,
                                         select_mode=mode, block_size=self.block_size)
        if dp != D:
            out = out[..., :D].contiguous()
        self._last_P = self._last_P_sparse = None
        if self._collect_last_P:
            self._export_last_P(q, k, w32, cu_seqlens, idx, lse, maxlen, mode, cu_list, scale)
        return self._apply_out_proj(out.view(total_len, self.d_model)), self._aux_zero(x.device, x.dtype)

    def _export_last_P(self, q, k, w32, cu_seqlens, idx, lse, maxlen, mode, cu_list, scale):
        """Attention probabilities of the first sequence (sparse; dense when short)."""
        from ..kernels.attention_probs import SparseAttentionProbs
        cu_h = list(cu_list) if cu_list is not None else cu_seqlens.detach().to("cpu").tolist()
        n0 = cu_h[1] - cu_h[0]
        p_win, p_lmk = ops.export_probs(q, k, w32, cu_seqlens, idx, lse, seq=0, rows=n0, seq_len=n0,
                                        w_cap=max(1, min(n0, self.n_max + 1)), scale=scale, max_seqlen=maxlen,
                                        select_mode=mode, block_size=self.block_size)
        sp = SparseAttentionProbs(p_win, p_lmk, idx[:, 0].long(), self.block_size if mode == ops.SELECT_BLOCK else 0)
        self._last_P_sparse = sp
        if n0 <= self.last_P_dense_max:
            self._last_P = sp.to_dense()

    def _packed(self, x, cu_seqlens, total_len, device, rope_cs=None, cu_list=None):
        if not self.training and not torch.is_grad_enabled():
            return self._packed_inference(x, cu_seqlens, total_len, device, rope_cs, cu_list)
        q = self.q_proj(x).view(total_len, self.n_heads, self.head_dim)
        k = self.k_proj(x).view(total_len, self.n_kv_heads, self.head_dim)
        v = self.v_proj(x).view(total_len, self.n_kv_heads, self.head_dim)
        if rope_cs is None:
            cu = cu_seqlens.long()
            lens = cu[1:] - cu[:-1]
            seq_ids = torch.repeat_interleave(torch.arange(lens.numel(), device=device), lens)
            pos = torch.arange(total_len, device=device) - cu[:-1][seq_ids]
            cos, sin = self.rope_cos[pos], self.rope_sin[pos]
        else:
            cos, sin = rope_cs
        cos, sin = cos.to(q.dtype), sin.to(q.dtype)
        q, k = apply_rotary_emb(q, k, cos.unsqueeze(1), sin.unsqueeze(1))
        self._last_P = None
        if self.training:
            out = self._packed_train_triton(q.contiguous(), k.contiguous(), v.contiguous(), x, cu_seqlens,
                                            total_len, device, cu_list)
            return self._apply_out_proj(out.view(total_len, self.d_model)), self._aux_zero(x.device, x.dtype)
        w = self._window_sizes(x, floor=True)
        alpha = self._alpha()
        lmk, _, _ = _compute_landmark_indices(x.detach(), self.v_proj.weight.detach(), alpha.detach().float(), w,
                                              cu_seqlens, self.k_lmk, self.n_min, total_len, cu_list,
                                              head_dim=self.head_dim, select_mode=self.select_mode,
                                              block_size=self.block_size, stats_scope=self.stats_scope)
        out = dsalt_attention(q.contiguous(), k.contiguous(), v.contiguous(), lmk, None, w, cu_seqlens,
                              cu_list=cu_list, block_size=self.block_size)
        self._last_P = None
        return self._apply_out_proj(out.view(total_len, self.d_model)), self._aux_zero(x.device, x.dtype)

"""Sparse export of the attention matrix behind the reference's analysis metrics.

The reference keeps, in eval mode, the dense ``[H, L, L]`` attention matrix of the first
sequence (``DSALTAttention._last_P``, ``dsalt/modules/dsalt_attention.py:636-702``) for the
trainer's metrics (``dsalt/training/trainer.py:88-135,186-190``: effective rank and second
singular value of the head mean, row entropy with probabilities clamped at 1e-9, the
spread of the per-head entropy, and the attention sink P[:, :, 0]).  Here the library
exports only the attended entries (``dsalt_export_probs``: the window band and the landmark
slots, O(L (w + k)) memory) and this class computes the same metrics from them; the dense
matrix is rebuilt on request (``to_dense``), e.g. for the SVD.

Deliberate difference: the values are the probabilities the forward used (its landmark
sets and float32 scores), where the reference re-selects landmarks in float32 for the first
sequence alone and recomputes the scores in the input dtype.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class SparseAttentionProbs:
    p_win: torch.Tensor             # [H, L, W]: p_win[h, i, c] = P(i, i - c), 0 past the row's window
    p_lmk: torch.Tensor | None      # [H, L, K]: P(i, landmark of the slot), 0 when not visible
    lmk_pos: torch.Tensor | None    # [H, n_sets, K] int64 landmark positions (sequence-relative, -1 empty)
    block_size: int = 0             # query rows per landmark set (0: one set per sequence)

    @property
    def n_heads(self) -> int:
        return self.p_win.shape[0]

    @property
    def length(self) -> int:
        return self.p_win.shape[1]

    def _lmk_cols(self) -> torch.Tensor:
        """[H, L, K] key column of every landmark slot of every row (-1 empty)."""
        H, L = self.n_heads, self.length
        if self.block_size:
            sets = (torch.arange(L, device=self.p_win.device) // self.block_size).clamp(max=self.lmk_pos.shape[1] - 1)
            return self.lmk_pos[:, sets]
        return self.lmk_pos[:, 0:1].expand(H, L, self.lmk_pos.shape[-1])

    def to_dense(self) -> torch.Tensor:
        """The dense [H, L, L] float32 attention matrix."""
        H, L, W = self.p_win.shape
        dev = self.p_win.device
        dense = torch.zeros(H, L, L + 1, dtype=torch.float32, device=dev)  # column L collects padding
        i = torch.arange(L, device=dev)[:, None]
        col = i - torch.arange(W, device=dev)[None, :]
        col = torch.where(col >= 0, col, torch.full_like(col, L))
        dense.scatter_add_(2, col.expand(H, L, W), self.p_win)
        if self.p_lmk is not None:
            lc = self._lmk_cols()
            lc = torch.where(lc >= 0, lc, torch.full_like(lc, L))
            dense.scatter_add_(2, lc, self.p_lmk)
        return dense[:, :, :L]

    def row_entropy(self, eps: float = 1e-9) -> torch.Tensor:
        """[H, L] entropy of every row, -sum_j max(P, eps) log max(P, eps) over all L keys
        (the trainer's clamp): stored entries plus the zeros of the unstored columns."""
        def g(p):
            c = p.clamp(min=eps)
            return c * c.log()
        H, L, W = self.p_win.shape
        s = g(self.p_win).sum(-1)
        n_stored = W
        if self.p_lmk is not None:
            s = s + g(self.p_lmk).sum(-1)
            n_stored += self.p_lmk.shape[-1]
        return -(s + (L - n_stored) * (eps * math.log(eps)))

    def sink(self) -> torch.Tensor:
        """[H, L] probability each row puts on key 0."""
        H, L, W = self.p_win.shape
        dev = self.p_win.device
        i = torch.arange(L, device=dev)
        out = torch.zeros(H, L, dtype=torch.float32, device=dev)
        m = i < W
        out[:, m] = self.p_win[:, m, i[m]]
        if self.p_lmk is not None:
            out = out + (self.p_lmk * (self._lmk_cols() == 0)).sum(-1)
        return out

    def metrics(self, eps: float = 1e-9) -> dict:
        """The trainer's metrics of this matrix: sigma2 and effective rank of the head mean
        (dense SVD), mean row entropy, std over heads of the per-head entropy, sink."""
        ent = self.row_entropy(eps)
        sv = torch.linalg.svdvals(self.to_dense().mean(dim=0))
        svn = sv / (sv.sum() + 1e-9)
        per_head = ent.mean(dim=-1)
        return {"sigma2": sv[1].item() if sv.shape[0] > 1 else 0.0,
                "eff_rank": torch.exp(-(svn * (svn + 1e-9).log()).sum()).item(),
                "entropy": ent.mean().item(),
                "head_spec_std": per_head.std(correction=0).item(),
                "sink": self.sink().mean().item()}

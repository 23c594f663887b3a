"""Serializable configuration of the DSALT language model.

Mirrors ``DSALTConfig`` of ``dsalt/model/config.py:10-91`` (same fields, defaults, checks
and JSON round trip), plus the attention layer's landmark variant: ``select_mode``
("global" or "block"), ``block_size`` and ``stats_scope``.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, fields
from pathlib import Path


@dataclass
class DSALTConfig:
    vocab_size: int
    d_model: int
    n_layers: int
    n_heads: int
    n_min: int
    n_max: int
    k_lmk: int
    max_seq_len: int
    d_ff: int | None = None
    dropout: float = 0.0
    yarn_scale: float = 1.0
    tie_weights: bool = True
    n_kv_heads: int | None = None
    qkv_bias: bool = False
    rope_base: float = 10000.0
    padding_idx: int | None = None
    lm_head_chunk_size: int = 2048
    loss_fn: str = "chunked"
    aux_loss_weight: float = 0.0
    select_mode: str = "global"
    block_size: int = 512
    stats_scope: str = "packed"

    def __post_init__(self) -> None:
        if self.d_model % self.n_heads != 0:
            raise ValueError(f"{self.n_heads} heads do not split a model width of {self.d_model} evenly")
        if not (0 <= self.n_min <= self.n_max):
            raise ValueError(f"window bounds out of order: n_min={self.n_min}, n_max={self.n_max} (need 0 <= n_min <= n_max)")
        if self.k_lmk < 0:
            raise ValueError(f"negative landmark count k_lmk={self.k_lmk}")
        if self.n_kv_heads is not None and (self.n_kv_heads <= 0 or self.n_heads % self.n_kv_heads != 0):
            raise ValueError(f"n_heads ({self.n_heads}) must be a positive multiple of n_kv_heads "
                             f"({self.n_kv_heads}) for grouped-query attention")
        if self.loss_fn not in ("auto", "chunked", "liger"):
            raise ValueError(f"unknown loss_fn {self.loss_fn!r} (one of 'auto', 'chunked', 'liger')")
        if self.select_mode not in ("global", "block"):
            raise ValueError(f"select_mode must be 'global' or 'block', got {self.select_mode!r}")

    def to_dict(self) -> dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, data: dict) -> "DSALTConfig":
        known = {f.name for f in fields(cls)}
        return cls(**{k: v for k, v in data.items() if k in known})

    def save(self, path: str | Path) -> None:
        Path(path).write_text(json.dumps(self.to_dict(), indent=2), encoding="utf-8")

    @classmethod
    def load(cls, path: str | Path) -> "DSALTConfig":
        return cls.from_dict(json.loads(Path(path).read_text(encoding="utf-8")))


def qwen25_3b_config(max_seq_len: int = 32768, **overrides) -> DSALTConfig:
    """The Qwen2.5-3B shape the DSALT graft uses: 36 layers, hidden 2048, 16 query heads
    and 2 key/value heads (head_dim 128), SwiGLU 11008, vocab 151936, q/k/v bias, RoPE base
    1e6, tied embeddings; DSALT windows up to 512 with block-causal landmarks (k = 128)."""
    cfg = dict(vocab_size=151936, d_model=2048, n_layers=36, n_heads=16, n_kv_heads=2, n_min=32, n_max=512,
               k_lmk=128, max_seq_len=max_seq_len, d_ff=11008, qkv_bias=True, rope_base=1e6, tie_weights=True,
               select_mode="block", block_size=512)
    cfg.update(overrides)
    return DSALTConfig(**cfg)

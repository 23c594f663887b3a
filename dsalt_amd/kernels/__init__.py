"""Kernel-level API of DSALT on MI355X, under the names of ``dsalt/kernels/__init__.py``.

Every compute entry point runs the gfx950 HIP library (``libdsalt_amd.so``); there is no CPU
fallback.  ``_HIP_OK`` tells whether the library is loadable; ``_TRITON_OK`` is kept as an
alias of it so code that tests the reference's flag picks the GPU path.
"""
from .autotune import autotune_blocks, get_tuned_config
from .dsalt_attn import DSALTAttentionFunction, dsalt_attention, dsalt_triton_attention
from .dsalt_bwd import dsalt_backward, dsalt_triton_backward
from .dsalt_train import DSALTTrainFunction, dsalt_train_attention, dsalt_triton_train_attention
from .landmark_tokens_ker import hybrid_scores_per_head
from .selectors import _build_landmark_kv, _build_seq_block_map, _compute_landmark_indices, _seq_meta
from .sparse_attn import sparse_attention_forward, sparse_attention_forward_packed
from .window_utils import (apply_rotary_emb, build_local_window_mask, build_local_window_mask_packed,
                           build_rope_cache)


def _library_loadable() -> bool:
    try:
        from .._lib import load
        load()
        return True
    except Exception:
        return False


_HIP_OK = _library_loadable()
_TRITON_OK = _HIP_OK

__all__ = [
    "dsalt_attention", "dsalt_triton_attention", "DSALTAttentionFunction",
    "dsalt_backward", "dsalt_triton_backward",
    "dsalt_train_attention", "dsalt_triton_train_attention", "DSALTTrainFunction",
    "hybrid_scores_per_head", "_compute_landmark_indices", "_build_landmark_kv", "_seq_meta",
    "_build_seq_block_map", "sparse_attention_forward", "sparse_attention_forward_packed",
    "build_local_window_mask", "build_local_window_mask_packed", "apply_rotary_emb", "build_rope_cache",
    "autotune_blocks", "get_tuned_config",
]

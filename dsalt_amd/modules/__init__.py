"""Layers built on the DSALT operator."""
from .dsalt_attention import DSALTAttention

__all__ = ["DSALTAttention"]

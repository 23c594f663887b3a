"""The DSALT language model (the reference's dsalt.model names)."""
from .config import DSALTConfig, qwen25_3b_config
from .dsalt_lm import DSALTLMHeadModel

__all__ = ["DSALTConfig", "DSALTLMHeadModel", "qwen25_3b_config"]

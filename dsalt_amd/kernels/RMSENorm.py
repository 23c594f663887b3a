"""RMSNorm with the reference's name and numerics.

Mirrors ``RMSENorm`` of ``dsalt/kernels/RMSENorm.py:6-21``: ``F.rms_norm`` over the last
dimension with a learnable per-channel scale (the input promoted to float32 with the float32
weight), the result cast back to the input dtype.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSENorm(nn.Module):
    def __init__(self, d_model: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))
        self.normalized_shape = (d_model,)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, self.normalized_shape, self.weight, self.eps).to(x.dtype)

"""RMSENorm of dsalt/kernels/RMSENorm.py:6-22 (the LM consumer's norm).

``F.rms_norm`` over the last dimension with a learnable per-channel scale; the result is
returned in the input's dtype (F.rms_norm promotes a 16-bit input with an fp32 weight).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSENorm(nn.Module):
    def __init__(self, d_model: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.normalized_shape = (d_model,)
        self.weight = nn.Parameter(torch.ones(d_model))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = F.rms_norm(x, self.normalized_shape, self.weight, self.eps)
        return y if y.dtype == x.dtype else y.to(x.dtype)

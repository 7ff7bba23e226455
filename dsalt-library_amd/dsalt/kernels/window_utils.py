"""RoPE helpers used by DSALTAttention upstream of the sparse-attention kernels.

``build_rope_cache`` and ``apply_rotary_emb`` follow dsalt/kernels/window_utils.py:73-107
(half-split rotation, positions divided by the YaRN scale). The reference wraps
``apply_rotary_emb`` in ``torch.compile``; here it runs eagerly, so no generated
kernels enter the path.
"""
from __future__ import annotations

import torch


def apply_rotary_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate ``q`` and ``k`` with the precomputed ``(cos, sin)`` (half-split convention)."""
    half = q.shape[-1] // 2

    def _rot(x: torch.Tensor) -> torch.Tensor:
        return torch.cat([-x[..., half:], x[..., :half]], dim=-1)

    return q * cos + _rot(q) * sin, k * cos + _rot(k) * sin


def build_rope_cache(seq_len: int, head_dim: int, device: torch.device,
                     dtype: torch.dtype = torch.float32, base: float = 10000.0,
                     scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE ``(cos, sin)`` of shape ``[seq_len, head_dim]``; ``scale`` divides positions."""
    theta = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device, dtype=dtype) / head_dim))
    positions = torch.arange(seq_len, device=device, dtype=dtype) / scale
    emb = torch.cat([torch.outer(positions, theta)] * 2, dim=-1)
    return emb.cos(), emb.sin()

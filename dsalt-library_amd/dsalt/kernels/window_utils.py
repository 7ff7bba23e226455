"""RoPE helpers used by DSALTAttention upstream of the sparse-attention kernels.

``build_rope_cache`` and ``apply_rotary_emb`` follow dsalt/kernels/window_utils.py:73-107
(half-split rotation, positions divided by the YaRN scale). The reference wraps
``apply_rotary_emb`` in ``torch.compile``; here it runs eagerly, so no generated
kernels enter the path. The module itself uses :func:`apply_rotary_emb_packed`, the
HIP kernel ``dsalt_rope`` (one pass over q and k, positions from cu_seqlens in-kernel,
the compiled function's fp32 arithmetic with one rounding), with its transposed
rotation as the backward.
"""
from __future__ import annotations

import torch

from .. import _hip


class _RopeFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin, cu_seqlens):
        ctx.save_for_backward(cos, sin, cu_seqlens)
        ctx.has_cu = cu_seqlens is not None
        return _hip.rope(q, k, cos, sin, cu_seqlens)

    @staticmethod
    def backward(ctx, gq, gk):
        cos, sin, cu = ctx.saved_tensors
        q_shape, k_shape = gq.shape if gq is not None else None, gk.shape if gk is not None else None
        gq = gq if gq is not None else torch.zeros(q_shape or gk.shape, device=gk.device, dtype=gk.dtype)
        gk = gk if gk is not None else torch.zeros(k_shape or gq.shape, device=gq.device, dtype=gq.dtype)
        dq, dk = _hip.rope(gq, gk, cos, sin, cu if ctx.has_cu else None, transpose=True)
        return dq, dk, None, None, None


def rotate_packed(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  cu_seqlens: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE of one packed tensor ``[T, H, D]`` with the HIP kernel (no autograd): for the
    inference path, where only k is rotated ahead of the attention kernel (which rotates q
    itself) and for the first-sequence diagnostic."""
    return _hip.rope(None, x, cos, sin, cu_seqlens)[1]


def apply_rotary_emb_packed(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                            cu_seqlens: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE of packed ``q [T, Hq, D]``, ``k [T, Hk, D]`` on the GPU (differentiable in q and
    k). ``cos``/``sin`` are fp32 tables ``[rows, D]``: with ``cu_seqlens`` row p is the
    position p inside a sequence (the module's rope_cos / rope_sin,
    dsalt_attention.py:570-585); without, row t is token t (the module's ``rope_cs``).
    They are rounded to q's dtype, as the module's ``cos.to(q.dtype)`` does."""
    return _RopeFunction.apply(q, k, cos, sin, cu_seqlens)


def compute_window_sizes(x_prev: torch.Tensor, n_min: int, n_max: int) -> torch.Tensor:
    """A fixed window ``(n_min + n_max) // 2`` for each of the ``x_prev.shape[0]`` tokens,
    fp32 on ``x_prev``'s device (window_utils.py:4-16 of the reference; the module predicts
    its windows with ``win_gate`` instead)."""
    return torch.full((x_prev.shape[0],), float((n_min + n_max) // 2), dtype=torch.float32, device=x_prev.device)


def _band(rows: torch.Tensor, starts: torch.Tensor, w: torch.Tensor, n_cols: int) -> torch.Tensor:
    """Boolean ``[len(rows), n_cols]``: row r admits columns ``max(starts[r], rows[r] - w[r] + 1)
    .. rows[r]`` (absolute indices)."""
    lo = torch.maximum(rows - w + 1, starts)
    cols = torch.arange(n_cols, device=rows.device)
    return (cols[None, :] >= lo[:, None]) & (cols[None, :] <= rows[:, None])


def build_local_window_mask(seq_len: int, window_sizes: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Causal local-window mask ``[T, T]`` of one sequence, True = attend: row i admits
    keys ``max(0, i - w_i + 1) .. i`` with ``w_i`` clamped to ``[1, T]`` and truncated
    to an integer (window_utils.py:19-38 of the reference)."""
    rows = torch.arange(seq_len, device=device)
    w = window_sizes.to(device).clamp(min=1, max=seq_len).long()
    return _band(rows, torch.zeros_like(rows), w, seq_len)


def build_local_window_mask_packed(cu_seqlens: torch.Tensor, window_sizes: torch.Tensor, total_len: int,
                                   device: torch.device) -> torch.Tensor:
    """Local-window mask ``[T, T]`` over packed sequences, True = attend: token t of a
    sequence starting at s admits ``max(s, t - w_t + 1) .. t`` (``w_t`` clamped below at 1,
    truncated), so never a key of another sequence (window_utils.py:41-70 of the
    reference)."""
    cu = cu_seqlens.to(device=device, dtype=torch.long)
    lens = cu[1:] - cu[:-1]
    starts = torch.repeat_interleave(cu[:-1], lens, output_size=total_len)
    rows = torch.arange(total_len, device=device)
    w = window_sizes.to(device).clamp(min=1).long()
    return _band(rows, starts, w, total_len)


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

"""DSALT inference attention (HARD selectors) on the gfx950 HIP kernels.

Drop-in for dsalt/kernels/dsalt_triton_attn.py: same entry point
``dsalt_triton_attention(q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens)`` and the
same ``DSALTAttentionFunction`` (returns fp32 output, gradients in q's dtype; fp32
inputs compute as fp16, dsalt_triton_attn.py:259-328). The module name is kept for
import compatibility; nothing here uses Triton.

Semantics (dsalt_triton_attn.py:69-169): query i of a sequence attends to keys
``[i - w + 1, i]`` with ``w = max(1, trunc(w_sizes[i]))`` and to landmark slot p when
``0 <= p <= i - w``, with logit ``q.k / sqrt(D) + lmk_bias[h, s, slot]``.
"""
from __future__ import annotations

import torch

from .. import _hip
from . import _sparse
from .autotune import autotune_blocks, get_tuned_config  # noqa: F401  (re-exports)
from .dsalt_triton_bwd import dsalt_triton_backward  # noqa: F401
from .landmark_tokens_ker import hybrid_scores_per_head  # noqa: F401
from .selectors import (  # noqa: F401  (re-exported like the reference, :18-24)
    _build_landmark_kv,
    _build_seq_block_map,
    _compute_landmark_indices,
    _score_block,
    _seq_meta,
)


class DSALTAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens):
        return _sparse._forward(ctx, _hip.MODE_HARD, q, k, v, lmk_indices, lmk_bias, w_sizes,
                                cu_seqlens, 1.0, 4.0, out_f32=True)

    @staticmethod
    def backward(ctx, grad_out):
        dq, dk, dv, d_bias, _ = _sparse._backward(ctx, grad_out, need_dw=False)
        return dq, dk, dv, None, d_bias, None, None


def _dynamo_opaque(fn):
    disable = getattr(getattr(torch, "_dynamo", None), "disable", None)
    return disable(fn) if disable is not None else fn


@_dynamo_opaque
def dsalt_triton_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    lmk_indices: torch.Tensor,
    lmk_bias: torch.Tensor,
    w_sizes: torch.Tensor,
    cu_seqlens: torch.Tensor,
) -> torch.Tensor:
    """HARD DSALT attention over packed ``[T, H, D]`` q/k/v; returns fp32 ``[T, H, D]``."""
    return DSALTAttentionFunction.apply(q, k, v, lmk_indices, lmk_bias, w_sizes, cu_seqlens)

"""Dense-mask attention helpers exported by dsalt.kernels (dsalt/kernels/sparse_attn.py:5-57
of the reference).

These are generic utilities: boolean ``[.., T, T]`` mask in, ``scaled_dot_product_attention``
out, on whatever device the tensors live. They are kept so that code importing them from
``dsalt.kernels`` keeps working. The DSALT attention path never calls them: the module and
``dsalt_triton_attention`` run the HIP kernels only and raise ``DsaltError`` without them.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _additive(mask: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """0 where ``mask`` is True (attend), -inf elsewhere, in ``dtype``."""
    zero = torch.zeros((), dtype=dtype, device=mask.device)
    return torch.where(mask, zero, torch.full((), float("-inf"), dtype=dtype, device=mask.device))


def sparse_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: torch.Tensor,
                             dropout_p: float = 0.0, training: bool = False) -> torch.Tensor:
    """Masked SDPA on batched ``[B, H, T, D]`` tensors; ``attn_mask`` is boolean
    ``[T, T]``, ``[H, T, T]`` (broadcast over the batch) or ``[B, H, T, T]``, True =
    attend. Dropout applies only when ``training``."""
    bias = _additive(attn_mask, q.dtype)
    if bias.dim() == 3:
        bias = bias[None]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=bias, dropout_p=dropout_p if training else 0.0)


def sparse_attention_forward_packed(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: torch.Tensor,
                                    dropout_p: float = 0.0, training: bool = False) -> torch.Tensor:
    """Masked SDPA on packed ``[T, H, D]`` tensors with one boolean ``[T, T]`` mask shared
    by every head; returns a contiguous ``[T, H, D]``."""
    def heads_first(t: torch.Tensor) -> torch.Tensor:
        return t.permute(1, 0, 2)[None]  # [1, H, T, D]

    out = F.scaled_dot_product_attention(heads_first(q), heads_first(k), heads_first(v),
                                         attn_mask=_additive(attn_mask, q.dtype)[None, None],
                                         dropout_p=dropout_p if training else 0.0)
    return out[0].permute(1, 0, 2).contiguous()

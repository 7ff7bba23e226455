"""Hybrid-energy landmark score (the single definition of the DSALT selection score).

For token j and head h::

    s[j, h] = alpha_h * z(||x_j W_V,h||_2) + (1 - alpha_h) * z(||x_j||_2)

where z(.) standardises over all T packed tokens (mean and unbiased std, the std
clamped at 1e-6). Mirrors ``hybrid_scores_per_head`` of
dsalt/kernels/landmark_tokens_ker.py:19-61 (same signature, same arithmetic order:
the norms are taken in the input dtype and upcast to fp32). The ``x @ W_V^T`` product
is a plain library GEMM (hipBLASLt through torch); its fp32 output feeds the HIP
selection kernel, which is bit-exact with respect to these scores.
"""
from __future__ import annotations

import torch


def hybrid_scores_per_head(
    x: torch.Tensor,
    W_V: torch.Tensor,
    alpha: torch.Tensor,
    n_heads: int,
    dh: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-head hybrid score and the standardised signals.

    Args:
        x: hidden states ``[T, d]``.
        W_V: value projection ``[n_kv_heads*dh, d]`` (``v_proj.weight``).
        alpha: per-head balance ``[n_heads]`` in (0, 1).
        n_heads: number of query heads (width of the returned score).
        dh: per-head dimension.

    Returns ``(scores [T, n_heads], z_x [T], z_v [T, n_heads])``; under GQA the value
    norm is computed per kv group and repeated to the query heads of each group
    (landmark_tokens_ker.py:56-59).
    """
    T = x.shape[0]
    x_norm = x.norm(dim=-1).float()
    z_x = (x_norm - x_norm.mean()) / x_norm.std().clamp(min=1e-6)

    n_kv = W_V.shape[0] // dh
    xwv = (x @ W_V.T).view(T, n_kv, dh).norm(dim=-1).float()
    mu_v = xwv.mean(0, keepdim=True)
    std_v = xwv.std(0, keepdim=True).clamp(min=1e-6)
    z_v = (xwv - mu_v) / std_v
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)

    scores = alpha * z_v + (1.0 - alpha) * z_x.unsqueeze(1)
    return scores, z_x, z_v


def hybrid_scores_from_v(
    x: torch.Tensor,
    v: torch.Tensor,
    alpha: torch.Tensor,
    n_heads: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The same score from the value projection ``v = x W_V^T`` ``[T, n_kv, dh]``
    (pre-RoPE, as the attention module computes it), without a second GEMM.

    Differentiable in x, v (hence W_V) and alpha; identical arithmetic to
    :func:`hybrid_scores_per_head` once ``v`` equals its ``x @ W_V.T``. The no-gradient
    selection path uses the HIP kernel ``dsalt_hybrid_scores`` instead
    (:func:`dsalt._hip.hybrid_scores`).
    """
    x_norm = x.norm(dim=-1).float()
    z_x = (x_norm - x_norm.mean()) / x_norm.std().clamp(min=1e-6)

    n_kv = v.shape[1]
    xwv = v.norm(dim=-1).float()
    mu_v = xwv.mean(0, keepdim=True)
    std_v = xwv.std(0, keepdim=True).clamp(min=1e-6)
    z_v = (xwv - mu_v) / std_v
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)

    scores = alpha * z_v + (1.0 - alpha) * z_x.unsqueeze(1)
    return scores, z_x, z_v

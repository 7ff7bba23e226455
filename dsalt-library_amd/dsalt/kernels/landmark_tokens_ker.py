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
import torch.nn as nn


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


def compute_hybrid_scores(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    """The hybrid score under the older ``(x, W_V, alpha)`` signature
    (landmark_tokens_ker.py:64-84 of the reference).

    A 0-d ``alpha`` scores whole vectors: ``alpha * z(||x W_V^T||) + (1 - alpha) * z(||x||)``
    over the T rows, returned as ``[T]``. A vector ``alpha [n_heads]`` is the per-head
    score of :func:`hybrid_scores_per_head` with ``dh = W_V.shape[0] // n_heads``,
    returned as ``[T, n_heads]``.
    """
    if alpha.ndim > 0:
        n_heads = alpha.shape[0]
        return hybrid_scores_per_head(x, W_V, alpha, n_heads, W_V.shape[0] // n_heads)[0]

    def standardise(t: torch.Tensor) -> torch.Tensor:
        return (t - t.mean()) / t.std().clamp(min=1e-6)

    return alpha * standardise((x @ W_V.T).norm(dim=-1)) + (1.0 - alpha) * standardise(x.norm(dim=-1))


def _excluded(scores: torch.Tensor, exclude_mask: torch.Tensor | None) -> torch.Tensor:
    return scores if exclude_mask is None else torch.where(exclude_mask, float("-inf"), scores)


def select_landmarks(scores: torch.Tensor, k: int, exclude_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Indices of the ``min(k, #finite)`` best scores along the last dimension, with the
    ``exclude_mask`` positions set to ``-inf`` first (landmark_tokens_ker.py:87-103 of the
    reference; slot order unspecified, as ``topk(sorted=False)``). An empty int64 tensor
    when nothing is admissible. The attention module selects with the HIP kernel
    (``dsalt.kernels.selectors._compute_landmark_indices``); this is the generic helper."""
    s = _excluded(scores, exclude_mask)
    take = min(k, int(torch.isfinite(s).sum()) if s.numel() else 0)
    if take <= 0:
        return torch.empty(0, dtype=torch.long, device=scores.device)
    return s.topk(take, dim=-1, sorted=False).indices


def soft_landmark_weights(scores: torch.Tensor, k: int, exclude_mask: torch.Tensor | None = None,
                          temperature: float = 1.0) -> torch.Tensor:
    """Softmax of ``scores / temperature`` over the last dimension with excluded positions
    at weight 0 (landmark_tokens_ker.py:106-116 of the reference; ``k`` is accepted for
    signature compatibility and does not truncate)."""
    return torch.softmax(_excluded(scores, exclude_mask) / temperature, dim=-1)


class HybridEnergyLandmarkSelector(nn.Module):
    """Stand-alone landmark selector with a learnable balance ``alpha [n_layers, n_heads]``
    (sigmoid-parameterised, starting at 0.6 like ``DSALTAttention.alpha_w``),
    landmark_tokens_ker.py:119-150 of the reference.

    ``forward(x, W_V, layer_idx, head_idx, k, window_mask)`` scores the T rows with the
    scalar-alpha hybrid score, excludes every key that any row's window covers
    (``window_mask.any(0)``) and returns ``(indices, weights)``."""

    def __init__(self, n_layers: int, n_heads: int):
        super().__init__()
        # the float32 logit of 0.6, as the reference computes it (one ulp from log(1.5))
        self.alpha = nn.Parameter(torch.full((n_layers, n_heads), torch.logit(torch.tensor(0.6)).item()))

    def forward(self, x: torch.Tensor, W_V: torch.Tensor, layer_idx: int, head_idx: int, k: int,
                window_mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        scores = compute_hybrid_scores(x, W_V, torch.sigmoid(self.alpha[layer_idx, head_idx]))
        covered = window_mask.any(dim=0)
        return (select_landmarks(scores, k, exclude_mask=covered),
                soft_landmark_weights(scores, k, exclude_mask=covered))

"""Selector helpers: packed metadata, landmark top-k and the landmark K/V gather.

Same names and signatures as dsalt/kernels/selectors.py. The landmark top-k runs in the
HIP selection kernel (bit-exact on the fp32 scores, positions returned in ascending
order with -1 in the unused slots). The HIP attention kernels derive the packed block
layout from cu_seqlens and gather landmark rows themselves; ``_seq_meta``,
``_build_seq_block_map`` and ``_build_landmark_kv`` remain for callers of the
reference's helper API. Their caches are keyed by the packing itself (the reference
keys them by (total_len, num_seqs[, block]) only, which goes stale across packings of
equal total length).
"""
from __future__ import annotations

import torch

from .. import _hip
from .landmark_tokens_ker import hybrid_scores_per_head

_SEQ_BLOCK_MAP_CACHE: dict = {}
_SEQ_META_CACHE: dict = {}
_CACHE_LIMIT = 64


def _cu_key(cu_seqlens: torch.Tensor, cu_list: list | None) -> tuple:
    if cu_list is not None:
        return tuple(int(c) for c in cu_list)
    return tuple(int(c) for c in cu_seqlens.detach().to("cpu").tolist())


def _cache_put(cache: dict, key, val) -> None:
    if len(cache) >= _CACHE_LIMIT:
        cache.pop(next(iter(cache)))
    cache[key] = val


def _seq_meta(cu_seqlens: torch.Tensor, total: int, device: torch.device, cu_list: list | None = None):
    """``(num_seqs, lens, starts, seq_ids, seq_off, max_len)`` of a packing
    (selectors.py:15-34)."""
    key = (_cu_key(cu_seqlens, cu_list), str(device))
    if key in _SEQ_META_CACHE:
        return _SEQ_META_CACHE[key]
    cu = torch.tensor(key[0], dtype=torch.long, device=device)
    num_seqs = cu.shape[0] - 1
    lens = cu[1:] - cu[:-1]
    starts = cu[:-1]
    seq_ids = torch.repeat_interleave(torch.arange(num_seqs, device=device), lens)
    seq_off = torch.arange(total, device=device) - starts[seq_ids]
    max_len = max((key[0][b + 1] - key[0][b] for b in range(num_seqs)), default=0)
    val = (num_seqs, lens, starts, seq_ids, seq_off, max_len)
    _cache_put(_SEQ_META_CACHE, key, val)
    return val


def _build_seq_block_map(cu_seqlens: torch.Tensor, block_m: int, device: torch.device,
                         cu_list: list | None = None) -> tuple[torch.Tensor, int]:
    """``(seq_block_map [total_blocks, 2] int32, total_blocks)``: each ``block_m`` block of
    queries mapped to ``(sequence, block-in-sequence)`` (selectors.py:37-67)."""
    cu = _cu_key(cu_seqlens, cu_list)
    key = (cu, int(block_m), str(device))
    if key in _SEQ_BLOCK_MAP_CACHE:
        return _SEQ_BLOCK_MAP_CACHE[key]
    lens = torch.tensor([cu[b + 1] - cu[b] for b in range(len(cu) - 1)], dtype=torch.long)
    blocks_per = (lens + block_m - 1) // block_m
    total_blks = int(blocks_per.sum())
    seq_col = torch.repeat_interleave(torch.arange(lens.shape[0], dtype=torch.int32), blocks_per)
    blk_col = (torch.arange(total_blks, dtype=torch.int32)
               - torch.repeat_interleave(blocks_per.cumsum(0) - blocks_per, blocks_per).int())
    result = torch.stack([seq_col, blk_col], dim=1).contiguous().to(device)
    _cache_put(_SEQ_BLOCK_MAP_CACHE, key, (result, total_blks))
    return result, total_blks


def _score_block(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int):
    return hybrid_scores_per_head(x, W_V, alpha, n_heads, dh)


def _compute_landmark_indices(
    x: torch.Tensor,
    W_V: torch.Tensor,
    alpha: torch.Tensor,
    w_sizes: torch.Tensor,
    cu_seqlens: torch.Tensor,
    k_lmk: int,
    n_min: int,
    total_len: int,
    cu_list: list | None = None,
    head_dim: int | None = None,
    v: torch.Tensor | None = None,
):
    """Top-``k_lmk`` landmark positions per (head, sequence), excluding covered tokens.

    Returns ``(lmk [H, S, k_lmk] int64, z_x, z_v)`` like selectors.py:75-134. A token at
    offset ``o`` of its sequence is covered (never a landmark) when ``o < trunc(w)``.
    The selection runs in the HIP kernel over the fp32 hybrid scores; slots are filled
    in ascending position order and padded with ``-1`` (the reference's
    ``topk(sorted=False)`` leaves slot order unspecified, so the set is what matches).
    ``n_min`` and ``total_len`` are accepted for signature compatibility.

    ``v`` (optional, not in the reference's signature): the value projection
    ``x @ W_V.T`` as ``[T, n_kv, dh]``, which the attention module already holds. With
    it the scores come from the fused HIP kernel ``dsalt_hybrid_scores`` (norms and
    standardisation in one pass over x and v) and the ``x @ W_V.T`` GEMM is skipped.
    """
    n_heads = alpha.shape[0]
    if v is not None:
        scores, z_x, z_v = _hip.hybrid_scores(x.detach(), v.detach(), alpha, n_heads)
        lmk = _hip.select_landmarks(scores, w_sizes, cu_seqlens, int(k_lmk))
        return lmk, z_x, z_v
    dh = head_dim if head_dim is not None else W_V.shape[0] // n_heads
    scores, z_x, z_v = _score_block(x, W_V, alpha, n_heads, dh)
    lmk = _hip.select_landmarks(scores.float(), w_sizes, cu_seqlens, int(k_lmk))
    return lmk, z_x, z_v


def _build_landmark_kv(K: torch.Tensor, V: torch.Tensor, lmk_indices: torch.Tensor,
                       cu_seqlens: torch.Tensor, k_lmk: int, n_heads: int,
                       head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather landmark keys/values into ``[H, S, k, D]``; empty slots are zero
    (selectors.py:137-159). The HIP kernels do this gather in-kernel; this helper only
    serves callers of the reference's API."""
    starts = cu_seqlens[:-1].to(K.device).long()
    safe_idx = lmk_indices.clamp(min=0)
    abs_idx = starts[None, :, None] + safe_idx
    h_idx = torch.arange(n_heads, device=K.device)[:, None, None]
    invalid = (lmk_indices < 0).unsqueeze(-1)
    lmk_K = K[abs_idx, h_idx, :].masked_fill(invalid, 0.0)
    lmk_V = V[abs_idx, h_idx, :].masked_fill(invalid, 0.0)
    return lmk_K.contiguous(), lmk_V.contiguous()

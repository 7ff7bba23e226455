"""Selector helpers: packed metadata, landmark top-k and the landmark K/V gather.

Same names, signatures and results as dsalt/kernels/selectors.py. The landmark top-k
runs in the HIP selection kernel (bit-exact on the fp32 scores, positions returned in
ascending order with -1 in the unused slots). The HIP attention kernels derive the
packed block layout from cu_seqlens and gather landmark rows themselves, so
``_seq_meta``, ``_build_seq_block_map`` and ``_build_landmark_kv`` only serve callers
of the reference's helper API. Their caches are keyed by the packing itself (the
reference keys them by (total_len, num_seqs[, block]) only, which goes stale across
packings of equal total length).
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _hip
from .landmark_tokens_ker import hybrid_scores_from_v, hybrid_scores_per_head

_CACHE: dict = {}
_CACHE_LIMIT = 128


def _boundaries(cu_seqlens: torch.Tensor, cu_list: list | None) -> tuple:
    """The packing as a tuple of ints (the host hint when given, else one device read)."""
    src = cu_list if cu_list is not None else cu_seqlens.detach().cpu().tolist()
    return tuple(int(c) for c in src)


def _memo(key, make):
    hit = _CACHE.get(key)
    if hit is None:
        if len(_CACHE) >= _CACHE_LIMIT:
            _CACHE.clear()
        hit = _CACHE[key] = make()
    return hit


def _seq_meta(cu_seqlens: torch.Tensor, total: int, device: torch.device, cu_list: list | None = None):
    """``(num_seqs, lens, starts, seq_ids, seq_off, max_len)`` of a packing
    (selectors.py:15-34): per-token sequence id and offset inside the sequence."""
    bounds = _boundaries(cu_seqlens, cu_list)

    def make():
        cu = torch.tensor(bounds, dtype=torch.long, device=device)
        tok = torch.arange(total, dtype=torch.long, device=device)
        # sequence of token t: the number of sequence ends <= t
        seq_ids = torch.searchsorted(cu[1:], tok, right=True)
        seq_off = tok - cu[seq_ids]
        lens = cu[1:] - cu[:-1]
        spans = np.diff(np.asarray(bounds, dtype=np.int64))
        return (len(bounds) - 1, lens, cu[:-1], seq_ids, seq_off, int(spans.max()) if spans.size else 0)

    return _memo(("meta", bounds, int(total), str(device)), make)


def _build_seq_block_map(cu_seqlens: torch.Tensor, block_m: int, device: torch.device,
                         cu_list: list | None = None) -> tuple[torch.Tensor, int]:
    """``(seq_block_map [total_blocks, 2] int32, total_blocks)``: block b of ``block_m``
    queries, counted over the sequences in order, is (sequence, block inside it)
    (selectors.py:37-67)."""
    bounds = _boundaries(cu_seqlens, cu_list)

    def make():
        spans = np.diff(np.asarray(bounds, dtype=np.int64))
        nblk = -(-spans // int(block_m))            # ceil(L_s / block_m)
        first = np.concatenate(([0], np.cumsum(nblk)))
        b = np.arange(first[-1], dtype=np.int64)
        seq = np.searchsorted(first[1:], b, side="right")
        table = np.stack((seq, b - first[seq]), axis=1).astype(np.int32)
        return torch.from_numpy(table).to(device), int(first[-1])

    return _memo(("blocks", bounds, int(block_m), str(device)), make)


def _score_block(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int):
    return hybrid_scores_per_head(x, W_V, alpha, n_heads, dh)


def selection_scores(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int,
                     v: torch.Tensor | None = None, hip_scores: bool = False):
    """``(scores [T, H] fp32, z_x, z_v)`` for the landmark selection.

    * ``v is None``: the reference's route, ``x @ W_V.T`` then the torch norms.
    * ``v`` given (the module's pre-RoPE value projection ``x W_V^T`` as ``[T, n_kv, dh]``):
      the same torch norms on ``v`` (torch forms ``v_proj(x)`` with the same matmul, so
      the scores are bit-identical and the second GEMM is saved).
    * ``hip_scores``: the one-pass HIP kernel over x and v (deterministic; its fp32 norm
      sums run in another order than torch's, so a score can differ from the torch
      route's in its last bits - a near-tie landmark could move; the landmark sets of
      configs 2 and 4 are those of the torch route, set for set). Shapes the kernel does
      not take (``_hip.scores_supported``) use the torch norms on ``v``.
    """
    if v is None:
        return _score_block(x, W_V, alpha, n_heads, dh)
    if hip_scores and _hip.scores_supported(x, v):
        return _hip.hybrid_scores(x.detach(), v.detach(), alpha, n_heads)
    return hybrid_scores_from_v(x, v, alpha, n_heads)


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
    hip_scores: bool = False,
):
    """Top-``k_lmk`` landmark positions per (head, sequence), excluding covered tokens.

    Returns ``(lmk [H, S, k_lmk] int64, z_x, z_v)`` like selectors.py:75-134. A token at
    offset ``o`` of its sequence is covered (never a landmark) when ``o < trunc(w)``.
    The selection runs in the HIP kernel over the fp32 hybrid scores; slots are filled
    in ascending position order and padded with ``-1`` (the reference's
    ``topk(sorted=False)`` leaves slot order unspecified, so the set is what matches).
    ``n_min`` and ``total_len`` are accepted for signature compatibility.

    ``v`` and ``hip_scores`` (not in the reference's signature) pick the score route of
    :func:`selection_scores`.
    """
    n_heads = alpha.shape[0]
    dh = head_dim if head_dim is not None else W_V.shape[0] // n_heads
    with torch.no_grad():
        scores, z_x, z_v = selection_scores(x, W_V, alpha, n_heads, dh, v, hip_scores)
        max_len = None if cu_list is None else max((b - a for a, b in zip(cu_list[:-1], cu_list[1:])), default=0)
        lmk = _hip.select_landmarks(scores.float(), w_sizes, cu_seqlens, int(k_lmk), max_seqlen=max_len)
    return lmk, z_x, z_v


def _landmarks_and_windows(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, w_cont: torch.Tensor | None,
                           cu_seqlens: torch.Tensor, k_lmk: int, cu_list: list | None = None,
                           head_dim: int | None = None, v: torch.Tensor | None = None,
                           hip_scores: bool = False, gate=None):
    """``(w_sizes [T] fp32, lmk [H, S, k_lmk] int64)``: the window quantisation of
    ``DSALTAttention._window_sizes(floor=True)`` (dsalt_attention.py:277-284 of the
    reference) and :func:`_compute_landmark_indices` on those windows, with the
    quantisation done by the selection launch itself (``w_cont`` is the continuous
    ``w~``; or ``gate = (window-gate logits [T], n_min, n_max)``, from which the launch
    also forms ``w~`` with torch's roundings). Same results as the steps apart. On the HIP
    score route the scores are formed inside the selection launch (``_hip.select_hybrid``:
    the norms pass, then the selection; no [T, H] score tensor), with the same bits."""
    n_heads = alpha.shape[0]
    dh = head_dim if head_dim is not None else W_V.shape[0] // n_heads
    with torch.no_grad():
        max_len = None if cu_list is None else max((b - a for a, b in zip(cu_list[:-1], cu_list[1:])), default=0)
        if v is not None and hip_scores and _hip.scores_supported(x, v):
            w_sizes, lmk, _ = _hip.select_hybrid(x.detach(), v.detach(), alpha, n_heads,
                                                 None if w_cont is None else w_cont.detach(), cu_seqlens, int(k_lmk),
                                                 max_seqlen=max_len, gate=gate)
            return w_sizes, lmk
        scores, _, _ = selection_scores(x, W_V, alpha, n_heads, dh, v, hip_scores)
        return _hip.select_landmarks_quantize(scores.float(), None if w_cont is None else w_cont.detach(),
                                              cu_seqlens, int(k_lmk), max_seqlen=max_len, gate=gate)


def _build_landmark_kv(K: torch.Tensor, V: torch.Tensor, lmk_indices: torch.Tensor,
                       cu_seqlens: torch.Tensor, k_lmk: int, n_heads: int,
                       head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Landmark keys/values ``[H, S, k, D]`` (selectors.py:137-159); empty slots are zero.
    The HIP kernels do this gather in-kernel; this helper only serves callers of the
    reference's API."""
    H, S, k = lmk_indices.shape
    T = K.shape[0]
    first = cu_seqlens[:-1].to(device=K.device, dtype=torch.long)
    empty = lmk_indices < 0
    # flat row of (token first[s] + pos, head h) in a [T * H, D] view
    token = first.view(1, S, 1) + lmk_indices.clamp_min(0)
    flat = (token * H + torch.arange(H, device=K.device).view(H, 1, 1)).reshape(-1)

    def take(src: torch.Tensor) -> torch.Tensor:
        rows = src.reshape(T * H, src.shape[-1]).index_select(0, flat).view(H, S, k, src.shape[-1])
        return torch.where(empty.unsqueeze(-1), torch.zeros((), dtype=rows.dtype, device=rows.device), rows)

    return take(K).contiguous(), take(V).contiguous()

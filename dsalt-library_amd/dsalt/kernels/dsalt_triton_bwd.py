"""Backward of the HARD DSALT attention on the gfx950 HIP kernels.

Same entry point as dsalt/kernels/dsalt_triton_bwd.py:219-324. The HIP backward is
deterministic (no atomics) and gathers landmark rows itself, so ``lmk_K``/``lmk_V``,
the block map and the Triton tile arguments are accepted and ignored. Returns
``(dq, dk, dv, d_bias)`` in fp32 like the reference.
"""
from __future__ import annotations

import torch

from .. import _hip


def dsalt_triton_backward(
    grad_out: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    lmk_K: torch.Tensor | None,
    lmk_V: torch.Tensor | None,
    lmk_pos: torch.Tensor,
    lmk_bias: torch.Tensor,
    w_sizes: torch.Tensor,
    cu_seqlens: torch.Tensor,
    scale: float,
    seq_block_map: torch.Tensor | None = None,
    total_blk: int | None = None,
    BLOCK_M: int | None = None,
    BLOCK_N: int | None = None,
    HEAD_DIM_C: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    dt = _hip.compute_dtype(q.dtype)
    q_c = _hip.as_kernel_operand(q, dt)
    k_c = _hip.as_kernel_operand(k, dt)
    v_c = _hip.as_kernel_operand(v, dt)
    o_c = _hip.as_kernel_operand(out, dt)
    lp = lmk_pos if lmk_pos is not None and lmk_pos.shape[-1] > 0 else None
    dq, dk, dv, d_bias, _ = _hip.bwd(_hip.MODE_HARD, q_c, k_c, v_c, o_c, lse.float(), grad_out,
                                     w_sizes, lp, None if lp is None else lmk_bias, cu_seqlens,
                                     float(scale), grad_dtype=torch.float32)
    if d_bias is None:
        H, S = q.shape[1], cu_seqlens.shape[0] - 1
        d_bias = torch.zeros((H, S, 0 if lmk_pos is None else lmk_pos.shape[-1]),
                             device=q.device, dtype=torch.float32)
    return dq, dk, dv, d_bias

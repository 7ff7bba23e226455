"""Autograd glue shared by the HARD (inference) and SOFT (training) entry points.

Forward: one HIP launch (fused band + landmark attention, in-kernel landmark gather,
no output memset). Backward: one ``dsalt_bwd`` call (deterministic, atomic-free).
Saved for backward: the kernel operands, O and the fp32 LSE, as DSALTAttentionFunction /
DSALTTrainFunction do (dsalt_triton_attn.py:300, dsalt_triton_train.py:647). The
``dsalt.kernels`` entry points return O in fp32 (like the reference); the kernel writes
it in fp32 directly, and the backward's Delta = rowsum(O * dO) then uses the unrounded O.
"""
from __future__ import annotations

import math

import torch

from .. import _hip


def _forward(ctx, mode: int, q, k, v, lmk_pos, lmk_bias, w, cu_seqlens, tau_win, win_edge,
             out_f32: bool = False, rope=None):
    _hip.require_gpu(q, k, v, w, cu_seqlens)
    if rope is not None and torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise _hip.DsaltError("the RoPE of q on load is forward-only; rotate q beforehand when gradients are needed")
    if q.dim() != 3:
        raise _hip.DsaltError(f"q must be packed [T, H, D], got {tuple(q.shape)}")
    scale = 1.0 / math.sqrt(q.shape[-1])
    dt = _hip.compute_dtype(q.dtype)
    q_c = _hip.as_kernel_operand(q.detach(), dt)
    k_c = _hip.as_kernel_operand(k.detach(), dt)
    v_c = _hip.as_kernel_operand(v.detach(), dt)
    w_f = w.detach().float()
    lp = None
    if lmk_pos is not None and lmk_pos.shape[-1] > 0:
        lp = lmk_pos.detach()
    lb = None if (lmk_bias is None or lp is None) else lmk_bias.detach().float()
    out, lse = _hip.fwd(mode, q_c, k_c, v_c, w_f, lp, lb, cu_seqlens, scale, tau_win, win_edge,
                        out_dtype=torch.float32 if out_f32 else None, rope=rope)
    ctx.save_for_backward(q_c, k_c, v_c, out, lse, lp, lb, w_f, cu_seqlens)
    ctx.dsalt_mode = mode
    ctx.dsalt_scale = scale
    ctx.dsalt_tau = float(tau_win)
    ctx.dsalt_edge = float(win_edge)
    ctx.dsalt_q_dtype = q.dtype
    ctx.dsalt_k_lmk = 0 if lmk_pos is None else lmk_pos.shape[-1]
    return out


def _backward(ctx, grad_out, need_dw: bool):
    q_c, k_c, v_c, out, lse, lp, lb, w_f, cu = ctx.saved_tensors
    od = ctx.dsalt_q_dtype
    # gradients come back in q's dtype; fp32 inputs (computed in fp16) get fp32 gradients
    # written directly by the kernels, and so do grouped K/V heads (per-query-head dK/dV
    # are summed over each group in fp32)
    n_kv = k_c.shape[1]
    gdt = torch.float32 if (od == torch.float32 or n_kv != q_c.shape[1]) else q_c.dtype
    dq, dk, dv, d_bias, d_w = _hip.bwd(
        ctx.dsalt_mode, q_c, k_c, v_c, out, lse, grad_out, w_f, lp, lb, cu,
        ctx.dsalt_scale, ctx.dsalt_tau, ctx.dsalt_edge, need_dw=need_dw, grad_dtype=gdt)
    dk, dv = _hip.group_sum(dk, n_kv), _hip.group_sum(dv, n_kv)
    return (dq.to(od), dk.to(od), dv.to(od),
            None if d_bias is None else d_bias.to(od),
            None if d_w is None else d_w.to(od))


class _SparseAttention(torch.autograd.Function):
    """Module-path variant: returns O in the compute dtype (no fp32 round trip)."""

    @staticmethod
    def forward(ctx, mode, q, k, v, lmk_pos, lmk_bias, w, cu_seqlens, tau_win, win_edge, rope):
        return _forward(ctx, mode, q, k, v, lmk_pos, lmk_bias, w, cu_seqlens, tau_win, win_edge, rope=rope)

    @staticmethod
    def backward(ctx, grad_out):
        need_dw = ctx.dsalt_mode == _hip.MODE_SOFT and ctx.needs_input_grad[6]
        dq, dk, dv, d_bias, d_w = _backward(ctx, grad_out, need_dw)
        if not ctx.needs_input_grad[5]:
            d_bias = None
        return None, dq, dk, dv, None, d_bias, d_w, None, None, None, None


def sparse_attention(mode: int, q, k, v, lmk_pos, lmk_bias, w, cu_seqlens,
                     tau_win: float = 1.0, win_edge: float = 4.0, rope=None) -> torch.Tensor:
    """Differentiable DSALT attention returning O [T, H, D] in the compute dtype. With
    ``rope = (cos, sin)`` q is the un-rotated query and the kernel rotates it on load
    (forward only; k must be rotated already)."""
    return _SparseAttention.apply(mode, q, k, v, lmk_pos, lmk_bias, w, cu_seqlens, tau_win, win_edge, rope)

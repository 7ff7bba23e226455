"""Autograd glue of the dense batched variant (DSALT_MODE_DENSE).

DSALTAttention._batched (dsalt/modules/dsalt_attention.py:371-401) forms the [H, T, T]
union log-bias (soft window tail of every causal key, landmark weights at the selected
keys left of floor(w~)) and a dense softmax over it, differentiable in w~ (through the
soft tail) and in the landmark weights. Here one HIP forward and one HIP backward compute
the same attention without materialising [H, T, T]: the bias is recomputed per element
from w~ [T] and the [H, T] landmark-bias table. Saved for backward: the kernel operands,
O, the fp32 LSE, w~ and the table.
"""
from __future__ import annotations

import math

import torch

from .. import _hip


class _DenseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, w_cont, lmk_bias, tau_win, win_edge):
        _hip.require_gpu(q, k, v, w_cont, lmk_bias)
        if q.dim() != 3:
            raise _hip.DsaltError(f"q must be [T, H, D], got {tuple(q.shape)}")
        scale = 1.0 / math.sqrt(q.shape[-1])
        dt = _hip.compute_dtype(q.dtype)
        q_c = _hip.as_kernel_operand(q.detach(), dt)
        k_c = _hip.as_kernel_operand(k.detach(), dt)
        v_c = _hip.as_kernel_operand(v.detach(), dt)
        w_f = w_cont.detach().float()
        lb = None if lmk_bias is None else lmk_bias.detach().float()
        out, lse = _hip.dense_fwd(q_c, k_c, v_c, w_f, lb, scale, tau_win, win_edge)
        ctx.save_for_backward(q_c, k_c, v_c, out, lse, w_f, lb)
        ctx.dsalt_scale = scale
        ctx.dsalt_tau = float(tau_win)
        ctx.dsalt_edge = float(win_edge)
        ctx.dsalt_q_dtype = q.dtype
        ctx.dsalt_w_dtype = w_cont.dtype
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q_c, k_c, v_c, out, lse, w_f, lb = ctx.saved_tensors
        od = ctx.dsalt_q_dtype
        n_kv = k_c.shape[1]
        gdt = torch.float32 if (od == torch.float32 or n_kv != q_c.shape[1]) else q_c.dtype
        need_dw = ctx.needs_input_grad[3]
        dq, dk, dv, d_lb, d_w = _hip.dense_bwd(q_c, k_c, v_c, out, lse, grad_out, w_f, lb, ctx.dsalt_scale,
                                               ctx.dsalt_tau, ctx.dsalt_edge, need_dw=need_dw, grad_dtype=gdt)
        dk, dv = _hip.group_sum(dk, n_kv), _hip.group_sum(dv, n_kv)
        if not ctx.needs_input_grad[4]:
            d_lb = None
        return (dq.to(od), dk.to(od), dv.to(od),
                None if d_w is None else d_w.to(ctx.dsalt_w_dtype),
                None if d_lb is None else d_lb, None, None)


def dense_attention(q, k, v, w_cont, lmk_bias, tau_win: float = 1.0, win_edge: float = 4.0) -> torch.Tensor:
    """Differentiable dense DSALT attention of one sequence: q [T, H, D], k/v [T, n_kv, D]
    (n_kv divides H; grouped heads share K/V without a copy), w_cont [T],
    lmk_bias [H, T] (natural log, -inf off the landmarks) or None. Returns O [T, H, D] in
    the compute dtype."""
    return _DenseAttention.apply(q, k, v, w_cont, lmk_bias, tau_win, win_edge)


@torch.no_grad()
def dense_probabilities(q, k, w_cont, lmk_bias, tau_win: float = 1.0, win_edge: float = 4.0) -> torch.Tensor:
    """The dense attention probabilities [H, T, T] (fp32) of the same bias, formed with
    torch as the reference's diagnostic ``_last_P`` (dsalt_attention.py:385-397): logits
    q.k in q's dtype, then fp32 scaling, bias and softmax. O(H T^2) memory."""
    T, H, D = q.shape
    dev = q.device
    qh = q.transpose(0, 1).contiguous()
    kt = k.transpose(0, 1).transpose(1, 2).contiguous()
    sc = torch.matmul(qh, kt).float() * (1.0 / math.sqrt(D))
    idx = torch.arange(T, device=dev)
    d = (idx.view(T, 1) - idx.view(1, T)).float()
    w = w_cont.detach().float().view(T, 1)
    g = torch.sigmoid((w - d) / tau_win)
    logb = torch.log(g.clamp(min=1e-20))
    logb = torch.where(d <= (w - win_edge), torch.zeros_like(logb), logb).masked_fill(d < 0, float("-inf"))
    bias = logb.unsqueeze(0).expand(H, T, T)
    if lmk_bias is not None:
        valid = (d >= 0) & (d >= torch.floor(w).clamp(min=1))
        lmk = torch.where(valid.unsqueeze(0), lmk_bias.float().unsqueeze(1).expand(H, T, T),
                          torch.full((1, 1, 1), float("-inf"), device=dev))
        bias = torch.maximum(bias, lmk)
    return torch.softmax(sc + bias, dim=-1)

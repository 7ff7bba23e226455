"""DSALT training attention (SOFT selectors) on the gfx950 HIP kernels.

Drop-in for dsalt/kernels/dsalt_triton_train.py: same entry point
``dsalt_triton_train_attention(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens,
tau_win=1.0, win_edge=4.0, n_max=256, cu_list=None)`` and the same
``DSALTTrainFunction`` (fp32 output; gradients dq, dk, dv, d_logw, d_w~ in q's dtype,
:751-760). The module name is kept for import compatibility; nothing here uses Triton.

Semantics (dsalt_triton_train.py:116-198): band ``0 <= d = i - j <= w~(i)`` with logit
bias 0 in the core ``d <= w~ - win_edge`` and ``log sigmoid((w~ - d) / tau_win)`` on the
edge; landmark p admitted when ``p <= i`` and ``(float)p < (float)i - w~(i)`` with bias
``lmk_logw[h, s, slot]``. The band is the exact set ``j >= i - floor(w~)``: the
reference kernel's scan can skip key ``i - w~`` when w~ is integral, while its dense
reference (dsalt_attention.py:540) includes it; this path follows the dense
definition. The HIP backward bounds its key-parallel scan by the actual largest window,
so ``n_max`` is accepted but not needed for correctness.
"""
from __future__ import annotations

import torch

from .. import _hip
from . import _sparse
from .dsalt_triton_attn import _dynamo_opaque


class DSALTTrainFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens, tau_win, win_edge, n_max,
                cu_list=None):
        return _sparse._forward(ctx, _hip.MODE_SOFT, q, k, v, lmk_pos, lmk_logw, w_cont,
                                cu_seqlens, float(tau_win), float(win_edge), out_f32=True)

    @staticmethod
    def backward(ctx, grad_out):
        dq, dk, dv, d_logw, d_w = _sparse._backward(ctx, grad_out, need_dw=ctx.needs_input_grad[5])
        return dq, dk, dv, None, d_logw, d_w, None, None, None, None, None


@_dynamo_opaque
def dsalt_triton_train_attention(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens,
                                 tau_win=1.0, win_edge=4.0, n_max=256, cu_list=None):
    """Differentiable SOFT DSALT attention; returns fp32 ``[T, H, D]``. ``lmk_logw``
    receives d_logw and ``w_cont`` receives d_w~ (summed over heads)."""
    return DSALTTrainFunction.apply(q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens,
                                    tau_win, win_edge, n_max, cu_list)

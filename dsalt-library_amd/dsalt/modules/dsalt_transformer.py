"""Pre-norm transformer block around DSALTAttention (dsalt/modules/dsalt_transformer.py).

The LM consumer of the attention path: x + attn(norm(x)), then x + ffn(norm(x)), with a
SwiGLU feed-forward. Parameter names and creation order follow the reference
(attn_norm, ffn_norm, attn, ffn; gate_proj, up_proj, down_proj) so state dicts load and
seeded initialisations agree. The attention runs on the HIP kernels; the projections are
torch (hipBLASLt GEMMs). Without autograd on the GPU, the FFN's gated product and each
residual add with the norm after it are HIP passes too; with autograd they are torch ops.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

from .. import _hip
from ..kernels.RMSENorm import RMSENorm
from .dsalt_attention import DSALTAttention


class SwiGLUFFN(nn.Module):
    """``down_proj(silu(gate_proj(x)) * up_proj(x))`` (dsalt_transformer.py:10-21). Without
    autograd, on the GPU, the gated product is one HIP pass (``dsalt_swiglu``) with torch's
    roundings, instead of torch's silu and product passes."""

    def __init__(self, d_model: int, d_ff: int, dropout: float = 0.0):
        super().__init__()
        self.gate_proj = nn.Linear(d_model, d_ff, bias=False)
        self.up_proj = nn.Linear(d_model, d_ff, bias=False)
        self.down_proj = nn.Linear(d_ff, d_model, bias=False)
        self.drop = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g, u = self.gate_proj(x), self.up_proj(x)
        if not torch.is_grad_enabled() and _hip.swiglu_supported(g, u):
            h = _hip.swiglu(g, u)  # one pass, the same bits as the two torch ops below
        else:
            h = F.silu(g) * u
        return self.drop(self.down_proj(h))


class DSALTTransformerBlock(nn.Module):
    """RMSNorm -> DSALTAttention -> residual, RMSNorm -> SwiGLU -> residual
    (dsalt_transformer.py:24-88); ``gradient_checkpointing`` recomputes the attention and
    the FFN in the backward when training. ``_fuse_norms`` (default True): at inference
    without autograd, with 16-bit rows, a residual add and the norm after it run as one
    HIP pass (``dsalt_add_rms_norm``: the sum is torch's add bit for bit, the norm can
    differ from F.rms_norm in an output's last bit)."""

    _fuse_norms = True

    def __init__(self, d_model: int, n_heads: int, n_min: int, n_max: int, k_lmk: int, max_seq_len: int,
                 d_ff: int, dropout: float = 0.0, yarn_scale: float = 1.0, layer_idx: int = 0,
                 n_kv_heads: int | None = None, qkv_bias: bool = False, rope_base: float = 10000.0):
        super().__init__()
        self.layer_idx = layer_idx
        self.attn_norm = RMSENorm(d_model)
        self.ffn_norm = RMSENorm(d_model)
        self.attn = DSALTAttention(d_model=d_model, n_heads=n_heads, n_min=n_min, n_max=n_max, k_lmk=k_lmk,
                                   max_seq_len=max_seq_len, dropout=dropout, yarn_scale=yarn_scale,
                                   layer_idx=layer_idx, n_kv_heads=n_kv_heads, qkv_bias=qkv_bias,
                                   rope_base=rope_base)
        self.ffn = SwiGLUFFN(d_model=d_model, d_ff=d_ff, dropout=dropout)

    def forward(self, x: torch.Tensor, cu_seqlens: torch.Tensor | None = None, max_seqlen: int | None = None,
                gradient_checkpointing: bool = False, rope_cs: tuple | None = None,
                cu_list: list | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        aux_box = []

        def attend(h):
            o, a = self.attn(h, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, rope_cs=rope_cs, cu_list=cu_list)
            aux_box.append(a)
            return o

        recompute = gradient_checkpointing and self.training
        h = self.attn_norm(x)
        x_attn = torch.utils.checkpoint.checkpoint(attend, h, use_reentrant=False) if recompute else attend(h)
        if self._norms_fusable(x, x_attn, self.ffn_norm):
            # the residual add and the FFN's norm in one HIP pass (inference)
            x, h = _hip.add_rms_norm(x, x_attn, self.ffn_norm.weight, self.ffn_norm.eps)
        else:
            x = x + x_attn
            h = self.ffn_norm(x)
        x = x + (torch.utils.checkpoint.checkpoint(self.ffn, h, use_reentrant=False) if recompute else self.ffn(h))
        return x, aux_box[0]

    def _norms_fusable(self, x: torch.Tensor, h: torch.Tensor | None, norm: nn.Module) -> bool:
        """Whether x (+ h) and the RMSENorm `norm` can run as one dsalt_add_rms_norm pass:
        inference without autograd, 16-bit rows on the GPU, a weight of x's dtype."""
        if self.training or torch.is_grad_enabled() or not self._fuse_norms:
            return False
        if h is not None and (h.shape != x.shape or h.dtype != x.dtype or not h.is_contiguous()
                              or h.data_ptr() % 16):
            return False
        return _hip.add_rms_norm_supported(x, norm.weight)

    def _forward_fused(self, x: torch.Tensor, delta: torch.Tensor | None, cu_seqlens=None, max_seqlen=None,
                       rope_cs=None, cu_list=None):
        """Inference forward that leaves its last residual add to the caller: returns
        (x + attention, the FFN output, aux - None on the packed path, where the attention
        makes no zero aux tensor), so that the next block's norm (or the final norm) takes
        that add in its own pass. `delta` is the previous block's pending FFN
        output (None for the first block). The caller checks `_norms_fusable` first."""
        x_sum, h = _hip.add_rms_norm(x, delta, self.attn_norm.weight, self.attn_norm.eps)
        if x_sum is not None:
            x = x_sum
        x_attn, aux = self.attn(h, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, rope_cs=rope_cs, cu_list=cu_list,
                                _need_aux=False)
        if self._norms_fusable(x, x_attn, self.ffn_norm):
            x, h = _hip.add_rms_norm(x, x_attn, self.ffn_norm.weight, self.ffn_norm.eps)
        else:
            x = x + x_attn
            h = self.ffn_norm(x)
        return x, self.ffn(h), aux

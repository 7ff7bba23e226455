"""DSALTLMHeadModel (dsalt/model/dsalt_lm.py:64-284): the causal-LM consumer of the
attention path.

Token embedding -> ``n_layers`` pre-norm DSALT blocks -> final RMSNorm -> LM head (tied
to the embedding by default). Constructor arguments, parameter names, module creation
order and the initialisation rule (every Linear weight N(0, 0.02), out_proj/down_proj
N(0, 0.02 / sqrt(2 n_layers)), biases 0, embedding N(0, 0.02); dsalt_lm.py:164-172)
follow the reference, so seeded models and state dicts agree.

Input: packed ``input_ids [T]`` with ``cu_seqlens`` (sparse HIP attention), or
``[1, T]`` without (the dense batched variant; the reference's batched attention fails
for B > 1 and so does this one, with a clear error). The packed RoPE positions are
derived in the HIP RoPE kernel from cu_seqlens, so no per-token cos/sin gather is built;
the host copy of cu_seqlens is taken once per forward and shared by every layer.
``labels`` gives the mean token cross-entropy (ignore index -100), computed over
``lm_head_chunk_size``-token chunks so that at most [chunk, vocab] logits exist at once.
The Triton-only "liger" loss is not available (as in the reference without Triton).

Inference without autograd in bf16/fp16 runs every residual add in the pass of the
RMSNorm after it (dsalt_add_rms_norm: each block hands its FFN output to the next
block's norm, the last one to the final norm); the FFN's gated product and the window
gate run as HIP passes too (SwiGLUFFN, DSALTAttention).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _hip
from ..kernels.RMSENorm import RMSENorm
from ..modules.dsalt_transformer import DSALTTransformerBlock

_LOSS_FNS = ("auto", "liger", "chunked")


def _chunked_cross_entropy(x: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                           chunk_size: int = 512) -> torch.Tensor:
    """Sum of token cross-entropies over chunks of rows of ``x @ weight.T``, divided by
    the number of labels other than -100 (at least 1)."""
    total = torch.zeros((), device=x.device, dtype=torch.float32)
    for a in range(0, x.shape[0], chunk_size):
        logits = F.linear(x[a:a + chunk_size], weight)
        total = total + F.cross_entropy(logits, labels[a:a + chunk_size], ignore_index=-100, reduction="sum")
    n = (labels != -100).sum().clamp(min=1).to(torch.float32)
    return total / n


class DSALTLMHeadModel(nn.Module):
    def __init__(self, vocab_size: int, d_model: int, n_layers: int, n_heads: int, n_min: int, n_max: int,
                 k_lmk: int, max_seq_len: int, d_ff: int | None = None, dropout: float = 0.0,
                 yarn_scale: float = 1.0, tie_weights: bool = True, padding_idx: int | None = None,
                 lm_head_chunk_size: int = 2048, loss_fn: str = "chunked", aux_loss_weight: float = 0.0,
                 n_kv_heads: int | None = None, qkv_bias: bool = False, rope_base: float = 10000.0):
        super().__init__()
        if loss_fn not in _LOSS_FNS:
            raise ValueError(f"loss_fn must be one of {list(_LOSS_FNS)}, got {loss_fn!r}")
        if loss_fn == "liger":
            raise RuntimeError("loss_fn='liger' needs the Triton fused cross-entropy, which this build does "
                               "not have; use loss_fn='chunked'")
        self.d_model = d_model
        self.n_layers = n_layers
        self.vocab_size = vocab_size
        self.lm_head_chunk_size = lm_head_chunk_size
        self.loss_fn = loss_fn
        self.aux_loss_weight = aux_loss_weight
        if d_ff is None:  # about 8/3 d_model, rounded up to a multiple of 128
            d_ff = -(-int(8 / 3 * d_model) // 128) * 128

        self.embed_tokens = nn.Embedding(vocab_size, d_model, padding_idx=padding_idx)
        self.embed_dropout = nn.Dropout(dropout)
        self.layers = nn.ModuleList(
            DSALTTransformerBlock(d_model=d_model, n_heads=n_heads, n_min=n_min, n_max=n_max, k_lmk=k_lmk,
                                  max_seq_len=max_seq_len, d_ff=d_ff, dropout=dropout, yarn_scale=yarn_scale,
                                  layer_idx=i, n_kv_heads=n_kv_heads, qkv_bias=qkv_bias, rope_base=rope_base)
            for i in range(n_layers))
        self.final_norm = RMSENorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        if tie_weights:
            self.lm_head.weight = self.embed_tokens.weight
        self._init_weights()

    @classmethod
    def from_config(cls, config) -> "DSALTLMHeadModel":
        """Build from a config object with ``to_dict()`` (the reference's DSALTConfig)."""
        return cls(**config.to_dict())

    def _init_weights(self) -> None:
        nn.init.normal_(self.embed_tokens.weight, std=0.02)
        deep = 0.02 / math.sqrt(2 * self.n_layers)
        for name, mod in self.named_modules():
            if not isinstance(mod, nn.Linear):
                continue
            nn.init.normal_(mod.weight, std=deep if ("out_proj" in name or "down_proj" in name) else 0.02)
            if mod.bias is not None:
                nn.init.zeros_(mod.bias)

    def set_collect_last_P(self, on: bool) -> None:
        """Turn the attention modules' ``_last_P`` diagnostic on or off."""
        for layer in self.layers:
            layer.attn._collect_last_P = on

    @staticmethod
    def _to_autocast_dtype(x: torch.Tensor) -> torch.Tensor:
        dev = x.device.type
        if torch.is_autocast_enabled(dev):
            dt = torch.get_autocast_dtype(dev)
            if x.dtype != dt:
                return x.to(dt)
        return x

    def forward(self, input_ids: torch.Tensor, cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None, labels: torch.Tensor | None = None,
                gradient_checkpointing: bool = False, padding_mask: torch.Tensor | None = None) -> dict:
        if max_seqlen is None:
            max_seqlen = input_ids.shape[-1]
        x = self._to_autocast_dtype(self.embed_dropout(self.embed_tokens(input_ids)))
        cu_list = None if cu_seqlens is None else cu_seqlens.detach().cpu().tolist()
        if labels is None and self._norms_fusable(x):
            # inference: each residual add runs in the pass of the norm that follows it
            delta = None
            for layer in self.layers:
                x, delta, _ = layer._forward_fused(x, delta, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen,
                                                   cu_list=cu_list)
            _, x = _hip.add_rms_norm(x, delta, self.final_norm.weight, self.final_norm.eps)
            return {"loss": None, "logits": self.lm_head(x), "aux_loss": None}
        aux = torch.zeros((), device=input_ids.device, dtype=x.dtype)
        for layer in self.layers:
            x, a = layer(x, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen,
                         gradient_checkpointing=gradient_checkpointing, cu_list=cu_list)
            if labels is not None:  # the layers' auxiliary losses are only returned with a loss
                aux = aux + a
        x = self.final_norm(x)
        if labels is None:
            return {"loss": None, "logits": self.lm_head(x), "aux_loss": None}
        loss = _chunked_cross_entropy(x.reshape(-1, self.d_model), self.lm_head.weight,
                                      labels.reshape(-1).long(), self.lm_head_chunk_size)
        return {"loss": loss + self.aux_loss_weight * aux, "logits": None, "aux_loss": aux.detach()}

    def _norms_fusable(self, x: torch.Tensor) -> bool:
        """Whether every residual add and norm of the forward can run as dsalt_add_rms_norm
        passes (inference without autograd, 16-bit rows, norm weights of x's dtype)."""
        if not self.layers or not _hip.add_rms_norm_supported(x, self.final_norm.weight):
            return False
        return all(layer._norms_fusable(x, None, layer.attn_norm) and layer._norms_fusable(x, None, layer.ffn_norm)
                   for layer in self.layers)

    def num_parameters(self, trainable_only: bool = True) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad or not trainable_only)

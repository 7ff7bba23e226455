"""DSALTAttention: adaptive local window plus content-selected landmarks, on gfx950.

Drop-in for dsalt/modules/dsalt_attention.py:147-704: same constructor, parameter
creation order (q, k, v, out projections, win_gate, alpha_w, so seeded inits match),
RoPE buffers, fixed attributes (tau_win = 1, tau_lmk = 2, win_edge = 4) and
``forward(x, cu_seqlens=None, max_seqlen=None, rope_cs=None, cu_list=None) -> (out, aux)``.

Packed input (``cu_seqlens`` given) runs the sparse path:
  * training: ``_train_selectors`` (continuous window, HIP landmark top-k, soft landmark
    weight log sigmoid(s/tau_lmk)) then the SOFT HIP kernels (forward + deterministic
    backward carrying d_w~ to win_gate and d_logw to alpha_w), dsalt_attention.py:440-487;
  * inference: floor-quantised windows (HIP), HIP hybrid scores from the value projection
    and HIP landmark top-k, the HARD HIP kernel,
    dsalt_attention.py:610-625; then the ``_last_P`` diagnostic of sequence 0 unless
    ``_collect_last_P`` is set to False (dsalt_attention.py:636-702).
The attention output stays in the compute dtype on the module path (the reference
round-trips it through fp32, which only the ``dsalt.kernels`` entry points keep).

There is no non-GPU fallback: CPU tensors raise. The reference's batched ``[B, T, d]``
path (a dense O(T^2) soft-tail variant) is not provided; pass packed tokens with
``cu_seqlens``.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from .. import _hip
from ..kernels._sparse import sparse_attention
from ..kernels.landmark_tokens_ker import hybrid_scores_from_v, hybrid_scores_per_head
from ..kernels.selectors import _compute_landmark_indices
from ..kernels.window_utils import apply_rotary_emb_packed, build_rope_cache


def _dynamo_opaque(fn):
    disable = getattr(getattr(torch, "_dynamo", None), "disable", None)
    return disable(fn) if disable is not None else fn


class DSALTAttention(nn.Module):
    """DSALT sparse attention: adaptive causal window plus k landmark tokens per head.

    Query i attends to ``A(i) = W(i) ∪ L(i)``: a causal local window of
    ``w~(i) = n_min + sigmoid(win_gate(x_i)) * (n_max - n_min)`` tokens and the
    landmarks left of the window, selected per (head, sequence) by the hybrid score
    with per-head balance ``alpha = sigmoid(alpha_w)``.

    ``_fused_selector`` (default True): with ``qkv_bias=False`` the landmark scores are
    formed from the module's own value projection ``v = x W_V^T`` (the fused HIP score
    kernel for the detached selection, the same formula in torch for the
    differentiable ``lmk_logw``) instead of a second ``x @ W_V.T`` GEMM. Set it to False
    for the reference's GEMM path.
    """

    _fused_selector = True

    def __init__(
        self,
        d_model: int,
        n_heads: int,
        n_min: int,
        n_max: int,
        k_lmk: int,
        max_seq_len: int,
        dropout: float = 0.0,
        yarn_scale: float = 1.0,
        layer_idx: int = 0,
        n_kv_heads: int | None = None,
        qkv_bias: bool = False,
        rope_base: float = 10000.0,
    ):
        super().__init__()
        assert d_model % n_heads == 0
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.n_kv_heads = n_kv_heads if n_kv_heads is not None else n_heads
        assert n_heads % self.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads"
        self.n_rep = n_heads // self.n_kv_heads
        self.kv_dim = self.n_kv_heads * self.head_dim
        self.n_min = n_min
        self.n_max = n_max
        self.k_lmk = k_lmk
        self.max_seq_len = max_seq_len
        self.dropout = dropout
        self.yarn_scale = yarn_scale
        self.rope_base = rope_base
        self.layer_idx = layer_idx

        self.q_proj = nn.Linear(d_model, d_model, bias=qkv_bias)
        self.k_proj = nn.Linear(d_model, self.kv_dim, bias=qkv_bias)
        self.v_proj = nn.Linear(d_model, self.kv_dim, bias=qkv_bias)
        self.out_proj = nn.Linear(d_model, d_model, bias=False)
        self.win_gate = nn.Linear(d_model, 1, bias=True)
        self.alpha_w = nn.Parameter(torch.full((n_heads,), math.log(0.6 / 0.4)))

        self.tau_win = 1.0
        self.tau_lmk = 2.0
        self.win_edge = 4

        self._last_P: torch.Tensor | None = None

        cos, sin = build_rope_cache(max_seq_len, self.head_dim, torch.device("cpu"),
                                    base=rope_base, scale=yarn_scale)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    # ---- small pieces (dsalt_attention.py:243-284, :331-342) ---------------------------
    def _alpha(self) -> torch.Tensor:
        return torch.sigmoid(self.alpha_w)

    def _apply_out_proj(self, out: torch.Tensor) -> torch.Tensor:
        return self.out_proj(out.to(self.out_proj.weight.dtype))

    def _repeat_kv(self, t: torch.Tensor) -> torch.Tensor:
        if self.n_rep == 1:
            return t
        T, _, D = t.shape
        return t.unsqueeze(2).expand(T, self.n_kv_heads, self.n_rep, D).reshape(T, self.n_heads, D)

    def _window_continuous(self, x: torch.Tensor) -> torch.Tensor:
        """``w~ = n_min + sigmoid(win_gate(x)) * (n_max - n_min)``, differentiable, ``[T]``."""
        win_logits = self.win_gate(x).squeeze(-1)
        return self.n_min + torch.sigmoid(win_logits) * (self.n_max - self.n_min)

    @torch.no_grad()
    def _window_sizes(self, x: torch.Tensor, floor: bool) -> torch.Tensor:
        """Integer-valued windows ``>= 1``: floor (HIP kernel) at inference, round otherwise."""
        w_cont = self._window_continuous(x)
        if floor:
            return _hip.quantize_windows(w_cont)
        return w_cont.round().clamp(min=1)

    @torch.no_grad()
    def _rope(self, n: int, device: torch.device):
        max_n = self.rope_cos.shape[0]
        if n <= max_n:
            return self.rope_cos[:n].to(device), self.rope_sin[:n].to(device)
        return self.rope_cos.to(device), self.rope_sin.to(device)

    def _aux_zero(self, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        return torch.zeros((), device=device, dtype=dtype)

    @torch.no_grad()
    def warmup(self, device: torch.device) -> None:
        was_training = self.training
        self.eval()
        dummy_T = max(self.n_min * 2, 16)
        x_w = torch.randn(dummy_T, self.d_model, device=device)
        cu_w = torch.tensor([0, dummy_T], dtype=torch.int32, device=device)
        self._packed(x_w, cu_w, dummy_T, device)
        torch.cuda.synchronize(device)
        self.train(was_training)

    # ---- forward -----------------------------------------------------------------------
    def forward(self, x: torch.Tensor, cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None, rope_cs: tuple | None = None,
                cu_list: list | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        if cu_seqlens is not None:
            return self._packed(x, cu_seqlens, x.shape[0], x.device, rope_cs, cu_list)
        raise NotImplementedError(
            "the dense batched [B, T, d] DSALT variant is not provided by the HIP path; pack "
            "the tokens to [T, d] and pass cu_seqlens (int32 [S + 1]) for sparse attention")

    @_dynamo_opaque
    def _train_selectors(self, x, cu_seqlens, total_len, device, cu_list=None, v=None):
        """``(w_cont [T], lmk_pos [H,S,k], lmk_logw [H,S,k])`` (dsalt_attention.py:457-487):
        the selection is detached; ``w_cont`` and ``lmk_logw`` carry the gradients.
        With ``v`` (the pre-RoPE value projection ``[T, n_kv, dh]``) the scores are
        formed from it instead of a second ``x @ W_V.T`` GEMM."""
        w_cont = self._window_continuous(x)
        alpha = self._alpha()
        fused = v is not None and self._fused_selector
        with torch.no_grad():
            w_disc = _hip.quantize_windows(w_cont.detach())
            lmk_pos, _, _ = _compute_landmark_indices(
                x.detach(), self.v_proj.weight.detach(), alpha.detach().float(),
                w_disc, cu_seqlens, self.k_lmk, self.n_min, total_len, cu_list,
                head_dim=self.head_dim, v=v.detach() if fused else None,
            )
        if fused:
            scores, _, _ = hybrid_scores_from_v(x, v, alpha, self.n_heads)
        else:
            scores, _, _ = hybrid_scores_per_head(x, self.v_proj.weight, alpha, self.n_heads, self.head_dim)
        starts = cu_seqlens[:-1].to(device).long()
        safe_pos = lmk_pos.clamp(min=0)
        abs_pos = starts[None, :, None] + safe_pos
        head_ix = torch.arange(self.n_heads, device=device)[:, None, None]
        s_sel = scores[abs_pos, head_ix]
        lmk_logw = torch.log(torch.sigmoid(s_sel / self.tau_lmk).clamp(min=1e-20))
        lmk_logw = torch.where(lmk_pos >= 0, lmk_logw, torch.full_like(lmk_logw, float("-inf")))
        return w_cont, lmk_pos, lmk_logw

    def _packed(self, x: torch.Tensor, cu_seqlens: torch.Tensor, total_len: int, device: torch.device,
                rope_cs: tuple | None = None, cu_list: list | None = None):
        _hip.require_gpu(x, cu_seqlens)
        q = self.q_proj(x).view(total_len, self.n_heads, self.head_dim)
        k = self.k_proj(x).view(total_len, self.n_kv_heads, self.head_dim)
        v = self.v_proj(x).view(total_len, self.n_kv_heads, self.head_dim)
        # x W_V^T before RoPE and the kv repeat: the selector's value norms come from it
        # (qkv_bias=False only; with a bias v is not x W_V^T)
        v_sel = v if self.v_proj.bias is None else None

        # RoPE in one HIP pass (dsalt_attention.py:570-585): positions from cu_seqlens
        # in-kernel, cos/sin rounded to q's dtype as the reference's cos.to(q.dtype)
        if rope_cs is None:
            q, k = apply_rotary_emb_packed(q, k, self.rope_cos, self.rope_sin, cu_seqlens)
        else:
            cos, sin = rope_cs
            q, k = apply_rotary_emb_packed(q, k, cos.reshape(total_len, -1), sin.reshape(total_len, -1))
        k = self._repeat_kv(k)
        v = self._repeat_kv(v)

        aux = self._aux_zero(x.device, x.dtype)

        if self.training:
            self._last_P = None
            w_cont, lmk_pos, lmk_logw = self._train_selectors(x, cu_seqlens, total_len, device, cu_list, v_sel)
            out = sparse_attention(_hip.MODE_SOFT, q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens,
                                   self.tau_win, float(self.win_edge))
            return self._apply_out_proj(out.reshape(total_len, self.d_model)), aux

        w_sizes = self._window_sizes(x, floor=True)
        alpha = self._alpha()
        lmk_indices, _, _ = _compute_landmark_indices(
            x.detach(), self.v_proj.weight.detach(), alpha.detach().float(), w_sizes,
            cu_seqlens, self.k_lmk, self.n_min, total_len, cu_list, head_dim=self.head_dim,
            v=v_sel.detach() if (self._fused_selector and v_sel is not None) else None,
        )
        # Hard A(i) = W(i) ∪ L(i): the score only selects (zero landmark bias).
        out = sparse_attention(_hip.MODE_HARD, q, k, v, lmk_indices, None, w_sizes, cu_seqlens)

        if not getattr(self, "_collect_last_P", True):
            self._last_P = None
        else:
            self._last_P = self._first_sequence_probs(x, q, k, w_sizes, alpha, cu_seqlens, cu_list, device)
        return self._apply_out_proj(out.reshape(total_len, self.d_model)), aux

    @torch.no_grad()
    def _first_sequence_probs(self, x, q, k, w_sizes, alpha, cu_seqlens, cu_list, device):
        """Dense ``[H, T0, T0]`` attention probabilities of sequence 0 under the HARD set,
        the metrics diagnostic of dsalt_attention.py:643-702 (landmarks re-selected on
        sequence 0 alone, in fp32). O(T0^2); disabled by ``_collect_last_P = False``."""
        if cu_list is not None:
            s0, e0 = int(cu_list[0]), int(cu_list[1])
        else:
            s0, e0 = (int(c) for c in cu_seqlens[:2].tolist())
        T0 = e0 - s0
        q0 = q[s0:e0].transpose(0, 1)
        k0 = k[s0:e0].transpose(0, 1)
        scale = 1.0 / math.sqrt(self.head_dim)
        cu0 = torch.tensor([0, T0], dtype=torch.int32, device=device)
        w0 = w_sizes[s0:e0]
        lmk_idx, _, _ = _compute_landmark_indices(
            x[s0:e0].float().detach(), self.v_proj.weight.float().detach(), alpha.detach().float(),
            w0.float(), cu0, self.k_lmk, self.n_min, T0, [0, T0], head_dim=self.head_dim)
        rows = torch.arange(T0, device=device)
        w0l = w0.long()
        in_win = (rows[None, :] >= rows[:, None] - w0l[:, None] + 1) & (rows[None, :] <= rows[:, None])
        lmk0 = lmk_idx[:, 0, :]
        col_is_lmk = torch.zeros(self.n_heads, T0 + 1, dtype=torch.bool, device=device)
        col_is_lmk.scatter_(1, torch.where(lmk0 >= 0, lmk0, T0), True)
        in_lmk = col_is_lmk[:, None, :T0] & (rows[None, None, :] <= rows[None, :, None])
        full_mask = in_win.unsqueeze(0) | in_lmk
        sc = torch.matmul(q0, k0.transpose(-2, -1).contiguous()) * scale
        additive = sc.new_full((self.n_heads, T0, T0), float("-inf")).masked_fill_(full_mask, 0.0)
        return torch.softmax(sc + additive, dim=-1).detach()

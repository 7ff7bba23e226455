"""DSALTAttention: adaptive local window plus content-selected landmarks, on gfx950.

Drop-in for dsalt/modules/dsalt_attention.py:147-704: same constructor, parameter
creation order (q, k, v, out projections, win_gate, alpha_w, so seeded inits match),
RoPE buffers, fixed attributes (tau_win = 1, tau_lmk = 2, win_edge = 4) and
``forward(x, cu_seqlens=None, max_seqlen=None, rope_cs=None, cu_list=None) -> (out, aux)``.

Packed input (``cu_seqlens`` given) runs the sparse path:
  * training: ``_train_selectors`` (continuous window, HIP landmark top-k, soft landmark
    weight log sigmoid(s/tau_lmk)) then the SOFT HIP kernels (forward + deterministic
    backward carrying d_w~ to win_gate and d_logw to alpha_w), dsalt_attention.py:440-487;
  * inference: two HIP launches select (dsalt_select_hybrid: a norms pass over x and the
    value projection that also rotates k, then one launch forming the hybrid scores, the
    floor-quantised windows from the gate logits and the landmark top-k), then the HARD
    HIP kernel rotating q as it loads it, dsalt_attention.py:610-625; then the
    ``_last_P`` diagnostic of sequence 0 unless ``_collect_last_P`` is set to False
    (dsalt_attention.py:636-702).
The attention output stays in the compute dtype on the module path (the reference
round-trips it through fp32, which only the ``dsalt.kernels`` entry points keep).

Unpacked input ``[1, T, d]`` (no ``cu_seqlens``) runs the dense batched variant of
dsalt_attention.py:371-438 on the DSALT_MODE_DENSE HIP kernels: every causal key with
the soft window tail, landmark weights log sigmoid(s/tau_lmk) at the top-k keys of each
head (selected by the HIP top-k over the whole sequence) left of floor(w~), union by
maximum; differentiable in w~ and the landmark weights in training and eval alike. In
eval ``_last_P`` holds the dense [H, T, T] probabilities unless ``_collect_last_P`` is
False. B > 1 raises (the reference's view of the [1, T, d] result fails there too), and
so does attention dropout in training.

There is no non-GPU fallback: CPU tensors raise.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _hip
from ..kernels._dense import dense_attention, dense_probabilities
from ..kernels._sparse import sparse_attention
from ..kernels.landmark_tokens_ker import hybrid_scores_from_v, hybrid_scores_per_head
from ..kernels.selectors import _compute_landmark_indices, _landmarks_and_windows
from ..kernels.window_utils import apply_rotary_emb_packed, build_rope_cache, rotate_packed


def _dynamo_opaque(fn):
    disable = getattr(getattr(torch, "_dynamo", None), "disable", None)
    return disable(fn) if disable is not None else fn


class DSALTAttention(nn.Module):
    """DSALT sparse attention: adaptive causal window plus k landmark tokens per head.

    Query i attends to ``A(i) = W(i) ∪ L(i)``: a causal local window of
    ``w~(i) = n_min + sigmoid(win_gate(x_i)) * (n_max - n_min)`` tokens and the
    landmarks left of the window, selected per (head, sequence) by the hybrid score
    with per-head balance ``alpha = sigmoid(alpha_w)``.

    ``_fused_selector`` (default True): without a projection bias the landmark scores are
    formed from the module's own value projection ``v = x W_V^T`` instead of a second
    ``x @ W_V.T`` GEMM. ``_hip_scores`` (default True) selects with the HIP norms pass over
    x and v, whose statistics, standardisation and hybrid combination the selection launch
    forms itself (no torch passes, no score tensor); it rounds its fp32 norm sums in another
    order than torch, so a score can differ in its last bits from the reference's route -
    the landmark sets of configs 2, 3 and 4 (fp32, bf16, autocast) are the reference
    route's, set for set, but a near-tie could move. ``_hip_scores = False`` keeps torch's own norm
    and standardisation ops on v, whose fp32 scores are bit-identical to the reference's
    route. The differentiable landmark weights of training always use the torch ops.
    ``_fuse_gate`` (default True): on that route's inference path, with 16-bit x and
    ``win_gate`` parameters of x's dtype, the norms pass also forms the window gate's
    logits (an fp32 dot product in its own fixed order, rounded once) instead of torch's
    GEMV; a logit can then differ from torch's in its last bit and move a window by one
    key - the windows of configs 2 and 5 are torch's, token for token.
    ``_fuse_qkv`` (default True): at inference without autograd or autocast, without
    projection biases and with ``_hip_scores`` (the reference-exact score route keeps the
    separate projections), q, k and v come from one GEMM against the three weights concatenated
    (cached until a weight changes; one extra copy of them in device memory) and are column
    views of its output - the kernels take their strides as they are. At configs 2 and 5 the
    columns equal the three separate projections bit for bit (hipBLASLt runs the same
    reduction order), and the one GEMM of 3x the width fills more of the chip. The cache
    follows each weight's pointer and version counter: in-place updates (optimizer steps,
    ``load_state_dict``, ``copy_`` under no_grad) are seen, but a change made through
    ``weight.data`` does not bump the counter - call ``invalidate_qkv_cache()`` after one.
    ``_last_selection`` holds the ``(windows, landmark positions)`` of the last forward.
    """

    _fused_selector = True
    _hip_scores = True
    _fuse_rope_k = True  # inference: k rotated by the selection's norms pass (when that route is taken)
    _fuse_gate = True    # inference: the window gate's logits formed by the same norms pass
    _fuse_qkv = True     # inference: q, k and v from one GEMM over the concatenated weights

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
        self._last_selection: tuple | None = None

        cos, sin = build_rope_cache(max_seq_len, self.head_dim, torch.device("cpu"),
                                    base=rope_base, scale=yarn_scale)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    # ---- small pieces (dsalt_attention.py:243-284) ---------------------------------------
    def invalidate_qkv_cache(self) -> None:
        """Drop the cached concatenation of the q/k/v weights (``_fuse_qkv``)."""
        self._qkv_weight_cache = None

    def _project_qkv(self, x: torch.Tensor):
        """``(q_proj(x), k_proj(x), v_proj(x))`` as [T, d_model], [T, kv_dim], [T, kv_dim]; with
        ``_fuse_qkv`` at inference one GEMM whose output columns the three are views of."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        if not (self._fuse_qkv and self._hip_scores and not self.training and not torch.is_grad_enabled() and x.is_cuda
                and not torch.is_autocast_enabled() and self.q_proj.bias is None and self.k_proj.bias is None
                and self.v_proj.bias is None and all(w.dtype == x.dtype and w.device == x.device for w in ws)
                and self.d_model % 8 == 0 and self.kv_dim % 8 == 0):
            return self.q_proj(x), self.k_proj(x), self.v_proj(x)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        cache = getattr(self, "_qkv_weight_cache", None)
        if cache is None or cache[0] != key:
            cache = (key, torch.cat([w.detach() for w in ws], 0))
            self._qkv_weight_cache = cache
        qkv = F.linear(x, cache[1])
        d, kv = self.d_model, self.kv_dim
        return qkv[:, :d], qkv[:, d:d + kv], qkv[:, d + kv:]

    def _alpha(self) -> torch.Tensor:
        return torch.sigmoid(self.alpha_w)

    def _alpha_selection(self) -> torch.Tensor:
        """``sigmoid(alpha_w)`` detached, in fp32 (rounded to ``alpha_w``'s dtype first, as
        the selection's scores see it): the per-head balance of the inference selection,
        which takes no gradient. Computed once per parameter storage and version."""
        p = self.alpha_w
        key = (p.data_ptr(), p._version, p.dtype)
        hit = getattr(self, "_alpha_sel_cache", None)
        if hit is None or hit[0] != key:
            with torch.no_grad():
                hit = (key, torch.sigmoid(p.detach()).float())
            self._alpha_sel_cache = hit
        return hit[1]

    def _rope_tables(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``rope_cos`` / ``rope_sin`` as the contiguous fp32 tables the HIP kernels read
        (they round each entry to the tensor dtype, so the values used are unchanged),
        converted once per buffer storage and version instead of on every call."""
        c, s = self.rope_cos, self.rope_sin
        key = (c.data_ptr(), s.data_ptr(), c._version, s._version, c.dtype)
        hit = getattr(self, "_rope_tables_cache", None)
        if hit is None or hit[0] != key:
            hit = (key, c.to(torch.float32).contiguous(), s.to(torch.float32).contiguous())
            self._rope_tables_cache = hit
        return hit[1], hit[2]

    def _apply_out_proj(self, out: torch.Tensor) -> torch.Tensor:
        """out_proj in its weight's dtype (the attention output may be fp32 or 16-bit)."""
        wdt = self.out_proj.weight.dtype
        return self.out_proj(out if out.dtype == wdt else out.to(wdt))

    def _repeat_kv(self, t: torch.Tensor) -> torch.Tensor:
        """[T, n_kv, D] -> [T, H, D]: kv head g serves query heads g*n_rep .. g*n_rep+n_rep-1."""
        if self.n_rep == 1:
            return t
        return t.repeat_interleave(self.n_rep, dim=1)

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
    def warmup(self, device: torch.device) -> None:
        """One small inference forward on ``device``: loads the HIP library and makes the
        first launches outside any timed region. The training flag is restored."""
        mode = self.training
        try:
            self.train(False)
            n = max(16, 2 * self.n_min)
            x = torch.randn(n, self.d_model, device=device, dtype=self.q_proj.weight.dtype)
            self._packed(x, torch.tensor([0, n], dtype=torch.int32, device=device), n, device)
            torch.cuda.synchronize(device)
        finally:
            self.train(mode)

    # ---- forward -----------------------------------------------------------------------
    def forward(self, x: torch.Tensor, cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None, rope_cs: tuple | None = None,
                cu_list: list | None = None, *, _need_aux: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
        # _need_aux=False (internal, packed path): return None instead of the zero aux loss,
        # so that a caller that discards it launches no fill for it
        if cu_seqlens is not None:
            return self._packed(x, cu_seqlens, x.shape[0], x.device, rope_cs, cu_list, need_aux=_need_aux)
        B, T, _ = x.shape
        return self._batched(x, B, T, x.device)

    def _batched(self, x: torch.Tensor, B: int, T: int, device: torch.device):
        """Dense batched forward of ``x [1, T, d]`` (dsalt_attention.py:371-438)."""
        _hip.require_gpu(x)
        if B != 1:
            raise ValueError(f"the dense batched path takes one sequence [1, T, d] (got B = {B}); pack "
                             "several sequences to [T, d] and pass cu_seqlens")
        if self.training and self.dropout > 0:
            raise NotImplementedError("attention dropout is not supported by the dense HIP path")
        xs = x[0]
        q = self.q_proj(xs).view(T, self.n_heads, self.head_dim)
        k = self.k_proj(xs).view(T, self.n_kv_heads, self.head_dim)
        v = self.v_proj(xs).view(T, self.n_kv_heads, self.head_dim)
        v_sel = v if (self.v_proj.bias is None and self._fused_selector) else None
        cu = torch.tensor([0, T], dtype=torch.int32, device=device)
        q, k = apply_rotary_emb_packed(q, k, *self._rope_tables(), cu)

        # grouped K/V heads go to the kernels as they are (query head h reads K/V head
        # h // n_rep); no repeated copy
        w_cont, lmk_bias, lmk_pos = self._dense_selectors(xs, T, device, v_sel)
        out = dense_attention(q, k, v, w_cont, lmk_bias, self.tau_win, float(self.win_edge))
        if not self.training and getattr(self, "_collect_last_P", True):
            self._last_P = dense_probabilities(q, self._repeat_kv(k), w_cont, lmk_bias, self.tau_win,
                                               float(self.win_edge))
        else:
            self._last_P = None
        self._last_selection = (w_cont.detach(), lmk_pos)
        aux = x.new_zeros(())
        return self._apply_out_proj(out.reshape(1, T, self.d_model)), aux

    @_dynamo_opaque
    def _dense_selectors(self, x, T, device, v=None):
        """``(w_cont [T], lmk_bias [H, T], lmk_pos [H, 1, k])`` of the dense variant
        (dsalt_attention.py:403-438): the top-min(k, T) keys of each head over the whole
        sequence by the detached fp32 hybrid score (nothing excluded: the window exclusion
        is per query, in the kernel), weight log(max(sigmoid(s / tau_lmk), 1e-20)) there
        and -inf elsewhere. ``w_cont`` and the weights carry the gradients."""
        w_cont = self._window_continuous(x)
        alpha = self._alpha()
        if v is not None:
            scores, _, _ = hybrid_scores_from_v(x, v, alpha, self.n_heads)
        else:
            scores, _, _ = hybrid_scores_per_head(x, self.v_proj.weight, alpha, self.n_heads, self.head_dim)
        k_act = min(self.k_lmk, T)
        with torch.no_grad():
            cu = torch.tensor([0, T], dtype=torch.int32, device=device)
            lmk_pos = _hip.select_landmarks(scores.detach().float().contiguous(),
                                            torch.zeros(T, device=device), cu, k_act, max_seqlen=T)
            sel = torch.zeros(self.n_heads, T + 1, dtype=torch.bool, device=device)
            sel.scatter_(1, torch.where(lmk_pos[:, 0] >= 0, lmk_pos[:, 0], T), True)
            sel = sel[:, :T]
        w_lmk = torch.log(torch.sigmoid(scores.float() / self.tau_lmk).clamp(min=1e-20)).t()   # [H, T]
        lmk_bias = torch.where(sel, w_lmk, torch.full_like(w_lmk, float("-inf")))
        return w_cont, lmk_bias, lmk_pos

    @_dynamo_opaque
    def _train_selectors(self, x, cu_seqlens, total_len, device, cu_list=None, v=None):
        """``(w_cont [T], lmk_pos [H,S,k], lmk_logw [H,S,k])`` (dsalt_attention.py:457-487):
        the selection is detached; ``w_cont`` and ``lmk_logw`` carry the gradients.
        With ``v`` (the pre-RoPE value projection ``[T, n_kv, dh]``, equal to ``x @ W_V.T``
        when the projection has no bias) the scores are formed from it instead of a second
        GEMM; the selection sees bit-identical scores either way."""
        w_cont = self._window_continuous(x)
        alpha = self._alpha()
        route_v = v if self._fused_selector else None
        with torch.no_grad():  # windows quantised by the selection launch
            w_disc, lmk_pos = _landmarks_and_windows(
                x.detach(), self.v_proj.weight.detach(), alpha.detach().float(), w_cont.detach(),
                cu_seqlens, self.k_lmk, cu_list, head_dim=self.head_dim,
                v=None if route_v is None else route_v.detach(), hip_scores=self._hip_scores)
        # the differentiable scores (the selection above ran on a detached copy of them)
        if route_v is not None:
            scores, _, _ = hybrid_scores_from_v(x, route_v, alpha, self.n_heads)
        else:
            scores, _, _ = hybrid_scores_per_head(x, self.v_proj.weight, alpha, self.n_heads, self.head_dim)
        H, S, k = lmk_pos.shape
        # score of each selected landmark: column h of scores at token cu[s] + pos
        first = cu_seqlens[:-1].to(device=device, dtype=torch.long)
        tok = (first.view(1, S, 1) + lmk_pos.clamp_min(0)).reshape(H, S * k)
        s_sel = scores.t().gather(1, tok).view(H, S, k)
        lmk_logw = torch.sigmoid(s_sel / self.tau_lmk).clamp(min=1e-20).log()
        lmk_logw = lmk_logw.masked_fill(lmk_pos < 0, float("-inf"))
        self._last_selection = (w_disc, lmk_pos)
        return w_cont, lmk_pos, lmk_logw

    def _packed(self, x: torch.Tensor, cu_seqlens: torch.Tensor, total_len: int, device: torch.device,
                rope_cs: tuple | None = None, cu_list: list | None = None, need_aux: bool = True):
        _hip.require_gpu(x, cu_seqlens)
        q, k, v = self._project_qkv(x)
        q = q.view(total_len, self.n_heads, self.head_dim)
        k = k.view(total_len, self.n_kv_heads, self.head_dim)
        v = v.view(total_len, self.n_kv_heads, self.head_dim)
        # x W_V^T before RoPE and the kv repeat: the selector's value norms come from it
        # (only without a projection bias, where v is exactly x W_V^T)
        v_sel = v if self.v_proj.bias is None else None

        # RoPE in one HIP pass (dsalt_attention.py:570-585): positions from cu_seqlens
        # in-kernel, cos/sin rounded to q's dtype as the reference's cos.to(q.dtype). At
        # inference without autograd only k is rotated here: the attention kernel rotates
        # q as it loads it (the same arithmetic), so q is never written back rotated.
        fuse_q = not self.training and rope_cs is None and not torch.is_grad_enabled()
        # ... and k is rotated by the launch that computes the selector norms from x and v,
        # when the selection takes that route (the HIP score kernels)
        fuse_k = (fuse_q and self._fuse_rope_k and self._hip_scores and self._fused_selector and v_sel is not None
                  and k.shape == v_sel.shape and _hip.scores_supported(x, v_sel))
        if fuse_q:
            if not fuse_k:
                k = rotate_packed(k, *self._rope_tables(), cu_seqlens)
        elif rope_cs is None:
            q, k = apply_rotary_emb_packed(q, k, *self._rope_tables(), cu_seqlens)
        else:
            cos, sin = rope_cs
            q, k = apply_rotary_emb_packed(q, k, cos.reshape(total_len, -1), sin.reshape(total_len, -1))
        # grouped K/V heads go to the kernels as they are (query head h reads K/V head
        # h // n_rep); no repeated copy

        aux = x.new_zeros(()) if need_aux else None

        if self.training:
            self._last_P = None
            w_cont, lmk_pos, lmk_logw = self._train_selectors(x, cu_seqlens, total_len, device, cu_list, v_sel)
            out = sparse_attention(_hip.MODE_SOFT, q, k, v, lmk_pos, lmk_logw, w_cont, cu_seqlens,
                                   self.tau_win, float(self.win_edge))
            return self._apply_out_proj(out.reshape(total_len, self.d_model)), aux

        alpha = self._alpha_selection()  # the HARD output takes no gradient from the scores
        route_v = v_sel if self._fused_selector else None
        # the windows are formed from the gate's logits and quantised by the selection
        # launch itself (same values as _window_sizes(floor=True) followed by
        # _compute_landmark_indices)
        gate_linear = None
        if fuse_k and self._fuse_gate and _hip.gate_linear_supported(x, self.win_gate.weight, self.win_gate.bias):
            # the norms pass forms the gate's logits: no GEMV
            bias = self.win_gate.bias
            gate_linear = (self.win_gate.weight.detach(), None if bias is None else bias.detach(), self.n_min,
                           self.n_max)
            gate = w_cont = None
        else:
            with torch.no_grad():
                logit = self.win_gate(x).squeeze(-1)
                # 16-bit logits: the launch forms the windows (torch's fp32 sigmoid is not
                # reproduced bit for bit, so fp32 logits take torch's window ops)
                gate = (logit, self.n_min, self.n_max) if logit.dtype in (torch.bfloat16, torch.float16) else None
                w_cont = None if gate is not None else self.n_min + torch.sigmoid(logit) * (self.n_max - self.n_min)
        if fuse_k:
            # two launches: the norms pass (which also rotates k), then the selection,
            # which forms the scores, the windows and the top-k
            with torch.no_grad():
                max_len = None if cu_list is None else max((b - a for a, b in zip(cu_list[:-1], cu_list[1:])),
                                                           default=0)
                w_sizes, lmk_indices, k = _hip.select_hybrid(
                    x.detach(), v_sel.detach(), alpha.detach().float(), self.n_heads, w_cont, cu_seqlens, self.k_lmk,
                    max_seqlen=max_len, gate=gate, rope_k=(k, *self._rope_tables(), cu_seqlens),
                    gate_linear=gate_linear)
        else:
            with torch.no_grad():
                w_sizes, lmk_indices = _landmarks_and_windows(
                    x.detach(), self.v_proj.weight.detach(), alpha.detach().float(), w_cont,
                    cu_seqlens, self.k_lmk, cu_list, head_dim=self.head_dim,
                    v=None if route_v is None else route_v.detach(), hip_scores=self._hip_scores, gate=gate)
        self._last_selection = (w_sizes, lmk_indices)
        # Hard A(i) = W(i) ∪ L(i): the score only selects (zero landmark bias).
        out = sparse_attention(_hip.MODE_HARD, q, k, v, lmk_indices, None, w_sizes, cu_seqlens,
                               rope=self._rope_tables() if fuse_q else None)

        if getattr(self, "_collect_last_P", True):
            if fuse_q:  # the diagnostic needs the rotated q of the first sequence
                n0 = int(cu_list[1]) if cu_list is not None else int(cu_seqlens[1])
                q = rotate_packed(q[:n0].contiguous(), *self._rope_tables(), cu_seqlens[:2])
            self._last_P = self._first_sequence_probs(x, q, k, w_sizes, alpha, cu_seqlens, cu_list)
        else:
            self._last_P = None
        return self._apply_out_proj(out.reshape(total_len, self.d_model)), aux

    @torch.no_grad()
    def _first_sequence_probs(self, x, q, k, w_sizes, alpha, cu_seqlens, cu_list):
        """Dense ``[H, L0, L0]`` attention probabilities of the first packed sequence under
        the HARD set (the metrics diagnostic of dsalt_attention.py:636-702): the landmarks
        are selected again on that sequence alone from fp32 scores, the logits are formed
        in q's dtype, and keys outside ``(i - w_i, i] ∪ {landmarks <= i}`` get probability
        0. O(L0^2); ``_collect_last_P = False`` turns it off."""
        bounds = cu_list if cu_list is not None else cu_seqlens[:2].tolist()
        a, b = int(bounds[0]), int(bounds[1])
        n = b - a
        dev = q.device
        seg = slice(a, b)
        w0 = w_sizes[seg]
        lmk, _, _ = _compute_landmark_indices(
            x[seg].detach().float(), self.v_proj.weight.detach().float(), alpha.detach().float(), w0.float(),
            torch.tensor([0, n], dtype=torch.int32, device=dev), self.k_lmk, self.n_min, n, [0, n],
            head_dim=self.head_dim)
        pos = torch.arange(n, device=dev)
        back = pos.view(n, 1) - pos.view(1, n)                      # i - j
        in_band = (back >= 0) & (back < w0.long().view(n, 1))       # i - w_i < j <= i
        is_lmk = torch.zeros(self.n_heads, n + 1, dtype=torch.bool, device=dev)
        is_lmk.scatter_(1, torch.where(lmk[:, 0] >= 0, lmk[:, 0], n), True)
        keep = in_band.unsqueeze(0) | (is_lmk[:, None, :n] & (back >= 0).unsqueeze(0))
        k0 = self._repeat_kv(k[seg])
        logits = torch.matmul(q[seg].transpose(0, 1), k0.transpose(0, 1).transpose(1, 2).contiguous())
        logits = logits * (1.0 / math.sqrt(self.head_dim))
        return logits.masked_fill(~keep, float("-inf")).softmax(dim=-1)

"""CPU oracle for the DSALT sparse-attention hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or the timed CPU baseline) - never as a product code
path. It restates, on the CPU, the reference algorithm of LeonardoCofone/dsalt-library
(files cited relative to the reference root):

  hybrid_scores          dsalt/kernels/landmark_tokens_ker.py:45-61
  window_continuous      dsalt/modules/dsalt_attention.py:270-275
  quantize_windows       dsalt/modules/dsalt_attention.py:277-284, :471
  select_landmarks       dsalt/kernels/selectors.py:105-134 (numpy, exact)
  attention_hard         dsalt/kernels/dsalt_triton_attn.py:69-169 (the HARD set; equal to
                         the _last_P mask of dsalt_attention.py:668-692)
  attention_soft         dsalt/kernels/dsalt_triton_train.py:116-214 with the exact band of
                         the dense reference dsalt_attention.py:520-563
  gradients              torch autograd through attention_hard / attention_soft in fp64
                         (the formulas of dsalt_triton_train.py:302-383, :439-476)
  attention_dense        the dense batched variant of _batched / _diff_logbias
                         (dsalt/modules/dsalt_attention.py:286-329, :371-438): soft window
                         tail on every causal key, landmarks admitted at d >= max(1, floor(w~)),
                         union = elementwise max of the two log-biases
  rope, seq_positions    dsalt/kernels/window_utils.py:73-88 as dsalt_attention.py:570-585
                         calls it (positions inside each packed sequence)
  hybrid_scores_from_v   hybrid_scores on the module's value projection v = x W_V^T
  module_train_forward   the packed training forward of DSALTAttention (dsalt_attention.py:
                         440-487, :565-609): projections, RoPE, SOFT selectors, attention
  module_eval_forward    the packed inference forward (dsalt_attention.py:610-625): the
                         same projections and RoPE, floor windows, top-k, HARD attention
  module_batched_forward dsalt_attention.py:371-401 (B = 1) from the module parameters
  effective_pairs,       the pair counts of F = 4 D P (band keys plus admitted landmark
  hard_mask              slots) and the dense HARD mask
  lm_forward             DSALTLMHeadModel eval logits (dsalt/model/dsalt_lm.py:237-280):
                         embedding, pre-norm blocks (RMSNorm, attention, SwiGLU), final
                         RMSNorm, tied head; lm_train_loss the packed training loss
  cpu_baseline_hard      the reference's CPU fallback cost model: dense per-sequence mask +
                         F.scaled_dot_product_attention in fp32 (dsalt_attention.py:95-144,
                         dsalt/kernels/sparse_attn.py:29-57), with the HARD kernel's mask

Pinning (tests/test_oracle.py): closed forms and library routines - causal attention via
F.scaled_dot_product_attention(is_causal=True) when k = 0 and the window covers the
sequence; O_i = V_i for w = 1, k = 0; the constant-landmark-bias reweighting closed
form; the soft edge against F.logsigmoid; selection against a brute-force Python sort
and against torch.topk as sets; scores against numpy's mean/std(ddof=1); gradients
against finite differences (torch.autograd.gradcheck) - and the committed golden
fixtures of tests/golden/ (module_train_forward, module_batched_forward, lm_forward,
lm_train_loss). module_eval_forward has no golden of its own: it composes the pinned
pieces above with module_train_forward's golden-pinned projections and RoPE. The pair
counts equal the entries of the masks attention_hard / attention_soft build
(tests/test_bench_counts.py). The reference ships no golden vectors of its own.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

# ---------------------------------------------------------------------------------------
# selectors
# ---------------------------------------------------------------------------------------


def hybrid_scores(x: torch.Tensor, W_V: torch.Tensor, alpha: torch.Tensor, n_heads: int, dh: int):
    """(scores [T,H], z_x [T], z_v [T,H]); landmark_tokens_ker.py:45-61."""
    T = x.shape[0]
    x_norm = x.norm(dim=-1).float()
    z_x = (x_norm - x_norm.mean()) / x_norm.std().clamp(min=1e-6)
    n_kv = W_V.shape[0] // dh
    xwv = (x @ W_V.T).view(T, n_kv, dh).norm(dim=-1).float()
    z_v = (xwv - xwv.mean(0, keepdim=True)) / xwv.std(0, keepdim=True).clamp(min=1e-6)
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)
    scores = alpha * z_v + (1.0 - alpha) * z_x.unsqueeze(1)
    return scores, z_x, z_v


def hybrid_scores_from_v(x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int):
    """(scores [T,H], z_x [T], z_v [T,H]) from the value projection v = x W_V^T
    [T, n_kv, dh] instead of W_V: landmark_tokens_ker.py:45-61 with its GEMM's output
    given (the module's pre-RoPE v). Norms in v's dtype, as the reference's."""
    x_norm = x.norm(dim=-1).float()
    z_x = (x_norm - x_norm.mean()) / x_norm.std().clamp(min=1e-6)
    n_kv = v.shape[1]
    xwv = v.norm(dim=-1).float()
    z_v = (xwv - xwv.mean(0, keepdim=True)) / xwv.std(0, keepdim=True).clamp(min=1e-6)
    if n_kv != n_heads:
        z_v = z_v.repeat_interleave(n_heads // n_kv, dim=1)
    scores = alpha * z_v + (1.0 - alpha) * z_x.unsqueeze(1)
    return scores, z_x, z_v


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
         dtype: torch.dtype | None = None):
    """Rotary embedding of the module path (window_utils.py:73-88 as called by
    dsalt_attention.py:570-585): rows cos/sin[pos[t]] rounded to `dtype` (the module's
    cos.to(q.dtype)), the half-split rotation computed in float64, the result rounded
    once to `dtype` (as the reference's compiled function rounds its fp32 result)."""
    dtype = dtype or q.dtype
    c = cos[pos].to(dtype).double().unsqueeze(1)
    s = sin[pos].to(dtype).double().unsqueeze(1)

    def rot(x):
        h = x.shape[-1] // 2
        return torch.cat([-x[..., h:], x[..., :h]], dim=-1)

    qd, kd = q.double(), k.double()
    return (qd * c + rot(qd) * s).to(dtype), (kd * c + rot(kd) * s).to(dtype)


def seq_positions(cu: list[int]) -> torch.Tensor:
    """Offset of every packed token inside its sequence."""
    return torch.cat([torch.arange(cu[i + 1] - cu[i]) for i in range(len(cu) - 1)])


def window_continuous(win_logits: torch.Tensor, n_min: int, n_max: int) -> torch.Tensor:
    """w~ = n_min + sigmoid(logit) * (n_max - n_min); dsalt_attention.py:270-275."""
    return n_min + torch.sigmoid(win_logits) * (n_max - n_min)


def quantize_windows(w_cont: np.ndarray | torch.Tensor) -> np.ndarray:
    """w = max(1, floor(w~)) in fp32, NaN kept (torch clamp semantics)."""
    w = np.asarray(w_cont.detach().cpu().numpy() if torch.is_tensor(w_cont) else w_cont, dtype=np.float32)
    out = np.maximum(np.floor(w), np.float32(1.0))
    out[np.isnan(w)] = np.nan
    return out.astype(np.float32)


def _rank_order(vals: np.ndarray) -> np.ndarray:
    """Indices of `vals` from the best to the worst pick: NaN first, then descending
    value (-0 == +0), ties broken by the lower index."""
    idx = np.arange(vals.shape[0])
    isnan = np.isnan(vals)
    v = np.where(isnan, 0.0, vals).astype(np.float64)
    # lexsort: last key is primary
    return np.lexsort((idx, -v, ~isnan))


def select_landmarks(scores: np.ndarray, w: np.ndarray, cu: np.ndarray, k: int) -> np.ndarray:
    """Landmark positions [H, S, k] int64 of selectors.py:105-134 with the build's
    deterministic slot order: selected finite positions ascending, then -1.

    Token j at offset o is covered when o < trunc(w_j) (its score becomes -inf); each
    (head, sequence) takes the top min(k, L) scores (NaN > +inf > finite, lower index
    first on ties); non-finite picks (NaN, +/-inf) become -1.
    """
    scores = np.asarray(scores, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    cu = np.asarray(cu, dtype=np.int64)
    T, H = scores.shape
    S = cu.shape[0] - 1
    out = np.full((H, S, k), -1, dtype=np.int64)
    for s in range(S):
        a, b = int(cu[s]), int(cu[s + 1])
        L = b - a
        if L <= 0 or k == 0:
            continue
        off = np.arange(L)
        with np.errstate(invalid="ignore"):
            covered = (off + 1).astype(np.float32) <= w[a:b]  # off < trunc(w)
        k_eff = min(k, L)
        for h in range(H):
            vals = scores[a:b, h].copy()
            vals[covered] = -np.inf
            order = _rank_order(vals)[:k_eff]
            picked = order[np.isfinite(vals[order])]
            picked.sort()
            out[h, s, :picked.shape[0]] = picked
    return out


def _covered(o: int, wv: float) -> bool:
    """Token at offset o is covered when o < trunc(w); NaN covers nothing, +inf all."""
    if math.isnan(wv):
        return False
    if math.isinf(wv):
        return wv > 0
    return o < math.trunc(wv)


def select_landmarks_bruteforce(scores, w, cu, k):
    """Pure-Python version of select_landmarks (one full sort per (head, sequence) by an
    explicit comparison key), used to pin the vectorised one on small inputs."""
    scores = np.asarray(scores, dtype=np.float32)
    w = [float(v) for v in np.asarray(w, dtype=np.float32)]
    cu = [int(c) for c in cu]
    H = scores.shape[1]
    S = len(cu) - 1
    res = np.full((H, S, k), -1, dtype=np.int64)
    for s in range(S):
        a, b = cu[s], cu[s + 1]
        L = b - a
        for h in range(H):
            cand = []
            for o in range(L):
                v = -math.inf if _covered(o, w[a + o]) else float(scores[a + o, h])
                cand.append((0, 0.0, o, v) if math.isnan(v) else (1, -v, o, v))
            cand.sort()
            picked = sorted(o for _, _, o, v in cand[:min(k, L)] if math.isfinite(v))
            res[h, s, :len(picked)] = picked
    return res


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------


def _seq_attention(qs, ks, vs, band_bias, band_ok, lk, lv, lmk_logit_bias, lmk_ok, scale):
    """Softmax over [band keys | landmark slots] for one sequence, all heads.

    qs [H,R,D] (R query rows), ks/vs [H,L,D]; band_bias [R,L] or scalar; band_ok [R,L]
    bool; lk/lv [H,k,D]; lmk_logit_bias [H,1,k]; lmk_ok [H,R,k] bool.
    Returns (O [H,R,D], LSE [H,R])."""
    logits_b = torch.matmul(qs, ks.transpose(-1, -2)) * scale + band_bias
    logits_b = logits_b.masked_fill(~band_ok, float("-inf"))
    parts = [logits_b]
    if lk is not None:
        logits_l = torch.matmul(qs, lk.transpose(-1, -2)) * scale + lmk_logit_bias
        logits_l = logits_l.masked_fill(~lmk_ok, float("-inf"))
        parts.append(logits_l)
    logits = torch.cat(parts, dim=-1)
    lse = torch.logsumexp(logits, dim=-1)
    nonempty = torch.isfinite(lse)
    lse_safe = torch.where(nonempty, lse, torch.zeros_like(lse))
    p = torch.exp(logits - lse_safe.unsqueeze(-1))
    L = ks.shape[1]
    o = torch.matmul(p[..., :L], vs)
    if lk is not None:
        o = o + torch.matmul(p[..., L:], lv)
    return o, lse


def _gather_landmarks(ks, vs, pos_hk, L):
    valid = (pos_hk >= 0) & (pos_hk < L)
    pc = pos_hk.clamp(0, max(L - 1, 0))
    idx = pc.unsqueeze(-1).expand(-1, -1, ks.shape[-1])
    lk = torch.gather(ks, 1, idx)
    lv = torch.gather(vs, 1, idx)
    return lk, lv, valid


def attention_hard(q, k, v, w, lmk_pos, lmk_bias, cu, scale=None, rows=None):
    """HARD sparse attention (dsalt_triton_attn.py:69-169).

    q/k/v [T,H,D] (any float dtype; computed in their dtype, use fp64 for the oracle);
    w [T] window sizes, w(i) = max(1, trunc(w)); lmk_pos [H,S,k] int; lmk_bias [H,S,k]
    or None. Band: j in [i-w+1, i]; landmark slot p: 0 <= p <= i - w, logit bias
    lmk_bias. Returns (O [T,H,D], LSE [T,H]) with O = 0, LSE = -inf on empty rows.
    Differentiable in q, k, v and lmk_bias. ``rows=(r0, r1)`` restricts every sequence
    to its query offsets [r0, r1) (the outputs then hold only those rows).
    """
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    cu = [int(c) for c in (cu.tolist() if torch.is_tensor(cu) else cu)]
    S = len(cu) - 1
    kl = 0 if lmk_pos is None else lmk_pos.shape[-1]
    w_np = np.asarray(w.detach().cpu().numpy() if torch.is_tensor(w) else w, dtype=np.float32)
    outs, lses = [], []
    for s in range(S):
        a, b = cu[s], cu[s + 1]
        L = b - a
        if L == 0:
            continue
        r0, r1 = (0, L) if rows is None else (min(rows[0], L), min(rows[1], L))
        if r1 <= r0:
            continue
        qs = q[a + r0:a + r1].transpose(0, 1)
        ks, vs = (t[a:b].transpose(0, 1) for t in (k, v))
        ws = w_np[a + r0:a + r1]
        with np.errstate(invalid="ignore"):
            wi = np.where(ws >= 1, np.trunc(np.minimum(ws, 2 ** 30)), 1).astype(np.int64)
        wi_t = torch.from_numpy(wi)
        i = torch.arange(r0, r1)
        j = torch.arange(L)
        lo = i - wi_t + 1
        band_ok = (j[None, :] <= i[:, None]) & (j[None, :] >= lo[:, None])
        lk = lv = lb = lmk_ok = None
        if kl > 0:
            pos = lmk_pos[:, s, :].to(torch.long).cpu()
            lk, lv, valid = _gather_landmarks(ks, vs, pos, L)
            lmk_ok = valid[:, None, :] & (pos[:, None, :] < lo[None, :, None])
            lb = (lmk_bias[:, s, :].unsqueeze(1).to(q.dtype) if lmk_bias is not None
                  else torch.zeros((H, 1, kl), dtype=q.dtype))
        o, lse = _seq_attention(qs, ks, vs, 0.0, band_ok, lk, lv, lb, lmk_ok, scale)
        outs.append(o.transpose(0, 1))
        lses.append(lse.transpose(0, 1))
    if not outs:
        return q.new_zeros((0, H, D)), q.new_zeros((0, H))
    return torch.cat(outs, 0), torch.cat(lses, 0)


def attention_soft(q, k, v, w_cont, lmk_pos, lmk_logw, cu, tau_win=1.0, win_edge=4.0, scale=None,
                   rows=None):
    """SOFT sparse attention (dsalt_triton_train.py:116-214).

    Band 0 <= d = i - j <= w~(i) (fp32 compare), bias 0 when d <= w~ - win_edge (fp32
    difference) else log sigmoid((w~ - d)/tau_win); landmark p admitted when p <= i and
    (float)p < (float)i - w~(i), bias lmk_logw. Differentiable in q, k, v, lmk_logw and
    w_cont (through the edge bias only; the set membership is a step function).
    ``rows=(r0, r1)`` restricts every sequence to its query offsets [r0, r1).
    """
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    cu = [int(c) for c in (cu.tolist() if torch.is_tensor(cu) else cu)]
    S = len(cu) - 1
    kl = 0 if lmk_pos is None else lmk_pos.shape[-1]
    w32_all = w_cont.detach().to(torch.float32).cpu()
    outs, lses = [], []
    for s in range(S):
        a, b = cu[s], cu[s + 1]
        L = b - a
        if L == 0:
            continue
        r0, r1 = (0, L) if rows is None else (min(rows[0], L), min(rows[1], L))
        if r1 <= r0:
            continue
        qs = q[a + r0:a + r1].transpose(0, 1)
        ks, vs = (t[a:b].transpose(0, 1) for t in (k, v))
        w32 = w32_all[a + r0:a + r1]
        w_hi = w_cont[a + r0:a + r1].to(q.dtype)
        i = torch.arange(r0, r1)
        j = torch.arange(L)
        d32 = (i[:, None] - j[None, :]).to(torch.float32)
        band_ok = (j[None, :] <= i[:, None]) & (d32 <= w32[:, None])
        core = d32 <= (w32 - torch.tensor(win_edge, dtype=torch.float32))[:, None]
        z = (w_hi[:, None] - d32.to(q.dtype)) / tau_win
        edge = F.logsigmoid(z)
        band_bias = torch.where(core, torch.zeros_like(edge), edge)
        band_bias = torch.where(band_ok, band_bias, torch.zeros_like(band_bias))
        lk = lv = lb = lmk_ok = None
        if kl > 0:
            pos = lmk_pos[:, s, :].to(torch.long).cpu()
            lk, lv, valid = _gather_landmarks(ks, vs, pos, L)
            thr = i.to(torch.float32) - w32  # (float)i - w~
            lmk_ok = (valid[:, None, :] & (pos[:, None, :] <= i[None, :, None])
                      & (pos.to(torch.float32)[:, None, :] < thr[None, :, None]))
            lw = lmk_logw[:, s, :].to(q.dtype)
            lb = torch.where(torch.isfinite(lw), lw, torch.zeros_like(lw)).unsqueeze(1)
            lmk_ok = lmk_ok & torch.isfinite(lw)[:, None, :]
        o, lse = _seq_attention(qs, ks, vs, band_bias, band_ok, lk, lv, lb, lmk_ok, scale)
        outs.append(o.transpose(0, 1))
        lses.append(lse.transpose(0, 1))
    if not outs:
        return q.new_zeros((0, H, D)), q.new_zeros((0, H))
    return torch.cat(outs, 0), torch.cat(lses, 0)


def effective_pairs(mode: str, w, lmk_pos, cu, H: int) -> int:
    """Exact number of (query, key) pairs of the sparse pattern (band + admitted
    landmark slots), summed over heads: the P of F_fwd = 4*D*P."""
    cu = [int(c) for c in (cu.tolist() if torch.is_tensor(cu) else cu)]
    w = np.asarray(w.detach().cpu().numpy() if torch.is_tensor(w) else w, dtype=np.float32)
    pos = None if lmk_pos is None else np.asarray(lmk_pos.detach().cpu().numpy() if torch.is_tensor(lmk_pos) else lmk_pos)
    total = 0
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        L = b - a
        if L == 0:
            continue
        i = np.arange(L)
        ws = w[a:b]
        if mode == "hard":
            with np.errstate(invalid="ignore"):
                wi = np.where(ws >= 1, np.trunc(np.minimum(ws, 2 ** 30)), 1).astype(np.int64)
            band = np.minimum(wi, i + 1)
            pmax = i - wi  # admissible p <= pmax
        else:
            with np.errstate(invalid="ignore"):
                fw = np.where(ws >= 0, np.floor(np.minimum(ws, 2 ** 30)), -1).astype(np.int64)
            band = np.clip(np.minimum(fw + 1, i + 1), 0, None)
            t = i.astype(np.float32) - ws
            with np.errstate(invalid="ignore"):
                pmax = np.where(np.isnan(t), -1, np.minimum(i, np.ceil(t).astype(np.int64) - 1))
        total += int(band.sum()) * H
        if pos is not None and pos.shape[-1] > 0:
            for h in range(H):
                p = pos[h, s]
                p = p[(p >= 0) & (p < L)]
                if p.size:
                    total += int((p[None, :] <= pmax[:, None]).sum())
    return total


# ---------------------------------------------------------------------------------------
# CPU baseline: the reference's dense masked-SDPA fallback, restated
# ---------------------------------------------------------------------------------------


def hard_mask(L: int, w: np.ndarray, pos_hk: np.ndarray) -> torch.Tensor:
    """[H, L, L] boolean HARD mask of one sequence: band [i-w+1, i] plus landmark
    columns p <= i - w (the set of dsalt_triton_attn.py:100-135)."""
    i = torch.arange(L)
    with np.errstate(invalid="ignore"):
        wi = torch.from_numpy(np.where(w >= 1, np.trunc(np.minimum(w, 2 ** 30)), 1).astype(np.int64))
    lo = i - wi + 1
    band = (i[None, :] <= i[:, None]) & (i[None, :] >= lo[:, None])
    H = pos_hk.shape[0]
    col = torch.zeros((H, L + 1), dtype=torch.bool)
    p = torch.from_numpy(np.where((pos_hk >= 0) & (pos_hk < L), pos_hk, L).astype(np.int64))
    col.scatter_(1, p, True)
    lmk = col[:, None, :L] & (i[None, None, :] < lo[None, :, None])
    return band.unsqueeze(0) | lmk


def cpu_baseline_hard(q32, k32, v32, w, lmk_pos, cu, seqs=None):
    """Dense masked SDPA in fp32 on the CPU for the listed sequences (default: all):
    per sequence, build the [H,L,L] HARD mask as an additive -inf mask and run
    F.scaled_dot_product_attention - the cost model of the reference's CPU path.
    Returns the list of per-sequence outputs [L,H,D]."""
    cu = [int(c) for c in cu]
    w = np.asarray(w, dtype=np.float32)
    pos = np.asarray(lmk_pos)
    outs = []
    for s in (range(len(cu) - 1) if seqs is None else seqs):
        a, b = cu[s], cu[s + 1]
        L = b - a
        mask = hard_mask(L, w[a:b], pos[:, s, :])
        additive = torch.zeros(mask.shape, dtype=torch.float32).masked_fill_(~mask, float("-inf"))
        qs, ks, vs = (t[a:b].transpose(0, 1).unsqueeze(0) for t in (q32, k32, v32))
        o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=additive.unsqueeze(0))
        outs.append(o.squeeze(0).transpose(0, 1))
    return outs


# ---------------------------------------------------------------------------------------
# module composition (training, packed): dsalt/modules/dsalt_attention.py:565-608 with
# _train_selectors (:457-487) and the dense SOFT attention of _packed_train (:489-563)
# ---------------------------------------------------------------------------------------


def rope_cache(seq_len: int, head_dim: int, base: float = 10000.0, scale: float = 1.0, dtype=torch.float64):
    """(cos, sin) [seq_len, head_dim]: half-split RoPE, positions divided by `scale`
    (dsalt/kernels/window_utils.py:91-107)."""
    theta = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(seq_len, dtype=torch.float32) / scale
    emb = torch.cat([torch.outer(pos, theta)] * 2, dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return x * cos + torch.cat([-x[..., half:], x[..., :half]], dim=-1) * sin


def module_train_forward(params: dict, cfg: dict, x: torch.Tensor, cu, tau_win=1.0, tau_lmk=2.0,
                         win_edge=4.0):
    """Packed training forward of DSALTAttention from its parameters (names as in
    named_parameters()). Differentiable in x and the parameters (leaf tensors in
    `params`). Returns (out [T, d_model], selectors (w_cont, lmk_pos, lmk_logw))."""
    cu = [int(c) for c in cu]
    T, d_model = x.shape
    H = cfg["n_heads"]
    D = d_model // H
    n_kv = cfg.get("n_kv_heads") or H

    def lin(name, inp):
        y = inp @ params[name + ".weight"].T
        b = params.get(name + ".bias")
        return y if b is None else y + b

    q = lin("q_proj", x).view(T, H, D)
    k = lin("k_proj", x).view(T, n_kv, D)
    v = lin("v_proj", x).view(T, n_kv, D)
    cos, sin = rope_cache(cfg["max_seq_len"], D, cfg.get("rope_base", 10000.0), cfg.get("yarn_scale", 1.0),
                          dtype=x.dtype)
    pos_ids = torch.cat([torch.arange(cu[s + 1] - cu[s]) for s in range(len(cu) - 1)])
    c, s_ = cos[pos_ids].unsqueeze(1), sin[pos_ids].unsqueeze(1)
    q, k = rotate(q, c, s_), rotate(k, c, s_)
    if n_kv != H:
        rep = H // n_kv
        k = k.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)
        v = v.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)

    w_cont = cfg["n_min"] + torch.sigmoid(lin("win_gate", x).squeeze(-1)) * (cfg["n_max"] - cfg["n_min"])
    alpha = torch.sigmoid(params["alpha_w"])
    with torch.no_grad():
        w_disc = quantize_windows(w_cont.detach().float())
        s32, _, _ = hybrid_scores(x.detach().float(), params["v_proj.weight"].detach().float(),
                                  alpha.detach().float(), H, D)
        lmk_pos = torch.from_numpy(select_landmarks(s32.numpy(), w_disc, np.array(cu), cfg["k_lmk"]))
    scores, _, _ = hybrid_scores(x, params["v_proj.weight"], alpha, H, D)
    starts = torch.tensor(cu[:-1])
    abs_pos = starts[None, :, None] + lmk_pos.clamp(min=0)
    s_sel = scores[abs_pos, torch.arange(H)[:, None, None]]
    lmk_logw = torch.log(torch.sigmoid(s_sel / tau_lmk).clamp(min=1e-20))
    lmk_logw = torch.where(lmk_pos >= 0, lmk_logw, torch.full_like(lmk_logw, float("-inf")))
    o, _ = attention_soft(q, k, v, w_cont, lmk_pos, lmk_logw, cu, tau_win=tau_win, win_edge=win_edge)
    out = o.reshape(T, d_model) @ params["out_proj.weight"].T
    return out, (w_cont, lmk_pos, lmk_logw)


def module_eval_forward(params: dict, cfg: dict, x: torch.Tensor, cu):
    """Packed inference forward of DSALTAttention (dsalt_attention.py:610-625): floor-
    quantised windows, landmark top-k on fp32 scores, HARD attention with zero landmark
    bias, out_proj. Returns (out, (w_sizes, lmk_pos))."""
    cu = [int(c) for c in cu]
    T, d_model = x.shape
    H = cfg["n_heads"]
    D = d_model // H
    n_kv = cfg.get("n_kv_heads") or H

    def lin(name, inp):
        y = inp @ params[name + ".weight"].T
        b = params.get(name + ".bias")
        return y if b is None else y + b

    q = lin("q_proj", x).view(T, H, D)
    k = lin("k_proj", x).view(T, n_kv, D)
    v = lin("v_proj", x).view(T, n_kv, D)
    cos, sin = rope_cache(cfg["max_seq_len"], D, cfg.get("rope_base", 10000.0), cfg.get("yarn_scale", 1.0),
                          dtype=x.dtype)
    pos_ids = torch.cat([torch.arange(cu[s + 1] - cu[s]) for s in range(len(cu) - 1)])
    c, s_ = cos[pos_ids].unsqueeze(1), sin[pos_ids].unsqueeze(1)
    q, k = rotate(q, c, s_), rotate(k, c, s_)
    if n_kv != H:
        rep = H // n_kv
        k = k.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)
        v = v.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)
    w_cont = cfg["n_min"] + torch.sigmoid(lin("win_gate", x).squeeze(-1)) * (cfg["n_max"] - cfg["n_min"])
    w_sizes = quantize_windows(w_cont.detach().float())
    alpha = torch.sigmoid(params["alpha_w"]).detach().float()
    s32, _, _ = hybrid_scores(x.detach().float(), params["v_proj.weight"].detach().float(), alpha, H, D)
    lmk_pos = torch.from_numpy(select_landmarks(s32.numpy(), w_sizes, np.array(cu), cfg["k_lmk"]))
    o, _ = attention_hard(q, k, v, w_sizes, lmk_pos, None, cu)
    return o.reshape(T, d_model) @ params["out_proj.weight"].T, (w_sizes, lmk_pos)


# ---------------------------------------------------------------------------------------
# dense batched variant: dsalt/modules/dsalt_attention.py:286-329 (log-biases), :371-401
# (_batched), :403-438 (_diff_logbias)
# ---------------------------------------------------------------------------------------


def dense_logbias(w_cont: torch.Tensor, lmk_bias_dense: torch.Tensor, T: int, tau_win: float = 1.0,
                  win_edge: float = 4.0) -> torch.Tensor:
    """The union log-bias [H, T, T] of the dense variant (natural-log units).

    Window (dsalt_attention.py:286-312): d = i - j; 0 in the core d <= w~_i - win_edge
    (fp32 compare), log(max(sigmoid((w~_i - d) / tau), 1e-20)) elsewhere for d >= 0, -inf
    for d < 0. Landmarks (:314-329, validity :420-433): lmk_bias_dense[h, j] (-inf for
    keys that are not landmarks of head h) where d >= 0 and d >= max(1, floor(w~_i)).
    Union (:389): the elementwise maximum (torch.maximum: ties split the gradient).
    Differentiable in w_cont (through the soft tail) and lmk_bias_dense."""
    idx = torch.arange(T)
    d = (idx.unsqueeze(1) - idx.unsqueeze(0)).to(torch.float32)            # [T, T] = i - j
    w32 = w_cont.detach().to(torch.float32).unsqueeze(1)
    core = d <= (w32 - torch.tensor(win_edge, dtype=torch.float32))
    w_i = w_cont.unsqueeze(1)
    g = torch.sigmoid((w_i - d.to(w_cont.dtype)) / tau_win)
    logb = torch.log(g.clamp(min=1e-20))
    logb = torch.where(core, torch.zeros_like(logb), logb)
    logb = logb.masked_fill(d < 0, float("-inf"))
    w_disc = torch.floor(w32).clamp(min=1)
    valid = (d >= 0) & (d >= w_disc)                                         # [T, T]
    lmk = lmk_bias_dense.unsqueeze(1).expand(-1, T, T)                       # [H, T(i), T(j)]
    lmk = torch.where(valid.unsqueeze(0), lmk, torch.full_like(lmk, float("-inf")))
    return torch.maximum(logb.unsqueeze(0), lmk)


def attention_dense(q, k, v, w_cont, lmk_bias_dense, tau_win=1.0, win_edge=4.0, scale=None):
    """Dense batched DSALT attention of one sequence (dsalt_attention.py:371-401):
    softmax over every causal key of q.k * scale + the union log-bias. q/k/v [T, H, D],
    w_cont [T], lmk_bias_dense [H, T]. Returns (O [T, H, D], LSE [T, H])."""
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    bias = dense_logbias(w_cont, lmk_bias_dense, T, tau_win, win_edge).to(q.dtype)
    logits = torch.matmul(q.transpose(0, 1), k.transpose(0, 1).transpose(-1, -2)) * scale + bias
    lse = torch.logsumexp(logits, dim=-1)                                      # [H, T]
    p = torch.exp(logits - lse.unsqueeze(-1))
    o = torch.matmul(p, v.transpose(0, 1))                                     # [H, T, D]
    return o.transpose(0, 1), lse.transpose(0, 1)


def dense_landmark_bias(scores: torch.Tensor, k_lmk: int, tau_lmk: float = 2.0) -> torch.Tensor:
    """lmk_bias_dense [H, T]: log(clamp(sigmoid(s / tau_lmk), 1e-20)) at the top-min(k, T)
    keys of each head over all T tokens (no covered exclusion; the selection is made on
    the detached fp32 scores), -inf elsewhere (dsalt_attention.py:318-329, :421-431)."""
    T, H = scores.shape
    sel = torch.zeros(H, T, dtype=torch.bool)
    k_act = min(k_lmk, T)
    if k_act > 0:
        s32 = scores.detach().to(torch.float32).numpy()
        w0 = np.zeros(T, dtype=np.float32)                                     # nothing covered
        pos = select_landmarks(s32, w0, np.array([0, T]), k_act)              # [H, 1, k]
        for h in range(H):
            p = pos[h, 0]
            sel[h, p[p >= 0]] = True
    w_lmk = torch.log(torch.sigmoid(scores / tau_lmk).clamp(min=1e-20)).transpose(0, 1)
    return torch.where(sel, w_lmk, torch.full_like(w_lmk, float("-inf")))


def module_batched_forward(params: dict, cfg: dict, x: torch.Tensor, tau_win=1.0, tau_lmk=2.0,
                           win_edge=4.0):
    """DSALTAttention.forward(x) without cu_seqlens for x [1, T, d_model]
    (dsalt_attention.py:371-401): q/k/v projections, RoPE at positions 0..T-1, GQA
    repeat, continuous windows, hybrid scores on x (GEMM route), the dense union
    log-bias, softmax, out_proj. Differentiable in x and the parameters. Returns
    (out [1, T, d_model], (w_cont, lmk_bias_dense))."""
    xs = x[0]
    T, d_model = xs.shape
    H = cfg["n_heads"]
    D = d_model // H
    n_kv = cfg.get("n_kv_heads") or H

    def lin(name, inp):
        y = inp @ params[name + ".weight"].T
        b = params.get(name + ".bias")
        return y if b is None else y + b

    q = lin("q_proj", xs).view(T, H, D)
    k = lin("k_proj", xs).view(T, n_kv, D)
    v = lin("v_proj", xs).view(T, n_kv, D)
    cos, sin = rope_cache(cfg["max_seq_len"], D, cfg.get("rope_base", 10000.0), cfg.get("yarn_scale", 1.0),
                          dtype=xs.dtype)
    c, s_ = cos[:T].unsqueeze(1), sin[:T].unsqueeze(1)
    q, k = rotate(q, c, s_), rotate(k, c, s_)
    if n_kv != H:
        rep = H // n_kv
        k = k.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)
        v = v.unsqueeze(2).expand(T, n_kv, rep, D).reshape(T, H, D)
    w_cont = cfg["n_min"] + torch.sigmoid(lin("win_gate", xs).squeeze(-1)) * (cfg["n_max"] - cfg["n_min"])
    alpha = torch.sigmoid(params["alpha_w"])
    scores, _, _ = hybrid_scores(xs, params["v_proj.weight"], alpha, H, D)
    with torch.no_grad():
        s_sel, _, _ = hybrid_scores(xs.detach().float(), params["v_proj.weight"].detach().float(),
                                    alpha.detach().float(), H, D)
    lb = dense_landmark_bias(scores, cfg["k_lmk"], tau_lmk)
    # the selection itself is made on the detached fp32 scores
    sel = dense_landmark_bias(s_sel, cfg["k_lmk"], tau_lmk) > float("-inf")
    lb = torch.where(sel, lb, torch.full_like(lb, float("-inf")))
    o, _ = attention_dense(q, k, v, w_cont, lb, tau_win, win_edge)
    out = o.reshape(T, d_model) @ params["out_proj.weight"].T
    return out.unsqueeze(0), (w_cont, lb)


# ---------------------------------------------------------------------------------------
# the LM consumer: dsalt/model/dsalt_lm.py:237-280, dsalt/modules/dsalt_transformer.py:
# 76-86, dsalt/kernels/RMSENorm.py:20-22
# ---------------------------------------------------------------------------------------

def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * weight over the last dimension (F.rms_norm)."""
    return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps) * weight


def _lm_trunk(params: dict, cfg: dict, input_ids: torch.Tensor, attend) -> torch.Tensor:
    """Embedding, the pre-norm blocks (attend(sub_params, h) is the attention module's
    output) and the final RMSNorm (dsalt_lm.py:254-272, dsalt_transformer.py:80-85)."""
    x = params["embed_tokens.weight"][input_ids]
    for li in range(cfg["n_layers"]):
        pre = f"layers.{li}."
        sub = {k[len(pre) + 5:]: v for k, v in params.items() if k.startswith(pre + "attn.")}
        x = x + attend(sub, rms_norm(x, params[pre + "attn_norm.weight"]))
        h = rms_norm(x, params[pre + "ffn_norm.weight"])
        g = h @ params[pre + "ffn.gate_proj.weight"].T
        u = h @ params[pre + "ffn.up_proj.weight"].T
        x = x + (F.silu(g) * u) @ params[pre + "ffn.down_proj.weight"].T
    return rms_norm(x, params["final_norm.weight"])


def lm_forward(params: dict, cfg: dict, input_ids: torch.Tensor, cu=None) -> torch.Tensor:
    """Logits of DSALTLMHeadModel in eval mode (tied head): packed ``input_ids [T]`` with
    ``cu`` (each attention is module_eval_forward: HARD set, zero landmark bias), or
    ``[1, T]`` without (each attention is module_batched_forward: the dense variant).
    ``params`` holds the model's state dict in the working dtype."""
    if cu is not None:
        x = _lm_trunk(params, cfg, input_ids, lambda sub, h: module_eval_forward(sub, cfg, h, cu)[0])
    else:
        x = _lm_trunk(params, cfg, input_ids, lambda sub, h: module_batched_forward(sub, cfg, h)[0])
    return x @ params["embed_tokens.weight"].T


def lm_train_loss(params: dict, cfg: dict, input_ids: torch.Tensor, cu, labels: torch.Tensor) -> torch.Tensor:
    """Training loss of DSALTLMHeadModel on packed input (tied head): each attention is
    module_train_forward (SOFT), then the mean token cross-entropy over labels other
    than -100 (dsalt_lm.py:19-39, :187-197). Differentiable in the parameters."""
    x = _lm_trunk(params, cfg, input_ids, lambda sub, h: module_train_forward(sub, cfg, h, cu)[0])
    logits = x @ params["embed_tokens.weight"].T
    return F.cross_entropy(logits, labels.long(), ignore_index=-100, reduction="sum") / (labels != -100).sum()

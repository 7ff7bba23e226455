"""Benchmark of the DSALT sparse-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c1|c4]

A step is one HARD DSALT attention forward (the fused HIP kernel) over the packed batch
of BASELINE.json config 2 (default): 4 x 2048 tokens, 16 heads x 64 head_dim,
n_min 32, n_max 512, k_lmk 64, with q/k/v, windows and landmarks produced by a
DSALTAttention module at random init (seed 1) from x ~ N(0, 1) [4, 2048, 1024].
Inputs are resident in HBM before the timed region. Prints one JSON line.

`mfma.achieved` counts only the FLOPs the sparse pattern needs: 4 * D * P, where P is
the exact number of (query, key) pairs (band + admitted landmarks) counted on the host
from the actual windows and landmarks. `roofline` is the HBM roofline of the launch:
algorithmic bytes (Q, K, V read and O written once in bf16, LSE, windows, landmark
positions) per launch over the measured launch time; `traffic` is the HBM bytes per
launch measured with rocprofv3 counters (recorded under profiles/). `cpu_baseline` times the reference's CPU
fallback cost model (dense mask + fp32 SDPA, restated in oracle/) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dsalt-library_amd"))

MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E

CONFIGS = {
    # name: (batch, seq_len, d_model, heads, n_min, n_max, k_lmk, seed)
    "c1": (1, 1024, 512, 8, 64, 256, 16, 0),
    "c2": (4, 2048, 1024, 16, 32, 512, 64, 1),
    "c4": (1, 16384, 2048, 16, 64, 1024, 128, 3),
}


def effective_pairs_hard(w: np.ndarray, lmk_pos: np.ndarray, cu: list[int]) -> int:
    """Exact (query, key) pairs of the HARD pattern summed over heads: per query
    min(w, i + 1) band keys plus the landmark slots p with 0 <= p <= i - w."""
    H = lmk_pos.shape[0]
    total = 0
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        L = b - a
        if L == 0:
            continue
        i = np.arange(L)
        ws = w[a:b]
        wi = np.where(ws >= 1, np.trunc(np.minimum(np.nan_to_num(ws, nan=1.0), 2 ** 30)), 1).astype(np.int64)
        total += int(np.minimum(wi, i + 1).sum()) * H
        pmax = np.sort(i - wi)  # landmark p admitted by query i iff p <= i - w(i)
        for h in range(H):
            p = lmk_pos[h, s]
            p = p[(p >= 0) & (p < L)]
            # number of queries admitting each p = #{i : i - w(i) >= p}
            total += int((L - np.searchsorted(pmax, p, side="left")).sum())
    return total


def make_workload(cfg: str, device: torch.device):
    from dsalt import _hip
    from dsalt.modules import DSALTAttention
    from dsalt.kernels.window_utils import apply_rotary_emb

    B, L, d_model, H, n_min, n_max, k_lmk, seed = CONFIGS[cfg]
    torch.manual_seed(seed)
    mod = DSALTAttention(d_model, H, n_min, n_max, k_lmk, max_seq_len=L)
    x = torch.randn(B, L, d_model)
    mod = mod.to(device).eval()
    T = B * L
    xp = x.reshape(T, d_model).to(device)
    cu = torch.arange(0, T + 1, L, dtype=torch.int32, device=device)
    with torch.no_grad():
        D = d_model // H
        q = mod.q_proj(xp).view(T, H, D)
        k = mod.k_proj(xp).view(T, H, D)
        v = mod.v_proj(xp).view(T, H, D)
        pos_ids = torch.arange(T, device=device) % L
        cos, sin = mod.rope_cos[pos_ids].unsqueeze(1), mod.rope_sin[pos_ids].unsqueeze(1)
        q, k = apply_rotary_emb(q, k, cos, sin)
        q, k, v = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
        w = mod._window_sizes(xp, floor=True)
        from dsalt.kernels.selectors import _compute_landmark_indices
        lmk, _, _ = _compute_landmark_indices(xp, mod.v_proj.weight, mod._alpha().float(), w, cu, k_lmk,
                                              n_min, T, cu.tolist(), head_dim=D)
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, w=w, lmk=lmk, cu=cu, T=T, H=H, D=D, B=B, L=L, k_lmk=k_lmk,
                n_min=n_min, n_max=n_max, xp=xp, mod=mod)


def effective_pairs_soft(w_cont: np.ndarray, lmk_pos: np.ndarray, cu: list[int]) -> int:
    """Exact (query, key) pairs of the SOFT pattern summed over heads: per query
    min(floor(w~), i) + 1 band keys (none when w~ < 0) plus the landmark slots p with
    p <= i and p < i - w~ (fp32 compare)."""
    H = lmk_pos.shape[0]
    total = 0
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        L = b - a
        if L == 0:
            continue
        i = np.arange(L)
        ws = w_cont[a:b].astype(np.float32)
        with np.errstate(invalid="ignore"):
            band = np.where(ws >= 0, np.minimum(np.floor(np.minimum(ws, 2.0 ** 30)), i) + 1, 0)
        total += int(band.sum()) * H
        thr = (i.astype(np.float32) - ws)  # p admitted iff p < thr (and p <= i)
        for h in range(H):
            p = lmk_pos[h, s]
            p = np.sort(p[(p >= 0) & (p < L)]).astype(np.float32)
            if p.size == 0:
                continue
            cnt = np.searchsorted(p, np.where(np.isnan(thr), -np.inf, thr), side="left")  # p < thr
            cnt = np.minimum(cnt, np.searchsorted(p, i.astype(np.float32), side="right"))  # p <= i
            total += int(cnt.sum())
    return total


def make_train_workload(device: torch.device):
    """eight sequences with lengths numpy.random.seed(2);
    randint(256, 2049, 8) packed into one stream (T = 9290), DSALTAttention(1024, 16, 32,
    512, 64) at random init (seed 2), x ~ N(0, 1), dO ~ N(0, 1); the SOFT (training)
    selection and attention inputs the module produces."""
    from dsalt.modules import DSALTAttention
    from dsalt.kernels.window_utils import apply_rotary_emb

    np.random.seed(2)
    lens = [int(x) for x in np.random.randint(256, 2049, 8)]
    d_model, H, n_min, n_max, k_lmk = 1024, 16, 32, 512, 64
    torch.manual_seed(2)
    mod = DSALTAttention(d_model, H, n_min, n_max, k_lmk, max_seq_len=2048).to(device).train()
    T = sum(lens)
    x = torch.randn(T, d_model).to(device)
    cu_list = [0]
    for L in lens:
        cu_list.append(cu_list[-1] + L)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=device)
    D = d_model // H
    with torch.no_grad():
        w_cont, lmk_pos, lmk_logw = mod._train_selectors(x, cu, T, device, cu_list)
        q = mod.q_proj(x).view(T, H, D)
        k = mod.k_proj(x).view(T, H, D)
        v = mod.v_proj(x).view(T, H, D)
        pos_ids = torch.cat([torch.arange(L, device=device) for L in lens])
        cos, sin = mod.rope_cos[pos_ids].unsqueeze(1), mod.rope_sin[pos_ids].unsqueeze(1)
        q, k = apply_rotary_emb(q, k, cos, sin)
        q, k, v = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
    dout = torch.randn(T, H, D, generator=torch.Generator().manual_seed(102)).to(torch.bfloat16).to(device)
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, w=w_cont.float().contiguous(), lmk=lmk_pos, logw=lmk_logw.float().contiguous(),
                cu=cu, cu_list=cu_list, T=T, H=H, D=D, lens=lens, k_lmk=k_lmk, dout=dout)


def measure_backward(device: torch.device, steps: int = 50, warmup: int = 20) -> dict:
    """SOFT forward and backward (dQ, dK, dV, d_lmk_logw, d_w~) at config 3, bf16 in and out."""
    from dsalt import _hip

    wl = make_train_workload(device)
    q, k, v, T, H, D = wl["q"], wl["k"], wl["v"], wl["T"], wl["H"], wl["D"]
    scale = 1.0 / math.sqrt(D)
    fwd = _hip.FwdLauncher(_hip.MODE_SOFT, q, k, v, wl["w"], wl["lmk"], wl["logw"], wl["cu"], scale)
    fwd_ms = time_launches(fwd, steps, warmup)
    bwd = _hip.BwdLauncher(_hip.MODE_SOFT, q, k, v, fwd.out, fwd.lse, wl["dout"], wl["w"], wl["lmk"], wl["logw"],
                           wl["cu"], scale, need_dw=True)
    bwd_ms = time_launches(bwd, steps, warmup)
    P = effective_pairs_soft(wl["w"].cpu().numpy(), wl["lmk"].cpu().numpy(), wl["cu_list"])
    t_b, t_f = bwd_ms * 1e-3, fwd_ms * 1e-3
    bytes_bwd = 2 * T * H * D * 8 + 8 * T * H  # read Q, K, V, O, dO; write dQ, dK, dV (16-bit); LSE, Delta
    bytes_fwd = 2 * T * H * D * 4 + 4 * T * H + 4 * T + 12 * H * len(wl["lens"]) * wl["k_lmk"]
    return {
        "workload": f"c3: SOFT DSALT attention forward + backward, {len(wl['lens'])} packed sequences "
                    f"(T = {T}), {H} heads x {D} head_dim, n_min 32, n_max 512, k_lmk 64, bf16",
        "pairs": P,
        "fwd_ms": fwd_ms,
        "bwd_ms": bwd_ms,
        "fwd_tflops": 4.0 * D * P / t_f / 1e12,
        "bwd_tflops": 10.0 * D * P / t_b / 1e12,
        "bwd_mfma_frac": 10.0 * D * P / t_b / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "bwd_hbm_GBs": bytes_bwd / t_b / 1e9,
        "bwd_hbm_frac": bytes_bwd / t_b / 1e9 / HBM_PEAK_GBS,
        "fwd_hbm_GBs": bytes_fwd / t_f / 1e9,
        "tokens_per_s_fwd_bwd": T / (t_f + t_b),
    }


def measure_dense(device: torch.device, steps: int = 50, warmup: int = 20) -> dict:
    """The dense batched variant (DSALT_MODE_DENSE) at config 1's shape on the GPU: module
    seed 0, x ~ N(0, 1) [1, 1024, 512], 8 heads x 64, bf16; q/k/v, w~ and the landmark
    table from the module's own projections and selector. Forward and backward launch
    times; FLOPs are the causal pairs' 4 D (forward) and 10 D (backward: S, dP, dV, dK,
    dQ) per pair."""
    from dsalt import _hip
    from dsalt.modules import DSALTAttention
    from dsalt.kernels.window_utils import apply_rotary_emb_packed

    B, L, d_model, H, n_min, n_max, k_lmk, seed = CONFIGS["c1"]
    torch.manual_seed(seed)
    mod = DSALTAttention(d_model, H, n_min, n_max, k_lmk, max_seq_len=L)
    x = torch.randn(B, L, d_model)
    mod = mod.to(device).to(torch.bfloat16)
    xs = x[0].to(device, torch.bfloat16)
    D = d_model // H
    with torch.no_grad():
        q = mod.q_proj(xs).view(L, H, D)
        k = mod.k_proj(xs).view(L, H, D)
        v = mod.v_proj(xs).view(L, H, D).contiguous()
        cu = torch.tensor([0, L], dtype=torch.int32, device=device)
        q, k = apply_rotary_emb_packed(q, k, mod.rope_cos, mod.rope_sin, cu)
        w_cont, lb, _ = mod._dense_selectors(xs, L, device, mod.v_proj(xs).view(L, H, D))
        w_cont, lb = w_cont.float(), lb.float().contiguous()
    scale = 1.0 / math.sqrt(D)
    fwd = _hip.DenseFwdLauncher(q.contiguous(), k.contiguous(), v, w_cont, lb, scale)
    fwd_ms = time_launches(fwd, steps, warmup)
    dout = torch.randn_like(q)
    bwd = _hip.DenseBwdLauncher(q.contiguous(), k.contiguous(), v, fwd.out, fwd.lse, dout, w_cont, lb, scale)
    bwd_ms = time_launches(bwd, steps, warmup)
    pairs = H * L * (L + 1) // 2
    bytes_fwd = 2 * L * H * D * 4 + 4 * L * H + 4 * L + 4 * H * L
    return {
        "workload": f"dense batched [1, {L}, {d_model}], {H} heads x {D}, module seed {seed}, bf16",
        "pairs": pairs,
        "fwd_us": fwd_ms * 1e3,
        "bwd_us": bwd_ms * 1e3,
        "fwd_mfma_frac": 4.0 * D * pairs / (fwd_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "bwd_mfma_frac": 10.0 * D * pairs / (bwd_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "fwd_hbm_frac": bytes_fwd / (fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s_fwd": L / (fwd_ms * 1e-3),
    }


def measure_lm(device: torch.device, steps: int = 5, warmup: int = 2) -> dict:
    """Config 5: DSALTLMHeadModel(32000, 1024, 24, 16, 32, 512, 64, 2048) inference forward
    in bf16 at random init (seed 4) on input_ids [8, 2048] packed to [16384] with
    cu_seqlens, _last_P off. End-to-end time per forward (logits included), timed without
    any instrumentation, and the share spent inside the attention modules (q/k/v
    projections, selection, the HIP attention kernel, out_proj) from a second set of
    forwards with CUDA events around each attention call (the 48 event records add
    ~0.5 ms per forward, so the share is taken within that set)."""
    from dsalt.model import DSALTLMHeadModel

    torch.manual_seed(4)
    with torch.device(device):  # parameters initialised on the GPU (the RoPE tables are built on the CPU)
        model = DSALTLMHeadModel(32000, 1024, 24, 16, 32, 512, 64, 2048)
    model = model.to(device, torch.bfloat16).eval()
    model.set_collect_last_P(False)
    ids = torch.randint(0, 32000, (8 * 2048,), device=device)
    cu = torch.arange(0, 8 * 2048 + 1, 2048, dtype=torch.int32, device=device)
    marks = []
    on = [False]

    def pre(_m, _a):
        if on[0]:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            marks.append([e, None])

    def post(_m, _a, _o):
        if on[0]:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            marks[-1][1] = e

    def timed() -> float:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            model(ids, cu_seqlens=cu)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    with torch.no_grad():
        for _ in range(warmup):
            model(ids, cu_seqlens=cu)
        torch.cuda.synchronize()
        ms = timed()
        hooks = []
        for layer in model.layers:
            hooks.append(layer.attn.register_forward_pre_hook(pre))
            hooks.append(layer.attn.register_forward_hook(post))
        on[0] = True
        ms_hooked = timed()
        on[0] = False
        for h in hooks:
            h.remove()
    attn_ms_hooked = sum(a.elapsed_time(b) for a, b in marks) / steps
    attn_share = attn_ms_hooked / ms_hooked
    attn_ms = attn_share * ms
    T = ids.numel()
    return {
        "workload": "c5: DSALTLMHeadModel(32000, 1024, 24 layers, 16 heads, n_min 32, n_max 512, k_lmk 64) "
                    "inference forward, bf16, 8 x 2048 packed tokens, random init seed 4",
        "ms_per_forward": ms,
        "tokens_per_s": T / (ms * 1e-3),
        "attn_module_ms": attn_ms,
        "attn_share": attn_share,
        "ms_per_forward_with_attn_events": ms_hooked,
        "steps": steps,
    }


def time_graph(fn, per_graph: int = 50, replays: int = 10) -> float:
    """Per-launch time of `fn` from a HIP graph of `per_graph` captured launches, replayed
    `replays` times: kernels shorter than the host's launch cost are timed on the GPU
    alone. `fn` must launch on the current stream and must not allocate or memset."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * per_graph)


WARMUP_MIN_S = 0.25  # the GPU clock ramps over ~10 ms of back-to-back launches


def time_launches(fn, steps: int, warmup: int) -> float:
    """Mean time per launch of `steps` launches, after `warmup` launches and then at least
    WARMUP_MIN_S seconds more of them (so the clock state does not depend on the flag)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARMUP_MIN_S:
        for _ in range(50):  # back to back: the clock ramps under sustained load
            fn()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def measure_front_end(wl, w, cu) -> dict:
    """The inference selection path in bf16 at the workload's shape: hybrid scores + top-k,
    by the reference's route (x @ W_V^T GEMM, norms and standardisation in torch,
    landmark_tokens_ker.py:45-61), by the torch ops on the module's value projection, by
    dsalt_hybrid_scores followed by the selection, and by the module's default,
    dsalt_select_hybrid. All eager, launch costs included; the HIP routes also from a HIP
    graph (GPU time alone). HBM bytes of the score kernels: x and v read once (bf16), norms
    and scores written and read back (fp32)."""
    from dsalt import _hip
    from dsalt.kernels.landmark_tokens_ker import hybrid_scores_per_head
    mod, T, H, D = wl["mod"], wl["T"], wl["H"], wl["D"]
    with torch.no_grad():
        xb = wl["xp"].to(torch.bfloat16)
        Wb = mod.v_proj.weight.to(torch.bfloat16)
        vb = (xb @ Wb.T).view(T, H, D)
        alpha = mod._alpha().float()
    k = wl["k_lmk"]

    def gemm_path():
        s, _, _ = hybrid_scores_per_head(xb, Wb, alpha, H, D)
        _hip.select_landmarks(s, w, cu, k, max_seqlen=wl["L"])

    scores = _hip.ScoresLauncher(xb, vb, alpha, H)
    sel_f = _hip.SelectLauncher(scores.scores, w, cu, k, max_seqlen=wl["L"])

    def hip_scores_path():
        scores()
        sel_f()

    from dsalt.kernels.landmark_tokens_ker import hybrid_scores_from_v

    def v_route_path():
        s, _, _ = hybrid_scores_from_v(xb, vb, alpha, H)
        _hip.select_landmarks(s, w, cu, k, max_seqlen=wl["L"])

    # the scores formed inside the selection launch (norms pass + selection: 2 launches
    # instead of 4); w is already quantised, so its quantisation is the identity
    hyb = _hip.SelectHybridLauncher(xb, vb, alpha, H, w, cu, k, max_seqlen=wl["L"], norms_f32=False)
    with torch.no_grad():
        hip_scores_path()
        hyb()
        torch.cuda.synchronize()
        if not (torch.equal(hyb.out, sel_f.out) and torch.equal(hyb.w_out, w.float())):
            raise RuntimeError("dsalt_select_hybrid differs from dsalt_hybrid_scores + dsalt_select_landmarks")
        gemm_ms = time_launches(gemm_path, 50, 10)
        v_route_ms = time_launches(v_route_path, 50, 10)
        hip_ms = time_launches(hip_scores_path, 50, 10)
        hyb_ms = time_launches(hyb, 50, 10)
        scores_graph_ms = time_graph(scores)
        two_step_graph_ms = time_graph(hip_scores_path)
        hyb_graph_ms = time_graph(hyb)
    d = xb.shape[1]
    bytes_scores = 2 * T * d + 2 * T * H * D + 4 * T * (1 + H) * 2 + 4 * T * H * 3
    return {
        "workload": "c2 inference selection (hybrid scores + top-k), bf16 x / W_V / v",
        "gemm_path_us": gemm_ms * 1e3,
        "torch_v_route_us": v_route_ms * 1e3,
        "hip_scores_path_us": hip_ms * 1e3,
        "select_hybrid_path_us": hyb_ms * 1e3,
        "hip_scores_graph_us": scores_graph_ms * 1e3,
        "hip_scores_then_select_graph_us": two_step_graph_ms * 1e3,
        "select_hybrid_graph_us": hyb_graph_ms * 1e3,
        "hip_scores_GB/s": bytes_scores / (scores_graph_ms * 1e-3) / 1e9,
        "gemm_flops_saved": 2.0 * T * d * H * D,
        "note": "gemm_path: the reference's x @ W_V^T route; torch_v_route: the same torch norms on the "
                "module's own value projection (no second GEMM, DSALTAttention._hip_scores = False); "
                "hip_scores_path: dsalt_hybrid_scores on x and v then dsalt_select_landmarks (4 launches); "
                "select_hybrid_path: the module's default, dsalt_select_hybrid (norms pass, then the selection "
                "forming each score itself: 2 launches, same sets, checked)",
    }


def measure_selection(device: torch.device) -> dict:
    """measure_front_end alone on the c2 workload (for kernel traces of the selection)."""
    wl = make_workload("c2", device)
    return measure_front_end(wl, wl["w"], wl["cu"])


def measure_host_launch(device: torch.device, calls: int = 4000) -> dict:
    """Host cost of one forward launch through the C ABI (argument block prebuilt, as the
    module's launcher reuses it): wall time of `calls` back-to-back launches of a forward
    so small (64 tokens, 16 heads) that the GPU finishes each before the host issues the
    next, so the wall time is the host's. The same for the HIP runtime alone (an empty
    torch fill launch) for reference."""
    from dsalt import _hip
    g = torch.Generator(device="cpu").manual_seed(0)
    T, H, D = 64, 16, 64
    q, k, v = (torch.randn(T, H, D, generator=g).to(device, torch.bfloat16) for _ in range(3))
    w = torch.full((T,), 16.0, device=device)
    cu = torch.tensor([0, T], dtype=torch.int32, device=device)
    lmk = torch.full((H, 1, 8), -1, dtype=torch.int64, device=device)
    f = _hip.FwdLauncher(_hip.MODE_HARD, q, k, v, w, lmk, None, cu, 0.125)
    buf = torch.empty(1, device=device)
    res = {}
    for name, fn in (("dsalt_fwd_us", f), ("torch_fill_us", lambda: buf.fill_(1.0))):
        for _ in range(200):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        res[name] = (time.perf_counter() - t0) / calls * 1e6
    return res


def measure_peaks(device: torch.device) -> dict:
    """What the box reaches of the published peaks, for context (the roofline fractions
    use the published 2.5 PFLOP/s and 8 TB/s): a large square bf16 GEMM through torch
    (hipBLASLt, MFMA), a 2 GiB device copy (bytes read + written) and a 2 GiB bf16 sum
    (bytes read)."""
    n = 8192
    a = torch.randn(n, n, device=device, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=device, dtype=torch.bfloat16)
    gemm_ms = time_launches(lambda: torch.matmul(a, b), 20, 5)
    del a, b
    nbytes = 2 << 30
    src = torch.empty(nbytes // 2, device=device, dtype=torch.bfloat16).normal_()
    dst = torch.empty_like(src)
    copy_ms = time_launches(lambda: dst.copy_(src), 20, 5)
    sum_ms = time_launches(lambda: src.sum(dtype=torch.float32), 20, 5)
    res = {
        "gemm_bf16_TFLOP/s": 2.0 * n ** 3 / (gemm_ms * 1e-3) / 1e12,
        "copy_GB/s": 2 * nbytes / (copy_ms * 1e-3) / 1e9,
        "sum_read_GB/s": nbytes / (sum_ms * 1e-3) / 1e9,
    }
    # the probe kernels of libdsalt_peaks.so: MFMA alone, and a plain streaming read
    import ctypes
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "dsalt-library_amd", "dsalt",
                                   "libdsalt_peaks.so"))
    lib.dsalt_bench_mfma.restype = ctypes.c_float
    lib.dsalt_bench_mfma.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.dsalt_bench_read.restype = ctypes.c_float
    lib.dsalt_bench_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    torch.cuda.synchronize()
    blocks, iters = 256 * 8, 32768  # 8 waves per SIMD; ~20 ms per launch, so the clock has ramped
    mfma_ms = lib.dsalt_bench_mfma(blocks, iters)
    read_ms = lib.dsalt_bench_read(src.data_ptr(), nbytes, 256 * 16)
    if mfma_ms <= 0 or read_ms <= 0:
        raise RuntimeError("peak probes failed")
    mfma_tf = blocks * 4 * iters * 4 * (32 * 32 * 16 * 2) / (mfma_ms * 1e-3) / 1e12
    res["mfma_loop_TFLOP/s"] = mfma_tf
    res["read_kernel_GB/s"] = nbytes / (read_ms * 1e-3) / 1e9
    res["mfma_loop_frac_of_published"] = mfma_tf / MFMA_BF16_PEAK_TFLOPS
    res["read_kernel_frac_of_published"] = res["read_kernel_GB/s"] / HBM_PEAK_GBS
    res["note"] = (f"torch.matmul {n}^3 bf16 (hipBLASLt); dst.copy_(src) and src.sum() over 2 GiB; "
                   f"mfma_loop: {blocks} x 4 waves, {iters} rounds of 4 independent 32x32x16 bf16 MFMAs; "
                   "read_kernel: one grid-stride 16-byte read of the 2 GiB")
    del src, dst
    torch.cuda.empty_cache()
    return res


def measure_module_path(wl, steps: int = 50, warmup: int = 10) -> dict:
    """The c2 inference forward as DSALTAttention runs it by default, in bf16 (module cast to
    bf16, _collect_last_P off, packed with cu_seqlens and its host copy): the whole
    module call, and each of its stages eager, launch costs included: the q/k/v projections
    (one GEMM over the concatenated weights, as the module runs them), the selection (dsalt_select_hybrid: the norms pass over x and the module's value
    projection, which also forms the window gate's logits and applies RoPE to k, then the
    selection launch forming the scores, the windows from the gate logits and the top-k),
    the HARD attention forward rotating q on load, out_proj. Beside them, not in the sum:
    the routes the default replaces (three separate projection GEMMs, the window gate's GEMV
    and the selection taking its logits, k RoPE alone, the score kernels then the selection
    on their scores, the torch score route)."""
    import copy
    from dsalt import _hip
    from dsalt.kernels._sparse import sparse_attention
    from dsalt.kernels.selectors import selection_scores
    from dsalt.kernels.window_utils import rotate_packed

    mod = copy.deepcopy(wl["mod"]).to(torch.bfloat16).eval()
    mod._collect_last_P = False
    T, H, D, L, kl = wl["T"], wl["H"], wl["D"], wl["L"], wl["k_lmk"]
    x = wl["xp"].to(torch.bfloat16)
    cu = wl["cu"]
    cu_list = cu.tolist()
    cos, sin = mod.rope_cos, mod.rope_sin
    with torch.no_grad():
        q, k, v = (t.view(T, H, D) for t in mod._project_qkv(x))
        kr = rotate_packed(k, cos, sin, cu)
        w = mod._window_sizes(x, floor=True)
        gl = mod.win_gate(x).squeeze(-1)
        alpha = mod._alpha().detach().float()
        sc, _, _ = selection_scores(x, mod.v_proj.weight, alpha, H, D, v=v, hip_scores=True)
        sc = sc.float()
        lmk = _hip.select_landmarks(sc, w, cu, kl, max_seqlen=L)
        out = sparse_attention(_hip.MODE_HARD, q, kr, v, lmk, None, w, cu, rope=(cos, sin))
    gate_linear = (mod.win_gate.weight, mod.win_gate.bias, mod.n_min, mod.n_max)
    stages = {
        "qkv_proj": lambda: mod._project_qkv(x),
        "qkv_proj_separate": lambda: (mod.q_proj(x), mod.k_proj(x), mod.v_proj(x)),
        "norms_gate_rope_k_and_select": lambda: _hip.select_hybrid(x, v, alpha, H, None, cu, kl, max_seqlen=L,
                                                                   rope_k=(k, cos, sin, cu), gate_linear=gate_linear),
        "window_gate_gemv": lambda: mod.win_gate(x),
        "norms_rope_k_and_select": lambda: _hip.select_hybrid(x, v, alpha, H, None, cu, kl, max_seqlen=L,
                                                              gate=(gl, mod.n_min, mod.n_max),
                                                              rope_k=(k, cos, sin, cu)),
        "rope_k_alone": lambda: rotate_packed(k, cos, sin, cu),
        "landmark_scores": lambda: selection_scores(x, mod.v_proj.weight, alpha, H, D, v=v, hip_scores=True),
        "landmark_scores_torch_route": lambda: selection_scores(x, mod.v_proj.weight, alpha, H, D, v=v),
        "select_topk_and_windows": lambda: _hip.select_landmarks_quantize(sc, None, cu, kl, max_seqlen=L,
                                                                          gate=(gl, mod.n_min, mod.n_max)),
        "attention_fwd_rotating_q": lambda: sparse_attention(_hip.MODE_HARD, q, kr, v, lmk, None, w, cu,
                                                             rope=(cos, sin)),
        "out_proj": lambda: mod._apply_out_proj(out.reshape(T, H * D)),
    }
    res = {"workload": "c2 DSALTAttention(1024, 16, 32, 512, 64) inference forward, bf16, packed 4 x 2048, "
                       "default routes (norms pass over x and v forming the window gate's logits and rotating k, "
                       "selection forming scores and windows from those logits, q rotated in the attention kernel)"}
    with torch.no_grad():
        res["module_forward_us"] = time_launches(lambda: mod(x, cu_seqlens=cu, cu_list=cu_list), steps,
                                                 warmup) * 1e3
        # the same call captured whole in a HIP graph and replayed: GPU time without the
        # host's per-call work
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            mod(x, cu_seqlens=cu, cu_list=cu_list)
        res["module_forward_graph_us"] = time_launches(graph.replay, steps, warmup) * 1e3
        for name, fn in stages.items():
            res[name + "_us"] = time_launches(fn, steps, warmup) * 1e3
    beside = ("module_forward_us", "module_forward_graph_us", "qkv_proj_separate_us", "window_gate_gemv_us",
              "norms_rope_k_and_select_us",
              "rope_k_alone_us", "landmark_scores_us", "landmark_scores_torch_route_us", "select_topk_and_windows_us")
    res["stages_sum_us"] = sum(v for kk, v in res.items() if kk.endswith("_us") and kk not in beside)
    return res


def measure_c4(device: torch.device, steps: int = 100, warmup: int = 100) -> dict:
    """the HARD forward on the seed-3 module's own windows and landmarks
    (DSALTAttention(2048, 16, 64, 1024, 128, 16384), x ~ N(0, 1) [1, 16384, 2048], bf16
    q/k/v), timed like the headline: MFMA fraction on the exact pair count, HBM fraction on
    the algorithmic bytes."""
    from dsalt import _hip

    wl = make_workload("c4", device)
    q, k, v, w, lmk, cu = wl["q"], wl["k"], wl["v"], wl["w"], wl["lmk"], wl["cu"]
    T, H, D = wl["T"], wl["H"], wl["D"]
    f = _hip.FwdLauncher(_hip.MODE_HARD, q, k, v, w, lmk, None, cu, 1.0 / math.sqrt(D))
    ms = time_launches(f, steps, warmup)
    P = effective_pairs_hard(w.float().cpu().numpy(), lmk.cpu().numpy(), cu.cpu().tolist())
    t = ms * 1e-3
    bytes_alg = 2 * T * H * D * 4 + 4 * T * H + 4 * T + 8 * H * wl["B"] * wl["k_lmk"]
    traffic, traffic_sha = load_traffic("c4")
    del wl, f
    torch.cuda.empty_cache()
    return {
        "workload": f"c4: HARD DSALT attention forward, 1 x 16384 tokens, {H} heads x {D} head_dim, n_min 64, "
                    "n_max 1024, k_lmk 128, module seed 3, bf16",
        "us_per_launch": ms * 1e3,
        "tokens_per_s": T / t,
        "pairs": P,
        "keys_per_query": P / (T * H),
        "mfma_tflops": 4.0 * D * P / t / 1e12,
        "mfma_frac": 4.0 * D * P / t / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "hbm_GBs": bytes_alg / t / 1e9,
        "hbm_frac": bytes_alg / t / 1e9 / HBM_PEAK_GBS,
        "bytes_per_launch": bytes_alg,
        "traffic": traffic,
        "traffic_source_sha16": traffic_sha,
    }


def measure_rope(wl, cu, fwd_ms: float) -> dict:
    """The module's RoPE at the workload's shape in bf16: the reference's route written
    eagerly (position gather, cos/sin cast, rotation in torch ops; the reference compiles
    it with Inductor, which is not used here) against dsalt_rope of q and k (one pass,
    from a HIP graph), and the inference path the module takes: dsalt_rope of k alone
    plus the HARD forward rotating q as it loads it (its time against the plain forward's
    `fwd_ms`). Bytes of dsalt_rope: q and k read and written once (bf16); the tables are a
    few hundred KB and stay in cache."""
    from dsalt import _hip
    from dsalt.kernels.window_utils import apply_rotary_emb
    mod, T, H, D = wl["mod"], wl["T"], wl["H"], wl["D"]
    g = torch.Generator(device=cu.device).manual_seed(5)
    q = torch.randn(T, H, D, device=cu.device, generator=g).to(torch.bfloat16)
    k = torch.randn(T, H, D, device=cu.device, generator=g).to(torch.bfloat16)
    cos_t, sin_t = mod.rope_cos.float().contiguous(), mod.rope_sin.float().contiguous()
    pos_ids = torch.arange(T, device=cu.device) % wl["L"]

    def eager():
        cos = cos_t[pos_ids].to(q.dtype)
        sin = sin_t[pos_ids].to(q.dtype)
        apply_rotary_emb(q, k, cos.unsqueeze(1), sin.unsqueeze(1))

    qo, ko = torch.empty_like(q), torch.empty_like(k)
    hip = lambda: _hip.rope(q, k, cos_t, sin_t, cu, q_out=qo, k_out=ko)
    hip_k = lambda: _hip.rope(None, k, cos_t, sin_t, cu, k_out=ko)
    # the HARD forward on the workload with q rotated on load (q of the workload serves as
    # the un-rotated input: the cost does not depend on the values)
    fused = _hip.FwdLauncher(_hip.MODE_HARD, wl["q"], wl["k"], wl["v"], wl["w"], wl["lmk"], None, cu,
                             1.0 / math.sqrt(D), rope=(cos_t, sin_t))
    with torch.no_grad():
        eager_ms = time_launches(eager, 50, 10)
        hip_ms = time_graph(hip)
        hip_k_ms = time_graph(hip_k)
        fused_ms = time_launches(fused, 200, 100)
    nbytes = 2 * (q.numel() + k.numel()) * 2
    return {"workload": "c2 RoPE of q and k, bf16", "eager_torch_us": eager_ms * 1e3, "hip_us": hip_ms * 1e3,
            "hip_GB/s": nbytes / (hip_ms * 1e-3) / 1e9,
            "module_path": {"rope_k_us": hip_k_ms * 1e3, "fwd_rotating_q_us": fused_ms * 1e3,
                            "fwd_plain_us": fwd_ms * 1e3,
                            "rope_plus_fwd_us": hip_k_ms * 1e3 + fused_ms * 1e3,
                            "unfused_rope_plus_fwd_us": hip_ms * 1e3 + fwd_ms * 1e3}}


def cpu_baseline(wl, budget_s: float = 10.0):
    """The reference's CPU fallback cost (dense HARD mask + fp32 SDPA), restated in
    oracle/, timed on this host over the whole workload (every sequence, all heads):
    runs of the full workload until about `budget_s` seconds (at least 5), median."""
    from oracle import dsalt_oracle as orc

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    T = wl["T"]
    q32, k32, v32 = (wl[n].float().cpu() for n in ("q", "k", "v"))
    w = wl["w"].float().cpu().numpy()
    pos = wl["lmk"].cpu().numpy()
    cu = wl["cu"].cpu().tolist()
    orc.cpu_baseline_hard(q32, k32, v32, w, pos, cu)  # warm-up
    times = []
    t_all = time.perf_counter()
    while len(times) < 5 or time.perf_counter() - t_all < budget_s:
        t0 = time.perf_counter()
        orc.cpu_baseline_hard(q32, k32, v32, w, pos, cu)
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    med = float(np.median(times))
    return {"value": T / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(), "torch": torch.__version__,
            "sample": f"median of {len(times)} runs ({sum(times):.1f} s) of the whole workload: "
                      f"{len(cu) - 1} sequences, {T} tokens, {wl['H']} heads (dense mask + fp32 SDPA)",
            "runs_s_min_max": [min(times), max(times)]}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


FWD_SOURCES = ("dsalt-library_amd/csrc/fwd.hip", "dsalt-library_amd/csrc/common.h",
               "dsalt-library_amd/csrc/tiles.h")


def source_hash(paths=FWD_SOURCES) -> str:
    import hashlib
    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic(cfg: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE, if recorded for
    the forward sources as they are now (None when the record is missing or stale)."""
    path = os.path.join(ROOT, "profiles", f"fwd_{cfg}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        rec = json.load(f)
    if rec.get("source_sha16") != source_hash():
        return None, rec.get("source_sha16")
    return rec.get("hbm_bytes_per_launch"), rec.get("source_sha16")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # the GPU clock ramps up over the first ~10 ms of back-to-back launches: the default
    # warmup (about 20 ms of forwards) makes the timed steps run at the sustained clock
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-backward", action="store_true", help="skip the config-3 backward measurement")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the config-4, dense-variant and config-5 LM measurements")
    ap.add_argument("--only-fwd", action="store_true",
                    help="time only the headline forward of --config and exit (for profiling)")
    ap.add_argument("--only", choices=("lm", "dense", "backward", "c4", "peaks", "selection", "module"), default=None,
                    help="run only that measurement and print its JSON (for profiling)")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    from dsalt import _hip

    dev = torch.device("cuda", 0)
    if args.copy_calib_mib > 0:
        n = args.copy_calib_mib * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only is not None:
        if args.only == "module":
            print(json.dumps(measure_module_path(make_workload("c2", dev))))
            return
        fn = {"lm": measure_lm, "dense": measure_dense, "backward": measure_backward, "c4": measure_c4,
              "peaks": measure_peaks, "selection": measure_selection}[args.only]
        print(json.dumps(fn(dev)))
        return
    wl = make_workload(args.config, dev)
    q, k, v, w, lmk, cu = wl["q"], wl["k"], wl["v"], wl["w"], wl["lmk"], wl["cu"]
    T, H, D = wl["T"], wl["H"], wl["D"]
    out = torch.empty_like(q)
    lse = torch.empty((H, T), device=dev, dtype=torch.float32).t()  # head-major storage
    scale = 1.0 / math.sqrt(D)

    step = _hip.FwdLauncher(_hip.MODE_HARD, q, k, v, w, lmk, None, cu, scale, out=out, lse=lse)
    ms = time_launches(step, args.steps, args.warmup)
    if args.only_fwd:  # the headline forward alone (for counter profiles of that kernel)
        print(json.dumps({"workload": args.config, "ms_per_step": ms, "steps": args.steps}))
        return

    # selection + quantisation (the rest of the inference hot path), reported alongside
    from dsalt.kernels.landmark_tokens_ker import hybrid_scores_per_head
    with torch.no_grad():
        mod = wl["mod"]
        scores, _, _ = hybrid_scores_per_head(wl["xp"], mod.v_proj.weight, mod._alpha().float(), H, D)
        w_cont = mod._window_continuous(wl["xp"]).float()
    sel = _hip.SelectLauncher(scores, w, cu, wl["k_lmk"], max_seqlen=wl["L"])
    sel_ms = time_graph(sel)
    qz_ms = time_graph(_hip.QuantizeLauncher(w_cont))
    # the module's inference path: the windows quantised by the selection launch itself
    selq = _hip.SelectLauncher(scores, w_cont, cu, wl["k_lmk"], max_seqlen=wl["L"], quantize=True)
    selq_ms = time_graph(selq)
    if not (torch.equal(selq.out, sel.out) and torch.equal(selq.w_out, w.float())):
        raise RuntimeError("fused selection + quantisation differs from the separate launches")
    bytes_sel = 4 * T * H + 4 * T + 4 * (wl["B"] + 1) + 8 * H * wl["B"] * wl["k_lmk"]
    front = measure_front_end(wl, w, cu)

    # cold HBM: launches rotate over input sets whose total (> 512 MB) exceeds the
    # 256 MB last-level cache, so every launch reads Q, K and V from HBM
    n_sets = max(2, int(math.ceil(544e6 / (4 * q.numel() * 2))))
    sets = []
    for _ in range(n_sets):
        qs, ks, vs = q.clone(), k.clone(), v.clone()
        os_ = torch.empty_like(q)
        ls = torch.empty((H, T), device=dev, dtype=torch.float32).t()
        sets.append(_hip.FwdLauncher(_hip.MODE_HARD, qs, ks, vs, w, lmk, None, cu, scale, out=os_, lse=ls))
    rot = [0]

    def cold_step():
        sets[rot[0] % n_sets]()
        rot[0] += 1

    cold_ms = time_launches(cold_step, max(args.steps, 4 * n_sets), 2 * n_sets)
    del sets

    P = effective_pairs_hard(w.float().cpu().numpy(), lmk.cpu().numpy(), cu.cpu().tolist())
    flops = 4.0 * D * P
    bytes_alg = 2 * T * H * D * 4 + 4 * T * H + 4 * T + 8 * H * wl["B"] * wl["k_lmk"]
    t_s = ms * 1e-3
    tflops = flops / t_s / 1e12
    traffic, traffic_sha = load_traffic(args.config)

    res = {
        "metric": "DSALT attn fwd tokens/s & % bf16 MFMA peak (16h×64d, seq 2048)",
        "value": T / t_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (DSALTAttention random init, x ~ N(0,1))",
        "config": {
            "workload": f"{args.config}: HARD DSALT attention forward, packed {wl['B']}x{wl['L']} tokens, "
                        f"{H} heads x {D} head_dim, n_min {wl['n_min']}, n_max {wl['n_max']}, k_lmk {wl['k_lmk']}",
            "tokens": T, "heads": H, "head_dim": D, "seqs": wl["B"], "seq_len": wl["L"],
            "k_lmk": wl["k_lmk"], "pairs": P, "keys_per_query": P / (T * H),
        },
        # The forward's compulsory arithmetic intensity at c2 (~137 FLOP/B) is below the
        # MI355X ridge (2.5 PFLOP/s / 8 TB/s = 312 FLOP/B), so its roofline bound is HBM;
        # the MFMA fraction is the headline metric and is reported next to it.
        "roofline": {
            "bound": "hbm",
            "achieved": bytes_alg / t_s / 1e9,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": bytes_alg / t_s / 1e9 / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source_sha16": traffic_sha,
            "source_sha16": source_hash(),
        },
        "mfma": {
            "achieved": tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": tflops / MFMA_BF16_PEAK_TFLOPS,
            "flops_per_launch": flops,
        },
        "bytes_per_launch": bytes_alg,
        # the same forward with every launch on a different input set (> 512 MB in total)
        "cold": {
            "ms_per_step": cold_ms,
            "tokens_per_s": T / (cold_ms * 1e-3),
            "mfma_frac": flops / (cold_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "hbm_frac": bytes_alg / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "input_sets": n_sets,
        },
        "select_ms": sel_ms,
        "select": {"us": sel_ms * 1e3, "GB/s": bytes_sel / (sel_ms * 1e-3) / 1e9, "bytes": bytes_sel},
        "quantize_ms": qz_ms,
        "select_quantize_us": selq_ms * 1e3,  # one launch: selection with the quantisation fused in
        "path_ms": ms + selq_ms,
        "selector_front_end": front,
        "rope": measure_rope(wl, cu, ms),
        "module_path_c2": measure_module_path(wl),
        "host_launch": measure_host_launch(dev),
        "peaks_measured": measure_peaks(dev),
    }
    if not args.no_extras and args.config == "c2":
        res["c4"] = measure_c4(dev)
    if not args.no_backward:
        res["backward"] = measure_backward(dev)
    if not args.no_extras:
        res["dense"] = measure_dense(dev)
        res["lm_c5"] = measure_lm(dev)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(wl)
    print(json.dumps(res))


if __name__ == "__main__":
    main()

"""Headline configurations on the selectors the module actually produces.

* Selection route parity at configs 2 (seed 1) and 4 (seed 3): the module's default
  route (the HIP score kernel over x and its own value projection v = x W_V^T) and the
  torch route on v must both pick exactly the landmark sets of the reference's route
  (x @ W_V.T, then torch's norms), per (head, sequence), for an fp32 module, a bf16
  module, an fp16 module (c2) and an fp32 module under bf16 autocast; the torch route on v also gives the
  same fp32 scores bit for bit.
* Forward parity at configs 2 and 4, HARD and SOFT, on the windows and landmarks the
  module produces (built as bench.py builds them: seed 1 / seed 3, x ~ N(0, 1)), against
  the fp64 oracle on a window of query rows of every sequence. Bar (north star):
  max-abs 2e-2 and relative L2 1e-2, absolute.
"""
import math

import pytest
import torch

import bench
import dsalt._hip as hip
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
MAX_ABS, REL_L2 = 2e-2, 1e-2


def _errs(got, ref):
    diff = got.double().cpu() - ref.double()
    return diff.abs().max().item(), (diff.norm() / ref.double().norm().clamp_min(1e-30)).item()


def _c2_module(dtype_mode, cfg="c2"):
    from dsalt.modules import DSALTAttention
    B, L, d_model, H, n_min, n_max, k_lmk, seed = bench.CONFIGS[cfg]
    torch.manual_seed(seed)
    mod = DSALTAttention(d_model, H, n_min, n_max, k_lmk, max_seq_len=L)
    x = torch.randn(B * L, d_model)
    mod = mod.to(DEV).eval()
    mod._collect_last_P = False
    x = x.to(DEV)
    if dtype_mode in ("bf16", "fp16"):
        dt = torch.bfloat16 if dtype_mode == "bf16" else torch.float16
        mod = mod.to(dt)
        x = x.to(dt)
    cu = torch.arange(0, B * L + 1, L, dtype=torch.int32, device=DEV)
    return mod, x, cu


def _run_route(mod, x, cu, fused, hip_scores, autocast):
    mod._fused_selector, mod._hip_scores = fused, hip_scores
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        mod(x, cu_seqlens=cu, cu_list=cu.tolist())
    w, lmk = mod._last_selection
    return w.clone(), lmk.clone()


@pytest.mark.parametrize("cfg,dtype_mode", [("c2", "fp32"), ("c2", "bf16"), ("c2", "fp16"), ("c2", "autocast"),
                                            ("c4", "bf16"), ("c4", "autocast")])
def test_default_selection_equals_gemm_route(cfg, dtype_mode):
    print(f"{cfg} selection routes {dtype_mode}", flush=True)
    mod, x, cu = _c2_module(dtype_mode, cfg)
    ac = dtype_mode == "autocast"
    w_g, lmk_g = _run_route(mod, x, cu, fused=False, hip_scores=False, autocast=ac)
    w_t, lmk_t = _run_route(mod, x, cu, fused=True, hip_scores=False, autocast=ac)
    w_h, lmk_h = _run_route(mod, x, cu, fused=True, hip_scores=True, autocast=ac)
    mod._fused_selector, mod._hip_scores = True, True
    assert torch.equal(w_g, w_t) and torch.equal(w_g, w_h)
    # the windows the selection launch formed from the gate logits are torch's own
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=ac):
        w_torch = mod._window_sizes(x, floor=True)
    assert torch.equal(w_g, w_torch), f"{int((w_g != w_torch).sum())} windows differ from _window_sizes"
    # slots are emitted in ascending position order, so equal sets are equal rows
    for name, lmk in (("torch route on v", lmk_t), ("HIP score kernel (default)", lmk_h)):
        same = (lmk_g == lmk).all(-1)
        print(f"  {name}: {int(same.sum())}/{same.numel()} (head, sequence) sets equal", flush=True)
        assert bool(same.all()), f"{name}: {int((~same).sum())} landmark sets differ from the x @ W_V.T route"


@pytest.mark.parametrize("dtype_mode", ["fp32", "bf16", "autocast"])
def test_c3_training_selection_equals_gemm_route(dtype_mode):
    """Config 3's training selection (the module's _train_selectors on its eight packed
    sequences): the default HIP score route and the torch route on v pick the landmark
    sets of the reference's x @ W_V.T route, and all three quantise the same windows."""
    import numpy as np
    from dsalt.modules import DSALTAttention
    print(f"c3 training selection routes {dtype_mode}", flush=True)
    np.random.seed(2)
    lens = [int(v) for v in np.random.randint(256, 2049, 8)]
    torch.manual_seed(2)
    mod = DSALTAttention(1024, 16, 32, 512, 64, max_seq_len=2048).to(DEV).train()
    T = sum(lens)
    x = torch.randn(T, 1024).to(DEV)
    if dtype_mode == "bf16":
        mod, x = mod.to(torch.bfloat16), x.to(torch.bfloat16)
    cu_list = [0]
    for L in lens:
        cu_list.append(cu_list[-1] + L)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=DEV)
    res = {}
    for name, fused, hip_scores in (("gemm", False, False), ("torch_v", True, False), ("hip", True, True)):
        mod._fused_selector, mod._hip_scores = fused, hip_scores
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype_mode == "autocast"):
            v = mod.v_proj(x).view(T, 16, 64)  # as the module forms it (in bf16 under autocast)
            w, lmk, _ = mod._train_selectors(x, cu, T, DEV, cu_list, v if fused else None)
        res[name] = (mod._last_selection[0].clone(), lmk.clone())
    mod._fused_selector, mod._hip_scores = True, True
    for name in ("torch_v", "hip"):
        assert torch.equal(res[name][0], res["gemm"][0])
        same = (res[name][1] == res["gemm"][1]).all(-1)
        print(f"  {name}: {int(same.sum())}/{same.numel()} (head, sequence) sets equal", flush=True)
        assert bool(same.all()), f"{name}: {int((~same).sum())} landmark sets differ from the x @ W_V.T route"


@pytest.mark.parametrize("cfg,windows", [("c2", [(0, 256), (1024, 1280), (1536, 1792)]),
                                         ("c4", [(0, 256), (8192, 8448), (15872, 16128)])])
@pytest.mark.parametrize("mode", ["hard", "soft"])
def test_headline_forward_on_module_selectors(cfg, windows, mode):
    """Rows at the start of every sequence (the band cut by the sequence start, few
    admissible landmarks), in the middle and near the end."""
    print(f"headline {cfg} {mode} on module selectors", flush=True)
    wl = bench.make_workload(cfg, DEV)
    q, k, v, cu = wl["q"], wl["k"], wl["v"], wl["cu"]
    scale = 1.0 / math.sqrt(wl["D"])
    if mode == "hard":
        w, lmk, bias = wl["w"], wl["lmk"], None
        out, lse = hip.fwd(hip.MODE_HARD, q, k, v, w, lmk, None, cu, scale, out_dtype=torch.float32)
    else:
        mod = wl["mod"].train()
        with torch.no_grad():
            w, lmk, bias = mod._train_selectors(wl["xp"], cu, wl["T"], DEV, cu.tolist())
        mod.eval()
        out, lse = hip.fwd(hip.MODE_SOFT, q, k, v, w, lmk, bias, cu, scale, mod.tau_win,
                           float(mod.win_edge), out_dtype=torch.float32)
    torch.cuda.synchronize()
    qc, kc, vc = (t.cpu().double() for t in (q, k, v))
    for rows in windows:
        if mode == "hard":
            o_ref, l_ref = orc.attention_hard(qc, kc, vc, w.cpu(), lmk.cpu(), None, cu.tolist(), rows=rows)
        else:
            o_ref, l_ref = orc.attention_soft(qc, kc, vc, w.cpu(), lmk.cpu(), bias.cpu().double(), cu.tolist(),
                                              rows=rows)
        sel = torch.cat([torch.arange(int(cu[s]) + rows[0], int(cu[s]) + rows[1]) for s in range(len(cu) - 1)])
        ma, rl = _errs(out[sel.to(DEV)], o_ref)
        lfin = torch.isfinite(l_ref)
        lerr = (lse[sel.to(DEV)].cpu().double()[lfin] - l_ref[lfin]).abs().max().item()
        print(f"  rows {rows}: out max-abs {ma:.2e} rel-L2 {rl:.2e}; lse max-abs {lerr:.2e}", flush=True)
        assert ma <= MAX_ABS and rl <= REL_L2, f"{cfg} {mode} rows {rows}: max-abs {ma:.3e}, rel-L2 {rl:.3e}"
        assert lerr <= 2e-2


def test_c3_backward_on_module_selectors():
    """Config 3 backward (SOFT) on the windows, landmarks and landmark weights the module
    produces (bench.make_train_workload: seed 2, the c3 packing), every gradient against
    fp64 autograd through the oracle. dQ/dK/dV and the window and landmark-weight
    gradients (d_w~ [T], d_logw [H, S, k]) are held to the north-star bar itself:
    max-abs 2e-2 (absolute) and relative L2 1e-2."""
    print("c3 backward on module selectors", flush=True)
    wl = bench.make_train_workload(DEV)
    q, k, v, w, lmk, logw, cu = wl["q"], wl["k"], wl["v"], wl["w"], wl["lmk"], wl["logw"], wl["cu"]
    scale = 1.0 / math.sqrt(wl["D"])
    out, lse = hip.fwd(hip.MODE_SOFT, q, k, v, w, lmk, logw, cu, scale, 1.0, 4.0, out_dtype=torch.float32)
    dq, dk, dv, dlw, dw = hip.bwd(hip.MODE_SOFT, q, k, v, out, lse, wl["dout"], w, lmk, logw, cu, scale, 1.0, 4.0,
                                  need_dw=True, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    q64, k64, v64 = (t.cpu().double().requires_grad_() for t in (q, k, v))
    w64 = w.cpu().double().requires_grad_()
    lw64 = logw.cpu().double().requires_grad_()
    o, _ = orc.attention_soft(q64, k64, v64, w64, lmk.cpu(), lw64, wl["cu_list"], tau_win=1.0, win_edge=4.0)
    (o * wl["dout"].cpu().double()).sum().backward()
    ref_lw = torch.where(torch.isfinite(logw.cpu().double()), lw64.grad, torch.zeros_like(lw64.grad))
    for name, got, ref in (("dq", dq, q64.grad), ("dk", dk, k64.grad), ("dv", dv, v64.grad),
                           ("d_w", dw, w64.grad), ("d_logw", dlw, ref_lw)):
        ma, rl = _errs(got, ref)
        print(f"  {name}: max-abs {ma:.3e} rel-L2 {rl:.3e} (max |ref| {ref.abs().max().item():.3e})", flush=True)
        assert ma <= MAX_ABS and rl <= REL_L2, f"c3 {name}: max-abs {ma:.3e}, rel-L2 {rl:.3e}"

"""Dense batched variant (DSALT_MODE_DENSE) on the GPU.

* Kernel parity: the HIP forward (O, LSE) and backward (dQ, dK, dV, the landmark-bias
  gradient [H, T] and d_w~ [T]) against the fp64 oracle (oracle.attention_dense and
  torch autograd through it) on the same bf16/fp16 inputs; ragged lengths (T = 1, 33,
  100, 257), head dims 64 and 128, windows below win_edge, below 1, integral, beyond
  T, landmark tables with and without entries, no table at all.
* Module parity: DSALTAttention on [1, T, d] input against the reference module's own
  golden vectors (tests/golden/module_batched_*.npz, written by make_golden.py):
  training output and every gradient, the landmark selection, the eval output and the
  diagnostic _last_P.
* Full size: T = 4096, H = 8, D = 128 against the oracle on every row.
Bar (north star): O and gradients relative L2 1e-2 and max-abs 2e-2 of the largest
reference value; LSE max-abs 2e-2.
"""
import glob
import json
import math
import os

import numpy as np
import pytest
import torch

import dsalt._hip as hip
from dsalt.modules import DSALTAttention
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BATCHED = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "module_batched_*.npz")))


def check(got, ref, what, rel=1e-2, frac=2e-2):
    got, ref = torch.as_tensor(got).double().cpu(), torch.as_tensor(ref).double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    diff = got - ref
    rl = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    ma = diff.abs().max().item() if diff.numel() else 0.0
    bar = frac * min(1.0, max(ref.abs().max().item() if ref.numel() else 0.0, 1e-3))
    print(f"  {what}: rel-L2 {rl:.2e} max-abs {ma:.2e} (bar {bar:.2e})", flush=True)
    assert rl <= rel and ma <= bar, f"{what}: rel-L2 {rl:.3e}, max-abs {ma:.3e} (bar {bar:.3e})"


def make_case(T, H, D, dtype, seed, w_kind="mixed", lmk="some"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    k = torch.randn(T, H, D, generator=g).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    if w_kind == "mixed":
        w = 2.0 + torch.rand(T, generator=g) * 40.0
        # special windows: below win_edge, below 1, integral, at and beyond T
        for j, val in enumerate((0.3, 1.0, 3.5, 4.0, 7.0, float(T), T + 5.5)):
            if j < T:
                w[(j * 7919) % T] = val
    elif w_kind == "small":
        w = 0.2 + torch.rand(T, generator=g) * 5.0
    else:
        w = float(T) + 10.0 * torch.rand(T, generator=g)
    if lmk == "none":
        lb = None
    else:
        s = torch.randn(T, H, generator=g)
        lb = torch.log(torch.sigmoid(s / 2.0).clamp(min=1e-20)).t().contiguous()
        if lmk == "some":
            keep = torch.rand(H, T, generator=g) < 0.15
        else:
            keep = torch.zeros(H, T, dtype=torch.bool)
        lb = torch.where(keep, lb, torch.full_like(lb, float("-inf")))
    return q, k, v, w.float(), lb


def oracle_grads(q, k, v, w, lb, dout, tau, edge):
    qd, kd, vd = (t.double().requires_grad_() for t in (q, k, v))
    wd = w.double().requires_grad_()
    lbd = (torch.full((q.shape[1], q.shape[0]), float("-inf"), dtype=torch.float64) if lb is None
           else lb.double()).requires_grad_()
    o, lse = orc.attention_dense(qd, kd, vd, wd, lbd, tau, edge, 1.0 / math.sqrt(q.shape[-1]))
    o.backward(dout.double())
    return o.detach(), lse.detach(), qd.grad, kd.grad, vd.grad, lbd.grad, wd.grad


CASES = [
    # T, H, D, dtype, seed, w_kind, lmk
    (1, 2, 64, torch.bfloat16, 1, "mixed", "some"),
    (33, 2, 64, torch.bfloat16, 2, "mixed", "some"),
    (100, 3, 64, torch.float16, 3, "small", "some"),
    (257, 2, 64, torch.bfloat16, 4, "mixed", "none"),
    (64, 2, 128, torch.bfloat16, 5, "large", "empty"),
    (200, 2, 128, torch.float16, 6, "mixed", "some"),
    (257, 1, 128, torch.bfloat16, 7, "small", "some"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"T{c[0]}-H{c[1]}-D{c[2]}-{str(c[3])[6:]}-{c[5]}-{c[6]}"
                                             for c in CASES])
def test_dense_kernels_match_oracle(case):
    T, H, D, dtype, seed, w_kind, lmk = case
    print(f"dense kernels {case}", flush=True)
    q, k, v, w, lb = make_case(T, H, D, dtype, seed, w_kind, lmk)
    tau, edge = 1.0, 4.0
    scale = 1.0 / math.sqrt(D)
    qg, kg, vg, wg = (t.to(DEV) for t in (q, k, v, w))
    lbg = None if lb is None else lb.to(DEV)
    out, lse = hip.dense_fwd(qg, kg, vg, wg, lbg, scale, tau, edge, out_dtype=torch.float32)
    dout = torch.randn(T, H, D, generator=torch.Generator().manual_seed(seed + 100)).to(dtype)
    dq, dk, dv, d_lb, d_w = hip.dense_bwd(qg, kg, vg, out, lse, dout.to(DEV), wg, lbg, scale, tau, edge,
                                          need_dw=True, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    o_r, l_r, dq_r, dk_r, dv_r, dlb_r, dw_r = oracle_grads(q, k, v, w, lb, dout, tau, edge)
    check(out, o_r, "O")
    assert (lse.cpu().double() - l_r).abs().max().item() <= 2e-2
    check(dq, dq_r, "dQ")
    check(dk, dk_r, "dK")
    check(dv, dv_r, "dV")
    if lb is None:
        assert d_lb is None
    else:
        check(d_lb, dlb_r, "d_lmk_bias")
        assert float(d_lb.cpu()[torch.isinf(lb)].abs().max() if torch.isinf(lb).any() else 0.0) == 0.0
    check(d_w, dw_r, "d_w")


@pytest.mark.parametrize("tau", [0.15, 0.25, 3.0])
@pytest.mark.parametrize("edge", [2.0, 8.0])
@pytest.mark.parametrize("case", [CASES[1], CASES[3], CASES[5]], ids=["T33-D64", "T257-D64", "T200-D128"])
def test_dense_edge_params(case, tau, edge):
    """Other window-edge temperatures and widths than the module default (tau = 1,
    win_edge = 4): tau = 0.15 takes one exp per tail element, tau = 0.25 also (its
    factored tail would overflow where the true bias is still above the clamp), tau = 3
    the factored tail; every output and gradient against the fp64 oracle."""
    T, H, D, dtype, seed, w_kind, lmk = case
    print(f"dense edge params T={T} D={D} tau={tau} edge={edge}", flush=True)
    q, k, v, w, lb = make_case(T, H, D, dtype, seed, w_kind, lmk)
    scale = 1.0 / math.sqrt(D)
    qg, kg, vg, wg = (t.to(DEV) for t in (q, k, v, w))
    lbg = None if lb is None else lb.to(DEV)
    out, lse = hip.dense_fwd(qg, kg, vg, wg, lbg, scale, tau, edge, out_dtype=torch.float32)
    dout = torch.randn(T, H, D, generator=torch.Generator().manual_seed(seed + 200)).to(dtype)
    dq, dk, dv, d_lb, d_w = hip.dense_bwd(qg, kg, vg, out, lse, dout.to(DEV), wg, lbg, scale, tau, edge,
                                          need_dw=True, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    o_r, l_r, dq_r, dk_r, dv_r, dlb_r, dw_r = oracle_grads(q, k, v, w, lb, dout, tau, edge)
    check(out, o_r, "O")
    assert (lse.cpu().double() - l_r).abs().max().item() <= 2e-2
    check(dq, dq_r, "dQ")
    check(dk, dk_r, "dK")
    check(dv, dv_r, "dV")
    if lb is not None:
        check(d_lb, dlb_r, "d_lmk_bias")
    check(d_w, dw_r, "d_w")


def test_dense_output_dtypes_and_relaunch():
    # 16-bit outputs and gradients equal the fp32 ones rounded; a second launch of the
    # same launcher reproduces the first bit for bit (deterministic, no stale state)
    q, k, v, w, lb = make_case(150, 2, 64, torch.bfloat16, 11)
    qg, kg, vg, wg, lbg = (t.to(DEV) for t in (q, k, v, w, lb))
    scale = 0.125
    o32, lse = hip.dense_fwd(qg, kg, vg, wg, lbg, scale, out_dtype=torch.float32)
    o16, lse16 = hip.dense_fwd(qg, kg, vg, wg, lbg, scale)
    assert o16.dtype == torch.bfloat16 and torch.equal(o16, o32.to(torch.bfloat16)) and torch.equal(lse, lse16)
    dout = torch.randn_like(qg)
    launcher = hip.DenseBwdLauncher(qg, kg, vg, o32, lse, dout, wg, lbg, scale, grad_dtype=torch.float32)
    launcher()
    first = [t.clone() for t in launcher.results]
    launcher()
    for a, b in zip(first, launcher.results):
        assert torch.equal(a, b)
    g16 = hip.dense_bwd(qg, kg, vg, o32, lse, dout, wg, lbg, scale)
    for a, b in zip(first[:3], g16[:3]):
        assert b.dtype == torch.bfloat16 and torch.equal(a.to(torch.bfloat16), b)


def test_dense_rejects_bad_arguments():
    q, k, v, w, lb = (t.to(DEV) for t in make_case(40, 2, 64, torch.bfloat16, 12))
    with pytest.raises(hip.DsaltError, match=r"\[H=2, T=40\]"):
        hip.dense_fwd(q, k, v, w, lb.t().contiguous(), 0.125)
    with pytest.raises(hip.DsaltError, match="scale > 0"):
        hip.dense_fwd(q, k, v, w, lb, -0.125)
    with pytest.raises(hip.DsaltError, match="tau_win"):
        hip.dense_fwd(q, k, v, w, lb, 0.125, tau_win=0.0)
    with pytest.raises(hip.DsaltError, match="head_dim"):
        hip.dense_fwd(q[..., :32].contiguous(), k[..., :32].contiguous(), v[..., :32].contiguous(), w, lb, 0.125)


def test_dense_full_size_every_row():
    # T = 4096, H = 8, D = 128 (bf16): every row against the oracle
    T, H, D = 4096, 8, 128
    print(f"dense full size T={T} H={H} D={D}", flush=True)
    q, k, v, w, lb = make_case(T, H, D, torch.bfloat16, 21)
    w = 16.0 + 240.0 * torch.rand(T, generator=torch.Generator().manual_seed(22))
    scale = 1.0 / math.sqrt(D)
    out, lse = hip.dense_fwd(q.to(DEV), k.to(DEV), v.to(DEV), w.to(DEV), lb.to(DEV), scale,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_r, l_r = orc.attention_dense(q.double(), k.double(), v.double(), w.double(), lb.double(), 1.0, 4.0, scale)
    check(out, o_r, "O full size")
    assert (lse.cpu().double() - l_r).abs().max().item() <= 2e-2


def build(d):
    cfg = json.loads(str(d["config"]))
    mod = DSALTAttention(cfg["d_model"], cfg["n_heads"], cfg["n_min"], cfg["n_max"], cfg["k_lmk"],
                         cfg["max_seq_len"], yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"],
                         qkv_bias=cfg["qkv_bias"], rope_base=cfg["rope_base"])
    with torch.no_grad():
        for name, p in mod.named_parameters():
            p.copy_(torch.from_numpy(d["p." + name]))
    return cfg, mod.to(DEV)


@pytest.mark.parametrize("path", BATCHED, ids=[os.path.basename(p) for p in BATCHED])
def test_module_batched_train_matches_reference_golden(path):
    print(f"module batched train {os.path.basename(path)}", flush=True)
    d = np.load(path, allow_pickle=False)
    cfg, mod = build(d)
    mod.train()
    x = torch.from_numpy(d["x"]).to(DEV).requires_grad_()
    out, aux = mod(x)
    assert float(aux) == 0.0
    w_cont, lmk_pos = mod._last_selection
    check(w_cont, d["w_cont"], "w_cont")
    H, T = d["lmk_sel"].shape
    sel = torch.zeros(H, T, dtype=torch.bool)
    for h in range(H):
        p = lmk_pos[h, 0].cpu()
        sel[h, p[p >= 0]] = True
    assert torch.equal(sel, torch.from_numpy(d["lmk_sel"]).bool()), "landmark selection differs from the reference"
    check(out.detach(), d["out"], "out")
    out.backward(torch.from_numpy(d["dout"]).to(DEV))
    check(x.grad, d["grad.x"], "grad x")
    for name, p in mod.named_parameters():
        check(p.grad, d["grad." + name], "grad " + name)


@pytest.mark.parametrize("path", BATCHED, ids=[os.path.basename(p) for p in BATCHED])
def test_module_batched_eval_matches_reference_golden(path):
    print(f"module batched eval {os.path.basename(path)}", flush=True)
    d = np.load(path, allow_pickle=False)
    cfg, mod = build(d)
    mod.eval()
    with torch.no_grad():
        out, _ = mod(torch.from_numpy(d["x"]).to(DEV))
    check(out, d["out_eval"], "eval out")
    P = mod._last_P
    assert P is not None and P.shape == tuple(d["last_P"].shape)
    check(P, d["last_P"], "_last_P")
    mod._collect_last_P = False
    with torch.no_grad():
        mod(torch.from_numpy(d["x"]).to(DEV))
    assert mod._last_P is None

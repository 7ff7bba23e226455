"""DSALTAttention on the GPU. Training mode (SOFT kernels, forward and backward) is
checked against golden vectors written from the reference's own module
(tests/golden/); inference mode (HARD kernel) against the oracle's composition, which
tests/test_golden.py pins to the same reference. fp32 modules compute attention in
fp16 as the reference's kernels do. Bar: relative L2 1e-2 and max-abs 2e-2 of the
largest reference value."""
import glob
import json
import os

import numpy as np
import pytest
import torch

from dsalt.modules import DSALTAttention
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "module_train_*.npz")))


def check(got, ref, what):
    got, ref = torch.as_tensor(got).double().cpu(), torch.as_tensor(ref).double()
    diff = got - ref
    rl = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    ma = diff.abs().max().item()
    bar = 2e-2 * min(1.0, max(ref.abs().max().item(), 1e-3))
    assert rl <= 1e-2 and ma <= bar, f"{what}: rel-L2 {rl:.3e}, max-abs {ma:.3e} (bar {bar:.3e})"


def build(d):
    cfg = json.loads(str(d["config"]))
    mod = DSALTAttention(cfg["d_model"], cfg["n_heads"], cfg["n_min"], cfg["n_max"], cfg["k_lmk"],
                         cfg["max_seq_len"], yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"],
                         qkv_bias=cfg["qkv_bias"], rope_base=cfg["rope_base"])
    with torch.no_grad():
        for name, p in mod.named_parameters():
            p.copy_(torch.from_numpy(d["p." + name]))
    return cfg, mod.to(DEV)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_module_train_matches_reference_golden(path):
    print(f"module train {os.path.basename(path)}", flush=True)
    d = np.load(path, allow_pickle=False)
    cfg, mod = build(d)
    mod.train()
    x = torch.from_numpy(d["x"]).to(DEV).requires_grad_()
    cu = torch.from_numpy(d["cu"]).to(DEV)
    w_cont, lmk_pos, lmk_logw = mod._train_selectors(x.detach(), cu, x.shape[0], DEV, d["cu"].tolist())
    for h in range(lmk_pos.shape[0]):
        for s in range(lmk_pos.shape[1]):
            assert sorted(lmk_pos[h, s].tolist()) == sorted(d["lmk_pos"][h, s].tolist())
    out, aux = mod(x, cu_seqlens=cu)
    # the selection the forward itself used (the module's default route) is the
    # reference's, set for set
    used = mod._last_selection[1].cpu()
    for h in range(used.shape[0]):
        for s in range(used.shape[1]):
            assert sorted(used[h, s].tolist()) == sorted(d["lmk_pos"][h, s].tolist())
    assert float(aux) == 0.0
    check(out.detach(), d["out"], "out")
    out.backward(torch.from_numpy(d["dout"]).to(DEV))
    check(x.grad, d["grad.x"], "grad x")
    for name, p in mod.named_parameters():
        check(p.grad, d["grad." + name], "grad " + name)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_module_eval_matches_oracle(path):
    print(f"module eval {os.path.basename(path)}", flush=True)
    d = np.load(path, allow_pickle=False)
    cfg, mod = build(d)
    mod.eval()
    x = torch.from_numpy(d["x"])
    cu = torch.from_numpy(d["cu"])
    with torch.no_grad():
        out, _ = mod(x.to(DEV), cu_seqlens=cu.to(DEV))
    params = {k[2:]: torch.from_numpy(d[k]).double() for k in d.files if k.startswith("p.")}
    ref, (w_sizes, lmk_pos) = orc.module_eval_forward(params, cfg, x.double(), d["cu"])
    check(out, ref, "eval out")
    # _last_P of sequence 0: dense softmax over the HARD set (rows sum to 1, zero off-set)
    P = mod._last_P.cpu()
    L0 = int(d["cu"][1])
    assert P.shape == (cfg["n_heads"], L0, L0)
    torch.testing.assert_close(P.sum(-1), torch.ones(cfg["n_heads"], L0), rtol=1e-4, atol=1e-4)
    mask = orc.hard_mask(L0, w_sizes[:L0], mod_lmk0(mod, x, cfg, L0))
    assert float(P.masked_select(~mask).abs().max()) == 0.0


def mod_lmk0(mod, x, cfg, L0):
    # landmarks of sequence 0 selected on sequence 0 alone (dsalt_attention.py:655-666)
    from dsalt.kernels.selectors import _compute_landmark_indices
    with torch.no_grad():
        xs = x[:L0].to(DEV)
        w = mod._window_sizes(xs, floor=True)
        lmk, _, _ = _compute_landmark_indices(xs, mod.v_proj.weight, mod._alpha().float(), w,
                                              torch.tensor([0, L0], dtype=torch.int32, device=DEV), mod.k_lmk,
                                              mod.n_min, L0, [0, L0], head_dim=mod.head_dim)
    return lmk[:, 0].cpu().numpy()


def test_module_rejects_cpu_and_unsupported_batched_input():
    mod = DSALTAttention(128, 2, 4, 40, 8, 256)
    x = torch.randn(64, 128)
    with pytest.raises(Exception, match="ROCm GPU"):
        mod(x, cu_seqlens=torch.tensor([0, 64], dtype=torch.int32))
    with pytest.raises(Exception, match="ROCm GPU"):
        mod(torch.randn(1, 64, 128))
    mod = mod.to(DEV)
    with pytest.raises(ValueError, match="one sequence"):
        mod(torch.randn(2, 64, 128, device=DEV))
    drop = DSALTAttention(128, 2, 4, 40, 8, 256, dropout=0.1).to(DEV).train()
    with pytest.raises(NotImplementedError, match="dropout"):
        drop(torch.randn(1, 64, 128, device=DEV))


def test_module_bf16_autocast_train_step():
    # a bf16 training step under autocast runs end to end and produces finite gradients
    torch.manual_seed(5)
    mod = DSALTAttention(256, 4, 8, 64, 16, 512).to(DEV).train()
    x = torch.randn(2 * 200, 256, device=DEV, requires_grad=True)
    cu = torch.tensor([0, 200, 400], dtype=torch.int32, device=DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, _ = mod(x, cu_seqlens=cu, cu_list=[0, 200, 400])
    out.float().square().mean().backward()
    for name, p in mod.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name
    assert mod.win_gate.weight.grad.abs().sum() > 0 and mod.alpha_w.grad.abs().sum() > 0


@pytest.mark.parametrize("T", [8192, 16384], ids=["c2", "c5"])
def test_fused_qkv_projection_equals_separate_at_headline_shapes(T):
    """At inference the module forms q, k and v with one GEMM over the concatenated weights
    (_fuse_qkv). At the d_model 1024 / 16-head shapes of configs 2 and 5 its columns are
    the three separate projections bit for bit, and so is the module's whole output."""
    print(f"fused qkv T={T}", flush=True)
    torch.manual_seed(11)
    mod = DSALTAttention(1024, 16, 32, 512, 64, 2048).to(DEV, torch.bfloat16).eval()
    mod._collect_last_P = False
    x = torch.randn(T, 1024, device=DEV).to(torch.bfloat16)
    L = 2048
    cu = torch.arange(0, T + 1, L, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        q, k, v = mod._project_qkv(x)
        assert q.data_ptr() + 1024 * 2 == k.data_ptr() and q.stride(0) == 3 * 1024  # one GEMM's columns
        assert torch.equal(q, mod.q_proj(x)) and torch.equal(k, mod.k_proj(x)) and torch.equal(v, mod.v_proj(x))
        fused, _ = mod(x, cu_seqlens=cu, cu_list=cu.tolist())
        try:
            DSALTAttention._fuse_qkv = False
            plain, _ = mod(x, cu_seqlens=cu, cu_list=cu.tolist())
        finally:
            DSALTAttention._fuse_qkv = True
    torch.cuda.synchronize()
    assert torch.equal(fused, plain)


def test_fused_qkv_projection_gqa_and_weight_updates():
    """The fused projection with grouped K/V heads (kv_dim < d_model) against the separate
    projections, before and after an in-place weight update (the cached concatenation is
    rebuilt), and the module's output with and without it."""
    print("fused qkv GQA", flush=True)
    torch.manual_seed(12)
    mod = DSALTAttention(512, 8, 16, 128, 16, 1024, n_kv_heads=2).to(DEV, torch.bfloat16).eval()
    mod._collect_last_P = False
    x = torch.randn(700, 512, device=DEV).to(torch.bfloat16)
    cu = torch.tensor([0, 300, 700], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        for step in range(2):
            q, k, v = mod._project_qkv(x)
            assert q.shape == (700, 512) and k.shape == (700, 128) and v.shape == (700, 128)
            for got, lin in ((q, mod.q_proj), (k, mod.k_proj), (v, mod.v_proj)):
                torch.testing.assert_close(got.float(), lin(x).float(), rtol=1e-2, atol=1e-2)
            mod.k_proj.weight.mul_(1.5)  # in place: the next call must see it
        mod.v_proj.weight.data.mul_(0.5)  # through .data: no version bump, so invalidate
        mod.invalidate_qkv_cache()
        _, _, v = mod._project_qkv(x)
        torch.testing.assert_close(v.float(), mod.v_proj(x).float(), rtol=1e-2, atol=1e-2)  # stale: 2x off
        fused, _ = mod(x, cu_seqlens=cu, cu_list=cu.tolist())
        try:
            DSALTAttention._fuse_qkv = False
            plain, _ = mod(x, cu_seqlens=cu, cu_list=cu.tolist())
        finally:
            DSALTAttention._fuse_qkv = True
    torch.cuda.synchronize()
    rel = float((fused.float() - plain.float()).norm() / plain.float().norm())
    assert rel < 1e-2, rel

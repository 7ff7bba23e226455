"""BASELINE config 1 on the GPU: the seed-0 module DSALTAttention(512, 8, 64, 256, 16,
max_seq_len=1024) in fp32 (the kernels compute fp32 inputs as fp16, as the reference's
do), x ~ N(0, 1) [1, 1024, 512] drawn after the module from the same seed, on the windows
and landmarks the module itself produces. Every row of the module output is compared with
the fp64 oracle fed the module's own selection (packed inference / HARD, packed training
/ SOFT, and the [1, T, d] dense variant), then the output projection. Bar (north star):
max-abs 2e-2 and relative L2 1e-2, absolute."""
import math

import pytest
import torch

import bench
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
MAX_ABS, REL_L2 = 2e-2, 1e-2


def _module():
    from dsalt.modules import DSALTAttention
    B, L, d_model, H, n_min, n_max, k_lmk, seed = bench.CONFIGS["c1"]
    torch.manual_seed(seed)
    mod = DSALTAttention(d_model, H, n_min, n_max, k_lmk, max_seq_len=L)
    x = torch.randn(B, L, d_model)
    params = {n: p.detach().double().clone() for n, p in mod.named_parameters()}
    mod = mod.to(DEV)
    mod._collect_last_P = False
    return mod, x, params, H, d_model // H


def _qkv(params, x, H, D, L):
    """q, k, v of the module in fp64 with RoPE at positions 0 .. L-1."""
    T = x.shape[0]
    q = (x @ params["q_proj.weight"].T).view(T, H, D)
    k = (x @ params["k_proj.weight"].T).view(T, H, D)
    v = (x @ params["v_proj.weight"].T).view(T, H, D)
    cos, sin = orc.rope_cache(L, D)
    c, s = cos[:T].unsqueeze(1), sin[:T].unsqueeze(1)
    return orc.rotate(q, c, s), orc.rotate(k, c, s), v


def _check(got, ref, what):
    diff = got.detach().double().cpu() - ref
    ma = diff.abs().max().item()
    rl = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    print(f"  {what}: max-abs {ma:.3e} rel-L2 {rl:.3e} (max |ref| {ref.abs().max().item():.3e})", flush=True)
    assert ma <= MAX_ABS and rl <= REL_L2, f"{what}: max-abs {ma:.3e}, rel-L2 {rl:.3e}"


def test_c1_packed_inference_on_module_selectors():
    print("c1 packed inference (HARD)", flush=True)
    mod, x, params, H, D = _module()
    mod.eval()
    xs = x[0].to(DEV)
    L = xs.shape[0]
    cu = torch.tensor([0, L], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        out, _ = mod(xs, cu_seqlens=cu, cu_list=[0, L])
    w, lmk = (t.cpu() for t in mod._last_selection)
    q, k, v = _qkv(params, x[0].double(), H, D, L)
    o, _ = orc.attention_hard(q, k, v, w, lmk, None, [0, L])
    _check(out, o.reshape(L, H * D) @ params["out_proj.weight"].T, "packed HARD module output")


def test_c1_packed_training_forward_on_module_selectors():
    print("c1 packed training forward (SOFT)", flush=True)
    mod, x, params, H, D = _module()
    mod.train()
    xs = x[0].to(DEV)
    L = xs.shape[0]
    cu = torch.tensor([0, L], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        w_cont, lmk, logw = mod._train_selectors(xs, cu, L, DEV, [0, L])
        out, _ = mod(xs, cu_seqlens=cu, cu_list=[0, L])
    assert torch.equal(mod._last_selection[1], lmk)  # the forward used these landmarks
    q, k, v = _qkv(params, x[0].double(), H, D, L)
    o, _ = orc.attention_soft(q, k, v, w_cont.double().cpu(), lmk.cpu(), logw.double().cpu(), [0, L],
                              tau_win=mod.tau_win, win_edge=float(mod.win_edge))
    _check(out, o.reshape(L, H * D) @ params["out_proj.weight"].T, "packed SOFT module output")


def test_c1_batched_inference_on_module_selectors():
    print("c1 [1, T, d] inference (dense variant)", flush=True)
    mod, x, params, H, D = _module()
    mod.eval()
    L = x.shape[1]
    with torch.no_grad():
        out, _ = mod(x.to(DEV))
    w_cont, lmk = mod._last_selection
    x64 = x[0].double()
    q, k, v = _qkv(params, x64, H, D, L)
    scores, _, _ = orc.hybrid_scores(x64, params["v_proj.weight"], torch.sigmoid(params["alpha_w"]), H, D)
    sel = torch.zeros(H, L, dtype=torch.bool)
    for h in range(H):
        p = lmk[h, 0].cpu()
        sel[h, p[p >= 0]] = True
    w_lmk = torch.log(torch.sigmoid(scores / mod.tau_lmk).clamp(min=1e-20)).t()
    lb = torch.where(sel, w_lmk, torch.full_like(w_lmk, float("-inf")))
    o, _ = orc.attention_dense(q, k, v, w_cont.double().cpu(), lb, mod.tau_win, float(mod.win_edge))
    _check(out[0], o.reshape(L, H * D) @ params["out_proj.weight"].T, "dense module output")

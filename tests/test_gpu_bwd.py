"""Backward parity: HIP dQ/dK/dV, landmark-bias gradient and (SOFT) window gradient
against fp64 autograd through the CPU oracle, on the same bf16 inputs and upstream
gradient. Tolerance: max-abs 2e-2 and relative L2 1e-2; the
landmark-bias and window gradients are sums over many pairs and are compared with
the same relative-L2 bar and a max-abs bar scaled by their magnitude."""
import math

import numpy as np
import pytest
import torch

import dsalt._hip as hip
from oracle import dsalt_oracle as orc
from test_gpu_fwd import close, make_inputs, summed_grad_bar

pytestmark = pytest.mark.gpu


def run_case(mode, lens, H, D, k, seed, n_min, n_max, kind="random", dtype=torch.bfloat16,
             tau=1.0, edge=4.0, grad_dtype=torch.float32, out_dtype=torch.float32):
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed, dtype=dtype, n_min=n_min,
                                             n_max=n_max, lmk_kind=kind)
    g = torch.Generator().manual_seed(seed + 1000)
    T = q.shape[0]
    dout = torch.randn(T, H, D, generator=g).to(dtype)
    dev = torch.device("cuda", 0)
    qd, kd, vd, dod = (t.to(dev) for t in (q, kk, v, dout))
    posd = pos.to(dev) if k > 0 else None
    biasd = bias.to(dev) if k > 0 else None
    scale = 1.0 / math.sqrt(D)
    out, lse = hip.fwd(mode, qd, kd, vd, w.to(dev), posd, biasd, cu.to(dev), scale, tau, edge,
                       out_dtype=out_dtype)
    dq, dk, dv, dbias, dw = hip.bwd(mode, qd, kd, vd, out, lse, dod, w.to(dev), posd, biasd, cu.to(dev),
                                    scale, tau, edge, need_dw=(mode == hip.MODE_SOFT), grad_dtype=grad_dtype)
    torch.cuda.synchronize()

    q64, k64, v64 = (t.double().requires_grad_() for t in (q, kk, v))
    b64 = bias.double().requires_grad_() if k > 0 else None
    if mode == hip.MODE_HARD:
        o, _ = orc.attention_hard(q64, k64, v64, w, pos if k > 0 else None, b64, cu.tolist())
        w64 = None
    else:
        w64 = w.double().requires_grad_()
        o, _ = orc.attention_soft(q64, k64, v64, w64, pos if k > 0 else None, b64, cu.tolist(),
                                  tau_win=tau, win_edge=edge)
    (o * dout.double()).sum().backward()
    for name, got, ref in (("dq", dq, q64.grad), ("dk", dk, k64.grad), ("dv", dv, v64.grad)):
        if grad_dtype == torch.float32:
            close(got.float().cpu(), ref, name)
        else:  # 16-bit O and gradients: never looser than the absolute bar
            close(got.float().cpu(), ref, name, max_abs=2e-2 * min(1.0, max(ref.abs().max().item(), 1e-3)))
    if k > 0:
        ref = b64.grad.clone()
        if mode == hip.MODE_SOFT:  # slots with lmk_logw = -inf carry no gradient
            ref = torch.where(torch.isfinite(bias.double()), ref, torch.zeros_like(ref))
        close(dbias.cpu(), ref, "d_lmk_bias", max_abs=summed_grad_bar(ref))
    if mode == hip.MODE_SOFT:
        close(dw.cpu(), w64.grad, "d_w", max_abs=summed_grad_bar(w64.grad))


CASES = [
    # lens, H, D, k, n_min, n_max, kind
    ([1, 2, 3, 130], 2, 64, 5, 1, 9, "random"),
    ([300, 77, 513], 3, 128, 20, 8, 96, "random"),
    ([200, 0, 129], 2, 64, 100, 4, 40, "messy"),
    ([64, 191], 2, 128, 0, 1, 300, "random"),
    ([700], 4, 64, 16, 64, 256, "random"),
]


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_bwd_matches_oracle(mode, case):
    lens, H, D, k, n_min, n_max, kind = CASES[case]
    print(f"bwd case={case} mode={mode} lens={lens} H={H} D={D} k={k}", flush=True)
    run_case(mode, lens, H, D, k, seed=20 + case, n_min=n_min, n_max=n_max, kind=kind)


def test_bwd_f16_soft_edge_params():
    print("bwd f16 soft tau=0.7 edge=3", flush=True)
    run_case(hip.MODE_SOFT, [333, 90], 2, 64, 12, seed=40, n_min=2, n_max=60, dtype=torch.float16, tau=0.7,
             edge=3.0)


@pytest.mark.parametrize("tau,edge,D", [(0.2, 4.0, 64), (0.25, 6.0, 128), (3.0, 1.0, 64)],
                         ids=["tau0.2-d64", "tau0.25-edge6-d128", "tau3-edge1-d64"])
def test_bwd_soft_edge_factor_paths(tau, edge, D):
    # the dq pass factors the edge's exp(-z) per lane and slot while (edge + 17) / tau < 80
    # and takes a per-element exp otherwise (tau 0.2 and 0.25 with edge 6)
    print(f"bwd soft tau={tau} edge={edge} D={D}", flush=True)
    run_case(hip.MODE_SOFT, [400, 130], 2, D, 8, seed=44, n_min=3, n_max=120, tau=tau, edge=edge)


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
def test_bwd_16bit_gradient_outputs(mode):
    print(f"bwd bf16 outputs mode={mode}", flush=True)
    run_case(mode, [257, 300], 4, 128, 16, seed=41, n_min=8, n_max=200, grad_dtype=torch.bfloat16,
             out_dtype=torch.bfloat16)


@pytest.mark.parametrize("mode,D,k", [(hip.MODE_SOFT, 64, 1024), (hip.MODE_HARD, 128, 300)],
                         ids=["soft-d64-k1024", "hard-d128-k300"])
def test_bwd_many_landmarks(mode, D, k):
    # landmark slots beyond 64 and up to DSALT_MAX_K_LMK: several slot groups of lmk_kv,
    # k_pad not a multiple of 64 slots per tile pair, a sequence shorter than k
    print(f"bwd many landmarks mode={mode} D={D} k={k}", flush=True)
    run_case(mode, [900, 45, 500], 2, D, k, seed=33, n_min=4, n_max=160)


@pytest.mark.parametrize("mode,D", [(hip.MODE_HARD, 64), (hip.MODE_SOFT, 64), (hip.MODE_SOFT, 128)],
                         ids=["hard-d64", "soft-d64", "soft-d128"])
def test_bwd_many_sequences(mode, D):
    # more than 64 sequences (block lookups scan cu_seqlens 64 entries at a time), empty
    # ones, lengths that cross the 64-query dq blocks and 64 / 128-key kv blocks anywhere
    rng = np.random.default_rng(17)
    lens = [int(x) for x in rng.integers(0, 150, size=90)]
    lens[5] = lens[70] = lens[89] = 0
    lens[66] = 420
    print(f"bwd many sequences mode={mode} D={D}", flush=True)
    run_case(mode, lens, 2, D, 7, seed=17, n_min=2, n_max=60)


def test_bwd_c3_packing():
    # 8 sequences, lengths numpy.random.seed(2); randint(256, 2049, 8)
    np.random.seed(2)
    lens = [int(x) for x in np.random.randint(256, 2049, 8)]
    assert sum(lens) == 9290
    print(f"bwd c3 lens={lens}", flush=True)
    run_case(hip.MODE_SOFT, lens, 16, 64, 64, seed=2, n_min=32, n_max=512)


def test_bwd_deterministic():
    lens, H, D, k = [400, 123], 4, 64, 24
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, hip.MODE_SOFT, 50, n_min=8, n_max=120)
    dev = torch.device("cuda", 0)
    dout = torch.randn_like(q.float()).to(torch.bfloat16).to(dev)
    args = [t.to(dev) for t in (q, kk, v)]
    out, lse = hip.fwd(hip.MODE_SOFT, *args, w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev), 0.125)
    r1 = hip.bwd(hip.MODE_SOFT, *args, out, lse, dout, w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev), 0.125,
                 need_dw=True)
    r2 = hip.bwd(hip.MODE_SOFT, *args, out, lse, dout, w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev), 0.125,
                 need_dw=True)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)

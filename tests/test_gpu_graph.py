"""The C-ABI calls under HIP graph capture. The library's launches allocate nothing, clear
no memory with hipMemsetAsync and run on the caller's stream, so a caller may capture
them: the module's inference chain (dsalt_select_hybrid with the k rotation, then the
HARD forward rotating q on load) and the SOFT backward are captured once and replayed
several times, with fresh inputs copied into the captured buffers and eager work and
synchronisations between the replays. Every replay must equal eager calls on the same
inputs, bit for bit."""
import math

import numpy as np
import pytest
import torch

from dsalt import _hip
from dsalt.kernels.window_utils import build_rope_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _capture(fn):
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("lens,k_lmk", [([700, 0, 333, 1100], 32), ([9000, 1500], 64)],
                         ids=["short", "long-chunked"])
def test_inference_chain_replays_match_eager(lens, k_lmk):
    print(f"graph inference chain lens={lens}", flush=True)
    H, D, d = 8, 64, 256
    cu_list = [0] + np.cumsum(lens).tolist()
    T = cu_list[-1]
    cu = torch.tensor(cu_list, dtype=torch.int32, device=DEV)
    L = max(lens)
    x = torch.empty(T, d, device=DEV, dtype=torch.bfloat16)
    q, k, v = (torch.empty(T, H, D, device=DEV, dtype=torch.bfloat16) for _ in range(3))
    logit = torch.empty(T, device=DEV, dtype=torch.bfloat16)
    alpha = torch.rand(H, device=DEV)
    cos, sin = build_rope_cache(L + 1, D, DEV)
    gate = (logit, 16.0, 400.0)

    def fill(seed):
        g = torch.Generator(device="cpu").manual_seed(seed)
        for t in (x, q, k, v):
            t.copy_(torch.randn(t.shape, generator=g).to(DEV, t.dtype))
        logit.copy_((torch.randn(T, generator=g) * 2).to(DEV, logit.dtype))

    fill(0)
    sel = _hip.SelectHybridLauncher(x, v, alpha, H, None, cu, k_lmk, max_seqlen=L, gate=gate, norms_f32=False,
                                    rope_k=(k, cos, sin, cu))
    fwd = _hip.FwdLauncher(_hip.MODE_HARD, q, sel.k_out, v, sel.w_out, sel.out, None, cu, 1 / math.sqrt(D),
                           rope=(cos, sin))
    graph = _capture(lambda: (sel(), fwd()))
    for seed in (1, 2, 3):
        fill(seed)
        w_e, lmk_e, k_e = _hip.select_hybrid(x, v, alpha, H, None, cu, k_lmk, max_seqlen=L, gate=gate,
                                             norms_f32=False, rope_k=(k, cos, sin, cu))
        o_e, l_e = _hip.fwd(_hip.MODE_HARD, q, k_e, v, w_e, lmk_e, None, cu, 1 / math.sqrt(D), rope=(cos, sin))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(sel.w_out, w_e) and torch.equal(sel.out, lmk_e) and torch.equal(sel.k_out, k_e)
        assert torch.equal(fwd.out, o_e)
        assert torch.equal(torch.nan_to_num(fwd.lse), torch.nan_to_num(l_e))
        assert bool((lmk_e >= 0).any())


def test_soft_backward_replays_match_eager():
    print("graph SOFT backward", flush=True)
    from test_gpu_fwd import make_inputs
    q, k, v, w, pos, bias, cu = make_inputs([600, 1, 423], 4, 64, 16, _hip.MODE_SOFT, seed=11, n_min=8, n_max=200)
    q, k, v, w, pos, bias, cu = (t.to(DEV) for t in (q, k, v, w, pos, bias, cu))
    scale = 1 / math.sqrt(64)
    out, lse = _hip.fwd(_hip.MODE_SOFT, q, k, v, w, pos, bias, cu, scale)
    dout = torch.empty_like(q)
    bwd = _hip.BwdLauncher(_hip.MODE_SOFT, q, k, v, out, lse, dout, w, pos, bias, cu, scale, need_dw=True)
    dout.copy_(torch.randn(q.shape, device=DEV).to(q.dtype))
    graph = _capture(bwd)
    for seed in (4, 5, 6):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        dout.copy_(torch.randn(q.shape, generator=gen).to(DEV, q.dtype))
        ref = _hip.bwd(_hip.MODE_SOFT, q, k, v, out, lse, dout, w, pos, bias, cu, scale, need_dw=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(bwd.results, ref):
            assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want))


def test_module_eval_forward_replays_match_eager():
    """DSALTAttention's packed inference forward (bf16, host cu_list, _last_P off) captured
    whole - projections, the two-launch selection, the forward, out_proj - and replayed."""
    print("graph module eval forward", flush=True)
    from dsalt.modules import DSALTAttention
    torch.manual_seed(7)
    mod = DSALTAttention(512, 8, 16, 300, 32, max_seq_len=1024).to(DEV).to(torch.bfloat16).eval()
    mod._collect_last_P = False
    lens = [600, 424, 1000]
    cu_list = [0] + np.cumsum(lens).tolist()
    cu = torch.tensor(cu_list, dtype=torch.int32, device=DEV)
    x = torch.randn(cu_list[-1], 512, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        mod(x, cu_seqlens=cu, cu_list=cu_list)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out_g, _ = mod(x, cu_seqlens=cu, cu_list=cu_list)
        for seed in (1, 2, 3):
            gen = torch.Generator(device="cpu").manual_seed(seed)
            x.copy_(torch.randn(x.shape, generator=gen).to(DEV, x.dtype))
            out_e, _ = mod(x, cu_seqlens=cu, cu_list=cu_list)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_e)

"""dsalt_bwd_noalloc (the backward with its scratch in a static device array, no
allocation) against dsalt_bwd with a caller workspace, through the C ABI: the kernels
are deterministic and atomic-free, so the results must be bit-identical. Two calls in a
row, the second on a smaller input, so the second runs on scratch the first left
behind; the caller's workspace fields are nulled to show they are not used."""
import ctypes
import math

import numpy as np
import pytest
import torch

import dsalt._hip as hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _case(lens, H, D, k, mode, seed, n_min, n_max):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T, S = int(cu[-1]), len(lens)
    q, kk, v = (torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    w = n_min + torch.rand(T, generator=g) * (n_max - n_min)
    if mode == hip.MODE_HARD:
        w = w.floor()
    pos = np.full((H, S, k), -1, dtype=np.int64)
    for h in range(H):
        for s, L in enumerate(lens):
            c = rng.choice(L, size=min(k, L), replace=False)
            pos[h, s, :len(c)] = c
    pos = torch.from_numpy(pos).to(DEV)
    bias = torch.nn.functional.logsigmoid(torch.randn(H, S, k, generator=g)).to(DEV)
    dout = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    return q, kk, v, w.to(DEV), pos, bias, cu.to(DEV), dout


def _both(mode, q, kk, v, w, pos, bias, cu, dout):
    scale = 1.0 / math.sqrt(q.shape[-1])
    out, lse = hip.fwd(mode, q, kk, v, w, pos, bias, cu, scale)
    need_dw = mode == hip.MODE_SOFT
    ref = hip.BwdLauncher(mode, q, kk, v, out, lse, dout, w, pos, bias, cu, scale, need_dw=need_dw)
    ref()
    nal = hip.BwdLauncher(mode, q, kk, v, out, lse, dout, w, pos, bias, cu, scale, need_dw=need_dw)
    nal.args.workspace, nal.args.workspace_bytes = None, 0
    rc = hip.lib().dsalt_bwd_noalloc(ctypes.byref(nal.args), hip.stream_handle(DEV))
    assert rc == 0, hip.lib().dsalt_last_error().decode()
    torch.cuda.synchronize()
    return ref.results, nal.results


@pytest.mark.parametrize("mode,D", [(hip.MODE_SOFT, 64), (hip.MODE_HARD, 128)], ids=["soft-d64", "hard-d128"])
def test_noalloc_matches_workspace_backward(mode, D):
    for lens, H, k, seed in (([700, 333, 1100], 4, 16, 3), ([200, 57], 2, 8, 4)):  # second call smaller
        print(f"noalloc bwd mode={mode} D={D} lens={lens}", flush=True)
        ref, got = _both(mode, *_case(lens, H, D, k, mode, seed, 8, 300))
        for name, a, b in zip(("dq", "dk", "dv", "d_bias", "d_w"), ref, got):
            if a is None:
                assert b is None
                continue
            assert torch.equal(a, b), f"{name} differs from the workspace backward"


def test_noalloc_rejects_oversized_scratch():
    # sizes whose scratch exceeds the static array: a clear error, nothing launched
    a = hip.BwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs, a.n_heads, a.head_dim, a.k_lmk = 0, 0, 1 << 20, 1, 64, 128, 1024
    rc = hip.lib().dsalt_bwd_noalloc(ctypes.byref(a), None)
    assert rc == 2 and b"above the static" in hip.lib().dsalt_last_error()

"""Grouped-query attention in the kernels: K/V with n_kv < H heads are read in place
(query head h reads K/V head h // (H // n_kv)) by the HARD / SOFT forward and backward
and by the dense variant; dK/dV come back per query head and are summed over each group.
Reference: the fp64 oracle on K/V repeated to H heads (dsalt_attention.py:254-268's
repeat), whose autograd sums the group gradients itself. Bar (north star): max-abs 2e-2
and relative L2 1e-2 (the summed d_lmk_bias / d_w with the max-abs bar scaled by their
largest value, as in test_gpu_bwd)."""
import math

import pytest
import torch

import dsalt._hip as hip
from oracle import dsalt_oracle as orc
from test_gpu_fwd import close, make_inputs, summed_grad_bar

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def rep_kv(t, n_rep):
    return t.repeat_interleave(n_rep, dim=1)


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
@pytest.mark.parametrize("H,n_kv,D", [(4, 2, 64), (6, 2, 128), (4, 1, 64)], ids=["4-2-d64", "6-2-d128", "4-1-d64"])
def test_gqa_fwd_bwd_match_oracle(mode, H, n_kv, D):
    print(f"gqa mode={mode} H={H} n_kv={n_kv} D={D}", flush=True)
    lens = [150, 333, 40]
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, 9, mode, seed=60 + H + D, n_min=4, n_max=90)
    n_rep = H // n_kv
    kk, v = kk[:, ::n_rep].contiguous(), v[:, ::n_rep].contiguous()  # [T, n_kv, D]
    T = q.shape[0]
    dout = torch.randn(T, H, D, generator=torch.Generator().manual_seed(7)).to(q.dtype)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, kk, v, dout))
    scale = 1.0 / math.sqrt(D)
    out, lse = hip.fwd(mode, qd, kd, vd, w.to(DEV), pos.to(DEV), bias.to(DEV), cu.to(DEV), scale,
                       out_dtype=torch.float32)
    dq, dk, dv, dbias, dw = hip.bwd(mode, qd, kd, vd, out, lse, dod, w.to(DEV), pos.to(DEV), bias.to(DEV),
                                    cu.to(DEV), scale, need_dw=(mode == hip.MODE_SOFT), grad_dtype=torch.float32)
    dk, dv = hip.group_sum(dk, n_kv), hip.group_sum(dv, n_kv)
    torch.cuda.synchronize()
    assert dk.shape == kk.shape and dv.shape == v.shape

    q64 = q.double().requires_grad_()
    k64, v64 = kk.double().requires_grad_(), v.double().requires_grad_()
    b64 = bias.double().requires_grad_()
    if mode == hip.MODE_HARD:
        o, l_ref = orc.attention_hard(q64, rep_kv(k64, n_rep), rep_kv(v64, n_rep), w, pos, b64, cu.tolist())
        w64 = None
    else:
        w64 = w.double().requires_grad_()
        o, l_ref = orc.attention_soft(q64, rep_kv(k64, n_rep), rep_kv(v64, n_rep), w64, pos, b64, cu.tolist())
    close(out.cpu(), o.detach(), "O")
    (o * dout.double()).sum().backward()
    close(dq.cpu(), q64.grad, "dq")
    close(dk.cpu(), k64.grad, "dk")
    close(dv.cpu(), v64.grad, "dv")
    ref_b = b64.grad if mode == hip.MODE_HARD else torch.where(torch.isfinite(bias.double()), b64.grad,
                                                                 torch.zeros_like(b64.grad))
    close(dbias.cpu(), ref_b, "d_lmk_bias", max_abs=summed_grad_bar(ref_b))
    if mode == hip.MODE_SOFT:
        close(dw.cpu(), w64.grad, "d_w", max_abs=summed_grad_bar(w64.grad))


@pytest.mark.parametrize("H,n_kv,D", [(4, 2, 64), (2, 1, 128)], ids=["4-2-d64", "2-1-d128"])
def test_gqa_dense_matches_oracle(H, n_kv, D):
    print(f"gqa dense H={H} n_kv={n_kv} D={D}", flush=True)
    T = 150
    g = torch.Generator().manual_seed(70 + D)
    n_rep = H // n_kv
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    kk = torch.randn(T, n_kv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, n_kv, D, generator=g).to(torch.bfloat16)
    w = 2.0 + 30.0 * torch.rand(T, generator=g)
    s = torch.randn(T, H, generator=g)
    lb = torch.log(torch.sigmoid(s / 2.0)).t().contiguous()
    lb = torch.where(torch.rand(H, T, generator=g) < 0.2, lb, torch.full_like(lb, float("-inf")))
    dout = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    out, lse = hip.dense_fwd(q.to(DEV), kk.to(DEV), v.to(DEV), w.to(DEV), lb.to(DEV), scale, out_dtype=torch.float32)
    dq, dk, dv, dlb, dw = hip.dense_bwd(q.to(DEV), kk.to(DEV), v.to(DEV), out, lse, dout.to(DEV), w.to(DEV),
                                        lb.to(DEV), scale, grad_dtype=torch.float32)
    dk, dv = hip.group_sum(dk, n_kv), hip.group_sum(dv, n_kv)
    torch.cuda.synchronize()
    q64, k64, v64 = q.double().requires_grad_(), kk.double().requires_grad_(), v.double().requires_grad_()
    w64, lb64 = w.double().requires_grad_(), lb.double().requires_grad_()
    o, _ = orc.attention_dense(q64, rep_kv(k64, n_rep), rep_kv(v64, n_rep), w64, lb64, 1.0, 4.0, scale)
    close(out.cpu(), o.detach(), "O")
    o.backward(dout.double())
    close(dq.cpu(), q64.grad, "dq")
    close(dk.cpu(), k64.grad, "dk")
    close(dv.cpu(), v64.grad, "dv")
    close(dlb.cpu(), lb64.grad, "d_lmk_bias", max_abs=summed_grad_bar(lb64.grad))
    close(dw.cpu(), w64.grad, "d_w", max_abs=summed_grad_bar(w64.grad))


def test_gqa_rejects_non_dividing_heads():
    q = torch.randn(64, 6, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(64, 4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.full((64,), 8.0, device=DEV)
    cu = torch.tensor([0, 64], dtype=torch.int32, device=DEV)
    with pytest.raises(hip.DsaltError, match="n_kv dividing H"):
        hip.fwd(hip.MODE_HARD, q, k, k, w, None, None, cu, 0.125)

"""The reference-compatible entry points on the GPU: dsalt.kernels.dsalt_triton_attention,
dsalt.kernels.dsalt_triton_train.dsalt_triton_train_attention (autograd forward and
backward), dsalt.kernels.dsalt_triton_backward and the selector helpers, against the
CPU oracle. Output/gradient conventions follow the reference: O is returned as fp32,
gradients in q's dtype (fp32 inputs compute as fp16 and get fp32 gradients)."""
import math

import numpy as np
import pytest
import torch

from dsalt.kernels import dsalt_triton_attention, dsalt_triton_backward
from dsalt.kernels.dsalt_triton_train import dsalt_triton_train_attention
from dsalt.kernels.selectors import _build_landmark_kv, _build_seq_block_map, _compute_landmark_indices
from oracle import dsalt_oracle as orc
from test_gpu_fwd import close, make_inputs, summed_grad_bar

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


SUMMED = ("d_bias", "d_logw", "d_w")  # sums over the queries of a landmark slot / heads and edge keys


def _grad_bar(ref):
    return 2e-2 * min(1.0, max(ref.abs().max().item(), 1e-3))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32-as-fp16"])
def test_dsalt_triton_attention_autograd(dtype):
    print(f"api hard {dtype}", flush=True)
    lens, H, D, k = [190, 333], 4, 64, 12
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, 0, seed=60, n_min=8, n_max=100)
    q, kk, v = (t.to(dtype) for t in (q, kk, v))
    g = torch.Generator().manual_seed(61)
    dout = torch.randn(q.shape, generator=g)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, kk, v))
    bd = bias.to(DEV).requires_grad_()
    out = dsalt_triton_attention(qd, kd, vd, pos.to(DEV), bd, w.to(DEV), cu.to(DEV))
    assert out.dtype == torch.float32 and out.shape == q.shape
    out.backward(dout.to(DEV))
    assert qd.grad.dtype == dtype and bd.grad.dtype == bias.dtype  # autograd casts to the input dtype

    cdt = torch.float16 if dtype == torch.float32 else dtype  # the kernels' compute dtype
    q64, k64, v64 = (t.to(cdt).double().requires_grad_() for t in (q, kk, v))
    b64 = bias.double().requires_grad_()
    o, _ = orc.attention_hard(q64, k64, v64, w, pos, b64, cu.tolist())
    (o * dout.to(cdt).double()).sum().backward()
    close(out.detach().cpu(), o.detach(), "out")
    for name, got, ref in (("dq", qd.grad, q64.grad), ("dk", kd.grad, k64.grad), ("dv", vd.grad, v64.grad),
                           ("d_bias", bd.grad, b64.grad)):
        close(got.float().cpu(), ref, name, max_abs=summed_grad_bar(ref) if name in SUMMED else _grad_bar(ref))


def test_dsalt_triton_train_attention_autograd():
    print("api train", flush=True)
    lens, H, D, k = [257, 64, 401], 3, 128, 16
    q, kk, v, w, pos, logw, cu = make_inputs(lens, H, D, k, 1, seed=62, n_min=4, n_max=90)
    g = torch.Generator().manual_seed(63)
    dout = torch.randn(q.shape, generator=g)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, kk, v))
    lw = logw.to(DEV).requires_grad_()
    wd = w.to(DEV).requires_grad_()
    out = dsalt_triton_train_attention(qd, kd, vd, pos.to(DEV), lw, wd, cu.to(DEV), tau_win=1.0, win_edge=4.0,
                                       n_max=90, cu_list=cu.tolist())
    assert out.dtype == torch.float32
    out.backward(dout.to(DEV))

    q64, k64, v64 = (t.double().requires_grad_() for t in (q, kk, v))
    l64 = logw.double().requires_grad_()
    w64 = w.double().requires_grad_()
    o, _ = orc.attention_soft(q64, k64, v64, w64, pos, l64, cu.tolist())
    (o * dout.to(torch.bfloat16).double()).sum().backward()
    close(out.detach().cpu(), o.detach(), "out")
    l_ref = torch.where(torch.isfinite(logw.double()), l64.grad, torch.zeros_like(l64.grad))
    for name, got, ref in (("dq", qd.grad, q64.grad), ("dk", kd.grad, k64.grad), ("dv", vd.grad, v64.grad),
                           ("d_logw", lw.grad, l_ref), ("d_w", wd.grad, w64.grad)):
        close(got.float().cpu(), ref, name, max_abs=summed_grad_bar(ref) if name in SUMMED else _grad_bar(ref))


def test_dsalt_triton_backward_signature():
    print("api dsalt_triton_backward", flush=True)
    lens, H, D, k = [300], 2, 64, 8
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, 0, seed=64, n_min=8, n_max=64)
    from dsalt import _hip
    qd, kd, vd = (t.to(DEV) for t in (q, kk, v))
    out, lse = _hip.fwd(0, qd, kd, vd, w.to(DEV), pos.to(DEV), bias.to(DEV), cu.to(DEV), 1 / math.sqrt(D),
                        out_dtype=torch.float32)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(65))
    sbm, nblk = _build_seq_block_map(cu, 64, DEV, cu.tolist())
    lk, lv = _build_landmark_kv(kd, vd, pos.to(DEV), cu.to(DEV), k, H, D)
    dq, dk, dv, db = dsalt_triton_backward(dout.to(DEV), qd, kd, vd, out, lse, lk, lv, pos.to(DEV), bias.to(DEV),
                                           w.to(DEV), cu.to(DEV), 1 / math.sqrt(D), sbm, nblk, 64, 32, 64)
    assert dq.dtype == dk.dtype == dv.dtype == db.dtype == torch.float32
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, kk, v))
    b64 = bias.double().requires_grad_()
    o, _ = orc.attention_hard(q64, k64, v64, w, pos, b64, cu.tolist())
    (o * dout.to(torch.bfloat16).double()).sum().backward()
    for name, got, ref in (("dq", dq, q64.grad), ("dk", dk, k64.grad), ("dv", dv, v64.grad), ("d_bias", db, b64.grad)):
        close(got.cpu(), ref, name, max_abs=summed_grad_bar(ref) if name in SUMMED else _grad_bar(ref))


def test_selector_helpers_match_reference_semantics():
    # _compute_landmark_indices on the GPU: same sets as the oracle (selectors.py:75-134)
    g = torch.Generator().manual_seed(66)
    lens = [300, 128, 40]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T, d, H, dh, k = int(cu[-1]), 256, 4, 64, 24
    x = torch.randn(T, d, generator=g)
    W = torch.randn(H * dh, d, generator=g) / 16
    alpha = torch.rand(H, generator=g)
    w = (torch.rand(T, generator=g) * 60 + 1).floor()
    lmk, z_x, z_v = _compute_landmark_indices(x.to(DEV), W.to(DEV), alpha.to(DEV), w.to(DEV), cu.to(DEV), k, 1, T,
                                              cu.tolist(), head_dim=dh)
    scores, _, _ = orc.hybrid_scores(x.to(DEV).cpu(), W, alpha, H, dh)
    # the GPU scores come from the same formula; compare selections as sets on GPU scores
    from dsalt.kernels.landmark_tokens_ker import hybrid_scores_per_head
    s_gpu, _, _ = hybrid_scores_per_head(x.to(DEV), W.to(DEV), alpha.to(DEV), H, dh)
    torch.testing.assert_close(s_gpu.cpu(), scores, rtol=1e-4, atol=1e-4)
    ref = orc.select_landmarks(s_gpu.cpu().numpy(), w.numpy(), cu.numpy(), k)
    np.testing.assert_array_equal(lmk.cpu().numpy(), ref)
    lk, lv = _build_landmark_kv(x.view(T, H, 64).to(DEV).to(torch.bfloat16), x.view(T, H, 64).to(DEV).to(torch.bfloat16),
                                lmk, cu.to(DEV), k, H, 64)
    assert lk.shape == (H, 3, k, 64)

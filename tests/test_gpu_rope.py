"""The module's RoPE on the GPU (dsalt_rope, window_utils.py:73-88 as called by
dsalt_attention.py:570-585) against the CPU oracle: positions from cu_seqlens,
per-token tables, in-place use, rows past the table, and the backward against fp64
autograd of the formula. The kernel computes in fp32 and rounds once; the oracle in
float64 and rounds once, so 16-bit results agree bit for bit except where the fp32
result sits on a rounding boundary (one ulp of the 16-bit type)."""
import math

import numpy as np
import pytest
import torch

from dsalt import _hip
from dsalt.kernels.window_utils import apply_rotary_emb, apply_rotary_emb_packed, build_rope_cache
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _case(lens, Hq, Hk, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    cu = [0] + np.cumsum(lens).tolist()
    T = cu[-1]
    q = torch.randn(T, Hq, D, generator=g).to(dtype)
    k = torch.randn(T, Hk, D, generator=g).to(dtype)
    cos, sin = build_rope_cache(max(lens) + 3, D, torch.device("cpu"), base=10000.0, scale=1.5)
    return q, k, cos, sin, cu


def _ulp_close(got, ref, dtype):
    if dtype == torch.float32:
        err = (got.double() - ref.double()).abs().max().item()
        assert err < 1e-5, err
        return
    eq = (got == ref).float().mean().item()
    assert eq > 0.999, f"only {eq:.5f} of the elements are bit-identical"
    ulp = (ref.float().abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)).clamp(min=1e-30)
    assert ((got.float() - ref.float()).abs() <= ulp * 1.01).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
def test_rope_forward_matches_oracle(dtype):
    print(f"rope fwd {dtype}", flush=True)
    q, k, cos, sin, cu = _case([700, 1, 333, 1024], 16, 4, 64, dtype, 80)
    cu_t = torch.tensor(cu, dtype=torch.int32)
    oq, ok = _hip.rope(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV), cu_t.to(DEV))
    rq, rk = orc.rope(q, k, cos, sin, orc.seq_positions(cu))
    _ulp_close(oq.cpu(), rq, dtype)
    _ulp_close(ok.cpu(), rk, dtype)


def test_rope_per_token_inplace_and_past_table():
    q, k, cos, sin, cu = _case([300, 200], 4, 4, 128, torch.bfloat16, 81)
    T = cu[-1]
    pos = orc.seq_positions(cu)
    # per-token tables (the module's rope_cs), in place
    qd, kd = q.to(DEV), k.to(DEV)
    _hip.rope(qd, kd, cos[pos].to(DEV), sin[pos].to(DEV), None, q_out=qd, k_out=kd)
    rq, rk = orc.rope(q, k, cos, sin, pos)
    _ulp_close(qd.cpu(), rq, torch.bfloat16)
    _ulp_close(kd.cpu(), rk, torch.bfloat16)
    # a 300-token sequence with a 250-row table: rows past it give NaN, the rest is exact
    oq, _ = _hip.rope(q.to(DEV), k.to(DEV), cos[:250].to(DEV), sin[:250].to(DEV),
                      torch.tensor(cu, dtype=torch.int32, device=DEV))
    bad = (pos >= 250)
    assert torch.isnan(oq.cpu()[bad].float()).all() and not torch.isnan(oq.cpu()[~bad].float()).any()
    assert T == 500


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_rope_backward_matches_autograd(dtype):
    q, k, cos, sin, cu = _case([400, 129], 8, 2, 64, dtype, 82)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=DEV)
    g = torch.Generator().manual_seed(83)
    gq, gk = torch.randn(q.shape, generator=g), torch.randn(k.shape, generator=g)
    qd, kd = q.to(DEV).requires_grad_(), k.to(DEV).requires_grad_()
    oq, ok = apply_rotary_emb_packed(qd, kd, cos.to(DEV), sin.to(DEV), cu_t)
    ((oq.float() * gq.to(DEV)).sum() + (ok.float() * gk.to(DEV)).sum()).backward()
    pos = orc.seq_positions(cu)
    q64, k64 = q.double().requires_grad_(), k.double().requires_grad_()
    c = cos[pos].to(dtype).double().unsqueeze(1)
    s = sin[pos].to(dtype).double().unsqueeze(1)
    r64q, r64k = apply_rotary_emb(q64, k64, c, s)
    ((r64q * gq.double()).sum() + (r64k * gk.double()).sum()).backward()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for got, ref in ((qd.grad, q64.grad), (kd.grad, k64.grad)):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err < tol * max(1.0, ref.abs().max().item()), err


@pytest.mark.parametrize("mode,D,dtype", [(0, 64, torch.bfloat16), (1, 64, torch.float16), (0, 128, torch.bfloat16),
                                          (1, 128, torch.bfloat16)],
                         ids=["hard-d64-bf16", "soft-d64-f16", "hard-d128-bf16", "soft-d128-bf16"])
@pytest.mark.parametrize("tables", ["rope_cache", "arbitrary"])
def test_forward_rotates_q_on_load_bit_identical(mode, D, dtype, tables):
    # the forward's RoPE of q on load equals dsalt_rope followed by the plain forward, bit
    # for bit (same arithmetic: tables rounded to the element type, fp32 products, no
    # contraction, one rounding), for packed sequences whose positions restart at 0
    from dsalt.kernels.window_utils import build_rope_cache
    from test_gpu_fwd import make_inputs
    print(f"rope on load mode={mode} D={D} {dtype}", flush=True)
    q, k, v, w, pos, bias, cu = make_inputs([300, 77, 512], 4, D, 12, mode, seed=90 + D, dtype=dtype,
                                            n_min=4, n_max=120)
    if tables == "rope_cache":  # halves repeat: the kernel reads half of each row
        cos, sin = build_rope_cache(600, D, torch.device("cpu"), base=10000.0)
    else:  # halves differ: every column read
        g = torch.Generator().manual_seed(D)
        cos, sin = torch.randn(600, D, generator=g), torch.randn(600, D, generator=g)
    qd, kd, vd, cud = (t.to(DEV) for t in (q, k, v, cu))
    cosd, sind = cos.to(DEV), sin.to(DEV)
    q_rot, k_rot = _hip.rope(qd, kd, cosd, sind, cud)
    args = (w.to(DEV), pos.to(DEV), bias.to(DEV), cud, 1.0 / math.sqrt(D))
    o_ref, l_ref = _hip.fwd(mode, q_rot, k_rot, vd, *args, out_dtype=torch.float32)
    o_fus, l_fus = _hip.fwd(mode, qd, k_rot, vd, *args, out_dtype=torch.float32, rope=(cosd, sind))
    torch.cuda.synchronize()
    assert torch.equal(o_ref, o_fus)
    assert torch.equal(torch.nan_to_num(l_ref), torch.nan_to_num(l_fus))


def test_rope_k_only_matches_pair():
    from dsalt.kernels.window_utils import build_rope_cache, rotate_packed
    q = torch.randn(200, 4, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(200, 2, 64, device=DEV, dtype=torch.bfloat16)
    cos, sin = build_rope_cache(256, 64, DEV)
    cu = torch.tensor([0, 120, 200], dtype=torch.int32, device=DEV)
    q2, k2 = _hip.rope(q, k, cos, sin, cu)
    assert torch.equal(rotate_packed(k, cos, sin, cu), k2)
    assert torch.equal(_hip.rope(q, None, cos, sin, cu)[0], q2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("n_kv,D", [(16, 64), (2, 128), (4, 64)])
def test_scores_pass_rotates_k_like_rope(dtype, n_kv, D):
    """The score pass with k given (the module's inference route) rotates k exactly as
    dsalt_rope rotates it alone - packed positions from cu_seqlens, the module's tables
    and arbitrary ones, a sequence longer than the table (NaN rows) - and its scores are
    those of the pass without k."""
    from dsalt.kernels.window_utils import build_rope_cache
    print(f"scores pass rotates k {dtype} n_kv={n_kv} D={D}", flush=True)
    g = torch.Generator().manual_seed(n_kv * D)
    lens = [300, 70, 230]
    T, d, H = sum(lens), 256, 16
    cu = torch.tensor([0, 300, 370, 600], dtype=torch.int32, device=DEV)
    x = torch.randn(T, d, generator=g).to(DEV, dtype)
    v = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
    k = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
    alpha = torch.rand(H, generator=g).to(DEV)
    for cos, sin in (build_rope_cache(512, D, DEV),
                     (torch.randn(280, D, generator=g).to(DEV), torch.randn(280, D, generator=g).to(DEV))):
        s0, zx0, zv0 = _hip.hybrid_scores(x, v, alpha, H)
        s1, zx1, zv1, k1 = _hip.hybrid_scores(x, v, alpha, H, rope_k=(k, cos, sin, cu))
        _, k_ref = _hip.rope(None, k, cos, sin, cu)
        torch.cuda.synchronize()
        assert torch.equal(s0, s1) and torch.equal(zx0, zx1) and torch.equal(zv0, zv1)
        assert torch.equal(torch.nan_to_num(k1.float(), 7.0), torch.nan_to_num(k_ref.float(), 7.0))
        assert bool(torch.isnan(k1).any()) == (cos.shape[0] < max(lens))

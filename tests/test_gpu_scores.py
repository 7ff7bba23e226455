"""The fused selector front-end on the GPU: dsalt_hybrid_scores (the hybrid landmark
score of landmark_tokens_ker.py:19-61 from the value projection v = x W_V^T) against the
CPU oracle, and its use by the selector and the module.

For fp32 inputs the scores match the float64-input oracle to fp32 rounding. For 16-bit
inputs each norm is rounded to the input dtype, as x.norm() returns it; the kernel's
fp32 sum of squares runs in another order than torch's, so a norm can land one unit in
the last place of the 16-bit type away (about 1 norm in 10^4). The tests bound the
fraction of such tokens instead of requiring equality. Under autocast torch keeps the
norms in fp32 (``norms_f32``), and the kernel matches the float64 oracle to fp32
rounding again.

The module's default inference selection takes this route in two launches
(dsalt_select_hybrid: the norms pass, which also rotates k and can form the window
gate's logits, then the selection forming the scores); its landmark sets equal the
reference's x @ W_V.T route at configs 2 to 4 (tests/test_gpu_headline.py)."""
import math

import numpy as np
import pytest
import torch

from dsalt import _hip
from dsalt.kernels.landmark_tokens_ker import hybrid_scores_from_v
from dsalt.kernels.selectors import _compute_landmark_indices
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _inputs(T, d, n_kv, dh, H, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g) * (1 + torch.rand(T, 1, generator=g))
    W = torch.randn(n_kv * dh, d, generator=g) / d ** 0.5
    alpha = torch.rand(H, generator=g)
    v = (x @ W.T).view(T, n_kv, dh)
    return x.to(dtype), v.to(dtype), alpha, W


@pytest.mark.parametrize("n_kv", [16, 4], ids=["mha", "gqa"])
def test_scores_fp32_match_oracle(n_kv):
    print(f"scores fp32 n_kv={n_kv}", flush=True)
    T, d, H, dh = 3000, 1024, 16, 64
    x, v, alpha, _ = _inputs(T, d, n_kv, dh, H, 70)
    s, zx, zv = _hip.hybrid_scores(x.to(DEV), v.to(DEV), alpha.to(DEV), H)
    rs, rzx, rzv = orc.hybrid_scores_from_v(x.double(), v.double(), alpha.double(), H)
    for got, ref, name in ((s, rs, "scores"), (zx, rzx, "z_x"), (zv, rzv, "z_v")):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err < 2e-5, f"{name} max-abs error {err}"


def test_scores_autocast_norms_f32():
    # under autocast .norm() of a bf16 tensor runs in fp32 and is not rounded back
    T, d, H, dh, n_kv = 4096, 1024, 16, 64, 16
    x, v, alpha, _ = _inputs(T, d, n_kv, dh, H, 76)
    x, v = x.to(torch.bfloat16), v.to(torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        s, zx, zv = _hip.hybrid_scores(x.to(DEV), v.to(DEV), alpha.to(DEV), H)
        # torch's own autocast route on the same operands, for the record
        ts, _, _ = hybrid_scores_from_v(x.to(DEV), v.to(DEV), alpha.to(DEV), H)
    rs, rzx, rzv = orc.hybrid_scores_from_v(x.double(), v.double(), alpha.double(), H)
    for got, ref, name in ((s, rs, "scores"), (zx, rzx, "z_x"), (zv, rzv, "z_v"), (ts, rs, "torch scores")):
        err = (got.cpu().double() - ref).abs().max().item()
        assert err < 5e-5, f"{name} max-abs error {err}"


@pytest.mark.parametrize("xdt,vdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.float32, torch.bfloat16)], ids=["bf16", "fp16", "mixed"])
def test_scores_16bit_match_oracle(xdt, vdt):
    print(f"scores {xdt} {vdt}", flush=True)
    T, d, H, dh, n_kv = 4096, 1024, 16, 64, 16
    x, v, alpha, _ = _inputs(T, d, n_kv, dh, H, 71)
    x, v = x.to(xdt), v.to(vdt)
    s, zx, zv = _hip.hybrid_scores(x.to(DEV), v.to(DEV), alpha.to(DEV), H, norms_f32=False)
    # the oracle takes the norms in the same 16-bit dtype (rounded there, then .float())
    rs, rzx, rzv = orc.hybrid_scores_from_v(x, v, alpha, H)
    for got, ref, name in ((s, rs, "scores"), (zx, rzx, "z_x"), (zv, rzv, "z_v")):
        diff = (got.cpu() - ref).abs()
        frac = (diff > 1e-4).float().mean().item()
        assert frac < 2e-3, f"{name}: {frac:.2e} of the entries differ by more than 1e-4"
        # one 16-bit ulp of a norm moves z by at most ulp(norm) / std
        assert diff.max().item() < 0.5, f"{name} max-abs error {diff.max().item()}"


def test_scores_deterministic_strided_and_tiny():
    T, d, H, dh, n_kv = 1000, 256, 8, 128, 2
    x, v, alpha, _ = _inputs(T, d, n_kv, dh, H, 72, torch.bfloat16)
    wide = torch.zeros(T, d + 64, dtype=torch.bfloat16)
    wide[:, 16:16 + d] = x  # row stride d + 64, 32-byte offset: still 16-byte aligned rows
    xs = wide.to(DEV)[:, 16:16 + d]
    a = _hip.hybrid_scores(xs, v.to(DEV), alpha.to(DEV), H)
    b = _hip.hybrid_scores(x.to(DEV), v.to(DEV), alpha.to(DEV), H)
    for p, q in zip(a, b):
        assert torch.equal(p, q)  # same values, run to run and across strides
    # one token: std = NaN (0/0), kept by the clamp, as torch.std gives
    s1, zx1, _ = _hip.hybrid_scores(x[:1].to(DEV), v[:1].to(DEV), alpha.to(DEV), H)
    assert torch.isnan(s1).all() and torch.isnan(zx1).all()
    rs1, _, _ = orc.hybrid_scores_from_v(x[:1], v[:1], alpha, H)
    assert torch.isnan(rs1).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_selection_from_v_matches_gemm_path(dtype):
    # v = x @ W.T formed on the GPU (as the module's v_proj does): the default v route
    # selects exactly the GEMM route's sets; the HIP score kernel's selection is bit-exact
    # on its own scores and agrees with the GEMM route up to near-ties
    g = torch.Generator().manual_seed(73)
    lens = [700, 333, 1100]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T, d, H, dh, k = int(cu[-1]), 512, 8, 64, 32
    x, _, alpha, W = _inputs(T, d, H, dh, H, 74)
    xd, Wd = x.to(DEV, dtype), W.to(DEV, dtype)
    vd = (xd @ Wd.T).view(T, H, dh)
    w = (torch.rand(T, generator=g) * 200 + 1).floor()
    args = (xd, Wd, alpha.to(DEV), w.to(DEV), cu.to(DEV), k, 1, T, cu.tolist())
    lmk_w, _, _ = _compute_landmark_indices(*args, head_dim=dh)
    lmk_v, _, _ = _compute_landmark_indices(*args, head_dim=dh, v=vd)
    assert torch.equal(lmk_v, lmk_w)
    lmk_h, _, _ = _compute_landmark_indices(*args, head_dim=dh, v=vd, hip_scores=True)
    s_v, _, _ = _hip.hybrid_scores(xd, vd, alpha.to(DEV), H)
    np.testing.assert_array_equal(lmk_h.cpu().numpy(), orc.select_landmarks(s_v.cpu().numpy(), w.numpy(), cu.numpy(), k))
    same = (lmk_h == lmk_w).float().mean().item()
    assert same > 0.99, f"only {same:.4f} of the landmark slots agree with the GEMM path"


def test_differentiable_scores_from_v_match_kernel_and_grad():
    T, d, H, dh, n_kv = 500, 256, 4, 64, 2
    x, v, alpha, W = _inputs(T, d, n_kv, dh, H, 75)
    xd, Wd, ad = x.to(DEV).requires_grad_(), W.to(DEV).requires_grad_(), alpha.to(DEV).requires_grad_()
    s_t, _, _ = hybrid_scores_from_v(xd, (xd @ Wd.T).view(T, n_kv, dh), ad, H)
    s_k, _, _ = _hip.hybrid_scores(x.to(DEV), v.to(DEV), alpha.to(DEV), H)
    assert (s_t.detach() - s_k).abs().max().item() < 1e-4
    s_t.square().sum().backward()
    xr, Wr, ar = x.double().requires_grad_(), W.double().requires_grad_(), alpha.double().requires_grad_()
    s_r, _, _ = orc.hybrid_scores(xr, Wr, ar, H, dh)
    s_r.square().sum().backward()
    for got, ref in ((xd.grad, xr.grad), (Wd.grad, Wr.grad), (ad.grad, ar.grad)):
        rel = (got.cpu().double() - ref).norm() / ref.norm()
        assert rel < 1e-4, rel


@pytest.mark.parametrize("training", [False, True], ids=["eval", "train"])
def test_module_fused_selector(training):
    from dsalt.modules import DSALTAttention
    torch.manual_seed(5)
    m = DSALTAttention(256, 4, 16, 128, 16, max_seq_len=1024).to(DEV)
    m.train(training)
    m._collect_last_P = False
    lens = [600, 424]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    x = torch.randn(int(cu[-1]), 256, device=DEV)
    outs, sels = [], []
    for fused, hip_scores in ((True, False), (False, False), (True, True)):
        m._fused_selector, m._hip_scores = fused, hip_scores
        out, _ = m(x, cu_seqlens=cu, cu_list=cu.tolist())
        outs.append(out.detach())
        sels.append(m._last_selection[1].clone())
    m._fused_selector, m._hip_scores = True, True
    # the torch route on v is the GEMM route's selection, hence the same output bit for
    # bit; the default HIP score route selects the same sets here
    assert torch.equal(sels[0], sels[1]) and torch.equal(outs[0], outs[1])
    assert torch.equal(sels[2], sels[1])
    err = (outs[2] - outs[1]).abs().max().item()
    assert err < 2e-2, f"HIP-score selector output differs by {err}"


SELECT_HYBRID_CASES = {
    # lens, d, H, n_kv, D, dtype, k, window source, norms_f32, rotate k
    "mha-bf16-gate": ([700, 0, 333, 1100], 512, 16, 16, 64, torch.bfloat16, 32, "gate", False, True),
    "gqa-f16-long-chunked": ([9000, 3000, 17], 256, 8, 2, 64, torch.float16, 128, "cont", False, False),
    "fp32-d128": ([600, 1500], 256, 8, 4, 128, torch.float32, 64, "cont", False, True),
    "bf16-autocast-norms": ([4096, 200], 1024, 16, 16, 64, torch.bfloat16, 64, "gate", True, True),
    "one-token-nan-std": ([1], 256, 4, 4, 64, torch.bfloat16, 8, "cont", False, False),
    "empty-seq-k0": ([50, 0, 80], 256, 4, 2, 64, torch.bfloat16, 0, "gate", False, False),
}


@pytest.mark.parametrize("case", list(SELECT_HYBRID_CASES), ids=list(SELECT_HYBRID_CASES))
def test_select_hybrid_equals_scores_then_select(case):
    """dsalt_select_hybrid (norms pass, then the selection forming each score itself) gives
    the windows, landmark sets and rotated k of dsalt_hybrid_scores followed by the
    selection on its scores, bit for bit: long chunked sequences, GQA, fp32 and 16-bit
    inputs, autocast's fp32 norms, a single token (NaN std), an empty sequence and k = 0."""
    from dsalt.kernels.window_utils import build_rope_cache
    lens, d, H, n_kv, D, dtype, k_lmk, src, nf32, rot = SELECT_HYBRID_CASES[case]
    print(f"select_hybrid {case}", flush=True)
    g = torch.Generator().manual_seed(len(case))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    T = int(cu[-1])
    x = (torch.randn(T, d, generator=g) * (1 + torch.rand(T, 1, generator=g))).to(DEV, dtype)
    v = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
    alpha = torch.rand(H, generator=g).to(DEV)
    if src == "gate":
        gdt = torch.float16 if dtype == torch.float16 else torch.bfloat16
        w_cont, gate = None, ((torch.randn(T, generator=g) * 3).to(DEV, gdt), 8.0, 700.0)
    else:
        w_cont, gate = (torch.rand(T, generator=g) * 300 + 0.5).to(DEV), None
    rope_k = None
    if rot:
        k = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
        cos, sin = build_rope_cache(max(lens) + 1, D, DEV)
        rope_k = (k, cos, sin, cu)
    for chunked in (True, False):
        ref = _hip.hybrid_scores(x, v, alpha, H, norms_f32=nf32, rope_k=rope_k)
        w_ref, lmk_ref = _hip.select_landmarks_quantize(ref[0], w_cont, cu, k_lmk, chunked=chunked, gate=gate)
        w_got, lmk_got, k_got = _hip.select_hybrid(x, v, alpha, H, w_cont, cu, k_lmk, chunked=chunked, gate=gate,
                                                   norms_f32=nf32, rope_k=rope_k)
        torch.cuda.synchronize()
        assert torch.equal(torch.nan_to_num(w_got, 7.0), torch.nan_to_num(w_ref, 7.0))
        assert torch.equal(lmk_got, lmk_ref), f"chunked={chunked}: landmark sets differ"
        if rot:
            assert torch.equal(k_got, ref[3])
        else:
            assert k_got is None
    if case == "one-token-nan-std":
        assert bool((lmk_got == -1).all())  # a NaN score is never a landmark


def _ulp(r: torch.Tensor, dtype) -> torch.Tensor:
    """Spacing of the 16-bit values around each float64 value r."""
    mant, emin = (7, -126) if dtype == torch.bfloat16 else (10, -14)
    e = torch.floor(torch.log2(r.abs().clamp(min=2.0 ** (emin - mant)))).clamp(min=emin)
    return torch.exp2(e - mant)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lens,d,bias", [([2048] * 4, 1024, True), ([300, 1, 777], 512, False),
                                         ([5000], 2048, True)], ids=["c2-shape", "ragged-no-bias", "long"])
def test_select_hybrid_window_gate_in_norms_pass(dtype, lens, d, bias):
    """The window gate's logits formed by the norms pass (gate_linear): each is x.w + b
    rounded once to the dtype from an fp32 sum, so it lies within half an ulp of the exact
    (float64) value plus the fp32 summation bound, and equals the correctly rounded value in
    all but a few tokens; the windows and landmark sets are those the selection forms from
    the same logits passed as `gate`, bit for bit; against torch's GEMV (win_gate), the
    logits differ in at most 0.5 % of the tokens, by one ulp."""
    from dsalt.kernels.window_utils import build_rope_cache
    print(f"gate in norms pass {dtype} lens={lens[:3]} d={d}", flush=True)
    g = torch.Generator().manual_seed(d + len(lens))
    H, n_kv, D, k_lmk, n_min, n_max = 16, 16, 64, 64, 32.0, 512.0
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    T = int(cu[-1])
    x = torch.randn(T, d, generator=g).to(DEV, dtype)
    v = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
    k = torch.randn(T, n_kv, D, generator=g).to(DEV, dtype)
    alpha = torch.rand(H, generator=g).to(DEV)
    # nn.Linear(d, 1)'s initialisation range, scaled up so that the logits span the sigmoid
    lin = torch.nn.Linear(d, 1).to(DEV, dtype)
    with torch.no_grad():
        lin.weight.copy_(((torch.rand(1, d, generator=g) * 2 - 1) * 4 / math.sqrt(d)).to(DEV, dtype))
        lin.bias.copy_(torch.tensor([0.3]).to(DEV, dtype))
    b = lin.bias if bias else None
    cos, sin = build_rope_cache(max(lens) + 1, D, DEV)
    f = _hip.SelectHybridLauncher(x, v, alpha, H, None, cu, k_lmk, gate_linear=(lin.weight, b, n_min, n_max),
                                  rope_k=(k, cos, sin, cu))
    f()
    with torch.no_grad():
        torch_logit = torch.nn.functional.linear(x, lin.weight, b).squeeze(-1)
    torch.cuda.synchronize()
    got = f.logit.double()
    exact = x.double() @ lin.weight.double()[0] + (b.double() if bias else 0.0)
    bound = 0.5 * _ulp(exact, dtype) + (d + 1) * 2.0 ** -24 * ((x.double().abs() @ lin.weight.double().abs()[0]) +
                                                                (b.double().abs() if bias else 0.0))
    assert bool(((got - exact).abs() <= bound).all()), "a logit is farther from x.w + b than its rounding allows"
    rounded = exact.float().to(dtype).double()
    off = int((got != rounded).sum())
    print(f"  {off}/{T} logits differ from the correctly rounded value", flush=True)
    assert off <= max(1, T // 500)
    n_torch = int((f.logit != torch_logit).sum())
    print(f"  {n_torch}/{T} logits differ from torch's GEMV", flush=True)
    assert n_torch <= max(2, T // 200)
    assert bool(((f.logit.double() - torch_logit.double()).abs() <= _ulp(torch_logit.double(), dtype)).all())
    # the selection on those logits, given explicitly
    w_ref, lmk_ref, k_ref = _hip.select_hybrid(x, v, alpha, H, None, cu, k_lmk, gate=(f.logit.clone(), n_min, n_max),
                                               rope_k=(k, cos, sin, cu))
    torch.cuda.synchronize()
    assert torch.equal(f.w_out, w_ref) and torch.equal(f.out, lmk_ref) and torch.equal(f.k_out, k_ref)

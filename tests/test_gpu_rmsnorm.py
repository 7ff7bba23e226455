"""dsalt_add_rms_norm (a residual add and the RMSENorm after it in one pass) against
torch's own ops: the sum equals torch's add bit for bit; the norm is F.rms_norm's
arithmetic with the sum of squares in another order, so an output may differ from
torch's in its last bit (up to ~3 in 10^6 in bf16, ~7 in 10^5 in fp16 here); every output lies within one 16-bit ulp of
the float64 norm of the rounded sum. The LM and the block with the fused passes against
the same modules with them off."""
import math

import pytest
import torch
import torch.nn.functional as F

from dsalt import _hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _ulp(r: torch.Tensor, dtype) -> torch.Tensor:
    mant, emin = (7, -126) if dtype == torch.bfloat16 else (10, -14)
    e = torch.floor(torch.log2(r.abs().clamp(min=2.0 ** (emin - mant)))).clamp(min=emin)
    return torch.exp2(e - mant)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("rows,d", [(16384, 1024), (3, 8), (777, 2816), (64, 4096)])
@pytest.mark.parametrize("add", [True, False], ids=["add", "norm"])
def test_add_rms_norm_matches_torch(dtype, rows, d, add):
    print(f"add_rms_norm {dtype} rows={rows} d={d} add={add}", flush=True)
    g = torch.Generator().manual_seed(rows + d)
    x = (torch.randn(rows, d, generator=g) * 2).to(DEV, dtype)
    h = (torch.randn(rows, d, generator=g) * 2).to(DEV, dtype) if add else None
    w = (1 + 0.2 * torch.randn(d, generator=g)).to(DEV, dtype)
    x_out, y = _hip.add_rms_norm(x, h, w, 1e-6)
    s = x + h if add else x
    ref = F.rms_norm(s, (d,), w, 1e-6)
    torch.cuda.synchronize()
    if add:
        assert torch.equal(x_out, s), "the sum differs from torch's add"
    else:
        assert x_out is None
    sd = s.double()
    exact = sd * torch.rsqrt(sd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert bool(((y.double() - exact).abs() <= _ulp(exact, dtype)).all()), "an output is more than one ulp off"
    off = int((y != ref).sum())
    print(f"  {off}/{y.numel()} outputs differ from F.rms_norm", flush=True)
    # a last-bit difference of a row's fp32 scale moves an output across a rounding boundary
    # ~8x as often in fp16 (10 fraction bits) as in bf16 (7)
    assert off <= max(2, y.numel() * (1e-4 if dtype == torch.float16 else 2e-5))
    assert bool(((y.double() - ref.double()).abs() <= _ulp(ref.double(), dtype)).all())


def test_add_rms_norm_in_place_sum():
    """x_out may alias x: the C ABI writes the sum over x."""
    import ctypes
    g = torch.Generator().manual_seed(5)
    x = torch.randn(100, 1024, generator=g).to(DEV, torch.bfloat16)
    h = torch.randn(100, 1024, generator=g).to(DEV, torch.bfloat16)
    w = torch.ones(1024, device=DEV, dtype=torch.bfloat16)
    want_s, want_y = _hip.add_rms_norm(x, h, w, 1e-5)
    y = torch.empty_like(x)
    rc = _hip.lib().dsalt_add_rms_norm(x.data_ptr(), h.data_ptr(), x.data_ptr(), y.data_ptr(), w.data_ptr(), 100,
                                       1024, ctypes.c_float(1e-5), _hip.DTYPE_BF16, _hip.stream_handle(DEV))
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(x, want_s) and torch.equal(y, want_y)


def test_lm_fused_norms_against_unfused():
    """A 2-layer LM's packed eval logits with the fused add + norm passes against the same
    model with them off (torch's add and F.rms_norm): the residual streams differ only
    through last-bit differences of the norms."""
    from dsalt.model import DSALTLMHeadModel
    from dsalt.modules.dsalt_transformer import DSALTTransformerBlock
    torch.manual_seed(9)
    with torch.device(DEV):
        model = DSALTLMHeadModel(1000, 256, 2, 4, 16, 128, 16, 512)
    model = model.to(DEV, torch.bfloat16).eval()
    model.set_collect_last_P(False)
    ids = torch.randint(0, 1000, (3 * 300,), device=DEV)
    cu = torch.tensor([0, 300, 600, 900], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        assert model._norms_fusable(model.embed_tokens(ids))
        fused = model(ids, cu_seqlens=cu)["logits"].float()
        try:
            DSALTTransformerBlock._fuse_norms = False
            assert not model._norms_fusable(model.embed_tokens(ids))
            plain = model(ids, cu_seqlens=cu)["logits"].float()
        finally:
            DSALTTransformerBlock._fuse_norms = True
    torch.cuda.synchronize()
    rel = float((fused - plain).norm() / plain.norm())
    print(f"  fused vs unfused logits rel-L2 {rel:.2e}", flush=True)
    assert torch.isfinite(fused).all() and rel < 2e-2


def test_block_declines_unaligned_residual():
    """A residual that is contiguous but not 16-byte aligned turns the block's fused pass
    off (torch's add and norm run), rather than reaching the C ABI, which rejects it."""
    from dsalt.modules.dsalt_transformer import DSALTTransformerBlock
    with torch.device(DEV):
        block = DSALTTransformerBlock(256, 4, 16, 128, 16, 512, 512)
    block = block.to(DEV, torch.bfloat16).eval()
    x = torch.randn(10, 256, device=DEV, dtype=torch.bfloat16)
    h = torch.randn(10 * 256 + 1, device=DEV, dtype=torch.bfloat16)[1:].view(10, 256)
    assert h.is_contiguous() and h.data_ptr() % 16
    with torch.no_grad():
        assert block._norms_fusable(x, h.clone(), block.ffn_norm)
        assert not block._norms_fusable(x, h, block.ffn_norm)
        with pytest.raises(_hip.DsaltError):
            _hip.add_rms_norm(x, h, block.ffn_norm.weight, block.ffn_norm.eps)

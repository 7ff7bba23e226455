"""dsalt_swiglu (the LM feed-forward's gated product in one pass) against torch's own two
ops, F.silu(gate) * up, bit for bit: every bf16 and every fp16 gate value against random
up values, fp32 on random values, NaN / inf included; and SwiGLUFFN's no-grad path, which
takes it, against the torch path."""
import pytest
import torch
import torch.nn.functional as F

from dsalt import _hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _same(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    nan = torch.isnan(a)
    assert torch.equal(nan, torch.isnan(b)), "NaN positions differ"
    assert torch.equal(a[~nan], b[~nan]), f"{int((a[~nan] != b[~nan]).sum())} values differ"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_swiglu_every_16bit_gate_value(dtype):
    print(f"swiglu exhaustive {dtype}", flush=True)
    gate = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype).to(DEV)
    g = torch.Generator(device="cpu").manual_seed(1)
    for up in (torch.ones(65536, dtype=dtype), (torch.randn(65536, generator=g) * 3).to(dtype),
               (torch.rand(65536, generator=g) * 1e4).to(dtype)):
        up = up.to(DEV)
        _same(_hip.swiglu(gate, up), F.silu(gate) * up)


def test_swiglu_fp32_and_shapes():
    g = torch.Generator(device="cpu").manual_seed(2)
    gate = (torch.randn(3, 1000, 64, generator=g) * 8).to(DEV)
    up = torch.randn(3, 1000, 64, generator=g).to(DEV)
    gate.view(-1)[:4] = torch.tensor([float("inf"), float("-inf"), float("nan"), 0.0])
    _same(_hip.swiglu(gate, up), F.silu(gate) * up)
    assert not _hip.swiglu_supported(gate[:, :, :63], up[:, :, :63])  # not contiguous
    with pytest.raises(_hip.DsaltError):
        _hip.swiglu(gate.to(torch.bfloat16), up)


def test_ffn_no_grad_path_equals_torch_ops():
    from dsalt.modules.dsalt_transformer import SwiGLUFFN
    torch.manual_seed(3)
    ffn = SwiGLUFFN(256, 704).to(DEV).to(torch.bfloat16).eval()
    x = torch.randn(1000, 256, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        got = ffn(x)  # the HIP gated product
        want = ffn.down_proj(F.silu(ffn.gate_proj(x)) * ffn.up_proj(x))
    _same(got, want)
    x.requires_grad_()
    ffn(x).float().sum().backward()  # with autograd the torch ops run
    assert x.grad is not None and torch.isfinite(x.grad).all()

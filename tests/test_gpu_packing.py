"""cu_seqlens that is not a plain packing of the T rows. The kernels read each sequence's
bounds clamped to [0, T], with every length at least 0 (seq_bounds in csrc/common.h), so
whatever cu_seqlens holds, every row they read or write lies inside the tensors:
- an end past T, or a negative start, gives exactly the result of the clamped packing;
- a first entry above 0 (rows before it belong to no sequence) gives the result of the
  sliced batch, and the rotations of those rows are NaN (no table row), as for positions
  past the table;
- out-of-order entries give, on the rows that only one sequence covers, the result of
  that sequence on its own.
The CPU side (tests/test_block_map.py) checks the bounds of every lookup for arbitrary
cu_seqlens content."""
import math

import numpy as np
import pytest
import torch

from dsalt import _hip
from dsalt.kernels.window_utils import build_rope_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
H, D = 4, 64


def _cu(v):
    return torch.tensor(v, dtype=torch.int32, device=DEV)


def _inputs(T, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q, k, v = (torch.randn(T, H, D, generator=g).to(DEV, torch.bfloat16) for _ in range(3))
    w = (8 + torch.rand(T, generator=g) * 300).floor().to(DEV)
    scores = torch.randn(T, H, generator=g).to(DEV)
    x = torch.randn(T, 128, generator=g).to(DEV, torch.bfloat16)
    logit = (torch.randn(T, generator=g) * 2).to(DEV, torch.bfloat16)
    return q, k, v, w, scores, x, logit


def _fwd(q, k, v, w, lmk, cu):
    return _hip.fwd(_hip.MODE_HARD, q, k, v, w, lmk, None, cu, 1 / math.sqrt(D), out_dtype=torch.float32)


@pytest.mark.parametrize("bad,equiv,T", [([0, 300, 900], [0, 300, 600], 600),
                                         ([-50, 300, 600], [0, 300, 600], 600),
                                         ([0, 5000, 12000], [0, 5000, 9000], 9000)],
                         ids=["end-past-T", "negative-start", "long-end-past-T"])
def test_clamped_packings_equal_their_equivalent(bad, equiv, T):
    print(f"packing {bad} ~ {equiv}", flush=True)
    q, k, v, w, scores, x, logit = _inputs(T, len(bad) + T)
    cb, ce = _cu(bad), _cu(equiv)
    lmk_b = _hip.select_landmarks(scores, w, cb, 16)
    lmk_e = _hip.select_landmarks(scores, w, ce, 16)
    torch.cuda.synchronize()
    assert torch.equal(lmk_b, lmk_e)
    ob, lb = _fwd(q, k, v, w, lmk_e, cb)
    oe, le = _fwd(q, k, v, w, lmk_e, ce)
    torch.cuda.synchronize()
    assert torch.equal(ob, oe) and torch.equal(lb, le)
    cos, sin = build_rope_cache(T + 1, D, DEV)
    gate = (logit, 8.0, 300.0)
    alpha = torch.full((H,), 0.5, device=DEV)
    rb = _hip.select_hybrid(x, v, alpha, H, None, cb, 16, gate=gate, rope_k=(k, cos, sin, cb))
    re = _hip.select_hybrid(x, v, alpha, H, None, ce, 16, gate=gate, rope_k=(k, cos, sin, ce))
    torch.cuda.synchronize()
    for got, want in zip(rb, re):
        assert torch.equal(torch.nan_to_num(got.float(), 7.0), torch.nan_to_num(want.float(), 7.0))


def test_rows_before_the_first_sequence():
    print("packing [100, 400, 600]", flush=True)
    T, off = 600, 100
    q, k, v, w, scores, x, logit = _inputs(T, 3)
    cu, cs = _cu([off, 400, 600]), _cu([0, 300, 500])
    lmk = _hip.select_landmarks(scores, w, cu, 16)
    lmk_s = _hip.select_landmarks(scores[off:].contiguous(), w[off:].contiguous(), cs, 16)
    torch.cuda.synchronize()
    assert torch.equal(lmk, lmk_s)
    o, l = _fwd(q, k, v, w, lmk, cu)
    o_s, l_s = _fwd(q[off:].contiguous(), k[off:].contiguous(), v[off:].contiguous(), w[off:].contiguous(), lmk, cs)
    torch.cuda.synchronize()
    assert torch.equal(o[off:], o_s) and torch.equal(l[off:], l_s)
    cos, sin = build_rope_cache(T, D, DEV)
    qr, kr = _hip.rope(q, k, cos, sin, cu)
    qr_s, kr_s = _hip.rope(q[off:].contiguous(), k[off:].contiguous(), cos, sin, cs)
    torch.cuda.synchronize()
    assert torch.equal(qr[off:], qr_s) and torch.equal(kr[off:], kr_s)
    assert bool(torch.isnan(qr[:off].float()).all()) and bool(torch.isnan(kr[:off].float()).all())
    _, _, k_h = _hip.select_hybrid(x, v, torch.full((H,), 0.5, device=DEV), H, None, cu, 16, gate=(logit, 8.0, 300.0),
                                   rope_k=(k, cos, sin, cu))
    torch.cuda.synchronize()
    assert torch.equal(k_h[off:], kr_s) and bool(torch.isnan(k_h[:off].float()).all())


def test_out_of_order_entries():
    """[0, 500, 300, 600]: sequence 0 is rows [0, 500), sequence 1 is empty, sequence 2 is
    rows [300, 600). Rows [0, 300) belong to sequence 0 alone and rows [500, 600) to
    sequence 2 alone; there the results are those of each sequence on its own."""
    print("packing [0, 500, 300, 600]", flush=True)
    T = 600
    q, k, v, w, scores, x, logit = _inputs(T, 4)
    cu = _cu([0, 500, 300, 600])
    lmk = _hip.select_landmarks(scores, w, cu, 16)
    l0 = _hip.select_landmarks(scores[:500].contiguous(), w[:500].contiguous(), _cu([0, 500]), 16)
    l2 = _hip.select_landmarks(scores[300:].contiguous(), w[300:].contiguous(), _cu([0, 300]), 16)
    torch.cuda.synchronize()
    assert torch.equal(lmk[:, 0], l0[:, 0]) and torch.equal(lmk[:, 2], l2[:, 0])
    assert bool((lmk[:, 1] == -1).all())
    o, _ = _fwd(q, k, v, w, lmk, cu)
    o0, _ = _fwd(q[:500].contiguous(), k[:500].contiguous(), v[:500].contiguous(), w[:500].contiguous(), l0,
                 _cu([0, 500]))
    o2, _ = _fwd(q[300:].contiguous(), k[300:].contiguous(), v[300:].contiguous(), w[300:].contiguous(), l2,
                 _cu([0, 300]))
    torch.cuda.synchronize()
    assert torch.equal(o[:300], o0[:300]) and torch.equal(o[500:], o2[200:])
    cos, sin = build_rope_cache(T, D, DEV)
    qr, _ = _hip.rope(q, k, cos, sin, cu)
    assert bool(torch.isfinite(qr.float()).all())
    np.testing.assert_array_equal(lmk.shape, (H, 3, 16))

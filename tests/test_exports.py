"""The reference's generic helpers exported by dsalt / dsalt.kernels (mask builders, masked
SDPA, older landmark helpers): checked on the CPU against brute-force loops and the oracle.
They are plain torch utilities; the DSALT attention path never calls them."""
import math

import numpy as np
import pytest
import torch

import dsalt
from dsalt import kernels as K
from oracle import dsalt_oracle as orc

REFERENCE_EXPORTS = [
    "dsalt_triton_attention", "RMSENorm", "compute_window_sizes", "build_local_window_mask",
    "build_local_window_mask_packed", "apply_rotary_emb", "build_rope_cache", "hybrid_scores_per_head",
    "compute_hybrid_scores", "select_landmarks", "soft_landmark_weights", "HybridEnergyLandmarkSelector",
    "sparse_attention_forward", "sparse_attention_forward_packed", "DSALTAttention", "DSALTTransformerBlock",
    "SwiGLUFFN", "DSALTLMHeadModel",
]


def test_reference_export_names():
    """Every name of the reference's dsalt/__init__.py:22-47 and kernels/__init__.py:1-19 that
    lies on or beside the attention path is importable (the Triton loss, the config
    dataclass and the trainer are out of scope)."""
    for name in REFERENCE_EXPORTS:
        assert hasattr(dsalt, name), name
    for name in REFERENCE_EXPORTS[1:14]:
        assert hasattr(K, name), name


def _band_loops(rows, starts, w, n):
    m = np.zeros((len(rows), n), dtype=bool)
    for r, (i, s, wi) in enumerate(zip(rows, starts, w)):
        for j in range(n):
            m[r, j] = max(s, i - wi + 1) <= j <= i
    return m


def test_local_window_mask_bruteforce():
    T = 23
    w = torch.tensor([0.0, 0.4, 1.0, 1.9, 2.0, 3.7, 30.0] + [float(x) for x in range(1, 17)])
    got = K.build_local_window_mask(T, w, torch.device("cpu"))
    wi = np.clip(w.numpy(), 1, T).astype(np.int64)  # clamp to [1, T], then truncate
    assert np.array_equal(got.numpy(), _band_loops(range(T), [0] * T, wi, T))


def test_local_window_mask_packed_bruteforce():
    lens = [7, 1, 12, 5]
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32)
    T = int(cu[-1])
    w = torch.tensor(np.random.default_rng(3).uniform(0, 9, T), dtype=torch.float32)
    got = K.build_local_window_mask_packed(cu, w, T, torch.device("cpu"))
    starts = np.repeat(cu[:-1].numpy(), lens)
    wi = np.maximum(w.numpy(), 1).astype(np.int64)
    assert np.array_equal(got.numpy(), _band_loops(range(T), starts, wi, T))


def test_sparse_attention_packed_is_hard_window_attention():
    """Masked SDPA over the packed local-window mask = the oracle's HARD attention without
    landmarks (scale 1/sqrt(D), fp64)."""
    lens = [19, 6, 11]
    cu = np.cumsum([0] + lens)
    T, H, D = int(cu[-1]), 3, 8
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(T, H, D, generator=g, dtype=torch.float64) for _ in range(3))
    w = torch.tensor(np.random.default_rng(4).integers(1, 9, T), dtype=torch.float32)
    mask = K.build_local_window_mask_packed(torch.tensor(cu, dtype=torch.int32), w, T, torch.device("cpu"))
    got = K.sparse_attention_forward_packed(q, k, v, mask)
    ref, _ = orc.attention_hard(q, k, v, w, None, None, cu)
    assert got.shape == (T, H, D) and got.is_contiguous()
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)


def test_sparse_attention_batched_masks():
    B, H, T, D = 2, 3, 10, 4
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(3))
    mask = K.build_local_window_mask(T, torch.full((T,), 4.0), torch.device("cpu"))
    for m in (mask, mask.expand(H, T, T), mask.expand(B, H, T, T)):
        got = K.sparse_attention_forward(q, k, v, m)
        s = q @ k.transpose(-1, -2) / math.sqrt(D)
        ref = torch.softmax(s.masked_fill(~mask, float("-inf")), -1) @ v
        torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)


def test_compute_window_sizes():
    w = K.compute_window_sizes(torch.zeros(5, 3), 32, 61)
    assert w.dtype == torch.float32 and w.tolist() == [46.0] * 5


def test_compute_hybrid_scores_vector_and_scalar_alpha():
    g = torch.Generator().manual_seed(6)
    T, H, dh, d = 40, 4, 8, 32
    x, W = torch.randn(T, d, generator=g, dtype=torch.float64), torch.randn(H * dh, d, generator=g, dtype=torch.float64)
    alpha = torch.rand(H, generator=g, dtype=torch.float64)
    ref, _, _ = orc.hybrid_scores(x, W, alpha, H, dh)
    torch.testing.assert_close(K.compute_hybrid_scores(x, W, alpha), ref, rtol=0, atol=0)
    a = torch.tensor(0.3, dtype=torch.float64)
    xn, vn = np.linalg.norm(x.numpy(), axis=1), np.linalg.norm((x @ W.T).numpy(), axis=1)
    z = lambda t: (t - t.mean()) / max(t.std(ddof=1), 1e-6)
    np.testing.assert_allclose(K.compute_hybrid_scores(x, W, a).numpy(), 0.3 * z(vn) + 0.7 * z(xn), rtol=1e-12)


def test_select_landmarks_and_weights():
    s = torch.tensor([0.5, 3.0, -1.0, 2.0, 7.0, 1.0])
    excl = torch.tensor([False, False, False, False, True, False])
    idx = K.select_landmarks(s, 3, exclude_mask=excl)
    assert sorted(idx.tolist()) == [1, 3, 5]  # the best three after excluding position 4
    assert K.select_landmarks(s, 10, exclude_mask=torch.ones(6, dtype=torch.bool)).numel() == 0
    assert sorted(K.select_landmarks(s, 10).tolist()) == list(range(6))  # k capped at the finite count
    wts = K.soft_landmark_weights(s, 3, exclude_mask=excl, temperature=2.0)
    ref = np.exp(s.numpy() / 2.0) * ~excl.numpy()
    np.testing.assert_allclose(wts.numpy(), ref / ref.sum(), rtol=1e-6)


def test_hybrid_energy_selector():
    sel = K.HybridEnergyLandmarkSelector(n_layers=2, n_heads=3)
    assert sel.alpha.shape == (2, 3)
    assert torch.equal(sel.alpha, torch.full((2, 3), torch.logit(torch.tensor(0.6)).item()))
    g = torch.Generator().manual_seed(7)
    x, W = torch.randn(20, 16, generator=g), torch.randn(16, 16, generator=g)
    wm = K.build_local_window_mask(20, torch.full((20,), 3.0), torch.device("cpu"))[:5]  # rows 0..4 cover keys 0..4
    idx, wts = sel(x, W, 1, 2, 4, wm)
    assert idx.numel() == 4 and (idx >= 5).all()
    assert torch.allclose(wts[:5], torch.zeros(5)) and abs(wts.sum().item() - 1) < 1e-6

"""bench.py's exact pair counts (the P of F = 4*D*P and 10*D*P) against the oracle's
count and, for HARD, against the number of True entries of the dense mask. CPU only."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402
from oracle import dsalt_oracle as orc  # noqa: E402


def _case(seed, soft):
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(0, 90, size=5)]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, H, k = int(cu[-1]), 3, 7
    w = (rng.random(T) * 60 - (5 if soft else 0)).astype(np.float32)
    if not soft:
        w = np.floor(np.maximum(w, 1)).astype(np.float32)
    w[::11] = np.nan if soft else w[::11]
    pos = rng.integers(-2, 95, size=(H, len(lens), k)).astype(np.int64)  # holes, out-of-range, duplicates
    return w, pos, cu.tolist(), H


@pytest.mark.parametrize("seed", range(5))
def test_hard_pairs(seed):
    w, pos, cu, H = _case(seed, soft=False)
    got = bench.effective_pairs_hard(w, pos, cu)
    assert got == orc.effective_pairs("hard", w, pos, cu, H)
    dense = 0
    for s in range(len(cu) - 1):
        L = cu[s + 1] - cu[s]
        if L:
            p = pos[:, s]
            m = orc.hard_mask(L, w[cu[s]:cu[s + 1]], p)
            # the dense mask de-duplicates landmark columns; count slots instead
            band = int(sum(min(int(x), i + 1) for i, x in enumerate(w[cu[s]:cu[s + 1]]))) * H
            lm = sum(int(((pp >= 0) & (pp < L) & (pp <= i - int(w[cu[s] + i]))).sum())
                     for h in range(H) for i in range(L) for pp in [p[h]])
            dense += band + lm
            assert int(m.sum()) <= band + lm
    assert got == dense


@pytest.mark.parametrize("seed", range(5))
def test_soft_pairs(seed):
    w, pos, cu, H = _case(seed, soft=True)
    assert bench.effective_pairs_soft(w, pos, cu) == orc.effective_pairs("soft", w, pos, cu, H)


@pytest.mark.parametrize("mode", ["hard", "soft"])
@pytest.mark.parametrize("seed", range(4))
def test_pair_counts_equal_the_attention_masks(mode, seed, monkeypatch):
    """The counted pairs are the pairs the oracle's attention actually admits: wrap the
    oracle's per-sequence softmax, record the band and landmark masks that
    attention_hard / attention_soft build (NaN and sub-1 windows, holes and out-of-range
    landmark slots included) and count their entries, one per head and landmark slot."""
    import torch
    w, pos, cu, H = _case(seed, soft=mode == "soft")
    T, k = int(cu[-1]), pos.shape[-1]
    g = torch.Generator().manual_seed(seed)
    q, kk, v = (torch.randn(T, H, 4, generator=g, dtype=torch.float64) for _ in range(3))
    counted = [0]
    inner = orc._seq_attention

    def recording(qs, ks, vs, band_bias, band_ok, lk, lv, lmk_logit_bias, lmk_ok, scale):
        counted[0] += int(band_ok.sum()) * qs.shape[0]  # band_ok [R, L] is shared by the heads
        if lmk_ok is not None:
            counted[0] += int(lmk_ok.sum())  # [H, R, k]: one entry per admitted slot
        return inner(qs, ks, vs, band_bias, band_ok, lk, lv, lmk_logit_bias, lmk_ok, scale)

    monkeypatch.setattr(orc, "_seq_attention", recording)
    pos_t = torch.from_numpy(pos)
    if mode == "hard":
        orc.attention_hard(q, kk, v, torch.from_numpy(w), pos_t, None, cu)
        want = bench.effective_pairs_hard(w, pos, cu)
    else:
        logw = torch.zeros(pos.shape, dtype=torch.float64)  # finite weights: every valid slot counts
        orc.attention_soft(q, kk, v, torch.from_numpy(w), pos_t, logw, cu)
        want = bench.effective_pairs_soft(w, pos, cu)
    assert counted[0] == want == orc.effective_pairs(mode, w, pos, cu, H)

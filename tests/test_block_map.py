"""The workgroup -> (sequence, block) numbering the HIP kernels compute in-kernel from
cu_seqlens (find_block in csrc/common.h): sequence s owns the ceil(L_s/bm) consecutive
ids starting at first(s) = floor(cu[s]/bm) + s. Checked here on the host, by brute
force over random packings, for the properties the launches rely on: every block has
exactly one id, ids of one sequence are consecutive, and every id is below the grid
size block_upper_bound = ceil(T/bm) + S. CPU only."""
import numpy as np
import pytest


def first_ids(cu, bm):
    return [int(cu[s]) // bm + s for s in range(len(cu) - 1)]


def lookup(cu, bm, target):
    """Device algorithm: the last sequence with first(s) <= target, then a range check."""
    f = first_ids(cu, bm)
    cand = max((s for s in range(len(f)) if f[s] <= target), default=-1)
    if cand < 0:
        return None
    L = int(cu[cand + 1] - cu[cand])
    blk = target - f[cand]
    return (cand, blk) if blk < (L + bm - 1) // bm else None


@pytest.mark.parametrize("bm", [64, 128])
@pytest.mark.parametrize("seed", range(6))
def test_block_ids_cover_every_block_once(bm, seed):
    rng = np.random.default_rng(seed)
    S = int(rng.integers(1, 200))
    lens = rng.integers(0, 3 * bm, size=S)
    lens[rng.random(S) < 0.2] = 0
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    grid = (T + bm - 1) // bm + S  # block_upper_bound
    seen = {}
    for g in range(grid):
        r = lookup(cu, bm, g)
        if r is not None:
            assert r not in seen
            seen[r] = g
    want = {(s, b) for s in range(S) for b in range((int(lens[s]) + bm - 1) // bm)}
    assert set(seen) == want
    for s in range(S):  # consecutive ids inside a sequence
        ids = [seen[(s, b)] for b in range((int(lens[s]) + bm - 1) // bm)]
        assert ids == list(range(ids[0], ids[0] + len(ids))) if ids else True

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


def lookup_desc(cu, bm, rank, n_rank):
    """Device algorithm of find_block_desc: blocks in decreasing block index (ties in
    increasing sequence), through the binary search over C(b) = sum_s max(0, n_s - b)."""
    S = len(cu) - 1
    if S > 64:
        return lookup(cu, bm, n_rank - 1 - rank)
    n = [max(int(cu[s + 1] - cu[s]) + bm - 1, 0) // bm for s in range(S)]
    if rank >= sum(n):
        return None
    C = lambda b: sum(max(x - b, 0) for x in n)  # noqa: E731
    lo, hi = 0, max(n)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if C(mid) > rank:
            lo = mid
        else:
            hi = mid
    j = rank - C(lo + 1)
    level = [s for s in range(S) if n[s] > lo]
    return (level[j], lo)


def head_rank(bid, grid, n_heads, n_rank):
    if n_heads % 8 == 0:
        hpx, j = n_heads // 8, bid >> 3
        return (bid & 7) * hpx + j % hpx, j // hpx
    per = grid >> 3
    logical = (bid & 7) * per + (bid >> 3)
    return logical // n_rank, logical % n_rank


@pytest.mark.parametrize("bm", [64, 128])
@pytest.mark.parametrize("seed", range(8))
def test_desc_order_covers_every_block_once(bm, seed):
    rng = np.random.default_rng(100 + seed)
    S = int(rng.integers(1, 70)) if seed < 6 else int(rng.integers(65, 120))
    lens = rng.integers(0, 6 * bm, size=S)
    lens[rng.random(S) < 0.2] = 0
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    n_rank = (T + bm - 1) // bm + S  # block_upper_bound
    got = [lookup_desc(cu, bm, r, n_rank) for r in range(n_rank)]
    blocks = [g for g in got if g is not None]
    want = {(s, b) for s in range(S) for b in range((int(lens[s]) + bm - 1) // bm)}
    assert len(blocks) == len(want) and set(blocks) == want
    if S <= 64:
        # decreasing block index, ties by sequence; every empty rank after the blocks
        assert blocks == sorted(want, key=lambda x: (-x[1], x[0]))
        assert all(g is not None for g in got[:len(want)])


@pytest.mark.parametrize("n_heads", [16, 8, 32, 12, 3])
def test_head_rank_covers_grid(n_heads):
    n_rank = 37
    grid = (n_heads * n_rank + 7) // 8 * 8
    seen = [head_rank(b, grid, n_heads, n_rank) for b in range(grid)]
    real = [x for x in seen if x[0] < n_heads]
    assert sorted(real) == [(h, r) for h in range(n_heads) for r in range(n_rank)]
    if n_heads % 8 == 0:
        for b, (h, r) in enumerate(seen):  # each XCD owns whole heads, rank-major
            assert h // (n_heads // 8) == b % 8
        for x in range(8):
            ranks = [seen[b][1] for b in range(x, grid, 8)]
            assert ranks == sorted(ranks)

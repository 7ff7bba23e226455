"""The workgroup -> (sequence, block) numbering the HIP kernels compute in-kernel from
cu_seqlens (find_block in csrc/common.h): sequence s owns the ceil(L_s/bm) consecutive
ids starting at first(s) = floor(cu[s]/bm) + s. Checked here on the host, by brute
force over random packings, for the properties the launches rely on: every block has
exactly one id, ids of one sequence are consecutive, and every id is below the grid
size block_upper_bound = ceil(T/bm) + S. CPU only."""
import numpy as np
import pytest


def bounds(cu, s, T):
    """seq_bounds: the entries clamped to [0, T], the end to at least the start."""
    c0 = min(max(int(cu[s]), 0), T)
    return c0, max(min(int(cu[s + 1]), T), c0)


def first_ids(cu, bm, T=None):
    T = int(cu[-1]) if T is None else T
    return [bounds(cu, s, T)[0] // bm + s for s in range(len(cu) - 1)]


def lookup(cu, bm, target, T=None, with_bounds=False):
    """Device algorithm of find_block: per group of 64 sequences, the last one whose
    first(s) <= target (the next group only when the group's last one qualifies), then a
    range check."""
    T = int(cu[-1]) if T is None else T
    f = first_ids(cu, bm, T)
    cand = -1
    for base in range(0, len(f), 64):
        lanes = [l for l in range(min(64, len(f) - base)) if f[base + l] <= target]
        if not lanes:
            break
        cand = base + lanes[-1]
        if lanes[-1] < 63:
            break
    if cand < 0:
        return None
    c0, c1 = bounds(cu, cand, T)
    blk = target - f[cand]
    if blk >= (c1 - c0 + bm - 1) // bm:
        return None
    return (cand, blk, c0, c1 - c0) if with_bounds else (cand, blk)


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


def lookup_desc(cu, bm, rank, n_rank, T=None, with_bounds=False):
    """Device algorithm of find_block_desc: blocks in decreasing block index (ties in
    increasing sequence), through the binary search over C(b) = sum_s max(0, n_s - b)."""
    T = int(cu[-1]) if T is None else T
    S = len(cu) - 1
    if S > 64:
        return lookup(cu, bm, n_rank - 1 - rank, T, with_bounds)
    bnd = [bounds(cu, s, T) for s in range(S)]
    n = [(c1 - c0 + bm - 1) // bm for c0, c1 in bnd]
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
    s = level[j]
    return (s, lo, bnd[s][0], bnd[s][1] - bnd[s][0]) if with_bounds else (s, lo)


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


@pytest.mark.parametrize("desc", [False, True], ids=["find_block", "find_block_desc"])
@pytest.mark.parametrize("seed", range(12))
def test_any_cu_seqlens_content_stays_inside_the_rows(desc, seed):
    """Whatever cu_seqlens holds (negative entries, entries past T, decreasing runs, a
    first entry above 0), every block the lookup returns lies inside the T rows: start >= 0,
    start + length <= T and block * bm < length, for every id of the launch's grid. For
    valid packings the clamps change nothing (the tests above)."""
    rng = np.random.default_rng(500 + seed)
    bm = 64
    S = int(rng.integers(1, 70)) if seed % 3 else int(rng.integers(65, 140))
    T = int(rng.integers(1, 40 * bm))
    cu = rng.integers(-3 * bm, T + 3 * bm, size=S + 1)
    if seed % 2:  # mostly increasing with a few disorders
        cu = np.sort(cu)
        for _ in range(3):
            i, j = rng.integers(0, S + 1, size=2)
            cu[i], cu[j] = cu[j], cu[i]
    n_rank = (T + bm - 1) // bm + S
    for r in range(n_rank):
        got = lookup_desc(cu, bm, r, n_rank, T, True) if desc else lookup(cu, bm, r, T, True)
        if got is None:
            continue
        s, blk, start, length = got
        assert 0 <= s < S and blk >= 0
        assert 0 <= start and start + length <= T and blk * bm < length

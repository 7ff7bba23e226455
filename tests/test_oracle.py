"""Pins the CPU oracle (oracle/dsalt_oracle.py) against closed forms, library routines,
brute force and finite differences. CPU only."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dsalt_oracle as orc


def _rand_qkv(T, H, D, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(T, H, D, generator=g, dtype=dtype) for _ in range(3)]


# ---------------------------------------------------------------- attention closed forms

@pytest.mark.parametrize("lens", [[37], [16, 1, 29]])
def test_hard_full_window_is_causal_attention(lens):
    cu = np.cumsum([0] + lens)
    T, H, D = int(cu[-1]), 3, 8
    q, k, v = _rand_qkv(T, H, D, 1)
    w = torch.full((T,), 1e6)
    o, lse = orc.attention_hard(q, k, v, w, None, None, cu)
    for s in range(len(lens)):
        a, b = cu[s], cu[s + 1]
        ref = F.scaled_dot_product_attention(*(t[a:b].transpose(0, 1) for t in (q, k, v)), is_causal=True)
        torch.testing.assert_close(o[a:b], ref.transpose(0, 1), rtol=1e-10, atol=1e-10)
        sc = torch.einsum("ihd,jhd->hij", q[a:b], k[a:b]) / math.sqrt(D)
        sc = sc.masked_fill(torch.ones(b - a, b - a, dtype=torch.bool).triu(1), float("-inf"))
        torch.testing.assert_close(lse[a:b], torch.logsumexp(sc, -1).T, rtol=1e-10, atol=1e-10)


def test_soft_full_window_is_causal_attention():
    T, H, D = 40, 2, 16
    q, k, v = _rand_qkv(T, H, D, 2)
    w = torch.full((T,), 1000.5, dtype=torch.float64)
    o, _ = orc.attention_soft(q, k, v, w, None, None, [0, T])
    ref = F.scaled_dot_product_attention(*(t.transpose(0, 1) for t in (q, k, v)), is_causal=True)
    torch.testing.assert_close(o, ref.transpose(0, 1), rtol=1e-10, atol=1e-10)


def test_window_one_no_landmarks_is_identity():
    T, H, D = 23, 4, 8
    q, k, v = _rand_qkv(T, H, D, 3)
    o, lse = orc.attention_hard(q, k, v, torch.ones(T), None, None, [0, 10, T])
    torch.testing.assert_close(o, v, rtol=0, atol=1e-12)
    torch.testing.assert_close(lse, (q * k).sum(-1) / math.sqrt(D), rtol=1e-12, atol=1e-12)


def test_constant_landmark_bias_closed_form():
    # w = 1 and every position a landmark with bias c:
    # O_i = (e^{s_ii} v_i + e^c sum_{j<i} e^{s_ij} v_j) / (e^{s_ii} + e^c sum_{j<i} e^{s_ij})
    T, H, D, c = 12, 2, 4, 0.7
    q, k, v = _rand_qkv(T, H, D, 4)
    pos = torch.arange(T).repeat(H, 1).unsqueeze(1)
    bias = torch.full((H, 1, T), c, dtype=torch.float64)
    o, _ = orc.attention_hard(q, k, v, torch.ones(T), pos, bias, [0, T])
    for h in range(H):
        for i in range(T):
            num = torch.zeros(D, dtype=torch.float64)
            den = 0.0
            for j in range(i + 1):
                e = math.exp(float(q[i, h] @ k[j, h]) / math.sqrt(D) + (0.0 if j == i else c))
                num += e * v[j, h]
                den += e
            torch.testing.assert_close(o[i, h], num / den, rtol=1e-12, atol=1e-12)


def test_soft_sharp_edge_limit_is_hard():
    # tau -> 0 with non-integral w~: the soft band becomes [i - floor(w~), i] and the
    # landmark rule p < i - w~ becomes p <= i - (floor(w~) + 1): HARD with w = floor(w~)+1.
    T, H, D = 48, 2, 8
    q, k, v = _rand_qkv(T, H, D, 5)
    g = torch.Generator().manual_seed(6)
    w_cont = (torch.rand(T, generator=g) * 20 + 1.0).to(torch.float32)
    w_cont = torch.where((w_cont - w_cont.floor()) < 0.05, w_cont + 0.25, w_cont).double()
    pos = torch.stack([torch.randperm(T, generator=g)[:6] for _ in range(H)]).unsqueeze(1)
    logw = torch.zeros(H, 1, 6, dtype=torch.float64)
    o_s, _ = orc.attention_soft(q, k, v, w_cont, pos, logw, [0, T], tau_win=1e-4, win_edge=4.0)
    o_h, _ = orc.attention_hard(q, k, v, w_cont.floor() + 1, pos, logw, [0, T])
    torch.testing.assert_close(o_s, o_h, rtol=1e-9, atol=1e-9)


def test_soft_edge_two_keys_closed_form():
    # one query at i = 3 with w~ = 1.3: keys j = 3 (d = 0) and j = 2 (d = 1) are in the band,
    # both on the edge (win_edge = 4); bias log(1 / (1 + exp(-(w~ - d)/tau))).
    D, tau, wt = 4, 0.8, 1.3
    q, k, v = _rand_qkv(4, 1, D, 7)
    w = torch.tensor([1.3, 1.3, 1.3, wt], dtype=torch.float64)
    o, _ = orc.attention_soft(q, k, v, w, None, None, [0, 4], tau_win=tau, win_edge=4.0)
    logit = {}
    for j, d in ((3, 0.0), (2, 1.0)):
        b = math.log(1.0 / (1.0 + math.exp(-(wt - d) / tau)))
        logit[j] = float(q[3, 0] @ k[j, 0]) / math.sqrt(D) + b
    m = max(logit.values())
    den = sum(math.exp(x - m) for x in logit.values())
    ref = sum(math.exp(logit[j] - m) * v[j, 0] for j in logit) / den
    torch.testing.assert_close(o[3, 0], ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- selection

def _rand_select_case(seed, S=3, H=4, maxlen=40):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, maxlen, S)
    lens[0] = max(lens[0], 1)
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    scores = rng.standard_normal((T, H)).astype(np.float32)
    scores = np.round(scores * 2) / 2  # many ties
    scores[rng.random((T, H)) < 0.05] = np.nan
    scores[rng.random((T, H)) < 0.05] = np.inf
    scores[rng.random((T, H)) < 0.05] = -np.inf
    scores[rng.random((T, H)) < 0.05] = -0.0
    w = (rng.random(T) * 12).astype(np.float32)
    w[rng.random(T) < 0.05] = np.nan
    return scores, w, cu


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("k", [1, 5, 16])
def test_select_matches_bruteforce(seed, k):
    scores, w, cu = _rand_select_case(seed)
    np.testing.assert_array_equal(orc.select_landmarks(scores, w, cu, k),
                                  orc.select_landmarks_bruteforce(scores, w, cu, k))


@pytest.mark.parametrize("seed", range(4))
def test_select_matches_torch_topk_as_sets(seed):
    # the reference's own computation (selectors.py:105-134), no ties: sets must agree
    rng = np.random.default_rng(100 + seed)
    lens = [33, 50, 17]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, H, k = int(cu[-1]), 3, 20
    scores = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.random(T) * 25 + 1).astype(np.float32)
    got = orc.select_landmarks(scores, w, cu, k)
    sc = torch.from_numpy(scores)
    off = torch.cat([torch.arange(l) for l in lens])
    sc = sc.masked_fill((off < torch.from_numpy(w).long()).unsqueeze(1), float("-inf"))
    for s, L in enumerate(lens):
        k_eff = min(k, L)
        vals, idx = torch.topk(sc[cu[s]:cu[s + 1]].T, k_eff, dim=1, sorted=False)
        idx = torch.where(torch.isfinite(vals), idx, -1)
        for h in range(H):
            ref = sorted(i for i in idx[h].tolist() if i >= 0)
            mine = [i for i in got[h, s].tolist() if i >= 0]
            assert mine == ref
            assert all(x == -1 for x in got[h, s, len(mine):])


def test_select_covered_never_chosen_and_short_sequences():
    cu = np.array([0, 3, 10])
    scores = np.arange(10 * 2, dtype=np.float32).reshape(10, 2)
    w = np.array([2, 2, 2, 0.5, 0.5, 6.9, 6.9, 6.9, 6.9, 6.9], dtype=np.float32)
    got = orc.select_landmarks(scores, w, cu, 4)
    # seq 0: offsets 0,1 covered (o < 2); only offset 2 left
    assert got[0, 0].tolist() == [2, -1, -1, -1]
    # seq 1: offsets o with o < trunc(w): o=2 (w=6.9 -> 6): covered; 0,1 (w=.5 -> 0) not
    assert got[1, 1].tolist() == [0, 1, 6, -1]


def test_quantize():
    w = np.array([0.2, 1.0, 1.99, 2.5, 255.999, np.nan, -3.0], dtype=np.float32)
    q = orc.quantize_windows(w)
    np.testing.assert_array_equal(q[[0, 1, 2, 3, 4, 6]], np.array([1, 1, 1, 2, 255, 1], dtype=np.float32))
    assert np.isnan(q[5])
    t = torch.from_numpy(w).floor().clamp(min=1).numpy()
    np.testing.assert_array_equal(np.isnan(t), np.isnan(q))
    np.testing.assert_array_equal(t[~np.isnan(t)], q[~np.isnan(q)])


def test_hybrid_scores_against_numpy():
    rng = np.random.default_rng(3)
    T, d, H, dh = 50, 32, 4, 8
    x = rng.standard_normal((T, d))
    W = rng.standard_normal((H * dh, d))
    alpha = rng.random(H)
    s, zx, zv = orc.hybrid_scores(torch.from_numpy(x), torch.from_numpy(W), torch.from_numpy(alpha), H, dh)
    xn = np.linalg.norm(x, axis=1)
    zx_ref = (xn - xn.mean()) / xn.std(ddof=1)
    vn = np.linalg.norm((x @ W.T).reshape(T, H, dh), axis=2)
    zv_ref = (vn - vn.mean(0)) / vn.std(0, ddof=1)
    np.testing.assert_allclose(zx.numpy(), zx_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(zv.numpy(), zv_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(s.numpy(), alpha * zv_ref + (1 - alpha) * zx_ref[:, None], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n_kv", [4, 2, 1], ids=["mha", "gqa2", "mqa"])
def test_hybrid_scores_from_v_is_the_gemm_path(n_kv):
    # given v = x W_V^T, the from-v restatement is the same computation as hybrid_scores
    # (landmark_tokens_ker.py:45-61), bit for bit in float64; GQA repeats z_v per group
    rng = np.random.default_rng(4)
    T, d, H, dh = 40, 32, 4, 8
    x = torch.from_numpy(rng.standard_normal((T, d)))
    W = torch.from_numpy(rng.standard_normal((n_kv * dh, d)))
    alpha = torch.from_numpy(rng.random(H))
    ref = orc.hybrid_scores(x, W, alpha, H, dh)
    got = orc.hybrid_scores_from_v(x, (x @ W.T).view(T, n_kv, dh), alpha, H)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    # and against numpy, with the group repeat written out
    vn = np.linalg.norm((x.numpy() @ W.numpy().T).reshape(T, n_kv, dh), axis=2)
    zv = np.repeat((vn - vn.mean(0)) / vn.std(0, ddof=1), H // n_kv, axis=1)
    np.testing.assert_allclose(got[2].numpy(), zv, rtol=1e-5, atol=1e-5)  # .float(): fp32 norms


def test_hybrid_scores_single_token_is_nan():
    # one token: the unbiased std is 0/0 = NaN, clamp(min=1e-6) keeps it (torch semantics)
    x = torch.ones(1, 8, dtype=torch.float64)
    s, zx, zv = orc.hybrid_scores_from_v(x, torch.ones(1, 2, 4, dtype=torch.float64),
                                         torch.full((2,), 0.5, dtype=torch.float64), 2)
    assert torch.isnan(s).all() and torch.isnan(zx).all()


def test_rope_oracle_pins():
    # against the package's eager restatement of window_utils.py:73-88 (float64), the
    # identity at cos = 1, sin = 0, and norm preservation of every rotated pair
    import sys
    sys.path.insert(0, "dsalt-library_amd")
    from dsalt.kernels.window_utils import apply_rotary_emb, build_rope_cache
    g = torch.Generator().manual_seed(9)
    cu = [0, 5, 12]
    T, H, D = 12, 3, 8
    q, k = torch.randn(T, H, D, generator=g, dtype=torch.float64), torch.randn(T, 2, D, generator=g, dtype=torch.float64)
    cos, sin = build_rope_cache(16, D, torch.device("cpu"), dtype=torch.float64)
    pos = orc.seq_positions(cu)
    assert pos.tolist() == [0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 5, 6]
    rq, rk = orc.rope(q, k, cos, sin, pos)
    eq, ek = apply_rotary_emb(q, k, cos[pos].unsqueeze(1), sin[pos].unsqueeze(1))
    assert torch.allclose(rq, eq, atol=1e-14) and torch.allclose(rk, ek, atol=1e-14)
    iq, _ = orc.rope(q, k, torch.ones_like(cos), torch.zeros_like(sin), pos)
    assert torch.equal(iq, q)
    pair = lambda x: x[..., : D // 2] ** 2 + x[..., D // 2:] ** 2
    assert torch.allclose(pair(rq), pair(q), atol=1e-12)


# ---------------------------------------------------------------- gradients

def test_gradcheck_hard():
    T, H, D = 9, 2, 4
    q, k, v = (t.requires_grad_() for t in _rand_qkv(T, H, D, 8))
    pos = torch.tensor([[[0, 2, 5]], [[1, -1, 3]]])
    bias = torch.randn(H, 1, 3, dtype=torch.float64, requires_grad=True)
    w = torch.tensor([1, 2, 3, 1, 2, 3, 1, 2, 3], dtype=torch.float32)

    def f(q, k, v, bias):
        return orc.attention_hard(q, k, v, w, pos, bias, [0, T])[0]

    assert torch.autograd.gradcheck(f, (q, k, v, bias))


def test_gradcheck_soft():
    T, H, D = 10, 2, 4
    q, k, v = (t.requires_grad_() for t in _rand_qkv(T, H, D, 9))
    pos = torch.tensor([[[0, 2]], [[1, 4]]])
    logw = torch.randn(H, 1, 2, dtype=torch.float64, requires_grad=True)
    w = torch.tensor([1.3, 2.6, 5.5, 4.2, 6.7, 1.8, 3.3, 7.4, 2.2, 4.9], dtype=torch.float64,
                     requires_grad=True)

    def f(q, k, v, logw, w):
        return orc.attention_soft(q, k, v, w, pos, logw, [0, T], tau_win=0.7, win_edge=2.0)[0]

    assert torch.autograd.gradcheck(f, (q, k, v, logw, w))


# ---------------------------------------------------------------- counting / baseline

def test_effective_pairs_counts_the_mask():
    rng = np.random.default_rng(11)
    lens = [30, 7, 45]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, H, k = int(cu[-1]), 3, 6
    w = (rng.random(T) * 12 + 1).astype(np.float32)
    pos = np.full((H, 3, k), -1)
    for h in range(H):
        for s, L in enumerate(lens):
            c = rng.choice(L, size=min(k, L), replace=False)
            pos[h, s, :len(c)] = np.sort(c)
    total = sum(int(orc.hard_mask(L, w[cu[s]:cu[s + 1]], pos[:, s]).sum()) for s, L in enumerate(lens))
    assert orc.effective_pairs("hard", w, pos, cu, H) == total


def test_cpu_baseline_matches_hard_oracle():
    rng = np.random.default_rng(12)
    lens = [64, 40]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, H, D, k = int(cu[-1]), 2, 16, 5
    q, k_, v = _rand_qkv(T, H, D, 13, torch.float32)
    w = (rng.random(T) * 10 + 1).astype(np.float32)
    pos = np.stack([np.stack([np.sort(rng.choice(L, k, replace=False)) for L in lens]) for _ in range(H)])
    outs = orc.cpu_baseline_hard(q, k_, v, w, pos, cu)
    o, _ = orc.attention_hard(q.double(), k_.double(), v.double(), w, torch.from_numpy(pos), None, cu)
    torch.testing.assert_close(torch.cat(outs).double(), o, rtol=1e-5, atol=1e-5)

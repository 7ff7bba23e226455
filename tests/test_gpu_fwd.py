"""Forward parity: HIP sparse attention (through the C ABI via dsalt._hip) against the
fp64 CPU oracle on the same bf16/fp16 inputs. Tolerance (north star): max-abs 2e-2 and
relative L2 1e-2 of the outputs; LSE within 2e-2 and -inf exactly on empty rows."""
import math

import numpy as np
import pytest
import torch

import dsalt._hip as hip
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, LSE_ABS = 2e-2, 1e-2, 2e-2


def close(got, ref, what, max_abs=MAX_ABS, rel_l2=REL_L2):
    got, ref = got.double().cpu(), ref.double().cpu()
    diff = got - ref
    ma = diff.abs().max().item() if diff.numel() else 0.0
    rl = (diff.norm() / ref.norm().clamp_min(1e-30)).item() if diff.numel() else 0.0
    mr = ref.abs().max().item() if ref.numel() else 0.0
    print(f"  {what}: max-abs {ma:.3e} (bar {max_abs:.3e}), rel-L2 {rl:.3e}, max |ref| {mr:.3e}", flush=True)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max-abs {ma:.3e}, rel-L2 {rl:.3e}"


def summed_grad_bar(ref):
    """Max-abs bar of a gradient that is a sum over every query attending to a key or a
    landmark slot (d_lmk_bias / d_logw, d_w~): 2e-2 times the largest reference value,
    at least the absolute 2e-2. Each summand carries the 16-bit rounding of P and dS, so
    the error of the sum grows with its magnitude (these synthetic inputs reach |ref| ~ 10);
    the relative-L2 bar stays 1e-2. The measured errors are printed by close()."""
    return 2e-2 * max(ref.abs().max().item() if ref.numel() else 0.0, 1.0)


def lse_close(got, ref, what):
    got, ref = got.double().cpu(), ref.double().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin), f"{what}: empty-row pattern differs"
    if fin.any():
        d = (got[fin] - ref[fin]).abs().max().item()
        assert d <= LSE_ABS, f"{what}: LSE max-abs {d:.3e}"


def make_inputs(lens, H, D, k, mode, seed, dtype=torch.bfloat16, n_min=8, n_max=64,
                lmk_kind="random"):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, S = int(cu[-1]), len(lens)
    q, kk, v = (torch.randn(T, H, D, generator=g).to(dtype) for _ in range(3))
    w_cont = (n_min + torch.rand(T, generator=g) * (n_max - n_min)).float()
    w = w_cont.floor().clamp(min=1) if mode == hip.MODE_HARD else w_cont
    pos = np.full((H, S, k), -1, dtype=np.int64)
    for h in range(H):
        for s, L in enumerate(lens):
            if L == 0 or k == 0:
                continue
            if lmk_kind == "random":
                c = rng.choice(L, size=min(k, L), replace=False)
                pos[h, s, :len(c)] = c  # unsorted
            elif lmk_kind == "messy":  # unsorted, duplicates, -1 holes, out-of-range
                c = rng.integers(-2, L + 3, size=k)
                pos[h, s] = c
    pos = torch.from_numpy(pos)
    if mode == hip.MODE_HARD:
        bias = torch.randn(H, S, k, generator=g)
    else:
        bias = torch.nn.functional.logsigmoid(torch.randn(H, S, k, generator=g) / 2)
        bias = torch.where(pos >= 0, bias, torch.full_like(bias, float("-inf")))
    return q, kk, v, w, pos, bias, torch.from_numpy(cu).to(torch.int32)


def run_hip(mode, q, k, v, w, pos, bias, cu, **kw):
    dev = torch.device("cuda", 0)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    posd = pos.to(dev) if pos is not None and pos.shape[-1] > 0 else None
    biasd = bias.to(dev) if posd is not None and bias is not None else None
    out, lse = hip.fwd(mode, qd, kd, vd, w.to(dev), posd, biasd, cu.to(dev), 1.0 / math.sqrt(q.shape[-1]), **kw)
    torch.cuda.synchronize()
    return out.float().cpu(), lse.cpu()


def run_oracle(mode, q, k, v, w, pos, bias, cu, rows=None, **kw):
    q64, k64, v64 = (t.double() for t in (q, k, v))
    if mode == hip.MODE_HARD:
        return orc.attention_hard(q64, k64, v64, w, pos, None if bias is None else bias.double(), cu.tolist(),
                                  rows=rows, **kw)
    return orc.attention_soft(q64, k64, v64, w.double(), pos, None if bias is None else bias.double(),
                              cu.tolist(), rows=rows, **kw)


CASES = [
    # lens, H, D, k, n_min, n_max, lmk_kind
    ([1, 2, 3, 130], 2, 64, 5, 1, 9, "random"),
    ([300, 77, 513], 3, 128, 20, 8, 96, "random"),
    ([200, 0, 129], 2, 64, 100, 4, 40, "messy"),
    ([64, 191], 2, 128, 0, 1, 300, "random"),
    ([1024], 8, 64, 16, 64, 256, "random"),
]


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_fwd_matches_oracle(mode, case):
    lens, H, D, k, n_min, n_max, kind = CASES[case]
    print(f"fwd case={case} mode={mode} lens={lens} H={H} D={D} k={k}", flush=True)
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed=case, n_min=n_min, n_max=n_max,
                                             lmk_kind=kind)
    out, lse = run_hip(mode, q, kk, v, w, pos, bias, cu)
    o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu)
    close(out, o_ref, f"out case {case}")
    lse_close(lse, l_ref, f"lse case {case}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_fwd_dtypes(dtype):
    lens, H, D, k = [257, 100], 2, 64, 12
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, hip.MODE_HARD, seed=7, dtype=dtype, n_max=120)
    out, lse = run_hip(hip.MODE_HARD, q, kk, v, w, pos, bias, cu)
    o_ref, l_ref = run_oracle(hip.MODE_HARD, q, kk, v, w, pos, bias, cu)
    close(out, o_ref, f"out {dtype}")
    lse_close(lse, l_ref, f"lse {dtype}")


def test_fwd_soft_edges_and_empty_rows():
    # integral w~ (exact band j >= i - w~), negative w~ (empty band), tiny w~ (edge only)
    lens, H, D, k = [150], 2, 64, 8
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, hip.MODE_SOFT, seed=8, n_min=2, n_max=30)
    w = w.clone()
    w[::3] = w[::3].floor()           # integral windows
    w[5:20] = -3.0                     # no band keys
    w[20:30] = 0.5                     # only d = 0, on the soft edge
    out, lse = run_hip(hip.MODE_SOFT, q, kk, v, w, pos, bias, cu, tau_win=0.7, win_edge=3.0)
    o_ref, l_ref = run_oracle(hip.MODE_SOFT, q, kk, v, w, pos, bias, cu, tau_win=0.7, win_edge=3.0)
    close(out, o_ref, "soft edges")
    lse_close(lse, l_ref, "soft edges lse")


def test_fwd_full_window_equals_causal_sdpa():
    lens, H, D = [333], 4, 128
    q, kk, v, _, _, _, cu = make_inputs(lens, H, D, 0, hip.MODE_HARD, seed=9)
    w = torch.full((333,), 1e6)
    out, _ = run_hip(hip.MODE_HARD, q, kk, v, w, None, None, cu)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().transpose(0, 1) for t in (q, kk, v)), is_causal=True).transpose(0, 1)
    close(out, ref, "causal")


def test_fwd_strided_operands():
    # q/k/v as views of one [T, 3, H, D] buffer (row stride 3*H*D), output written in place
    T, H, D = 300, 4, 64
    g = torch.Generator().manual_seed(10)
    qkv = torch.randn(T, 3, H, D, generator=g).to(torch.bfloat16)
    q, kk, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    cu = torch.tensor([0, 120, 300], dtype=torch.int32)
    w = (torch.rand(T, generator=g) * 50 + 1).floor()
    pos = torch.stack([torch.stack([torch.randperm(120, generator=g)[:10], torch.randperm(180, generator=g)[:10]])
                       for _ in range(H)])
    bias = torch.randn(H, 2, 10, generator=g)
    dev = torch.device("cuda", 0)
    qkv_d = qkv.to(dev)
    out = torch.empty(T, H, 2 * D, device=dev, dtype=torch.bfloat16)[:, :, :D]  # strided output
    o, lse = hip.fwd(hip.MODE_HARD, qkv_d[:, 0], qkv_d[:, 1], qkv_d[:, 2], w.to(dev), pos.to(dev), bias.to(dev),
                     cu.to(dev), 1.0 / math.sqrt(D), out=out)
    torch.cuda.synchronize()
    o_ref, _ = run_oracle(hip.MODE_HARD, q, kk, v, w, pos, bias, cu)
    close(o.float().cpu(), o_ref, "strided")


@pytest.mark.parametrize("cfg", ["c2", "c4"])
def test_fwd_headline_shapes_on_row_subsets(cfg):
    # full-size launches; the oracle checks a window of query rows of every sequence
    if cfg == "c2":
        lens, H, D, k, n_min, n_max, rows = [2048] * 4, 16, 64, 64, 32, 512, (1536, 1792)
    else:
        lens, H, D, k, n_min, n_max, rows = [16384], 16, 128, 128, 64, 1024, (15872, 16128)
    print(f"fwd headline {cfg}", flush=True)
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, hip.MODE_HARD, seed=11, n_min=n_min, n_max=n_max)
    out, lse = run_hip(hip.MODE_HARD, q, kk, v, w, pos, bias, cu)
    o_ref, l_ref = run_oracle(hip.MODE_HARD, q, kk, v, w, pos, bias, cu, rows=rows)
    sel = torch.cat([torch.arange(int(cu[s]) + rows[0], int(cu[s]) + rows[1]) for s in range(len(lens))])
    close(out[sel], o_ref, cfg)
    lse_close(lse[sel], l_ref, cfg + " lse")


def test_fwd_many_sequences():
    # more than 64 sequences (the block lookup scans cu_seqlens 64 entries at a time),
    # empty ones included, lengths not multiples of the 128-query block
    rng = np.random.default_rng(13)
    lens = [int(x) for x in rng.integers(0, 70, size=150)]
    lens[3] = lens[77] = lens[149] = 0
    lens[64] = 300
    for mode in (hip.MODE_HARD, hip.MODE_SOFT):
        print(f"fwd many sequences mode={mode}", flush=True)
        q, kk, v, w, pos, bias, cu = make_inputs(lens, 2, 64, 6, mode, seed=13, n_min=2, n_max=40)
        out, lse = run_hip(mode, q, kk, v, w, pos, bias, cu)
        o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu)
        close(out, o_ref, f"many sequences {mode}")
        lse_close(lse, l_ref, f"many sequences {mode} lse")


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
def test_fwd_negative_scale(mode):
    lens, H, D, k = [200, 61], 2, 64, 9
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed=14, n_min=4, n_max=90)
    dev = torch.device("cuda", 0)
    scale = -0.3
    out, lse = hip.fwd(mode, q.to(dev), kk.to(dev), v.to(dev), w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev),
                       scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu, scale=scale)
    close(out.cpu(), o_ref, "negative scale")
    lse_close(lse.cpu(), l_ref, "negative scale lse")


# ------------------------------------------------------------------- selection

def _select_case(seed, lens, H, tie=True):
    rng = np.random.default_rng(seed)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    scores = rng.standard_normal((T, H)).astype(np.float32)
    if tie:
        scores = np.round(scores * 4) / 4
        scores[rng.random((T, H)) < 0.02] = np.nan
        scores[rng.random((T, H)) < 0.02] = np.inf
        scores[rng.random((T, H)) < 0.02] = -np.inf
        scores[rng.random((T, H)) < 0.02] = -0.0
    w = (rng.random(T) * 60).astype(np.float32)
    w[rng.random(T) < 0.02] = np.nan
    return scores, w, cu


@pytest.mark.parametrize("lens,H,k", [
    ([50, 0, 7, 300], 4, 16),
    ([2048] * 4, 16, 64),
    ([1448, 783, 749, 1864, 1814, 555, 722, 1355], 16, 64),
    ([20000, 33], 2, 128),     # longer than the LDS key cache
    ([5, 900], 3, 1024),
])
@pytest.mark.parametrize("tie", [True, False], ids=["ties", "distinct"])
def test_select_bit_exact(lens, H, k, tie):
    print(f"select lens={lens[:3]} H={H} k={k} tie={tie}", flush=True)
    scores, w, cu = _select_case(len(lens) * 31 + k, lens, H, tie)
    dev = torch.device("cuda", 0)
    got = hip.select_landmarks(torch.from_numpy(scores).to(dev), torch.from_numpy(w).to(dev),
                               torch.from_numpy(cu).to(torch.int32).to(dev), k).cpu().numpy()
    np.testing.assert_array_equal(got, orc.select_landmarks(scores, w, cu, k))


@pytest.mark.parametrize("k", [64, 65, 63, 100])
def test_select_clusters(k):
    """Clusters of equal scores: the first radix pass can already hold exactly the keys
    still needed (k = 64: the top cluster), or the boundary falls inside a cluster of
    ties (k = 63, 65) or on a cluster edge deeper down (k = 100)."""
    rng = np.random.default_rng(k)
    lens, H = [700, 2048, 150], 3
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    scores = np.ones((T, H), np.float32)
    for s0, L in zip(cu[:-1], lens):
        idx = rng.permutation(L)
        scores[s0 + idx[:64]] = 5.0           # top cluster of 64 equal scores
        scores[s0 + idx[64:100]] = 3.0        # next cluster of 36
        scores[s0 + idx[100:130]] = rng.standard_normal((30, H)).astype(np.float32)
    w = np.zeros(T, np.float32)               # nothing covered
    dev = torch.device("cuda", 0)
    got = hip.select_landmarks(torch.from_numpy(scores).to(dev), torch.from_numpy(w).to(dev),
                               torch.from_numpy(cu).to(torch.int32).to(dev), k).cpu().numpy()
    np.testing.assert_array_equal(got, orc.select_landmarks(scores, w, cu, k))


def test_select_strided_scores():
    scores, w, cu = _select_case(5, [100, 60], 8)
    dev = torch.device("cuda", 0)
    big = torch.zeros(scores.shape[0], 16, device=dev)
    big[:, ::2] = torch.from_numpy(scores).to(dev)
    got = hip.select_landmarks(big[:, ::2], torch.from_numpy(w).to(dev), torch.from_numpy(cu).int().to(dev), 9)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.select_landmarks(scores, w, cu, 9))


def _select_gpu(scores, w, cu, k, chunked=True):
    dev = torch.device("cuda", 0)
    return hip.select_landmarks(torch.from_numpy(scores).to(dev), torch.from_numpy(w).to(dev),
                                torch.from_numpy(cu).to(torch.int32).to(dev), k, chunked=chunked).cpu().numpy()


@pytest.mark.parametrize("lens,H,k", [
    ([4097, 6000, 50, 16384], 2, 64),      # just past the chunk-wise threshold, ragged last chunks
    ([8193, 4096, 12000], 3, 1),
    ([6000, 16384], 2, 896),               # 8 chunks x (896 + 128) slots: the gather's capacity
    ([20000, 5000], 2, 1024),              # 10 x 1152 slots > capacity: one workgroup per sequence
    ([300, 4500, 7, 9000], 2, 128),
])
@pytest.mark.parametrize("tie", [True, False], ids=["ties", "distinct"])
def test_select_chunked_bit_exact(lens, H, k, tie):
    """Sequences longer than 4096 tokens go through the per-chunk candidates (the chunk's
    top k, or a superset of at most k + min(k, 128) when the first radix pass bounds one)
    and the top-k of the chunks' candidates; same bar as the single-workgroup path: the
    oracle exactly."""
    print(f"select chunked lens={lens} H={H} k={k} tie={tie}", flush=True)
    scores, w, cu = _select_case(sum(lens) % 997 + k, lens, H, tie)
    np.testing.assert_array_equal(_select_gpu(scores, w, cu, k), orc.select_landmarks(scores, w, cu, k))


def test_select_chunked_concentrated_and_tied():
    """The top k all in one chunk (ascending scores: the last chunk supplies every pick,
    the others candidates that lose), one cluster of equal scores spanning every chunk
    (ties across chunk boundaries go to the lower position), and windows that cover
    most of a chunk (chunks with fewer than k candidates)."""
    lens, H, k = [10000, 9000, 6000], 3, 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    scores = np.zeros((T, H), np.float32)
    w = np.zeros(T, np.float32)
    for s, (s0, L) in enumerate(zip(cu[:-1], lens)):
        off = np.arange(L, dtype=np.float32)
        scores[s0:s0 + L, 0] = off                       # ascending
        scores[s0:s0 + L, 1] = 2.0                       # one cluster of ties
        scores[s0:s0 + L, 2] = -off                      # descending (first chunk wins)
        if s == 2:
            w[s0:s0 + L] = np.where(off < 4000, off + 1.0, 0.0)  # first 4000 tokens: every key covered
    np.testing.assert_array_equal(_select_gpu(scores, w, cu, k), orc.select_landmarks(scores, w, cu, k))


def test_select_chunked_equals_single_workgroup_c4():
    """Config 4's selection shape (one 16384-token sequence, 16 heads, k = 128): the
    chunk-wise and the single-workgroup selections agree bit for bit, and with the oracle."""
    print("select c4 chunked vs single", flush=True)
    scores, w, cu = _select_case(44, [16384], 16, tie=False)
    got = _select_gpu(scores, w, cu, 128)
    np.testing.assert_array_equal(got, _select_gpu(scores, w, cu, 128, chunked=False))
    np.testing.assert_array_equal(got, orc.select_landmarks(scores, w, cu, 128))


@pytest.mark.parametrize("lens,H,k", [
    ([50, 0, 7, 300], 4, 16),
    ([2048] * 4, 16, 64),                  # config 2's shape
    ([4097, 6000, 50, 16384], 2, 64),      # chunk-wise sequences write their windows from the chunks
    ([20000, 33], 2, 128),                 # longer than the LDS key cache (keys re-read)
    ([30, 70], 3, 0),                      # nothing to select: only the quantisation
])
def test_select_with_quantize_bit_exact(lens, H, k):
    """Selection with the window quantisation fused in (w_out): the quantised windows are
    the oracle's max(1, floor(w~)) (NaN kept) bit for bit, and the selection is the
    oracle's on those windows - including continuous windows below 1 (a token at offset
    0 is then covered) and NaN windows (never covered). In place (w_out = w) gives the
    same."""
    print(f"select+quantize lens={lens[:3]} H={H} k={k}", flush=True)
    scores, _, cu = _select_case(len(lens) * 7 + k, lens, H, tie=True)
    rng = np.random.default_rng(k + 3)
    T = scores.shape[0]
    w = (rng.random(T) * 80 - 10).astype(np.float32)   # includes w~ < 1 and negative
    w[rng.random(T) < 0.02] = np.nan
    w[rng.random(T) < 0.01] = np.inf
    dev = torch.device("cuda", 0)
    st = torch.from_numpy(scores).to(dev)
    cut = torch.from_numpy(cu).to(torch.int32).to(dev)
    wq, got = hip.select_landmarks_quantize(st, torch.from_numpy(w).to(dev), cut, k)
    wq_ref = orc.quantize_windows(w)
    np.testing.assert_array_equal(wq.cpu().numpy(), wq_ref)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.select_landmarks(scores, wq_ref, cu, k))
    # in place: the windows buffer receives the quantised values
    wbuf = torch.from_numpy(w).to(dev)
    out = torch.empty((H, len(lens), k), device=dev, dtype=torch.int64)
    a, _keep = hip._select_args(st, wbuf, cut, k, out, True, None, wbuf)
    assert hip.lib().dsalt_select_landmarks(hip.ctypes.byref(a), hip.stream_handle(dev)) == 0
    np.testing.assert_array_equal(wbuf.cpu().numpy(), wq_ref)
    np.testing.assert_array_equal(out.cpu().numpy(), got.cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("n_min,n_max", [(32, 512), (64, 1024), (7, 1000)])
def test_select_windows_from_gate_logits_bit_exact(dtype, n_min, n_max):
    """Windows formed in the selection launch from the window gate's 16-bit logits equal
    torch's own n_min + sigmoid(logits) * (n_max - n_min) in the logits' dtype, then
    max(1, floor(.)), bit for bit, for every logit value (65536 bit patterns, NaN and
    infinities included). (7, 1000): a span that bf16 cannot hold exactly. The selection
    on those windows equals the selection on torch's windows. (fp32 logits are refused:
    torch's fp32 sigmoid differs from 1 / (1 + exp(-x)) in the last bit for about one
    value in 10^6.)"""
    print(f"gate windows dtype={dtype} n_min={n_min} n_max={n_max}", flush=True)
    dev = torch.device("cuda", 0)
    logit = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(dtype).to(dev)
    T = logit.numel()
    with torch.no_grad():
        w_torch = n_min + torch.sigmoid(logit) * (n_max - n_min)   # the module's _window_continuous
        wq_ref = hip.quantize_windows(w_torch)
    lens = [T // 3, T - T // 3]
    cu = torch.tensor([0, lens[0], T], dtype=torch.int32, device=dev)
    scores = torch.randn(T, 2, device=dev)
    wq, lmk = hip.select_landmarks_quantize(scores, None, cu, 8, gate=(logit, n_min, n_max))
    same = (wq == wq_ref) | (torch.isnan(wq) & torch.isnan(wq_ref))
    assert bool(same.all()), f"{int((~same).sum())} windows differ from torch's, e.g. logit " \
                             f"{logit[~same][:4].tolist()}: {wq[~same][:4].tolist()} vs {wq_ref[~same][:4].tolist()}"
    assert torch.equal(lmk, hip.select_landmarks(scores, wq_ref, cu, 8))
    with pytest.raises(hip.DsaltError):
        hip.select_landmarks_quantize(scores, None, cu, 8, gate=(logit.float(), n_min, n_max))


def test_quantize_bit_exact():
    rng = np.random.default_rng(1)
    w = np.concatenate([rng.random(10000).astype(np.float32) * 600 - 50,
                        np.array([np.nan, 1.0, 0.999999, 2 ** 31, -np.inf, np.inf], dtype=np.float32)])
    dev = torch.device("cuda", 0)
    wq, wi = hip.quantize_windows(torch.from_numpy(w).to(dev), want_int=True)
    ref = orc.quantize_windows(w)
    np.testing.assert_array_equal(wq.cpu().numpy(), ref)
    exp_i = np.where(w >= 1, np.minimum(np.floor(np.nan_to_num(w, posinf=2 ** 30)), 2 ** 30), 1).astype(np.int32)
    np.testing.assert_array_equal(wi.cpu().numpy(), exp_i)


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
def test_fwd_fp32_output(mode):
    lens, H, D, k = [300, 45], 3, 128, 10
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed=12, n_min=4, n_max=80)
    dev = torch.device("cuda", 0)
    out, lse = hip.fwd(mode, q.to(dev), kk.to(dev), v.to(dev), w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev),
                       1.0 / math.sqrt(D), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu)
    close(out.cpu(), o_ref, "fp32 out")
    lse_close(lse.cpu(), l_ref, "fp32 out lse")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
@pytest.mark.parametrize("case", ["large", "small", "tiny", "underflow"])
def test_fwd_extreme_logits(mode, case, dtype):
    """Logits far from 0: tile sums beyond the 16-bit range ("large"), row totals of
    about 2^-40 ("small": kept as they are in bf16), about 2^-72 ("tiny") and P that all
    underflow in fp32 ("underflow") must still match the oracle."""
    print(f"extreme logits mode={mode} case={case} dtype={dtype}", flush=True)
    lens, H, D, k = [200, 77], 2, 64, 8
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed=21, dtype=dtype, n_min=4, n_max=90)
    scale = 1.0 / math.sqrt(D)
    if case == "large":
        scale = 8.0
    else:
        # Q and K along opposite directions: every q.k is about -a^2
        a = {"small": 15.0, "tiny": 20.0, "underflow": 40.0}[case]
        g = torch.Generator().manual_seed(5)
        u = torch.randn(D, generator=g)
        u = u / u.norm()
        q = (a * u + 0.1 * torch.randn(q.shape, generator=g)).to(dtype)
        kk = (-a * u + 0.1 * torch.randn(kk.shape, generator=g)).to(dtype)
    dev = torch.device("cuda", 0)
    out, lse = hip.fwd(mode, q.to(dev), kk.to(dev), v.to(dev), w.to(dev), pos.to(dev), bias.to(dev), cu.to(dev),
                       scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu, scale=scale)
    assert torch.isfinite(out).all()
    close(out.cpu(), o_ref, f"extreme {case}")
    lse_close(lse.cpu(), l_ref, f"extreme {case} lse")


@pytest.mark.parametrize("mode", [hip.MODE_HARD, hip.MODE_SOFT], ids=["hard", "soft"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("k", [300, 1024])
def test_fwd_many_landmarks(mode, D, k):
    """Up to DSALT_MAX_K_LMK landmark slots (k_pad 320: an odd number of 32-slot tiles;
    1024: 32 landmark tiles), with a sequence shorter than k (slots past its length stay
    empty)."""
    lens, H = [1300, 45, 700], 2
    print(f"fwd many landmarks mode={mode} D={D} k={k}", flush=True)
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, mode, seed=31, n_min=4, n_max=200)
    out, lse = run_hip(mode, q, kk, v, w, pos, bias, cu)
    o_ref, l_ref = run_oracle(mode, q, kk, v, w, pos, bias, cu)
    close(out, o_ref, f"many landmarks k={k}")
    lse_close(lse, l_ref, f"many landmarks k={k} lse")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("tau,edge", [(1.0, 4.0), (0.5, 2.5), (0.15, 4.0), (1.0, 8.0), (3.0, 9.0), (0.15, 12.0)],
                         ids=["t1-e4", "t0.5-e2.5", "t0.15-e4", "t1-e8", "t3-e9", "t0.15-e12"])
def test_fwd_soft_edge_params(D, tau, edge):
    """SOFT edge bias log sigmoid((w~ - d) / tau) over tau and win_edge. win_edge <= 4
    starts the scores from per-query rows of edge biases (the first three cases); wider
    edges bias every band element in the loop, with the factored exp(-z) = E * ec[j] (one
    log per element) where (win_edge + 1 + 16 NRB) / tau < 80 (win_edge 8 and 9) and the
    per-element exp otherwise (tau = 0.15, win_edge 12)."""
    print(f"fwd soft edge D={D} tau={tau} edge={edge}", flush=True)
    lens, H, k = [400, 130], 2, 12
    q, kk, v, w, pos, bias, cu = make_inputs(lens, H, D, k, hip.MODE_SOFT, seed=41, n_min=2, n_max=120)
    out, lse = run_hip(hip.MODE_SOFT, q, kk, v, w, pos, bias, cu, tau_win=tau, win_edge=edge)
    o_ref, l_ref = run_oracle(hip.MODE_SOFT, q, kk, v, w, pos, bias, cu, tau_win=tau, win_edge=edge)
    close(out, o_ref, f"soft edge tau={tau}")
    lse_close(lse, l_ref, f"soft edge tau={tau} lse")

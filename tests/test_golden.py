"""Pins the oracle's module compositions against golden vectors written from the
reference's own DSALTAttention (tests/golden/make_golden.py): the packed training
forward (oracle.module_train_forward: output, selectors, gradients with respect to x
and every parameter) and the dense batched variant for x [1, T, d_model]
(oracle.module_batched_forward: training output and every gradient, the selected
landmark keys, the eval output and the dense _last_P probabilities); and the LM
consumer (oracle.lm_forward on [1, T] input, oracle.lm_train_loss on packed input with
its gradients) against the reference's DSALTLMHeadModel. CPU only."""
import glob
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import dsalt_oracle as orc

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "module_train_*.npz")))
BATCHED = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "module_batched_*.npz")))
LM = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "lm_*.npz")))


def load(path):
    d = np.load(path, allow_pickle=False)
    cfg = json.loads(str(d["config"]))
    params = {k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p.")}
    return d, cfg, params


def rel_l2(a, b):
    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_module_matches_reference_golden(path):
    d, cfg, params = load(path)
    p64 = {k: v.double().requires_grad_() for k, v in params.items()}
    x = torch.from_numpy(d["x"]).double().requires_grad_()
    out, (w_cont, lmk_pos, lmk_logw) = orc.module_train_forward(p64, cfg, x, d["cu"])
    # selectors: identical landmark sets per (head, sequence), same windows and weights
    for h in range(lmk_pos.shape[0]):
        for s in range(lmk_pos.shape[1]):
            assert sorted(lmk_pos[h, s].tolist()) == sorted(d["lmk_pos"][h, s].tolist())
    np.testing.assert_allclose(w_cont.detach().numpy(), d["w_cont"], rtol=1e-5)
    ref_logw = {(h, s, int(p)): d["lmk_logw"][h, s, j] for h in range(lmk_pos.shape[0])
                for s in range(lmk_pos.shape[1]) for j, p in enumerate(d["lmk_pos"][h, s]) if p >= 0}
    for h in range(lmk_pos.shape[0]):
        for s in range(lmk_pos.shape[1]):
            for j, p in enumerate(lmk_pos[h, s].tolist()):
                if p >= 0:
                    assert abs(lmk_logw[h, s, j].item() - ref_logw[(h, s, p)]) < 1e-5
    assert rel_l2(out.detach(), d["out"]) < 1e-5
    out.backward(torch.from_numpy(d["dout"]).double())
    assert rel_l2(x.grad, d["grad.x"]) < 1e-4
    for name, p in p64.items():
        assert rel_l2(p.grad, d["grad." + name]) < 1e-4, name


@pytest.mark.parametrize("path", BATCHED, ids=[os.path.basename(p) for p in BATCHED])
def test_oracle_batched_module_matches_reference_golden(path):
    d, cfg, params = load(path)
    p64 = {k: v.double().requires_grad_() for k, v in params.items()}
    x = torch.from_numpy(d["x"]).double().requires_grad_()
    out, (w_cont, lb) = orc.module_batched_forward(p64, cfg, x)
    # the same landmark keys per head (sets over all T tokens)
    assert torch.equal(torch.isfinite(lb), torch.from_numpy(d["lmk_sel"]).bool())
    np.testing.assert_allclose(w_cont.detach().numpy(), d["w_cont"], rtol=1e-5)
    assert rel_l2(out.detach(), d["out"]) < 1e-5
    out.backward(torch.from_numpy(d["dout"]).double())
    assert rel_l2(x.grad, d["grad.x"]) < 1e-4
    for name, p in p64.items():
        assert rel_l2(p.grad, d["grad." + name]) < 1e-4, name


@pytest.mark.parametrize("path", BATCHED, ids=[os.path.basename(p) for p in BATCHED])
def test_oracle_batched_eval_and_probabilities(path):
    d, cfg, params = load(path)
    p64 = {k: v.double() for k, v in params.items()}
    x = torch.from_numpy(d["x"]).double()
    out, (w_cont, lb) = orc.module_batched_forward(p64, cfg, x)
    assert rel_l2(out, d["out_eval"]) < 1e-5
    T = x.shape[1]
    bias = orc.dense_logbias(w_cont, lb, T)
    assert torch.isfinite(bias).sum() > 0
    # _last_P rows sum to 1 and vanish exactly where the union bias is -inf (after i)
    P = torch.from_numpy(d["last_P"]).double()
    np.testing.assert_allclose(P.sum(-1).numpy(), np.ones(P.shape[:2]), rtol=1e-5)
    assert float(P.masked_select(torch.isinf(bias)).abs().max()) == 0.0


def test_dense_bias_special_cases():
    # the soft tail against logsigmoid, the 1e-20 clamp, the core, the causal cut, and a
    # landmark winning the union only at d >= max(1, floor(w~))
    T = 70
    w = torch.full((T,), 10.5, dtype=torch.float64)
    lb = torch.full((1, T), float("-inf"), dtype=torch.float64)
    lb[0, 3] = -0.25
    b = orc.dense_logbias(w, lb, T)[0]
    i = 60
    for j in range(T):
        dd = i - j
        if dd < 0:
            assert b[i, j] == float("-inf")
        elif dd <= 10.5 - 4:
            assert b[i, j] == 0.0
        else:
            ref = max(torch.nn.functional.logsigmoid(torch.tensor((10.5 - dd) / 1.0, dtype=torch.float64)).item(),
                      math.log(1e-20))
            if j == 3:
                ref = max(ref, -0.25)
            assert abs(b[i, j].item() - ref) < 1e-12, (j, b[i, j].item(), ref)
    assert b[i, 3] == -0.25
    # key 3 from rows 8 / 12 / 13: d = 5 (core), 9 (< floor(10.5) = 10: window only,
    # log sigmoid(1.5)), 10 (landmark admitted: max(log sigmoid(0.5), -0.25))
    assert b[8, 3] == 0.0
    assert abs(b[12, 3].item() - torch.nn.functional.logsigmoid(torch.tensor(1.5, dtype=torch.float64)).item()) < 1e-12
    assert b[13, 3] == -0.25


@pytest.mark.parametrize("path", LM, ids=[os.path.basename(p) for p in LM])
def test_oracle_lm_matches_reference_golden(path):
    d, cfg, params = load(path)
    p64 = {k: v.double() for k, v in params.items()}
    ids_b = torch.from_numpy(d["ids_batched"]).long()
    with torch.no_grad():
        logits_b = orc.lm_forward(p64, cfg, ids_b)
    assert rel_l2(logits_b, d["logits_batched"]) < 1e-5
    # the training loss on packed input and its gradients (tied head: one leaf)
    leaves = {k: v.clone().requires_grad_() for k, v in p64.items() if k != "lm_head.weight"}
    loss = orc.lm_train_loss(leaves, cfg, torch.from_numpy(d["ids"]).long(), d["cu"],
                             torch.from_numpy(d["labels"]))
    assert abs(loss.item() - float(d["loss"])) < 1e-5
    loss.backward()
    # the reference ran in fp32 through two blocks: its gradients carry ~3e-4 relative
    # rounding on the smallest ones (alpha_w ~ 4e-5)
    for k in d.files:
        if k.startswith("grad."):
            assert rel_l2(leaves[k[5:]].grad, d[k]) < 1e-3, k

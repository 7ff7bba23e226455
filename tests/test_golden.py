"""Pins the oracle's module composition (oracle.module_train_forward) against golden
vectors written from the reference's own DSALTAttention (tests/golden/make_golden.py):
training forward output, selectors, and gradients with respect to x and every
parameter. CPU only."""
import glob
import json
import os

import numpy as np
import pytest
import torch

from oracle import dsalt_oracle as orc

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "module_*.npz")))


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

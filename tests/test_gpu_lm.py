"""The LM consumer (DSALTLMHeadModel over the HIP attention) on the GPU.

* Reference golden (tests/golden/lm_small.npz, two blocks, written from the reference's
  own DSALTLMHeadModel): the state dict loads with the reference's names; eval logits of
  [1, T] input (dense batched attention per layer); the training loss of packed input
  with labels and the gradients the fixture holds (SOFT attention per layer).
* Packed eval logits (sparse HARD attention per layer) against the fp64 oracle
  composition oracle.lm_forward, which tests/test_golden.py pins to the same golden.
* Config 5 at full size (bf16, 24 layers, vocab 32000, 8 x 2048 packed tokens, seed 4):
  finite logits and bit-identical reruns.
Bar: relative L2 1e-2 and max-abs 2e-2 of the largest reference value.
"""
import json
import os

import numpy as np
import pytest
import torch

from dsalt.model import DSALTLMHeadModel
from oracle import dsalt_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "lm_small.npz")


def check(got, ref, what):
    got, ref = torch.as_tensor(got).double().cpu(), torch.as_tensor(ref).double().cpu()
    diff = got - ref
    rl = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    ma = diff.abs().max().item()
    bar = 2e-2 * min(1.0, max(ref.abs().max().item(), 1e-3))
    print(f"  {what}: rel-L2 {rl:.2e} max-abs {ma:.2e} (bar {bar:.2e})", flush=True)
    assert rl <= 1e-2 and ma <= bar, f"{what}: rel-L2 {rl:.3e}, max-abs {ma:.3e} (bar {bar:.3e})"


def load_small():
    d = np.load(GOLDEN, allow_pickle=False)
    cfg = json.loads(str(d["config"]))
    model = DSALTLMHeadModel(cfg["vocab_size"], cfg["d_model"], cfg["n_layers"], cfg["n_heads"], cfg["n_min"],
                             cfg["n_max"], cfg["k_lmk"], cfg["max_seq_len"], d_ff=cfg["d_ff"],
                             yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"], qkv_bias=cfg["qkv_bias"],
                             rope_base=cfg["rope_base"])
    state = {k[2:]: torch.from_numpy(d[k]) for k in d.files if k.startswith("p.")}
    model.load_state_dict(state, strict=True)
    model.set_collect_last_P(False)
    return d, cfg, model.to(DEV), state


def test_lm_small_eval_matches_reference_and_oracle():
    print("lm small eval", flush=True)
    d, cfg, model, state = load_small()
    model.eval()
    with torch.no_grad():
        logits_b = model(torch.from_numpy(d["ids_batched"]).to(DEV))["logits"]
        ids = torch.from_numpy(d["ids"])
        cu = torch.from_numpy(d["cu"])
        logits = model(ids.to(DEV), cu_seqlens=cu.to(DEV))["logits"]
    check(logits_b, d["logits_batched"], "logits [1, T] (reference golden)")
    ref = orc.lm_forward({k: v.double() for k, v in state.items()}, cfg, ids.long(), d["cu"])
    check(logits, ref, "logits packed (oracle)")


def test_lm_small_train_loss_and_grads_match_reference():
    print("lm small train", flush=True)
    d, cfg, model, _ = load_small()
    model.train()
    out = model(torch.from_numpy(d["ids"]).to(DEV), cu_seqlens=torch.from_numpy(d["cu"]).to(DEV),
                labels=torch.from_numpy(d["labels"]).to(DEV))
    loss = out["loss"]
    print(f"  loss {loss.item():.6f} vs reference {float(d['loss']):.6f}", flush=True)
    assert abs(loss.item() - float(d["loss"])) <= 2e-2 * abs(float(d["loss"]))
    loss.backward()
    named = dict(model.named_parameters())
    for k in d.files:
        if k.startswith("grad."):
            check(named[k[5:]].grad, d[k], k)


def test_lm_config5_full_size_finite_and_deterministic():
    print("lm config 5 full size", flush=True)
    torch.manual_seed(4)
    model = DSALTLMHeadModel(32000, 1024, 24, 16, 32, 512, 64, 2048).to(DEV, torch.bfloat16).eval()
    model.set_collect_last_P(False)
    ids = torch.randint(0, 32000, (8 * 2048,), device=DEV)
    cu = torch.arange(0, 8 * 2048 + 1, 2048, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        a = model(ids, cu_seqlens=cu)["logits"]
        b = model(ids, cu_seqlens=cu)["logits"]
    torch.cuda.synchronize()
    assert a.shape == (8 * 2048, 32000) and a.dtype == torch.bfloat16
    assert bool(torch.isfinite(a).all())
    assert torch.equal(a, b)

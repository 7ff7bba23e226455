"""Writes golden vectors of the reference's DSALTAttention module composition.

Run in the build container only (where the reference checkout exists):

    TORCHDYNAMO_DISABLE=1 python tests/golden/make_golden.py [/path/to/reference]

What it pins: the part no closed form covers - the module composition of
dsalt/modules/dsalt_attention.py in training mode on packed uniform-length input
(q/k/v projections -> RoPE -> _train_selectors (continuous window, landmark top-k,
soft landmark weight) -> the dense SOFT attention of _packed_train ->
out_proj), and the gradients of the output with respect to x and every parameter;
and the dense batched variant forward(x) for x [1, T, d_model] (_batched /
_diff_logbias, :366-438) in training mode (output and every gradient) and in eval mode
(output and the dense _last_P), with the landmark keys each head selected; and the LM
consumer DSALTLMHeadModel (dsalt/model/dsalt_lm.py) with two blocks: eval logits of
[1, T] input, and the training loss of packed input with labels and some gradients.
On a CPU the reference takes its dense path (_packed_train, :489-563), which is the
reference's own definition of the training kernel's math. TORCHDYNAMO_DISABLE=1 runs
its torch.compile'd RoPE eagerly.

Each fixture is an .npz (no pickles) holding the config, the parameters, the inputs,
the upstream gradient and the reference's outputs and gradients.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    "module_train_mha": dict(d_model=128, n_heads=2, n_min=4, n_max=40, k_lmk=8, max_seq_len=256,
                             n_kv_heads=None, qkv_bias=False, yarn_scale=1.0, rope_base=10000.0,
                             lens=[64, 64], seed=0),
    "module_train_gqa": dict(d_model=128, n_heads=2, n_min=2, n_max=24, k_lmk=5, max_seq_len=128,
                             n_kv_heads=1, qkv_bias=True, yarn_scale=2.0, rope_base=500.0,
                             lens=[48, 48, 48], seed=1),
}


# the dense batched variant: DSALTAttention.forward(x) with x [1, T, d_model] and no
# cu_seqlens (dsalt/modules/dsalt_attention.py:366-438)
BATCHED_CASES = {
    "module_batched_mha": dict(d_model=128, n_heads=2, n_min=4, n_max=40, k_lmk=8, max_seq_len=256,
                               n_kv_heads=None, qkv_bias=False, yarn_scale=1.0, rope_base=10000.0,
                               T=96, seed=3),
    "module_batched_gqa": dict(d_model=128, n_heads=2, n_min=2, n_max=24, k_lmk=5, max_seq_len=128,
                               n_kv_heads=1, qkv_bias=True, yarn_scale=2.0, rope_base=500.0,
                               T=80, seed=4),
}


def write_batched(DSALTAttention, hybrid_scores_per_head) -> None:
    import torch

    for name, cfg in BATCHED_CASES.items():
        torch.manual_seed(cfg["seed"])
        mod = DSALTAttention(cfg["d_model"], cfg["n_heads"], cfg["n_min"], cfg["n_max"], cfg["k_lmk"],
                             cfg["max_seq_len"], yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"],
                             qkv_bias=cfg["qkv_bias"], rope_base=cfg["rope_base"])
        T = cfg["T"]
        x = torch.randn(1, T, cfg["d_model"])
        # the landmark keys of each head, selected over all T tokens (dsalt_attention.py:421-428)
        with torch.no_grad():
            scores, _, _ = hybrid_scores_per_head(x[0], mod.v_proj.weight, torch.sigmoid(mod.alpha_w),
                                                  cfg["n_heads"], cfg["d_model"] // cfg["n_heads"])
            _, top = torch.topk(scores, min(cfg["k_lmk"], T), dim=0, sorted=False)
            sel = torch.zeros(cfg["n_heads"], T, dtype=torch.bool)
            sel.scatter_(1, top.transpose(0, 1), True)
            w_cont = mod._window_continuous(x[0])
        mod.train()
        xg = x.clone().requires_grad_()
        out, _ = mod(xg)
        dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(200 + cfg["seed"]))
        out.backward(dout)
        mod.eval()
        with torch.no_grad():
            out_eval, _ = mod(x)
        arrays = {"config": np.array(json.dumps(cfg)), "x": x.numpy(), "out": out.detach().numpy(),
                  "dout": dout.numpy(), "grad.x": xg.grad.numpy(), "w_cont": w_cont.numpy(),
                  "lmk_sel": sel.numpy().astype(np.uint8), "out_eval": out_eval.numpy(),
                  "last_P": mod._last_P.numpy()}
        for pname, prm in mod.named_parameters():
            arrays["p." + pname] = prm.detach().numpy()
            arrays["grad." + pname] = prm.grad.numpy()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


# the LM consumer: DSALTLMHeadModel (dsalt/model/dsalt_lm.py:64-280) with two blocks,
# every attention module with _collect_last_P = False
LM_CASES = {
    "lm_small": dict(vocab_size=256, d_model=128, n_layers=2, n_heads=2, n_min=4, n_max=40, k_lmk=8,
                     max_seq_len=256, d_ff=128, n_kv_heads=None, qkv_bias=False, yarn_scale=1.0,
                     rope_base=10000.0, lens=[88, 88], T_batched=96, seed=5),
}
LM_GRADS = ("embed_tokens.weight", "layers.0.attn.win_gate.weight", "layers.0.attn.alpha_w",
            "layers.1.attn.q_proj.weight", "layers.1.ffn.down_proj.weight", "final_norm.weight")


def write_lm(DSALTLMHeadModel) -> None:
    """Eval logits of [1, T] input (the dense batched variant per layer) and the training
    loss of packed input with labels (SOFT attention per layer, the reference's CPU path)
    with the gradients of LM_GRADS. (Packed eval runs the reference's Triton kernel,
    which has no CPU path.)"""
    import torch

    for name, cfg in LM_CASES.items():
        torch.manual_seed(cfg["seed"])
        model = DSALTLMHeadModel(cfg["vocab_size"], cfg["d_model"], cfg["n_layers"], cfg["n_heads"], cfg["n_min"],
                                 cfg["n_max"], cfg["k_lmk"], cfg["max_seq_len"], d_ff=cfg["d_ff"],
                                 yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"],
                                 qkv_bias=cfg["qkv_bias"], rope_base=cfg["rope_base"])
        for layer in model.layers:
            layer.attn._collect_last_P = False
        T = sum(cfg["lens"])
        g = torch.Generator().manual_seed(300 + cfg["seed"])
        ids = torch.randint(0, cfg["vocab_size"], (T,), generator=g)
        labels = torch.randint(0, cfg["vocab_size"], (T,), generator=g)
        labels[::7] = -100
        ids_b = torch.randint(0, cfg["vocab_size"], (1, cfg["T_batched"]), generator=g)
        cu_list = [0]
        for L in cfg["lens"]:
            cu_list.append(cu_list[-1] + L)
        cu = torch.tensor(cu_list, dtype=torch.int32)
        model.eval()
        with torch.no_grad():
            logits_b = model(ids_b)["logits"]
        model.train()
        loss = model(ids, cu_seqlens=cu, labels=labels)["loss"]
        loss.backward()
        arrays = {"config": np.array(json.dumps(cfg)), "ids": ids.numpy(), "cu": cu.numpy(),
                  "labels": labels.numpy(), "ids_batched": ids_b.numpy(),
                  "logits_batched": logits_b.numpy(), "loss": np.array(loss.item(), dtype=np.float64)}
        for pname, prm in model.state_dict().items():
            arrays["p." + pname] = prm.detach().numpy()
        named = dict(model.named_parameters())
        for pname in LM_GRADS:
            arrays["grad." + pname] = named[pname].grad.numpy()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def main(ref_root: str) -> None:
    os.environ.setdefault("TORCHDYNAMO_DISABLE", "1")
    sys.path.insert(0, ref_root)
    import torch
    from dsalt.kernels.landmark_tokens_ker import hybrid_scores_per_head
    from dsalt.modules.dsalt_attention import DSALTAttention

    for name, cfg in CASES.items():
        torch.manual_seed(cfg["seed"])
        mod = DSALTAttention(cfg["d_model"], cfg["n_heads"], cfg["n_min"], cfg["n_max"], cfg["k_lmk"],
                             cfg["max_seq_len"], yarn_scale=cfg["yarn_scale"], n_kv_heads=cfg["n_kv_heads"],
                             qkv_bias=cfg["qkv_bias"], rope_base=cfg["rope_base"])
        T = sum(cfg["lens"])
        x = torch.randn(T, cfg["d_model"])
        cu_list = [0]
        for L in cfg["lens"]:
            cu_list.append(cu_list[-1] + L)
        cu = torch.tensor(cu_list, dtype=torch.int32)
        mod.train()
        with torch.no_grad():
            w_cont, lmk_pos, lmk_logw = mod._train_selectors(x, cu, T, x.device, cu_list)
        xg = x.clone().requires_grad_()
        out, _ = mod(xg, cu_seqlens=cu)
        dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(100 + cfg["seed"]))
        out.backward(dout)
        arrays = {"config": np.array(json.dumps(cfg)), "x": x.numpy(), "cu": cu.numpy(),
                  "out": out.detach().numpy(), "dout": dout.numpy(), "grad.x": xg.grad.numpy(),
                  "w_cont": w_cont.numpy(), "lmk_pos": lmk_pos.numpy(), "lmk_logw": lmk_logw.numpy()}
        for pname, p in mod.named_parameters():
            arrays["p." + pname] = p.detach().numpy()
            arrays["grad." + pname] = p.grad.numpy()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")
    write_batched(DSALTAttention, hybrid_scores_per_head)
    from dsalt.model.dsalt_lm import DSALTLMHeadModel
    write_lm(DSALTLMHeadModel)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

"""Static gfx950 tile configuration (name-compatible with dsalt/kernels/autotune.py).

The reference benchmarks Triton BLOCK_M/BLOCK_N/num_warps candidates once per
(head_dim, GPU) (autotune.py:192-238). The HIP kernels use fixed gfx950 tiles chosen
for 64-wide wavefronts and the 160 KB LDS, so ``autotune_blocks`` measures nothing and
``get_tuned_config`` reports the fixed configuration.
"""
from __future__ import annotations

import torch

# forward: 4 waves x 32 queries per workgroup, 64-key tiles, v_mfma_f32_32x32x16
_GFX950_CONFIG = {"BLOCK_M": 128, "BLOCK_N": 64, "BLOCK_N_BWD": 64, "num_warps": 4, "num_stages": 2}


def get_tuned_config(head_dim: int, device: torch.device | None = None) -> dict:
    """The fixed gfx950 tile configuration for ``head_dim`` (64 or 128)."""
    if head_dim not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {head_dim}")
    return dict(_GFX950_CONFIG)


def autotune_blocks(head_dim: int, device: torch.device | None = None, make_runner=None,
                    verbose: bool = False) -> dict:
    """Return the fixed configuration; ``make_runner`` is accepted and not called."""
    cfg = get_tuned_config(head_dim, device)
    if verbose:
        print(f"  [DSALT gfx950] head_dim={head_dim}: static tiles {cfg}")
    return cfg

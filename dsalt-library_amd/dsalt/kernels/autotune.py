"""Static gfx950 tile configuration (name-compatible with dsalt/kernels/autotune.py).

The reference benchmarks Triton BLOCK_M/BLOCK_N/num_warps candidates once per
(head_dim, GPU) (autotune.py:192-238). The HIP kernels use fixed gfx950 tiles chosen
for 64-wide wavefronts and the 160 KB LDS, so ``autotune_blocks`` measures nothing and
``get_tuned_config`` reports the fixed configuration.
"""
from __future__ import annotations

import torch

# Forward workgroups (the constants of csrc/launch.h): BLOCK_M queries = num_warps waves
# of 32, BLOCK_N keys per LDS tile, num_stages-deep LDS rings of K and of V tiles;
# BLOCK_N_BWD queries per tile of the band dK/dV pass (csrc/bwd.hip). All products are
# v_mfma_f32_32x32x16.
_GFX950_CONFIG = {
    64: {"BLOCK_M": 64, "BLOCK_N": 32, "BLOCK_N_BWD": 32, "num_warps": 2, "num_stages": 2},
    128: {"BLOCK_M": 64, "BLOCK_N": 32, "BLOCK_N_BWD": 64, "num_warps": 2, "num_stages": 2},
}


def get_tuned_config(head_dim: int, device: torch.device | None = None) -> dict:
    """The fixed gfx950 tile configuration for ``head_dim`` (64 or 128)."""
    if head_dim not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {head_dim}")
    return dict(_GFX950_CONFIG[head_dim])


def autotune_blocks(head_dim: int, device: torch.device | None = None, make_runner=None,
                    verbose: bool = False) -> dict:
    """Return the fixed configuration; ``make_runner`` is accepted and not called."""
    cfg = get_tuned_config(head_dim, device)
    if verbose:
        print(f"  [DSALT gfx950] head_dim={head_dim}: static tiles {cfg}")
    return cfg

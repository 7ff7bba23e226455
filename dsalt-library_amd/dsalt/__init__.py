"""DSALT sparse-attention hot path for AMD MI355X (gfx950).

Drop-in for the attention path of LeonardoCofone/dsalt-library: ``dsalt.modules.DSALTAttention``,
``dsalt.kernels.dsalt_triton_attention`` / ``dsalt_triton_backward``,
``dsalt.kernels.dsalt_triton_train.dsalt_triton_train_attention`` and the selector helpers,
all backed by hand-written HIP kernels in libdsalt_hip.so (see ``dsalt._hip``).
"""
from ._hip import DsaltError
from .kernels import (
    apply_rotary_emb,
    build_rope_cache,
    dsalt_triton_attention,
    dsalt_triton_backward,
    hybrid_scores_per_head,
)
from .kernels.dsalt_triton_train import dsalt_triton_train_attention
from .modules import DSALTAttention

__all__ = [
    "DSALTAttention",
    "DsaltError",
    "dsalt_triton_attention",
    "dsalt_triton_backward",
    "dsalt_triton_train_attention",
    "hybrid_scores_per_head",
    "apply_rotary_emb",
    "build_rope_cache",
]

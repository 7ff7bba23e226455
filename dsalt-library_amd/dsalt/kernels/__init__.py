"""DSALT kernel entry points on gfx950 HIP (names of dsalt/kernels/__init__.py that lie on
the sparse-attention path). Importing never needs a GPU; calling needs libdsalt_hip.so
and ROCm tensors, and raises ``DsaltError`` otherwise (there is no fallback path, so the
names are never ``None``)."""
from .autotune import autotune_blocks, get_tuned_config
from .dsalt_triton_attn import dsalt_triton_attention
from .dsalt_triton_bwd import dsalt_triton_backward
from .dsalt_triton_train import dsalt_triton_train_attention
from .landmark_tokens_ker import hybrid_scores_per_head
from .window_utils import apply_rotary_emb, build_rope_cache

__all__ = [
    "dsalt_triton_attention",
    "dsalt_triton_backward",
    "dsalt_triton_train_attention",
    "autotune_blocks",
    "get_tuned_config",
    "hybrid_scores_per_head",
    "apply_rotary_emb",
    "build_rope_cache",
]

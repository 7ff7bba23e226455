"""DSALT kernel entry points on gfx950 HIP (the names of dsalt/kernels/__init__.py that lie
on the sparse-attention path).

As in the reference (dsalt/kernels/__init__.py:23-35, where a failed Triton import
leaves them ``None``), ``dsalt_triton_attention``, ``dsalt_triton_backward``,
``autotune_blocks`` and ``get_tuned_config`` are ``None`` when libdsalt_hip.so cannot be
loaded; ``_HIP_OK`` says which case holds. Loading the library touches no GPU. Calls
need ROCm tensors and raise ``DsaltError`` otherwise: there is no CPU fallback.
"""
from .. import _hip
from .dsalt_triton_train import dsalt_triton_train_attention
from .landmark_tokens_ker import hybrid_scores_per_head
from .window_utils import apply_rotary_emb, build_rope_cache

try:
    _hip.lib()
    _HIP_OK = True
except (_hip.DsaltError, OSError):
    _HIP_OK = False

if _HIP_OK:
    from .autotune import autotune_blocks, get_tuned_config
    from .dsalt_triton_attn import dsalt_triton_attention
    from .dsalt_triton_bwd import dsalt_triton_backward
else:
    dsalt_triton_attention = None
    dsalt_triton_backward = None
    autotune_blocks = None
    get_tuned_config = None

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

"""DSALT kernel entry points on gfx950 HIP (the names of dsalt/kernels/__init__.py that lie
on the sparse-attention path).

As in the reference (dsalt/kernels/__init__.py:23-35, where a failed Triton import
leaves them ``None``), ``dsalt_triton_attention``, ``dsalt_triton_backward``,
``autotune_blocks`` and ``get_tuned_config`` are ``None`` when libdsalt_hip.so cannot be
loaded; ``_HIP_OK`` says which case holds. Loading the library touches no GPU. Calls
need ROCm tensors and raise ``DsaltError`` otherwise: there is no CPU fallback.

The reference's generic helpers are exported under their names too: the dense-mask
builders and masked SDPA (``window_utils``, ``sparse_attn``), the older landmark helpers
(``landmark_tokens_ker``) and ``RMSENorm``. They are plain torch utilities that the DSALT
attention path never calls. ``LigerFusedLinearCrossEntropyFunction`` (the Triton loss)
is not part of this package.
"""
from .. import _hip
from .RMSENorm import RMSENorm
from .dsalt_triton_train import dsalt_triton_train_attention
from .landmark_tokens_ker import (
    HybridEnergyLandmarkSelector,
    compute_hybrid_scores,
    hybrid_scores_per_head,
    select_landmarks,
    soft_landmark_weights,
)
from .sparse_attn import sparse_attention_forward, sparse_attention_forward_packed
from .window_utils import (
    apply_rotary_emb,
    build_local_window_mask,
    build_local_window_mask_packed,
    build_rope_cache,
    compute_window_sizes,
)

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
    "RMSENorm",
    "compute_window_sizes",
    "build_local_window_mask",
    "build_local_window_mask_packed",
    "apply_rotary_emb",
    "build_rope_cache",
    "hybrid_scores_per_head",
    "compute_hybrid_scores",
    "select_landmarks",
    "soft_landmark_weights",
    "HybridEnergyLandmarkSelector",
    "sparse_attention_forward",
    "sparse_attention_forward_packed",
]

"""DSALT sparse-attention hot path for AMD MI355X (gfx950).

Drop-in for the attention path of LeonardoCofone/dsalt-library: ``dsalt.modules.DSALTAttention``,
``dsalt.kernels.dsalt_triton_attention`` / ``dsalt_triton_backward``,
``dsalt.kernels.dsalt_triton_train.dsalt_triton_train_attention`` and the selector helpers,
all backed by hand-written HIP kernels in libdsalt_hip.so (see ``dsalt._hip``), and the
consumers ``DSALTTransformerBlock`` / ``DSALTLMHeadModel``. ``DSALTConfig`` and
``DSALTTrainer`` (configuration dataclass and training loop) are not part of it.
"""
from ._hip import DsaltError
from .kernels import (
    HybridEnergyLandmarkSelector,
    RMSENorm,
    apply_rotary_emb,
    build_local_window_mask,
    build_local_window_mask_packed,
    build_rope_cache,
    compute_hybrid_scores,
    compute_window_sizes,
    dsalt_triton_attention,
    dsalt_triton_backward,
    hybrid_scores_per_head,
    select_landmarks,
    soft_landmark_weights,
    sparse_attention_forward,
    sparse_attention_forward_packed,
)
from .kernels.dsalt_triton_train import dsalt_triton_train_attention
from .model import DSALTLMHeadModel
from .modules import DSALTAttention, DSALTTransformerBlock, SwiGLUFFN

__all__ = [
    "DSALTAttention",
    "DSALTTransformerBlock",
    "SwiGLUFFN",
    "DSALTLMHeadModel",
    "DsaltError",
    "dsalt_triton_attention",
    "dsalt_triton_backward",
    "dsalt_triton_train_attention",
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

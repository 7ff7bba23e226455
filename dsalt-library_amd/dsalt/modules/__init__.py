from .dsalt_attention import DSALTAttention

__all__ = ["DSALTAttention"]

from .dsalt_lm import DSALTLMHeadModel

__all__ = ["DSALTLMHeadModel"]

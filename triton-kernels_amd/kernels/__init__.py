"""MI355X-native ``flash_attention_v2`` (drop-in for harsh-vsingh/triton-kernels
``kernels/__init__.py:1-4``, which re-exports it from ``kernels.attention``)."""

from .attention import flash_attention_v2

__all__ = ["flash_attention_v2"]

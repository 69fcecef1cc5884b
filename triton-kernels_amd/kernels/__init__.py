"""MI355X-native attention kernels: drop-in for the attention entry points of
harsh-vsingh/triton-kernels ``kernels/__init__.py`` (flash_attention_v1/v2
from ``kernels.attention``, ``decode_attention`` from ``kernels.decode``,
``speculative_decode_attention`` from ``kernels.speculative_decode``)."""

from .attention import flash_attention_v1, flash_attention_v2
from .decode import decode_attention
from .speculative_decode import speculative_decode_attention

__all__ = [
    "flash_attention_v1",
    "flash_attention_v2",
    "speculative_decode_attention",
    "decode_attention",
]

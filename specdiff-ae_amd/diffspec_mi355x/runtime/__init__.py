"""Attention backend of the verification path (gfx950 kernels)."""

from .attention_compat import FLASH_ATTN_AVAILABLE, flash_attn_func, flash_attn_with_kvcache  # noqa: F401
from .tree_attention import prefix_attention_forward, tree_attention_forward, tree_verify  # noqa: F401

"""flash-attn compatible entry points backed by the gfx950 prefix kernel.

Mirrors the contract of the reference's ``diffspec/runtime/attention_compat.py``
(:103-132): ``flash_attn_with_kvcache(q, k_cache, v_cache, causal,
cache_seqlens, return_softmax_lse)`` returns ``out [B, M, H, D]`` and, when
asked, ``lse [B, H, M]`` in float32.  Only the non-causal form used by the
verification path (llama_target_model.py:838-845) is implemented; causal=True
raises.
"""

from __future__ import annotations

from typing import Optional

import torch

from .tree_attention import prefix_attention_forward

# The verification path never imports the flash-attn package; these flags keep
# callers that branch on them on the HIP path.
FLASH_ATTN_AVAILABLE = True
PYTORCH_FLASH_ATTN_AVAILABLE = False


def sdpa_backend_name() -> str:
    return "dsv_hip_gfx950"


def flash_attn_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dropout_p: float = 0.0,
                    causal: bool = False, window_size=None, **_: object) -> torch.Tensor:
    if causal:
        raise NotImplementedError("causal attention is not part of the tree-verification kernels")
    if dropout_p:
        raise NotImplementedError("dropout is not supported")
    B, M, H, D = q.shape
    out, _ = prefix_attention_forward(q, k, v, B, M, H, D)
    return out


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, causal: bool = False,
                            cache_seqlens: Optional[int] = None, return_softmax_lse: bool = False, **_: object):
    if causal:
        raise NotImplementedError("causal attention is not part of the tree-verification kernels")
    if isinstance(cache_seqlens, torch.Tensor):
        if cache_seqlens.numel() != 1:
            raise NotImplementedError("per-batch cache_seqlens are not supported")
        cache_seqlens = int(cache_seqlens.item())
    B, M, H, D = q.shape
    n = -1 if cache_seqlens is None else int(cache_seqlens)
    out, lse = prefix_attention_forward(q, k_cache, v_cache, B, M, H, D, n_keys=n)
    if return_softmax_lse:
        return out, lse
    return out

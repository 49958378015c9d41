"""flash-attn compatible entry points backed by the gfx950 prefix kernel.

Mirrors the contract of the reference's ``diffspec/runtime/attention_compat.py``
(:103-132): ``flash_attn_with_kvcache(q, k_cache, v_cache, causal,
cache_seqlens, return_softmax_lse)`` returns ``out [B, M, H, D]`` and, when
asked, ``lse [B, H, M]`` in float32.  ``cache_seqlens`` is an int or a
per-batch tensor (flash-attn's form; the reference's fallback takes only a
scalar), and ``causal=True`` aligns the mask to the end of each batch's keys
(query m sees keys n <= len - M + m), as flash-attn does.

"""

from __future__ import annotations

from typing import Optional, Union

import torch

from .. import _ext

# The verification path never imports the flash-attn package; these flags keep
# callers that branch on them on the HIP path.
FLASH_ATTN_AVAILABLE = True
PYTORCH_FLASH_ATTN_AVAILABLE = False


def sdpa_backend_name() -> str:
    return "dsv_hip_gfx950"


def _slice_len(n: int, N: int) -> int:
    """Keys kept by the reference's ``k_cache[:, :n]`` (attention_compat.py:113):
    Python slicing, so n > N keeps all N and a negative n drops -n from the end."""
    return len(range(N)[:n])


def flash_attn_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dropout_p: float = 0.0,
                    causal: bool = False, window_size=None, **_: object) -> torch.Tensor:
    if dropout_p:
        raise NotImplementedError("dropout is not supported")
    return flash_attn_with_kvcache(q, k, v, causal=causal)


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, causal: bool = False,
                            cache_seqlens: Optional[Union[int, torch.Tensor]] = None, return_softmax_lse: bool = False,
                            **_: object):
    dev = _ext.require_gpu(q, k_cache, v_cache)
    B, M, H, D = q.shape
    N, Hk = k_cache.shape[1], k_cache.shape[2]
    seqlens, n = None, N
    if isinstance(cache_seqlens, torch.Tensor):
        if cache_seqlens.numel() == 1 and cache_seqlens.dim() == 0:
            n = _slice_len(int(cache_seqlens.item()), N)
        else:
            seqlens = cache_seqlens.reshape(-1)
            if seqlens.numel() != B:
                raise ValueError(f"cache_seqlens must hold one length per batch ({B}), got {seqlens.numel()}")
            if seqlens.dtype not in (torch.int32, torch.int64):
                seqlens = seqlens.to(torch.int64)
            seqlens = seqlens.to(dev).contiguous()
    elif cache_seqlens is not None:
        n = _slice_len(int(cache_seqlens), N)
    lib = _ext.load()
    out = torch.empty_like(q)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=dev) if return_softmax_lse else None
    ws = _ext.workspace(lib.dsv_attn_workspace_bytes(B, M, H, Hk, D, n, 0, 0), dev)
    rc = lib.dsv_flash_attn_with_kvcache(_ext.desc(q), _ext.desc(k_cache), _ext.desc(v_cache), _ext.desc(seqlens),
                                         int(n), int(bool(causal)), _ext.desc(out), _ext.desc(lse), ws.data_ptr(),
                                         ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "flash_attn_with_kvcache")
    if return_softmax_lse:
        return out, lse
    return out

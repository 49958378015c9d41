"""Tree K/V append with RoPE into the cache (gfx950 kernel behind dsv_kv_append).

Per layer, the reference rotates the projected queries and keys
(``apply_rotary_pos_emb_L31``, llama_target_model.py:452-473 with
``rotate_half`` :408-427, applied at :768-771) and appends keys and values to
its preallocated cache (``KVCache.cat``, runtime/cache_state.py:52-66, used at
llama_target_model.py:781-783), or writes them token by token into the page
pool (``PagedKVCache.write_kv``, core/kv_cache/paged_kv.py:168-223).  Here
one launch does all of it for the tree's M tokens, with torch's rounding of
the 16-bit elementwise ops (each product, then the sum, rounded to the dtype).
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _ext

__all__ = ["append_tree_kv"]


def append_tree_kv(k: torch.Tensor, v: torch.Tensor, k_dst: torch.Tensor, v_dst: torch.Tensor, start: int,
                   cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                   page_table: Optional[torch.Tensor] = None,
                   q: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Write RoPE(k) and v of the tree tokens at logical tokens [start, start + M).

    Args:
      k, v: ``[M, Hk, D]`` or ``[1, M, Hk, D]`` bf16/f16, before RoPE.
      k_dst, v_dst: page-pool halves ``[P, Hk, page, D]`` (with ``page_table``)
        or dense caches ``[Hk, S, D]`` / ``[1, Hk, S, D]``.
      start: the cache length before the tree.
      cos, sin: ``[M, D]`` or ``[1, M, D]`` tables at the tree tokens'
        positions (the rotary embedding's output, in k's dtype); None: no RoPE.
      page_table: ``[n_logical]`` int32/int64.
      q: optional ``[M, H, D]`` / ``[1, M, H, D]`` queries, rotated the same way.

    Returns the rotated queries (shape of ``q``) when ``q`` is given.
    """
    _ext.require_gpu(k, v, k_dst, v_dst, cos, sin, page_table, q)
    q_out = torch.empty_like(q) if q is not None else None
    lib = _ext.load()
    rc = lib.dsv_kv_append(_ext.desc(k), _ext.desc(v), _ext.desc(cos), _ext.desc(sin), _ext.desc(k_dst),
                           _ext.desc(v_dst), _ext.desc(page_table), int(start), _ext.desc(q), _ext.desc(q_out),
                           _ext.stream_of(k.device))
    _ext.check(rc, "kv_append")
    return q_out

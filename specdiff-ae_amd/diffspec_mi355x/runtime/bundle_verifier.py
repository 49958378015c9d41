"""Bundle verification on MI355X: dense and paged KV, plus the fused tree path.

Drop-in for the reference's ``diffspec/runtime/bundle_verifier.py``:

  * ``FusedBundleVerifier(bundle_size, enable_triton, device)`` with
    ``verify_bundle(q, k, v, masks, shared_prefix_len) -> (o [B,M,H,D],
    lse [B,M,H])`` and ``get_statistics()`` (reference :142-331);
  * ``PagedBundleVerifier.verify_bundle_paged(q, kv_pages, page_table, masks,
    shared_prefix_len=0, layer_idx=0)`` (reference :338-366, where it raises
    NotImplementedError) reading K/V straight from the page pool
    ``[L, 2, P, Hk, page_size, D]`` through the page table;
  * ``PagedBundleVerifier.verify_tree_paged`` — the fused hybrid tree
    verification (prefix + ancestor-masked tree block + LSE merge) over the
    page pool, the fast path used by the benchmark.

As in the reference, only the first mask of ``masks`` is applied (reference
:196-205) and ``shared_prefix_len`` changes the statistics but not the
result (both reference phases apply the mask, :71-126).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from .. import _ext
from .tree_attention import tree_verify


def _byte_mask(m: torch.Tensor) -> torch.Tensor:
    # Non-zero = keep, the int1 conversion of the reference kernel (:94-95).
    if m.dtype in (torch.int8, torch.uint8, torch.bool):
        return m
    return (m != 0).to(torch.int8)


def _first_mask(masks: List[torch.Tensor], B: int) -> torch.Tensor:
    m = masks[0]
    if m.dim() == 2:
        m = m.unsqueeze(0)
    if m.size(0) not in (1, B):
        raise ValueError("mask batch must be 1 or B")
    return _byte_mask(m)


class FusedBundleVerifier:
    """Verify a bundle of tree nodes with the gfx950 masked-attention kernel."""

    def __init__(self, bundle_size: int = 3, enable_triton: bool = True, device: str = "cuda"):
        self.bundle_size = bundle_size
        # Kept for API compatibility: this backend never runs Triton.
        self.enable_triton = False
        self.requested_triton = enable_triton
        self.device = device
        self.total_verifications = 0
        self.total_bundles = 0
        self.prefix_reuse_count = 0

    def _count(self, masks, shared_prefix_len: int) -> None:
        self.total_verifications += len(masks)
        self.total_bundles += 1
        if shared_prefix_len > 0:
            self.prefix_reuse_count += 1

    def verify_bundle(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, masks: List[torch.Tensor],
                      shared_prefix_len: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
        """Masked attention of q [B,M,H,D] over k/v [B,N,Hk,D] -> (o [B,M,H,D], lse [B,M,H])."""
        self._count(masks, shared_prefix_len)
        dev = _ext.require_gpu(q, k, v, masks[0])
        B, M, H, D = q.shape
        mask = _first_mask(masks, B)
        lib = _ext.load()
        o = torch.empty_like(q)
        lse = torch.empty((B, M, H), dtype=torch.float32, device=dev)
        ws_bytes = lib.dsv_attn_workspace_bytes(B, M, H, k.shape[2], D, k.shape[1], 0, 0)
        ws = _ext.workspace(ws_bytes, dev)
        rc = lib.dsv_verify_bundle(_ext.desc(q), _ext.desc(k), _ext.desc(v), _ext.desc(mask), _ext.desc(o),
                                   _ext.desc(lse), ws.data_ptr(), ws.numel(), _ext.stream_of(dev))
        _ext.check(rc, "verify_bundle")
        return o, lse

    def get_statistics(self) -> Dict:
        return {
            "total_verifications": self.total_verifications,
            "total_bundles": self.total_bundles,
            "avg_bundle_size": self.total_verifications / self.total_bundles if self.total_bundles > 0 else 0,
            "prefix_reuse_rate": self.prefix_reuse_count / self.total_bundles if self.total_bundles > 0 else 0,
            "triton_enabled": self.enable_triton,
            "hip_enabled": True,
        }


class PagedBundleVerifier(FusedBundleVerifier):
    """Bundle verification read directly from paged KV storage."""

    def verify_bundle_paged(self, q: torch.Tensor, kv_pages: torch.Tensor, page_table: torch.Tensor,
                            masks: List[torch.Tensor], shared_prefix_len: int = 0,
                            layer_idx: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
        """Masked attention over the logical token sequence of ``page_table``.

        Args:
            q: [B, M, H, D]
            kv_pages: [L, 2, P, Hk, page_size, D] page pool (core/kv_cache/paged_kv.py:56-65)
            page_table: [n_pages] or [B, n_pages] logical -> physical page
            masks: list of [M, N] (or [B, M, N]) masks over the N logical tokens
        Returns:
            o [B, M, H, D], lse [B, M, H]
        """
        self._count(masks, shared_prefix_len)
        dev = _ext.require_gpu(q, kv_pages, page_table, masks[0])
        B, M, H, D = q.shape
        mask = _first_mask(masks, B)
        lib = _ext.load()
        o = torch.empty_like(q)
        lse = torch.empty((B, M, H), dtype=torch.float32, device=dev)
        ws_bytes = lib.dsv_attn_workspace_bytes(B, M, H, kv_pages.shape[3], D, mask.shape[-1], kv_pages.shape[4], 0)
        ws = _ext.workspace(ws_bytes, dev)
        rc = lib.dsv_verify_bundle_paged(_ext.desc(q), _ext.desc(kv_pages), _ext.desc(page_table), int(layer_idx),
                                         _ext.desc(mask), _ext.desc(o), _ext.desc(lse), ws.data_ptr(), ws.numel(),
                                         _ext.stream_of(dev))
        _ext.check(rc, "verify_bundle_paged")
        return o, lse

    def verify_tree_paged(self, q: torch.Tensor, kv_pages: torch.Tensor, page_table: torch.Tensor,
                          prefix_len: int, parent: torch.Tensor, layer_idx: int = 0,
                          row_perm: Optional[torch.Tensor] = None,
                          out_dtype: Optional[torch.dtype] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Fused tree verification over the page pool.

        The prefix is logical tokens [0, prefix_len); the tree's K/V rows are
        tokens [prefix_len, prefix_len + M).  ``parent`` ([M] or [B, M]) gives
        each node's parent (< 0 for the root).  Returns (o [B, M, H, D],
        lse [B, M, H]) of attention over prefix + ancestors-or-self.
        """
        self.total_verifications += q.shape[1]
        self.total_bundles += 1
        return tree_verify(q, kv_pages[layer_idx, 0], kv_pages[layer_idx, 1], prefix_len, parent,
                           page_table=page_table, row_perm=row_perm, out_dtype=out_dtype)

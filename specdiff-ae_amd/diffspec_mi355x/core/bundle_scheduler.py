"""Ancestor-based bundle scheduling, and the query packing order it induces.

Same public surface and results as the reference's
``diffspec/core/bundle_scheduler.py`` (BundleScheduler :15-288,
TreeDescriptorBuilder :291-392):

  * every leaf is assigned its nearest *branching* ancestor (the first
    ancestor with more than one child; a chain that reaches the root without
    one maps to the root) — reference :125-145;
  * leaves are bucketed by that ancestor in first-seen order, each bucket is
    stably sorted by depth and cut into bundles of ``bundle_size`` leaves,
    emitting at most ``max_bundles`` bundles — reference :42-123;
  * a bundle's shared prefix is the path from the ancestor to its first leaf
    (``_get_path_to_ancestor``, reference :147-171).

Unlike the reference, the child counts are computed once per call instead of
once per leaf, so scheduling is O(N) instead of O(leaves * N).

``bundle_row_order`` turns a schedule into the node permutation used by the
tree-attention kernel to pack query rows: nodes of one bundle (the union of
its leaves' root paths) become adjacent rows, so rows sharing ancestors share
K/V tiles of the tree block.  ``bundle_row_order_device`` computes the same
permutation on the GPU from a device parent tensor (one launch, no host round
trip between the draft tree and the verify launch).
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Dict, List, Optional, Sequence

import torch


def _child_counts(parent_map: Dict[int, int]) -> Dict[int, int]:
    counts: Dict[int, int] = {}
    for _, p in parent_map.items():
        if p >= 0:
            counts[p] = counts.get(p, 0) + 1
    return counts


class BundleScheduler:
    """Group tree leaves into prefix-coherent verification bundles."""

    def __init__(self, bundle_size: int = 3, max_bundles: int = 100, device: str = "cuda"):
        self.bundle_size = bundle_size
        self.max_bundles = max_bundles
        self.device = device
        self.total_scheduled = 0
        self.total_bundles = 0
        self.avg_prefix_length = 0.0

    # -- reference :125-145 --------------------------------------------------
    def _find_branching_ancestor(self, node: int, parent_map: Dict[int, int],
                                 _counts: Optional[Dict[int, int]] = None) -> int:
        counts = _child_counts(parent_map) if _counts is None else _counts
        cur = node
        while cur in parent_map:
            p = parent_map[cur]
            if p < 0:
                return cur
            if counts.get(p, 0) > 1:
                return p
            cur = p
        return 0

    # -- reference :147-171 --------------------------------------------------
    def _get_path_to_ancestor(self, node: int, ancestor: int, parent_map: Dict[int, int]) -> List[int]:
        rev: List[int] = []
        cur = node
        while cur != ancestor and cur in parent_map:
            rev.append(cur)
            p = parent_map[cur]
            if p < 0:
                break
            cur = p
        rev.append(ancestor)
        return rev[::-1]

    # -- reference :42-123 ---------------------------------------------------
    def schedule_bundles(self, tree_descriptor: Dict, return_tensors: bool = True) -> List[Dict]:
        leaf_ids = tree_descriptor["leaf_ids"]
        parent_map = tree_descriptor["parent_map"]
        depth_map = tree_descriptor.get("depth_map", {})
        if isinstance(leaf_ids, torch.Tensor):
            leaf_ids = leaf_ids.cpu().tolist()

        counts = _child_counts(parent_map)
        # dict semantics of the reference: a repeated leaf keeps its first slot
        leaf_anc: "OrderedDict[int, int]" = OrderedDict()
        for leaf in leaf_ids:
            leaf_anc[leaf] = self._find_branching_ancestor(leaf, parent_map, counts)
        buckets: "OrderedDict[int, List[int]]" = OrderedDict()
        for leaf, anc in leaf_anc.items():
            buckets.setdefault(anc, []).append(leaf)

        bundles: List[Dict] = []
        for anc, members in buckets.items():
            if depth_map:
                members = sorted(members, key=lambda x: depth_map.get(x, 0))
            for start in range(0, len(members), self.bundle_size):
                chunk = members[start:start + self.bundle_size]
                prefix = self._get_path_to_ancestor(chunk[0], anc, parent_map) if chunk else []
                bundles.append({
                    "leaves": chunk,
                    "br_anc": anc,
                    "shared_prefix": prefix,
                    "prefix_length": len(prefix),
                    "bundle_id": len(bundles),
                    "bucket_id": anc,
                })
                if len(bundles) >= self.max_bundles:
                    break
            if len(bundles) >= self.max_bundles:
                break

        self.total_scheduled += len(leaf_ids)
        self.total_bundles += len(bundles)
        if bundles:
            self.avg_prefix_length = sum(b["prefix_length"] for b in bundles) / len(bundles)
        if return_tensors:
            bundles = self._convert_to_tensors(bundles)
        return bundles

    def _convert_to_tensors(self, bundles: List[Dict]) -> List[Dict]:
        out = []
        for b in bundles:
            out.append({
                "leaves": torch.tensor(b["leaves"], dtype=torch.long, device=self.device),
                "br_anc": b["br_anc"],
                "shared_prefix": torch.tensor(b["shared_prefix"], dtype=torch.long, device=self.device),
                "prefix_length": b["prefix_length"],
                "bundle_id": b["bundle_id"],
                "bucket_id": b["bucket_id"],
            })
        return out

    def create_bundle_attention_masks(self, bundles: List[Dict], max_seq_len: int) -> List[torch.Tensor]:
        """One int8 [bundle_size, max_seq_len] mask per bundle; the shared prefix is visible."""
        masks = []
        for b in bundles:
            leaves, prefix = b["leaves"], b["shared_prefix"]
            n = leaves.size(0) if isinstance(leaves, torch.Tensor) else len(leaves)
            m = torch.zeros(n, max_seq_len, dtype=torch.int8, device=self.device)
            idx = prefix if isinstance(prefix, torch.Tensor) else torch.tensor(prefix, dtype=torch.long)
            if idx.numel() > 0:
                m[:, idx.to(m.device)] = 1
            masks.append(m)
        return masks

    def merge_bundle_logits(self, bundle_logits: List[torch.Tensor], bundles: List[Dict]) -> torch.Tensor:
        if not bundle_logits:
            return torch.empty(0, device=self.device)
        order = sorted(range(len(bundles)), key=lambda i: bundles[i]["bundle_id"])
        return torch.cat([bundle_logits[i] for i in order], dim=0)

    def get_statistics(self) -> Dict:
        return {
            "total_scheduled_leaves": self.total_scheduled,
            "total_bundles_created": self.total_bundles,
            "avg_bundle_size": self.total_scheduled / self.total_bundles if self.total_bundles > 0 else 0,
            "avg_prefix_length": self.avg_prefix_length,
            "bundle_size_config": self.bundle_size,
        }

    def reset_statistics(self) -> None:
        self.total_scheduled = 0
        self.total_bundles = 0
        self.avg_prefix_length = 0.0


class TreeDescriptorBuilder:
    """Build scheduler descriptors (reference :291-392)."""

    @staticmethod
    def from_draft_tree(tree, final_indices: Optional[torch.Tensor] = None) -> Dict:
        if final_indices is None:
            final_indices = torch.arange(tree.depth * tree.nnodes, device=tree.device)
        parent_map: Dict[int, int] = {}
        depth_map: Dict[int, int] = {}
        ids = final_indices.cpu().tolist()
        for idx in ids:
            row, col = divmod(idx, tree.nnodes)
            depth_map[idx] = row
            parent_map[idx] = -1
            if row > 0:
                pc = int(tree.parents_matrix[row, col].item())
                if pc >= 0:
                    parent_map[idx] = (row - 1) * tree.nnodes + pc
        nodes = set(ids)
        parents = set(parent_map.values()) - {-1}
        return {"leaf_ids": list(nodes - parents), "parent_map": parent_map, "depth_map": depth_map,
                "all_nodes": list(nodes)}

    @staticmethod
    def from_parent_tensor(parent: torch.Tensor, num_nodes: Optional[int] = None) -> Dict:
        if num_nodes is None:
            num_nodes = parent.size(0)
        plist = parent.cpu().tolist()
        parent_map = {i: (int(plist[i]) if i < len(plist) else -1) for i in range(num_nodes)}
        nodes = set(range(num_nodes))
        parents = {p for p in parent_map.values() if p >= 0}
        depth_map: Dict[int, int] = {}
        for node in range(num_nodes):
            d, cur, seen = 0, node, set()
            while cur in parent_map and parent_map[cur] >= 0 and cur not in seen:
                seen.add(cur)
                cur = parent_map[cur]
                d += 1
            depth_map[node] = d
        return {"leaf_ids": list(nodes - parents), "parent_map": parent_map, "depth_map": depth_map,
                "all_nodes": list(nodes)}


def descriptor_from_parents(parent: Sequence[int]) -> Dict:
    """Descriptor of a tree given per-node parents (node 0 = root, parent < 0 = none).

    Same construction as verify_new's scheduling block
    (draft/tree_verification.py:143-153): leaves are the nodes that are nobody's
    parent, in index order; depth comes from walking the parents.
    """
    n = len(parent)
    parent_map = {i: int(parent[i]) if int(parent[i]) != i else -1 for i in range(n)}
    parent_map[0] = -1
    has_child = {p for p in parent_map.values() if p >= 0}
    leaf_ids = [i for i in range(n) if i not in has_child]
    depth_map = {}
    for i in range(n):
        d, cur = 0, i
        while parent_map[cur] >= 0 and d <= n:
            cur = parent_map[cur]
            d += 1
        depth_map[i] = d
    return {"leaf_ids": leaf_ids, "parent_map": parent_map, "depth_map": depth_map}


def bundle_row_order(parent: Sequence[int], bundle_size: int = 3, max_bundles: int = 1 << 30,
                     num_bundles: Optional[int] = None) -> List[int]:
    """Node permutation that packs query rows bundle by bundle.

    The schedule is the reference's (leaves grouped by branching ancestor,
    depth-sorted, chunked); ``num_bundles`` picks bundle_size so that about
    that many bundles result.  For each bundle in order, the nodes on its
    leaves' root paths that are not placed yet are appended (root first);
    nodes on no leaf path (none, in a tree) follow in index order.
    """
    desc = descriptor_from_parents(parent)
    if num_bundles:
        nleaf = max(1, len(desc["leaf_ids"]))
        bundle_size = max(1, -(-nleaf // num_bundles))
    sched = BundleScheduler(bundle_size=bundle_size, max_bundles=max_bundles, device="cpu")
    bundles = sched.schedule_bundles(desc, return_tensors=False)
    pm = desc["parent_map"]
    placed, order = set(), []
    for b in bundles:
        for leaf in b["leaves"]:
            path, cur = [], leaf
            while cur >= 0 and cur not in placed and len(path) <= len(parent):
                path.append(cur)
                cur = pm[cur]
            for node in reversed(path):
                placed.add(node)
                order.append(node)
    order.extend(i for i in range(len(parent)) if i not in placed)
    return order


def bundle_row_order_device(parent: torch.Tensor, bundle_size: int = 3, max_bundles: int = 1 << 30,
                            num_bundles: Optional[int] = None, return_bundles: bool = False):
    """``bundle_row_order`` computed on the GPU (libdsv ``dsv_bundle_order``).

    ``parent``: device int32/int64 ``[M]`` or ``[B, M]`` per-node parents
    (< 0, equal to the node or >= M: none; node 0 is a root), M <= 1024.
    Returns the int32 permutation (same shape; row j packs node perm[..., j]),
    and with ``return_bundles`` also the int32 bundle id of the leaf through
    which each node was placed (-1 for nodes no emitted bundle covers).
    For a tree, the result equals ``bundle_row_order(parent.tolist(), ...)``
    (schedule of the reference's core/bundle_scheduler.py:42-171).
    """
    from .. import _ext

    _ext.require_gpu(parent)
    if parent.dim() not in (1, 2):
        raise ValueError("parent must be [M] or [B, M]")
    perm = torch.empty(parent.shape, dtype=torch.int32, device=parent.device)
    bof = torch.empty_like(perm) if return_bundles else None
    lib = _ext.load()
    rc = lib.dsv_bundle_order(_ext.desc(parent), int(bundle_size), int(num_bundles or 0), int(max_bundles),
                              _ext.desc(perm), _ext.desc(bof), _ext.stream_of(parent.device))
    _ext.check(rc, "bundle_order")
    return (perm, bof) if return_bundles else perm

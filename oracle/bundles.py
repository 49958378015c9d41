"""Bundle scheduling and the bundle-ordered query packing — ORACLE (test
infrastructure only; nothing in the product imports this module).

A sequential restatement, loop for loop, of the reference's scheduler:

  descriptor      verify_new's scheduling block (draft/tree_verification.py:139-159):
                  parent map with node 0 as the root, leaves = nodes that are
                  nobody's parent in index order, a depth per node (the
                  reference uses position ids, which are depth + a constant)
  branching_ancestor   BundleScheduler._find_branching_ancestor
                  (core/bundle_scheduler.py:125-145), child counts recomputed
                  per call as there
  path_to_ancestor     BundleScheduler._get_path_to_ancestor (:147-171)
  schedule        BundleScheduler.schedule_bundles (:42-123): buckets in
                  first-seen order, stable depth sort, chunks of bundle_size,
                  the max_bundles check after each bundle is added
  packing_order   the query-row order fed to the attention kernel: for each
                  bundle and each of its leaves, the leaf's root-path nodes
                  not placed yet, root first; then the unplaced nodes in index
                  order

Pinned by tests/test_oracle_bundles.py: the reference's own vectors
(tests/test_bundle_scheduler.py:20-46 of the reference), hand-worked trees,
and invariants on generated trees (a permutation, parents before children,
bundles contiguous in bundle order).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence


def descriptor(parent: Sequence[int]) -> Dict:
    """parent[i] < 0, == i, or >= len(parent): no parent; node 0 is a root."""
    n = len(parent)
    pm: Dict[int, int] = {}
    for i in range(n):
        p = int(parent[i])
        pm[i] = -1 if (i == 0 or p == i or p < 0 or p >= n) else p
    children = set(pm.values()) - {-1}
    leaves = [i for i in range(n) if i not in children]
    depth = {}
    for i in range(n):
        d, cur = 0, i
        while pm[cur] >= 0 and d <= n:
            cur = pm[cur]
            d += 1
        depth[i] = d
    return {"leaf_ids": leaves, "parent_map": pm, "depth_map": depth}


def branching_ancestor(node: int, parent_map: Dict[int, int]) -> int:
    counts: Dict[int, int] = {}
    for _, p in parent_map.items():
        if p >= 0:
            counts[p] = counts.get(p, 0) + 1
    cur = node
    steps = 0
    while cur in parent_map and steps <= len(parent_map):
        p = parent_map[cur]
        if p < 0:
            return cur
        if counts.get(p, 0) > 1:
            return p
        cur = p
        steps += 1
    return 0


def path_to_ancestor(node: int, ancestor: int, parent_map: Dict[int, int]) -> List[int]:
    path, cur = [], node
    while cur != ancestor and cur in parent_map:
        path.append(cur)
        p = parent_map[cur]
        if p < 0:
            break
        cur = p
    path.append(ancestor)
    return path[::-1]


def schedule(desc: Dict, bundle_size: int, max_bundles: int) -> List[Dict]:
    pm, depth = desc["parent_map"], desc["depth_map"]
    leaf_to_anc = {}
    for leaf in desc["leaf_ids"]:
        leaf_to_anc[leaf] = branching_ancestor(leaf, pm)
    buckets: Dict[int, List[int]] = {}
    for leaf, anc in leaf_to_anc.items():
        buckets.setdefault(anc, []).append(leaf)
    bundles: List[Dict] = []
    for anc, leaves in buckets.items():
        if depth:
            leaves = sorted(leaves, key=lambda x: depth.get(x, 0))
        for s in range(0, len(leaves), bundle_size):
            chunk = leaves[s:s + bundle_size]
            bundles.append({"leaves": chunk, "br_anc": anc,
                            "shared_prefix": path_to_ancestor(chunk[0], anc, pm) if chunk else [],
                            "bundle_id": len(bundles)})
            if len(bundles) >= max_bundles:
                break
        if len(bundles) >= max_bundles:
            break
    return bundles


def packing_order(parent: Sequence[int], bundle_size: int = 3, max_bundles: int = 1 << 30,
                  num_bundles: Optional[int] = None):
    """(order, bundle_of): order[j] = node packed in row j; bundle_of[i] = the
    bundle through whose leaf node i was placed, -1 if none."""
    desc = descriptor(parent)
    if num_bundles:
        bundle_size = max(1, -(-len(desc["leaf_ids"]) // num_bundles))
    bundles = schedule(desc, bundle_size, max_bundles)
    pm, n = desc["parent_map"], len(parent)
    placed = [False] * n
    order: List[int] = []
    bundle_of = [-1] * n
    for b in bundles:
        for leaf in b["leaves"]:
            seg, cur = [], leaf
            while cur >= 0 and not placed[cur] and len(seg) <= n:
                seg.append(cur)
                placed[cur] = True
                cur = pm[cur]
            for node in reversed(seg):
                order.append(node)
                bundle_of[node] = b["bundle_id"]
    order.extend(i for i in range(n) if not placed[i])
    return order, bundle_of

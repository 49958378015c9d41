"""Bundle scheduler (host logic of the query packing): the reference's own
pinned facts (tests/test_bundle_scheduler.py of the reference) plus
brute-force invariants and the row-packing permutation."""

import numpy as np
import pytest
import torch

from diffspec_mi355x.core.bundle_scheduler import (BundleScheduler, TreeDescriptorBuilder, bundle_row_order,
                                                   descriptor_from_parents)
from diffspec_mi355x import workloads as wl


def test_branching_ancestor_reference_vector():
    # reference tests/test_bundle_scheduler.py:20-37
    s = BundleScheduler(bundle_size=3, device="cpu")
    pm = {0: -1, 1: 0, 2: 1, 3: 2, 4: 2, 5: 2, 6: 3, 7: 4, 8: 5}
    assert [s._find_branching_ancestor(n, pm) for n in (6, 7, 8)] == [2, 2, 2]


def test_path_to_ancestor_reference_vector():
    # reference tests/test_bundle_scheduler.py:40-46
    s = BundleScheduler(bundle_size=3, device="cpu")
    assert s._get_path_to_ancestor(4, 1, {0: -1, 1: 0, 2: 1, 3: 2, 4: 3}) == [1, 2, 3, 4]


def test_basic_schedule_and_tensor_conversion():
    s = BundleScheduler(bundle_size=3, device="cpu")
    d = {"leaf_ids": [3, 4, 5, 6], "parent_map": {0: -1, 1: 0, 2: 0, 3: 1, 4: 1, 5: 2, 6: 2},
         "depth_map": {0: 0, 1: 1, 2: 1, 3: 2, 4: 2, 5: 2, 6: 2}}
    b = s.schedule_bundles(d, return_tensors=False)
    assert [x["leaves"] for x in b] == [[3, 4], [5, 6]]
    assert [x["br_anc"] for x in b] == [1, 2]
    assert [x["shared_prefix"] for x in b] == [[1, 3], [2, 5]]
    bt = BundleScheduler(bundle_size=2, device="cpu").schedule_bundles(d, return_tensors=True)
    assert all(isinstance(x["leaves"], torch.Tensor) and isinstance(x["shared_prefix"], torch.Tensor) for x in bt)


def test_statistics_accumulate():
    s = BundleScheduler(bundle_size=3, device="cpu")
    d = {"leaf_ids": [3, 4, 5, 6, 7, 8], "parent_map": {0: -1, 1: 0, 2: 0, 3: 1, 4: 1, 5: 2, 6: 2, 7: 1, 8: 2},
         "depth_map": {i: 1 if 0 < i < 3 else 2 for i in range(9)}}
    for _ in range(3):
        s.schedule_bundles(d, return_tensors=False)
    st = s.get_statistics()
    assert st["total_scheduled_leaves"] == 18 and st["total_bundles_created"] == 6


def test_max_bundles_truncates():
    s = BundleScheduler(bundle_size=1, max_bundles=2, device="cpu")
    d = {"leaf_ids": [3, 4, 5, 6], "parent_map": {0: -1, 1: 0, 2: 0, 3: 1, 4: 1, 5: 2, 6: 2}}
    assert len(s.schedule_bundles(d, return_tensors=False)) == 2


def test_masks_and_descriptor_builder():
    s = BundleScheduler(bundle_size=2, device="cpu")
    d = {"leaf_ids": [3, 4, 5, 6], "parent_map": {0: -1, 1: 0, 2: 0, 3: 1, 4: 1, 5: 2, 6: 2},
         "depth_map": {i: min(i, 2) for i in range(7)}}
    b = s.schedule_bundles(d, return_tensors=True)
    masks = s.create_bundle_attention_masks(b, max_seq_len=10)
    assert len(masks) == len(b) and all(m.shape[1] == 10 and m.dtype == torch.int8 for m in masks)
    assert masks[0][:, [1, 3]].all() and masks[0].sum() == 2 * masks[0].shape[0]
    desc = TreeDescriptorBuilder.from_parent_tensor(torch.tensor([0, 0, 0, 1, 1, 2, 2]), num_nodes=8)
    assert len(desc["parent_map"]) == 8 and len(desc["leaf_ids"]) > 0


def brute_branching(node, parent):
    """Nearest ancestor with > 1 child, root if none (independent formulation)."""
    kids = {}
    for c, p in enumerate(parent):
        if p >= 0:
            kids[p] = kids.get(p, 0) + 1
    cur = node
    while parent[cur] >= 0:
        if kids.get(parent[cur], 0) > 1:
            return parent[cur]
        cur = parent[cur]
    return cur


@pytest.mark.parametrize("seed,M,depth,deg", [(0, 64, 8, 4), (1, 128, 12, 6), (2, 32, 8, 4)])
def test_schedule_invariants_on_generated_trees(seed, M, depth, deg):
    parent, dep = wl.make_tree(M, max_depth=depth, max_outdeg=deg, seed=seed)
    desc = descriptor_from_parents(parent)
    s = BundleScheduler(bundle_size=3, max_bundles=10 ** 6, device="cpu")
    bundles = s.schedule_bundles(desc, return_tensors=False)
    leaves = [l for b in bundles for l in b["leaves"]]
    assert sorted(leaves) == sorted(desc["leaf_ids"])
    seen_anc = []
    for b in bundles:
        assert 1 <= len(b["leaves"]) <= 3
        assert all(brute_branching(l, parent) == b["br_anc"] for l in b["leaves"])
        ds = [dep[l] for l in b["leaves"]]
        assert ds == sorted(ds)
        assert b["shared_prefix"][0] == b["br_anc"] and b["shared_prefix"][-1] == b["leaves"][0]
        if b["br_anc"] not in seen_anc:
            seen_anc.append(b["br_anc"])
    # buckets appear in first-seen order of the ascending leaf list
    first_seen = []
    for l in desc["leaf_ids"]:
        a = brute_branching(l, parent)
        if a not in first_seen:
            first_seen.append(a)
    assert seen_anc == first_seen


@pytest.mark.parametrize("seed,M", [(0, 64), (2, 128)])
def test_bundle_row_order_is_a_parent_first_permutation(seed, M):
    parent, _ = wl.make_tree(M, max_depth=12, max_outdeg=6, seed=seed)
    order = bundle_row_order(parent, num_bundles=8)
    assert sorted(order) == list(range(M))
    where = {n: i for i, n in enumerate(order)}
    assert all(parent[n] < 0 or where[parent[n]] < where[n] for n in range(M))

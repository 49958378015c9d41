"""Oracle of the bundle order (oracle/bundles.py), pinned by the reference's
own scheduler vectors, hand-worked trees and invariants on generated trees."""

import numpy as np
import pytest

from oracle import bundles as ob
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.core.bundle_scheduler import bundle_row_order

# Tree of the reference's tests/test_bundle_scheduler.py:20-37 (0-1-2, node 2
# with children 3, 4, 5, each with one leaf child).
REF_PARENT = [-1, 0, 1, 2, 2, 2, 3, 4, 5]


def test_reference_vectors():
    pm = {0: -1, 1: 0, 2: 1, 3: 2, 4: 2, 5: 2, 6: 3, 7: 4, 8: 5}
    assert [ob.branching_ancestor(n, pm) for n in (6, 7, 8)] == [2, 2, 2]
    pm2 = {0: -1, 1: 0, 2: 1, 3: 2, 4: 3}
    assert ob.path_to_ancestor(4, 1, pm2) == [1, 2, 3, 4]


def test_hand_worked_orders():
    # one bucket (ancestor 2), leaves 6, 7, 8 at equal depth
    assert ob.packing_order(REF_PARENT, bundle_size=3) == ([0, 1, 2, 3, 6, 4, 7, 5, 8], [0] * 9)
    assert ob.packing_order(REF_PARENT, bundle_size=1)[1] == [0, 0, 0, 0, 1, 2, 0, 1, 2]
    # node 1 hangs below node 4 (a parent with a higher index); leaves 1, 2, 3
    # share ancestor 0; depth sort puts 2, 3 (depth 1) before 1 (depth 2)
    par = [-1, 4, 0, 0, 0]
    assert ob.packing_order(par, bundle_size=1) == ([0, 2, 3, 4, 1], [0, 2, 0, 1, 2])
    # two bundles emitted: nodes 1 and 4 are uncovered and follow in index order
    assert ob.packing_order(par, bundle_size=1, max_bundles=2) == ([0, 2, 3, 1, 4], [0, -1, 0, 1, -1])
    # the bound is checked after a bundle is added: 0 still emits one
    assert ob.packing_order(par, bundle_size=1, max_bundles=0) == ([0, 2, 1, 3, 4], [0, -1, 0, -1, -1])
    # num_bundles = 2 over 3 leaves: bundles of 2 leaves
    assert ob.packing_order(par, num_bundles=2)[1] == [0, 1, 0, 0, 1]
    # two buckets: leaf 2 (ancestor 0, first seen) before leaves 3, 4 (ancestor 1)
    par2 = [-1, 0, 5, 1, 1, 0]
    assert ob.packing_order(par2, bundle_size=1) == ([0, 5, 2, 1, 3, 4], [0, 1, 0, 1, 2, 0])
    # single node, chain, star
    assert ob.packing_order([-1]) == ([0], [0])
    assert ob.packing_order([-1, 0, 1, 2]) == ([0, 1, 2, 3], [0] * 4)
    assert ob.packing_order([-1, 0, 0, 0, 0], bundle_size=2) == ([0, 1, 2, 3, 4], [0, 0, 0, 1, 1])


def _relabel(parent, rng):
    """Same tree under a random labelling that keeps node 0 as the root."""
    M = len(parent)
    lab = np.concatenate([[0], 1 + rng.permutation(M - 1)])
    out = [-1] * M
    for i in range(1, M):
        out[lab[i]] = int(lab[parent[i]])
    return out


@pytest.mark.parametrize("seed,M,depth,deg", [(0, 64, 8, 4), (1, 128, 12, 6), (2, 300, 20, 3), (3, 17, 4, 8)])
def test_invariants_and_host_scheduler_agree(seed, M, depth, deg):
    rng = np.random.default_rng(seed)
    parent, _ = wl.make_tree(M, max_depth=depth, max_outdeg=deg, seed=seed)
    for par in (parent, _relabel(parent, rng)):
        for kw in ({"bundle_size": 3}, {"num_bundles": 8}, {"bundle_size": 1}, {"bundle_size": 2, "max_bundles": 3}):
            order, bof = ob.packing_order(par, **kw)
            assert sorted(order) == list(range(M))
            assert order == bundle_row_order(par, **kw)
            where = {n: j for j, n in enumerate(order)}
            covered = [n for n in range(M) if bof[n] >= 0]
            # parents before children; bundles contiguous and in bundle order
            assert all(par[n] < 0 or where[par[n]] < where[n] for n in covered)
            seq = [bof[n] for n in order if bof[n] >= 0]
            assert seq == sorted(seq)
            if "max_bundles" not in kw:
                assert len(covered) == M
            # uncovered nodes close the order, in index order
            tail = order[len(covered):]
            assert tail == sorted(n for n in range(M) if bof[n] < 0)

"""GPU parity of the bundle order (dsv_bundle_order) against the oracle
(bit-exact permutation and bundle ids)."""

import numpy as np
import pytest
import torch

from oracle import bundles as ob
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.core.bundle_scheduler import bundle_row_order_device

pytestmark = pytest.mark.gpu


def _relabel(parent, rng):
    M = len(parent)
    lab = np.concatenate([[0], 1 + rng.permutation(M - 1)])
    out = [-1] * M
    for i in range(1, M):
        out[lab[i]] = int(lab[parent[i]])
    return out


def _check(gpu, par, dtype=torch.int64, **kw):
    want_o, want_b = ob.packing_order(par, **kw)
    t = torch.tensor(par, dtype=dtype, device=gpu)
    perm, bof = bundle_row_order_device(t, return_bundles=True, **kw)
    torch.cuda.synchronize()
    assert perm.tolist() == want_o, kw
    assert bof.tolist() == want_b, kw


@pytest.mark.parametrize("seed,M,depth,deg", [(0, 64, 8, 4), (1, 128, 12, 6), (2, 300, 20, 3),
                                              (3, 17, 4, 8), (4, 1024, 16, 4), (5, 2, 1, 1)])
def test_generated_trees_match_oracle(gpu, seed, M, depth, deg):
    rng = np.random.default_rng(seed)
    parent, _ = wl.make_tree(M, max_depth=depth, max_outdeg=deg, seed=seed)
    for par in (parent, _relabel(parent, rng)):
        for kw in ({"bundle_size": 3}, {"num_bundles": 8}, {"bundle_size": 1}, {"bundle_size": 2, "max_bundles": 3},
                   {"bundle_size": 1, "max_bundles": 0}):
            _check(gpu, par, **kw)
    _check(gpu, parent, dtype=torch.int32, bundle_size=3)


def test_special_trees(gpu):
    M = 1024
    chain = [-1] + list(range(M - 1))          # deepest path: every jumping round is needed
    star = [-1] + [0] * (M - 1)                # one bucket of 1023 leaves
    for par in (chain, star, [-1], [-1, 0, 1, 2, 2, 2, 3, 4, 5], [-1, 4, 0, 0, 0]):
        for kw in ({"bundle_size": 3}, {"bundle_size": 1, "max_bundles": 2}, {"num_bundles": 5}):
            _check(gpu, par, **kw)
    # parents equal to the node, negative or outside the tree mean "no parent"
    _check(gpu, [5, 0, 2, -7, 1, 99, 4], bundle_size=2)


def test_batched_trees_and_strided_parent(gpu):
    M, B = 96, 5
    trees = [wl.make_tree(M, max_depth=10, max_outdeg=5, seed=s)[0] for s in range(B)]
    big = torch.full((B, 2 * M), 7, dtype=torch.int64)
    big[:, ::2] = torch.tensor(trees)
    par = big.to(gpu)[:, ::2]                  # element stride 2
    perm, bof = bundle_row_order_device(par, num_bundles=8, return_bundles=True)
    torch.cuda.synchronize()
    for b in range(B):
        o, bb = ob.packing_order(trees[b], num_bundles=8)
        assert perm[b].tolist() == o and bof[b].tolist() == bb


def test_cycle_still_gives_a_permutation(gpu):
    # 1 -> 2 -> 3 -> 1 never reaches the root: the order is unspecified, but
    # it is a permutation and the launch ends.
    par = torch.tensor([-1, 3, 1, 2, 0, 4], dtype=torch.int64, device=gpu)
    perm = bundle_row_order_device(par)
    torch.cuda.synchronize()
    assert sorted(perm.tolist()) == list(range(6))


def test_device_order_drives_tree_verify(gpu):
    from diffspec_mi355x.core.bundle_scheduler import bundle_row_order
    from diffspec_mi355x.runtime.tree_attention import tree_verify

    inp = wl.make_tree_verify_inputs(n_prefix=300, M=64, H=8, Hk=2, D=128, device=str(gpu), seed=3, max_depth=6)
    par_dev = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    p_dev = bundle_row_order_device(par_dev, num_bundles=8)
    p_host = torch.tensor(bundle_row_order(inp.parent, num_bundles=8), dtype=torch.int32, device=gpu)
    args = (inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 300, par_dev)
    o1, l1 = tree_verify(*args, page_table=inp.page_table, row_perm=p_dev)
    o2, l2 = tree_verify(*args, page_table=inp.page_table, row_perm=p_host)
    torch.cuda.synchronize()
    assert torch.equal(p_dev, p_host)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)

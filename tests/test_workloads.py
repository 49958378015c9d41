"""Seeded workload generators (CPU): tree shape rules, determinism, paging."""

import numpy as np
import pytest
import torch

from diffspec_mi355x import workloads as wl


@pytest.mark.parametrize("M,depth,deg,seed", [(64, 8, 4, 0), (128, 12, 6, 2), (64, 8, 4, 7)])
def test_tree_rules(M, depth, deg, seed):
    parent, dep = wl.make_tree(M, max_depth=depth, max_outdeg=deg, seed=seed)
    assert parent[0] == -1 and dep[0] == 0
    outdeg = np.bincount([p for p in parent if p >= 0], minlength=M)
    assert outdeg.max() <= deg
    assert max(dep) <= depth
    for i in range(1, M):
        assert 0 <= parent[i] < i and dep[i] == dep[parent[i]] + 1
    assert wl.make_tree(M, max_depth=depth, max_outdeg=deg, seed=seed) == (parent, dep)


def test_parent_reference_convention_roundtrip():
    parent, _ = wl.make_tree(20, seed=1)
    pref = wl.parent_to_reference(parent)
    ext = [0] + [p + 1 for p in pref]
    assert ext[1:] == parent[1:]


def test_paged_inputs_gather_cpu():
    inp = wl.make_tree_verify_inputs(n_prefix=100, M=8, H=4, Hk=2, D=64, page_size=16, device="cpu")
    assert sorted(inp.page_table.tolist()) == list(range(inp.kv_pages.shape[2]))
    k = inp.logical_kv(0, 0)
    ps = 16
    for t in [0, 15, 16, 99, 107]:
        assert torch.equal(k[0, t], inp.kv_pages[0, 0, inp.page_table[t // ps], :, t % ps])


def test_accept_inputs_cpu_plant_paths():
    a = wl.make_accept_inputs(T=2, M=16, V=300, dtype=torch.float32, device="cpu")
    for t in range(2):
        top = a.logits[t].argmax(-1)
        node = [i for i in range(16) if a.depths[t][i] == a.planted_len[t]]
        assert node
        assert 1 <= a.planted_len[t] <= 8

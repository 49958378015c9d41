"""Pins of the acceptance oracle (CPU): the restated greedy walk against an
independent brute force, the reference's torch op sequence, hand-made trees,
and closed forms of the typical-acceptance statistics."""

import math

import numpy as np
import pytest
import torch

from oracle import accept as oacc
from oracle import ref_cpu_path as rc
from diffspec_mi355x import workloads as wl


def planted_case(M, V, seed, plen, max_depth=8):
    rng = np.random.default_rng(seed)
    parent, depth = wl.make_tree(M, max_depth=max_depth, seed=seed)
    logits = rng.standard_normal((M, V)).astype(np.float32) * 3
    top = rng.integers(0, V, size=M)
    logits[np.arange(M), top] = 20.0
    draft = rng.integers(0, V, size=M)
    cands = [i for i in range(M) if depth[i] == plen] or [int(np.argmax(depth))]
    node = cands[int(rng.integers(len(cands)))]
    while node > 0:
        draft[node] = top[parent[node]]
        node = parent[node]
    pos = np.array([100 + d for d in depth])
    return logits, draft, parent, depth, pos


@pytest.mark.parametrize("seed", range(8))
def test_greedy_walk_matches_brute_force(seed):
    M, V = 64, 1000
    logits, draft, parent, depth, pos = planted_case(M, V, seed, plen=1 + seed % 8)
    toks, ids, alen, nxt, wid = oacc.greedy_walk(logits, draft, wl.parent_to_reference(parent), pos, max_depth=8)
    bpath, balen, bnxt = oacc.brute_force_greedy(logits, draft, parent, pos)
    assert ids == bpath and alen == balen and nxt == bnxt
    assert toks == [int(draft[i]) for i in ids]
    assert alen >= 1 + seed % 8 or alen == max(depth)


@pytest.mark.parametrize("seed", range(4))
def test_greedy_walk_matches_reference_torch_ops(seed):
    M, V = 32, 500
    logits, draft, parent, depth, pos = planted_case(M, V, seed, plen=3)
    pref = wl.parent_to_reference(parent)
    want = rc.greedy_walk_torch(torch.from_numpy(logits)[None], torch.from_numpy(draft)[None],
                                torch.tensor(pref), torch.from_numpy(pos), max_depth=8)
    got = oacc.greedy_walk(logits, draft, pref, pos, max_depth=8)
    assert tuple(got) == tuple(want)


def test_root_only_when_nothing_matches():
    V = 10
    logits = np.zeros((4, V), dtype=np.float32)
    logits[:, 3] = 1.0
    draft = [3, 5, 5, 5]
    toks, ids, alen, nxt, wid = oacc.greedy_walk(logits, draft, [-1, 0, 1], [7, 8, 9, 10], 8)
    assert ids == [0] and alen == 0 and nxt == 3 and wid == 0


def test_full_chain_accept():
    V = 10
    logits = np.zeros((4, V), dtype=np.float32)
    for i, t in enumerate([1, 2, 3, 4]):
        logits[i, t] = 5
    draft = [9, 1, 2, 3]
    _, ids, alen, nxt, wid = oacc.greedy_walk(logits, draft, [-1, 0, 1], [0, 1, 2, 3], 8)
    assert ids == [0, 1, 2, 3] and alen == 3 and nxt == 4 and wid == 3


def test_tie_on_depth_picks_lowest_index():
    V = 10
    logits = np.zeros((3, V), dtype=np.float32)
    logits[0, 4] = 1
    draft = [0, 4, 4]  # both children of the root match
    _, ids, alen, _, wid = oacc.greedy_walk(logits, draft, [-1, -1], [5, 6, 6], 8)
    assert wid == 1 and ids == [0, 1]


def test_argmax_ties_take_first_index():
    V = 8
    logits = np.zeros((2, V), dtype=np.float32)
    logits[0, [2, 5]] = 3.0  # tie between tokens 2 and 5
    _, ids, _, nxt, _ = oacc.greedy_walk(logits, [0, 2], [-1], [0, 1], 8)
    assert ids == [0, 1]
    _, ids, _, _, _ = oacc.greedy_walk(logits, [0, 5], [-1], [0, 1], 8)
    assert ids == [0]


def test_self_parent_means_root():
    V = 5
    logits = np.zeros((3, V), dtype=np.float32)
    logits[0, 1] = 1
    logits[1, 2] = 1
    # parent_ref[1] == 1 (self) -> node 2 hangs off the root
    _, ids, _, _, _ = oacc.greedy_walk(logits, [0, 1, 1], [-1, 1], [0, 1, 1], 8)
    assert oacc.parent_ext([-1, 1]).tolist() == [0, 0, 0]
    assert ids == [0, 1]


def test_bounded_closure_matches_reference_iteration_count():
    """A chain deeper than max_depth + 2 with a mismatch near the root: the
    reference's bounded closure cannot propagate it to the deep nodes."""
    M, V = 12, 4
    logits = np.zeros((M, V), dtype=np.float32)
    logits[:, 1] = 1
    draft = [1] * M
    draft[1] = 2  # edge root -> 1 fails
    pref = [-1] + list(range(M - 2))  # chain 0-1-2-...-11
    pos = list(range(M))
    want = rc.greedy_walk_torch(torch.from_numpy(logits)[None], torch.tensor([draft]), torch.tensor(pref),
                                torch.tensor(pos), max_depth=2)
    got = oacc.greedy_walk(logits, draft, pref, pos, max_depth=2)
    assert tuple(got) == tuple(want)
    assert got[4] > 4  # a deep node survives the 4-round closure


def test_entropy_closed_forms():
    p, ent = oacc.softmax_stats(np.zeros(1000))
    assert abs(ent - math.log(1000)) < 1e-12
    row = np.full(50, -1e4)
    row[7] = 0
    p, ent = oacc.softmax_stats(row)
    assert abs(ent) < 1e-9 and abs(p[7] - 1) < 1e-12
    # two-point distribution
    row = np.array([0.0, math.log(3.0)])
    p, ent = oacc.softmax_stats(row)
    assert abs(ent - (-(0.25 * math.log(0.25) + 0.75 * math.log(0.75)))) < 1e-12


def test_entropy_ignores_neg_inf_logits():
    # -inf logits have p = 0 and, by 0 log 0 = 0, leave the entropy of the rest
    row = np.array([0.0, -np.inf, math.log(3.0), -np.inf])
    p, ent = oacc.softmax_stats(row)
    assert p[1] == 0 and p[3] == 0
    assert abs(ent - (-(0.25 * math.log(0.25) + 0.75 * math.log(0.75)))) < 1e-12


def test_typical_threshold_rules():
    # uniform over V: p = 1/V, H = log V -> threshold min(eps, alpha / V) = alpha/V < 1/V when alpha < 1
    V = 100
    assert oacc.typical_accept(np.zeros(V), 3, 1.0, 0.09, 0.3)
    # peaked distribution: threshold is eps; a token with p < eps is rejected
    row = np.full(V, 0.0)
    row[0] = 10.0
    p, _ = oacc.softmax_stats(row)
    assert p[1] < 0.09 and not oacc.typical_accept(row, 1, 1.0, 0.09, 0.3)
    assert oacc.typical_accept(row, 0, 1.0, 0.09, 0.3)


def test_typical_accepts_non_argmax_candidate_greedy_rejects():
    V = 20
    logits = np.full((2, V), -5.0, dtype=np.float32)
    logits[0, 3] = 2.0
    logits[0, 4] = 1.9  # high-probability runner-up
    draft = [0, 4]
    _, ids_g, _, _, _ = oacc.greedy_walk(logits, draft, [-1], [0, 1], 8)
    _, ids_t, _, _, _ = oacc.typical_walk(logits, draft, [-1], [0, 1], 8)
    assert ids_g == [0] and ids_t == [0, 1]


def test_typical_with_planted_path_equals_greedy():
    M, V = 64, 2000
    logits, draft, parent, depth, pos = planted_case(M, V, 11, plen=5)
    pref = wl.parent_to_reference(parent)
    assert oacc.typical_walk(logits, draft, pref, pos, 8)[1] == oacc.greedy_walk(logits, draft, pref, pos, 8)[1]


def test_kv_commit_matches_row_by_row_copy_from_the_old_cache():
    # Brute force: every destination row reads the cache as it was before the
    # commit, including when a source slot is also a destination (path
    # [0, 2, 3, 5]: slot 2 is read for row 1 and written by row 2).
    rng = np.random.default_rng(3)
    cache = rng.standard_normal((2, 3, 40, 5))
    for path in ([0, 2, 3, 5], [0], list(range(12)), [0, 1, 7, 8, 11]):
        got = oacc.kv_commit(cache, 20, path)
        want = cache.copy()
        for lead in np.ndindex(*cache.shape[:-2]):
            for i, p in enumerate(path):
                want[lead + (20 + i,)] = cache[lead + (20 + p,)]
        assert np.array_equal(got, want)
        untouched = [t for t in range(40) if not 20 <= t < 20 + len(path)]
        assert np.array_equal(got[..., untouched, :], cache[..., untouched, :])

"""The sampling oracle (oracle/sampling.py) pinned without the GPU.

  * its counter RNG against the Random123 known-answer vectors of Philox4x32-10;
  * its deterministic ln / 2^x against numpy's log / exp2 (a few ulp);
  * its warpers against transformers' own TemperatureLogitsWarper /
    TopPLogitsWarper / TopKLogitsWarper on the committed fixture rows
    (tests/golden/sampling_warpers.json, written by make_sampling_fixtures.py);
  * the top-p cut against an independent float64 nucleus on random rows, and
    the tie rule (higher index first) and top-k ties on hand-made rows;
  * the Gumbel-max draw against the softmax by a chi-square test;
  * the walk with sampled tokens against the greedy walk's rule.
"""

import json
from pathlib import Path

import numpy as np
import pytest
from scipy import stats

from oracle import accept as oacc
from oracle import sampling as sp

GOLDEN = Path(__file__).resolve().parent / "golden" / "sampling_warpers.json"


# Known-answer vectors of philox4x32_10 published with the Random123 library
# (Salmon et al. 2011): (counter, key) -> output block.
PHILOX4X32_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX4X32_KAT)
def test_philox_known_answer_vectors(ctr, key, want):
    got = sp.philox4x32_10(*[np.array([c], dtype=np.uint64) for c in ctr], *key)
    assert [int(g[0]) for g in got] == list(want)


def test_uniforms_use_one_word_per_element_of_a_four_element_group():
    seed, tree, node = 0x0123456789ABCDEF, 3, 7
    u = sp.uniforms(seed, tree, node, 10)
    for v in range(10):
        w = sp.philox4x32_10(np.array([v >> 2], dtype=np.uint64), node, tree, 0, seed & 0xFFFFFFFF, seed >> 32)
        assert u[v] == (float(w[v & 3][0]) + 0.5) * 2.0 ** -32


def test_uniforms_are_open_unit_interval_and_uniform():
    u = sp.uniforms(12345, 3, 7, 200000)
    assert u.min() > 0.0 and u.max() < 1.0
    assert stats.kstest(u, "uniform").pvalue > 1e-4


def test_det_ln_and_exp2_against_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([np.exp(rng.uniform(-40, 40, 100000)), [2.0 ** -52, 1.0, 1 - 2 ** -53, 1 + 2 ** -52, 0.7071]])
    got, want = sp.det_ln(x), np.log(x)
    assert np.all(np.abs(got - want) <= 4e-16 * np.maximum(np.abs(want), 1.0))
    assert sp.det_ln(np.array([1.0]))[0] == 0.0
    u = np.concatenate([rng.uniform(-150, 0, 100000), [0.0, -1.0, -0.5, -199.9]])
    g, w = sp.det_exp2(u), np.exp2(u)
    assert np.all(np.abs(g - w) <= 4e-16 * w)
    assert np.array_equal(sp.det_exp2(np.array([-200.5, -np.inf, np.nan])), np.zeros(3))


def test_warpers_match_transformers_fixtures():
    data = json.loads(GOLDEN.read_text())
    assert data["source"].startswith("transformers")
    for case in data["cases"]:
        x = np.array(case["logits"], dtype=np.float32)
        for r in range(x.shape[0]):
            y = sp.warp_temperature(x[r], case["temperature"], case["dtype"])
            keep = sp.kept_mask(y, case["top_p"], case["top_k"])
            removed = np.array([c == "1" for c in case["removed"][r]])
            assert np.array_equal(~keep, removed), (case["name"], r)
            want = np.array([np.nan if v is None else v for v in case["warped"][r]], dtype=np.float32)
            got = np.where(removed, np.nan, y.astype(np.float32))
            assert np.array_equal(got, want, equal_nan=True), (case["name"], r)


def _float_nucleus(y, top_p):
    """Independent nucleus in float64: walk the order (value, then index,
    descending) accumulating softmax probabilities; keep while the mass
    before an element is below top_p."""
    order = sorted(range(y.size), key=lambda v: (y[v], v), reverse=True)
    p = np.exp(y - y.max())
    p = p / p.sum()
    keep = np.zeros(y.size, dtype=bool)
    acc = 0.0
    for v in order:
        if acc < np.float64(np.float32(top_p)):
            keep[v] = True
        acc += p[v]
    return keep, order, p


@pytest.mark.parametrize("top_p", [0.9, 0.5, 0.05, 0.999])
def test_top_p_matches_an_independent_float_nucleus(top_p):
    rng = np.random.default_rng(int(top_p * 1000))
    for _ in range(20):
        y = rng.normal(0, 2.5, 500).astype(np.float32).astype(np.float64)
        keep = sp.kept_mask(y, top_p, 0)
        want, order, p = _float_nucleus(y, top_p)
        # skip rows whose boundary lies within 1e-9 of top_p (fixed point vs float)
        cum = np.cumsum(p[order])
        if np.min(np.abs(cum - np.float32(top_p))) < 1e-9:
            continue
        assert np.array_equal(keep, want)


def test_top_p_ties_keep_the_higher_indices_first():
    # four equal top values of mass 1/4.2 each and two of 0.1/4.2: top_p 0.3
    # keeps two of the four, the highest indices (the warpers' stable
    # ascending sort removes low indices first)
    y = np.full(10, -np.inf)
    y[[1, 4, 6, 8]] = 0.0
    y[[0, 2]] = np.log(0.1)
    keep = sp.kept_mask(y, 0.3, 0)
    assert np.nonzero(keep)[0].tolist() == [6, 8]
    assert np.nonzero(sp.kept_mask(y, 0.85, 0))[0].tolist() == [1, 4, 6, 8]
    # mass above index 2 is 4/4.2 < 0.96, above index 0 it is 4.1/4.2
    assert np.nonzero(sp.kept_mask(y, 0.96, 0))[0].tolist() == [1, 2, 4, 6, 8]


def test_top_k_keeps_every_tie_of_the_kth_value():
    y = np.array([3.0, 1.0, 2.0, 2.0, 2.0, -1.0])
    assert np.nonzero(sp.kept_mask(y, 1.0, 2))[0].tolist() == [0, 2, 3, 4]
    assert sp.kept_mask(y, 1.0, 100).all()
    # top-p then top-k is the intersection
    k = sp.kept_mask(y, 0.6, 3)
    assert np.array_equal(k, sp.kept_mask(y, 0.6, 0) & sp.kept_mask(y, 1.0, 3))


@pytest.mark.parametrize("temperature,top_p,top_k", [(1.0, 1.0, 0), (0.7, 1.0, 0), (1.0, 0.8, 0), (1.3, 1.0, 3)])
def test_gumbel_max_draws_follow_the_warped_softmax(temperature, top_p, top_k):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1.0, 6).astype(np.float32)
    y = sp.warp_temperature(x, temperature, "f32")
    keep = sp.kept_mask(y, top_p, top_k)
    p = np.where(keep, np.exp(y - y.max()), 0.0)
    p /= p.sum()
    n = 6000
    draws = np.array([sp.sample_row(x, "f32", temperature, top_p, top_k, 99, t, 0) for t in range(n)])
    counts = np.bincount(draws, minlength=x.size)
    assert counts[~keep].sum() == 0
    kept = np.nonzero(keep)[0]
    if kept.size > 1:
        assert stats.chisquare(counts[kept], n * p[kept]).pvalue > 1e-4


def test_no_finite_logit_draws_token_zero():
    x = np.full(7, -np.inf, dtype=np.float32)
    assert sp.sample_row(x, "f32", 1.0, 0.9, 3, 1, 0, 0) == 0
    x[3] = np.nan
    assert sp.sample_row(x, "f32", 1.0, 1.0, 0, 1, 0, 0) == 0


def test_sample_walk_follows_the_greedy_rule_with_the_draws():
    rng = np.random.default_rng(3)
    M, V = 12, 50
    lg = rng.normal(0, 3.0, (M, V)).astype(np.float32)
    parent = [-1, 0, 1, 2, 0, 4, 5, 6, 3, 8, 9, 10]
    pref = [p - 1 for p in parent[1:]]
    pos = np.array([0, 1, 2, 3, 1, 2, 3, 4, 4, 5, 6, 7])
    draws = np.array([sp.sample_row(lg[i], "f32", 0.8, 0.95, 0, 77, 0, i) for i in range(M)])
    draft = rng.integers(0, V, M)
    for node in (1, 2, 3, 8, 9):  # plant the chain 0-1-2-3-8-9
        draft[node] = draws[parent[node]]
    res = sp.sample_walk(lg, "f32", draft, pref, pos, 8, 0.8, 0.95, 0, 77)
    assert np.array_equal(res[5], draws)
    # the greedy walk over logits whose argmax is each row's draw gives the same path
    onehot = np.full((M, V), -1.0, dtype=np.float32)
    onehot[np.arange(M), draws] = 1.0
    assert res[:5] == oacc.greedy_walk(onehot, draft, pref, pos, 8)
    assert res[1][:6] == [0, 1, 2, 3, 8, 9]


def test_reference_call_shape_and_the_per_row_rule():
    """The reference warps the target logits as one [1, M, V] tensor
    (draft/tree_verification.py:104).  transformers' TopPLogitsWarper scatters
    its removal mask along dim 1, so on that shape it raises (an index out of
    range for dimension 1): the reference's top-p branch fails there.  The temperature and top-k warpers
    work on [1, M, V] and give exactly what they give row by row.  This build
    defines sampling by the warpers applied to each [1, V] row, which the
    oracle restates: checked here against transformers on every row."""
    import torch
    from transformers.generation.logits_process import (LogitsProcessorList, TemperatureLogitsWarper,
                                                        TopKLogitsWarper, TopPLogitsWarper)
    g = torch.Generator().manual_seed(3)
    x = torch.randn((1, 4, 50), generator=g) * 2.0
    with pytest.raises((IndexError, RuntimeError), match="out of (range|bounds)"):
        TopPLogitsWarper(0.9)(None, x)
    rowwise = lambda lst, t: torch.cat([lst(None, t[:, r, :].clone()) for r in range(t.shape[1])])
    no_p = LogitsProcessorList([TemperatureLogitsWarper(0.7), TopKLogitsWarper(5)])
    assert torch.equal(no_p(None, x.clone())[0], rowwise(no_p, x))
    for temperature, top_p, top_k in [(0.7, 0.9, 0), (1.0, 0.5, 7), (1.3, 0.95, 3)]:
        lst = LogitsProcessorList()
        if temperature != 1.0:
            lst.append(TemperatureLogitsWarper(temperature))
        lst.append(TopPLogitsWarper(top_p))
        if top_k > 0:
            lst.append(TopKLogitsWarper(top_k))
        warped = rowwise(lst, x)
        for r in range(x.shape[1]):
            y = sp.warp_temperature(x[0, r].numpy(), temperature, "f32")
            keep = sp.kept_mask(y, top_p, top_k)
            assert np.array_equal(keep, torch.isfinite(warped[r]).numpy()), (temperature, top_p, top_k, r)

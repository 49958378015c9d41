"""Known-answer vectors of the reference's own tests (tests/golden/reference_test_vectors.json)
against the oracle and the host-side product code, on the CPU.

  * bundle scheduling: the branching ancestor and the ancestor path of the
    reference's scheduler tests, through oracle/bundles.py and the product's
    BundleScheduler;
  * paged KV: page counts, the contiguous token window and the physical block
    list of the reference's paged-cache tests, through the [P, Hk, page, D]
    pool layout the kernels read (oracle/attention.py::paged_gather and
    TreeVerifyInputs.logical_kv).
"""

import json
from pathlib import Path

import numpy as np
import torch

from oracle import attention as oa
from oracle import bundles as ob
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.core.bundle_scheduler import BundleScheduler

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "reference_test_vectors.json").read_text())


def _pm(d):
    return {int(k): int(v) for k, v in d.items()}


def test_branching_ancestor_vector():
    g = GOLDEN["bundle_scheduler"]["branching_ancestor"]
    pm = _pm(g["parent_map"])
    assert [ob.branching_ancestor(n, pm) for n in g["nodes"]] == g["expected"]
    s = BundleScheduler(bundle_size=g["bundle_size"], device="cpu")
    assert [s._find_branching_ancestor(n, pm) for n in g["nodes"]] == g["expected"]


def test_path_to_ancestor_vector():
    g = GOLDEN["bundle_scheduler"]["path_to_ancestor"]
    pm = _pm(g["parent_map"])
    assert ob.path_to_ancestor(g["node"], g["ancestor"], pm) == g["expected"]
    s = BundleScheduler(bundle_size=g["bundle_size"], device="cpu")
    assert s._get_path_to_ancestor(g["node"], g["ancestor"], pm) == g["expected"]


def test_pages_for_tokens_vector():
    g = GOLDEN["paged_kv"]["pages_for_tokens"]
    # the pool of a 50-token sequence (tree of 2 nodes after a 48-token prefix)
    inp = wl.make_tree_verify_inputs(n_prefix=g["num_tokens"] - 2, M=2, H=4, Hk=4, D=32,
                                     page_size=g["page_size"], device="cpu")
    assert inp.page_table.numel() == g["expected_pages"]
    assert inp.kv_pages.shape[2] == g["expected_pages"]


def test_contiguous_window_vector():
    g = GOLDEN["paged_kv"]["contiguous_window"]
    ps, Hk, D = g["page_size"], g["num_heads"], g["head_dim"]
    n_alloc, n_written = g["allocated_tokens"], g["written_tokens"]
    lo, hi = g["window"]
    n_pages = -(-n_alloc // ps)
    P = 50
    # logical pages on scattered physical pages of a larger pool
    pt = np.random.default_rng(3).permutation(P)[:n_pages]
    pool = np.zeros((P, Hk, ps, D), dtype=np.float32)
    for t in range(n_written):
        pool[pt[t // ps], :, t % ps, :] = float(t)
    keys = oa.paged_gather(pool, pt, n_alloc)[lo:hi].transpose(1, 0, 2)  # [heads, tokens, dim]
    assert list(keys.shape) == g["expected_shape_heads_tokens_dim"]
    assert keys[0, 0, 0] == g["expected_first_key_element"]
    assert np.array_equal(keys[:, :, 0], np.broadcast_to(np.arange(lo, hi, dtype=np.float32), (Hk, hi - lo)))
    # the product's logical view of the same pool reads the same window
    inp = wl.TreeVerifyInputs(q=torch.zeros(1, 1, Hk, D), kv_pages=torch.from_numpy(np.stack([pool, pool])[None]),
                              page_table=torch.from_numpy(pt.astype(np.int32)), n_prefix=n_alloc - 1, parent=[-1],
                              depth=[0], page_size=ps)
    view = inp.logical_kv(0, 0)[0, lo:hi].permute(1, 0, 2).numpy()
    assert np.array_equal(view, keys)


def test_physical_blocks_vector():
    g = GOLDEN["paged_kv"]["physical_blocks"]
    inp = wl.make_tree_verify_inputs(n_prefix=g["num_tokens"] - 2, M=2, H=4, Hk=4, D=32,
                                     page_size=g["page_size"], device="cpu")
    blocks = inp.page_table.tolist()
    assert len(blocks) == -(-g["num_tokens"] // g["page_size"])
    assert all(b >= 0 for b in blocks) and len(set(blocks)) == len(blocks)

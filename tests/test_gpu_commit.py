"""GPU parity of the accepted-path KV commit against the oracle (bit-exact).

The commit moves cache rows: tokens [start, start + n) of every row receive
tokens start + path[0..n), every read before any write, with n = info[3] and
path taken from device memory (as written by the acceptance kernel)."""

import numpy as np
import pytest
import torch

from oracle import accept as oacc
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.draft.tree_verification import kv_commit, tree_accept

pytestmark = pytest.mark.gpu


def _path_info(path, M, gpu, n=None):
    p = torch.full((1, M), -1, dtype=torch.int64)
    p[0, :len(path)] = torch.tensor(path, dtype=torch.int64)
    info = torch.tensor([[path[-1], len(path) - 1, 0, len(path) if n is None else n]], dtype=torch.int64)
    return p.to(gpu), info.to(gpu)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("path", [[0, 2, 3, 5], [0], list(range(24)), [0, 1, 7, 8, 15, 23]])
def test_dense_commit_matches_oracle(gpu, dtype, path):
    M, S, start = 24, 100, 61
    g = torch.Generator().manual_seed(len(path))
    cache = torch.randn((3, 2, 2, S, 64), generator=g).to(dtype)
    want = oacc.kv_commit(cache.float().numpy(), start, path)
    x = cache.to(gpu)
    p, info = _path_info(path, M, gpu)
    kv_commit(x, start, p, info)
    torch.cuda.synchronize()
    assert np.array_equal(x.float().cpu().numpy(), want)


def test_dense_commit_reference_layout_and_noop_cases(gpu):
    # [2, B, H, S, D] fp32 (the reference's past_key_values_data layout), D = 8.
    M, S, start = 16, 80, 60
    cache = torch.randn((2, 1, 2, S, 8))
    x = cache.to(gpu)
    # info[3] = -1 (malformed tree reported by the walk): nothing moves.
    p, info = _path_info([0, 3], M, gpu, n=-1)
    kv_commit(x, start, p, info)
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), cache)
    # Root only: token start onto itself.
    p, info = _path_info([0], M, gpu)
    kv_commit(x, start, p, info)
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), cache)
    p, info = _path_info([0, 4, 9, 15], M, gpu)
    kv_commit(x, start, p, info)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), oacc.kv_commit(cache.numpy(), start, [0, 4, 9, 15]))


def test_paged_commit_matches_oracle_on_the_logical_view(gpu):
    # Page pool [L, 2, P, Hk, 16, D] behind a random permutation; the tree's
    # tokens [start, start + M) straddle pages.
    inp = wl.make_tree_verify_inputs(n_prefix=150, M=40, H=8, Hk=2, D=128, layers=2, device=str(gpu), seed=4)
    start, M = 150, 40
    path = [0, 1, 5, 6, 17, 30, 39]
    before = [[inp.logical_kv(l, h)[0].float().cpu().numpy() for h in range(2)] for l in range(2)]
    p, info = _path_info(path, M, gpu)
    kv_commit(inp.kv_pages, start, p, info, page_table=inp.page_table)
    torch.cuda.synchronize()
    for l in range(2):
        for h in range(2):
            got = inp.logical_kv(l, h)[0].float().cpu().numpy()
            # logical view [n, Hk, D]: tokens on axis 0 -> move them to axis -2
            want = np.moveaxis(oacc.kv_commit(np.moveaxis(before[l][h], 0, -2), start, path), -2, 0)
            assert np.array_equal(got, want)


def test_commit_from_the_walk_output(gpu):
    # path and info straight from the acceptance kernel, no host round trip.
    a = wl.make_accept_inputs(T=1, M=16, V=3000, device=str(gpu), seed=9, pos_offset=50)
    r = tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10)
    n = int(r["info"][0, 3])
    path = r["path"][0, :n].tolist()
    cache = torch.randn((4, 2, 2, 70, 64)).to(torch.bfloat16)
    x = cache.to(gpu)
    kv_commit(x, 50, r["path"], r["info"])
    torch.cuda.synchronize()
    assert np.array_equal(x.float().cpu().numpy(), oacc.kv_commit(cache.float().numpy(), 50, path))


def test_out_of_range_path_entries_stay_inside_the_tree_slots(gpu):
    # Entries outside [0, M) are clamped to the tree; rows outside
    # [start, start + M) are never touched.
    M, S, start = 8, 40, 10
    cache = torch.randn((1, 2, S, 64)).to(torch.bfloat16)
    x = cache.to(gpu)
    p = torch.tensor([[0, 999, -5, 3, -1, -1, -1, -1]], dtype=torch.int64, device=gpu)
    info = torch.tensor([[3, 3, 0, 4]], dtype=torch.int64, device=gpu)
    kv_commit(x, start, p, info)
    torch.cuda.synchronize()
    got = x.float().cpu().numpy()
    want = oacc.kv_commit(cache.float().numpy(), start, [0, 7, 0, 3])
    assert np.array_equal(got, want)


def test_commit_random_layouts(gpu):
    """24 random commits, bit-exact: dense caches of 1-4 leading dimensions
    (layers, K/V, batch, heads) in bf16 / f16 / f32 with head_dim 8 to 256,
    and page pools of 1- to 64-token pages behind a random permutation; paths
    are random root-first increasing node lists of 1 to M nodes."""
    rng = np.random.default_rng(44)
    for case in range(24):
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        esize = 4 if dtype == torch.float32 else 2
        D = int(rng.choice([d for d in (8, 16, 64, 128, 256) if (d * esize) % 16 == 0]))
        M = int(rng.choice([1, 5, 24, 64, 128]))
        M = min(M, 65536 // (D * esize))                  # the kernel's row budget: M * row bytes <= 64 KiB
        n = int(rng.integers(1, M + 1))
        path = [0] + sorted(rng.choice(np.arange(1, M), size=n - 1, replace=False).tolist()) if M > 1 else [0]
        paged = bool(rng.integers(2))
        print(f"[commit random] case {case}: {dtype} D={D} M={M} path={len(path)} paged={paged}", flush=True)
        p, info = _path_info(path, M, gpu)
        if not paged:
            start = int(rng.integers(0, 100))
            lead = tuple(int(x) for x in rng.integers(1, 4, size=int(rng.integers(1, 5))))
            cache = torch.randn(lead + (start + M + int(rng.integers(0, 9)), D)).to(dtype)
            want = oacc.kv_commit(cache.float().numpy(), start, path)
            x = cache.to(gpu)
            kv_commit(x, start, p, info)
            torch.cuda.synchronize()
            assert np.array_equal(x.float().cpu().numpy(), want), f"case {case}"
        else:
            ps = int(rng.choice([1, 2, 16, 64]))
            start = int(rng.integers(0, 300))
            L, Hk = int(rng.integers(1, 3)), int(rng.integers(1, 4))
            n_pages = (start + M + ps - 1) // ps
            pool = torch.randn((L, 2, n_pages + 3, Hk, ps, D)).to(dtype).to(gpu)
            pt = torch.from_numpy(rng.permutation(n_pages + 3)[:n_pages].astype(np.int32)).to(gpu)
            tok = torch.arange(start + M, device=gpu)
            # the logical view: tokens first ([n, L, 2, Hk, D]), then on axis -2 for the oracle
            before = np.moveaxis(pool[:, :, pt[tok // ps].long(), :, tok % ps].float().cpu().numpy(), 0, -2)
            kv_commit(pool, start, p, info, page_table=pt)
            torch.cuda.synchronize()
            got = np.moveaxis(pool[:, :, pt[tok // ps].long(), :, tok % ps].float().cpu().numpy(), 0, -2)
            assert np.array_equal(got, oacc.kv_commit(before, start, path)), f"case {case}"

"""HIP graph capture of the hot-path entry points.

Each test runs an entry point eagerly, captures the same call once in a HIP
graph, then replays the graph three times. Between replays it runs eager work
of the same entry point on other data and synchronises the device. Every replay
must reproduce the eager result bit for bit, since the kernels are
deterministic. In-place entry points get their input restored before each
replay. Outputs are cleared before each replay, so a replay that writes nothing
fails.

Graph capture works because the library records no memset node and every
workspace comes from the caller: the wrappers allocate it from torch, so inside
a capture it comes from the graph's pool.
"""

import numpy as np
import pytest
import torch

from diffspec_mi355x import workloads as wl
from diffspec_mi355x.core.bundle_scheduler import bundle_row_order_device
from diffspec_mi355x.draft.tree_verification import kv_commit, lmhead_tree_accept, tree_accept
from diffspec_mi355x.runtime.cache_state import append_tree_kv
from diffspec_mi355x.runtime.tree_attention import tree_verify

pytestmark = pytest.mark.gpu


def _flat(x):
    if isinstance(x, dict):
        return [x[k] for k in sorted(x)]
    if isinstance(x, (tuple, list)):
        return list(x)
    return [x]


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, _flat(out)


def _replays_match(g, out, want, between, before=None):
    for r in range(3):
        if before is not None:
            before()
        for t in out:
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(out, want)):
            assert torch.equal(a, b), f"replay {r}: output {i} differs from the eager result"
        between()
        torch.cuda.synchronize()


def test_tree_verify_graph_replays(gpu):
    print("[graph] tree_verify paged 4096/64", flush=True)
    inp = wl.make_tree_verify_inputs(n_prefix=4096, M=64, device=str(gpu), seed=5, tree_seed=5)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    other = wl.make_tree_verify_inputs(n_prefix=1000, M=20, device=str(gpu), seed=6, tree_seed=6)
    opar = torch.tensor(other.parent, dtype=torch.int64, device=gpu)

    def fn():
        return tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 4096, par, page_table=inp.page_table)

    want = [t.clone() for t in _flat(fn())]
    g, out = _capture(fn)
    _replays_match(g, out, want, lambda: tree_verify(other.q, other.kv_pages[0, 0], other.kv_pages[0, 1], 1000, opar,
                                                     page_table=other.page_table))


_ACCEPT_KW = {"greedy": ("greedy", {}),
              "typical": ("typical", dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3)),
              "sample_top_p_top_k": ("sample", dict(temperature=0.7, top_p=0.9, top_k=50, seed=11)),
              "sample_temperature": ("sample", dict(temperature=1.3, seed=12))}


@pytest.mark.parametrize("case", list(_ACCEPT_KW))
def test_tree_accept_graph_replays(gpu, case):
    print(f"[graph] tree_accept {case}", flush=True)
    a = wl.make_accept_inputs(T=4, M=32, V=5000, device=str(gpu), seed=3)
    b = wl.make_accept_inputs(T=2, M=16, V=3000, device=str(gpu), seed=4)
    mode, kw = _ACCEPT_KW[case]

    def fn():
        return tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode=mode, return_next=True, **kw)

    want = [t.clone() for t in _flat(fn())]
    g, out = _capture(fn)
    _replays_match(g, out, want, lambda: tree_accept(b.logits, b.draft, b.parent_ref, b.pos, 10, mode=mode, **kw))


def test_lmhead_accept_graph_replays(gpu):
    print("[graph] lmhead_tree_accept greedy", flush=True)
    gen = torch.Generator().manual_seed(9)
    T, M, Dm, V = 2, 24, 256, 3000
    h = torch.randn((T, M, Dm), generator=gen).to(torch.bfloat16).to(gpu)
    w = (torch.randn((V, Dm), generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    parents = [wl.make_tree(M, max_depth=6, max_outdeg=4, seed=20 + t)[0] for t in range(T)]
    pref = torch.tensor([p[1:] for p in parents], dtype=torch.int64, device=gpu) - 1
    pref = torch.where(pref < 0, torch.full_like(pref, -1), pref)
    draft = torch.from_numpy(np.random.default_rng(1).integers(0, V, size=(T, M))).to(gpu)
    pos = torch.arange(M, device=gpu)

    def fn():
        return lmhead_tree_accept(h, w, draft, pref, pos, 8, return_next=True)

    want = [t.clone() for t in _flat(fn())]
    g, out = _capture(fn)
    _replays_match(g, out, want, lambda: lmhead_tree_accept(h[:1, :5], w, draft[:1, :5], pref[:1, :4], pos[:5], 4))


def test_bundle_order_graph_replays(gpu):
    print("[graph] bundle order", flush=True)
    par = torch.tensor(wl.make_tree(128, max_depth=12, max_outdeg=6, seed=7)[0], dtype=torch.int64, device=gpu)
    par2 = torch.tensor(wl.make_tree(40, seed=8)[0], dtype=torch.int64, device=gpu)

    def fn():
        return bundle_row_order_device(par, num_bundles=8, return_bundles=True)

    want = [t.clone() for t in _flat(fn())]
    g, out = _capture(fn)
    _replays_match(g, out, want, lambda: bundle_row_order_device(par2, bundle_size=2))


def test_kv_commit_graph_replays(gpu):
    print("[graph] kv_commit dense", flush=True)
    gen = torch.Generator().manual_seed(11)
    S, start, M = 100, 61, 24
    orig = torch.randn((3, 2, 2, S, 64), generator=gen).to(torch.bfloat16).to(gpu)
    path = torch.full((1, M), -1, dtype=torch.int64)
    path[0, :5] = torch.tensor([0, 1, 7, 8, 15])
    path = path.to(gpu)
    info = torch.tensor([[15, 4, 0, 5]], dtype=torch.int64, device=gpu)
    cache = orig.clone()
    kv_commit(cache, start, path, info)
    want = cache.clone()
    cache.copy_(orig)
    torch.cuda.synchronize()
    g, _ = _capture(lambda: kv_commit(cache, start, path, info))
    scratch = orig.clone()

    def between():
        kv_commit(scratch, start, path, info)

    def before():
        cache.copy_(orig)

    for r in range(3):
        before()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache, want), f"replay {r}: committed cache differs from the eager result"
        between()
        torch.cuda.synchronize()


def test_kv_append_graph_replays(gpu):
    print("[graph] kv append + RoPE dense", flush=True)
    gen = torch.Generator().manual_seed(12)
    M, Hk, H, D, S, start = 37, 4, 16, 128, 120, 70
    dt = torch.bfloat16
    k = (torch.randn((M, Hk, D), generator=gen) * 2).to(dt).to(gpu)
    v = torch.randn((M, Hk, D), generator=gen).to(dt).to(gpu)
    q = (torch.randn((1, M, H, D), generator=gen) * 2).to(dt).to(gpu)
    pos = torch.arange(5000, 5000 + M, dtype=torch.float32)
    inv = 1.0 / (5e5 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], -1)
    cos, sin = emb.cos().to(dt).to(gpu), emb.sin().to(dt).to(gpu)
    k0 = torch.randn((1, Hk, S, D), generator=gen).to(dt).to(gpu)
    v0 = torch.randn((1, Hk, S, D), generator=gen).to(dt).to(gpu)
    kc, vc = k0.clone(), v0.clone()
    q_want = append_tree_kv(k, v, kc, vc, start, cos=cos, sin=sin, q=q).clone()
    k_want, v_want = kc.clone(), vc.clone()
    kc.copy_(k0)
    vc.copy_(v0)
    torch.cuda.synchronize()
    g, out = _capture(lambda: append_tree_kv(k, v, kc, vc, start, cos=cos, sin=sin, q=q))
    ks, vs = k0.clone(), v0.clone()
    for r in range(3):
        kc.copy_(k0)
        vc.copy_(v0)
        out[0].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], q_want), f"replay {r}: rotated q differs from the eager result"
        assert torch.equal(kc, k_want) and torch.equal(vc, v_want), f"replay {r}: cache differs from the eager result"
        append_tree_kv(k[:5], v[:5], ks, vs, 3)
        torch.cuda.synchronize()

"""GPU parity of the attention kernels (1: split-K prefix, 2: tree block, 3: merge)
against the float64 oracle on identical seeded inputs.

Tolerances (attention outputs):
  * max-abs 2e-2 and mean-abs 2e-3 against the fp32/fp64 computation;
  * because that bar alone cannot see a zero output at 64K context (softmax is
    nearly uniform there), every case also asserts a relative error
    ||O - O*|| / ||O*|| <= 1e-2 (bf16 output) or 4e-3 (fp32 output) and a
    natural-log LSE error <= 2e-3, and tree-only / short-prefix cases check
    the tree block where it carries weight.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.core.bundle_scheduler import bundle_row_order
from diffspec_mi355x.runtime.bundle_verifier import FusedBundleVerifier, PagedBundleVerifier
from diffspec_mi355x.runtime.tree_attention import prefix_attention_forward, tree_attention_forward, tree_verify

pytestmark = pytest.mark.gpu


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_attn_close(got, want, rel=1e-2, max_abs=2e-2, mean_abs=2e-3, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    diff = np.abs(got - want)
    r = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert diff.max() <= max_abs, f"{what} max-abs {diff.max():.3e}"
    assert diff.mean() <= mean_abs, f"{what} mean-abs {diff.mean():.3e}"
    assert r <= rel, f"{what} relative {r:.3e}"


def assert_lse_close(got, want, tol=2e-3, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert np.array_equal(np.isneginf(got), np.isneginf(want)), f"{what} -inf pattern differs"
    fin = np.isfinite(want)
    if fin.any():
        err = np.abs(got[fin] - want[fin]).max()
        assert err <= tol, f"{what} lse err {err:.3e}"


def rand(shape, seed, dtype, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D,H,Hk,M,N,B", [(128, 32, 8, 64, 1000, 2), (64, 8, 8, 10, 20, 1), (128, 32, 8, 5, 4096, 1),
                                         (64, 16, 4, 33, 777, 1)])
def test_prefix_attention_matches_oracle(gpu, dtype, D, H, Hk, M, N, B):
    print(f"[prefix] dtype={dtype} D={D} H={H} Hk={Hk} M={M} N={N} B={B}", flush=True)
    q, k, v = rand((B, M, H, D), 1, dtype, gpu), rand((B, N, Hk, D), 2, dtype, gpu), rand((B, N, Hk, D), 3, dtype, gpu)
    out, lse = prefix_attention_forward(q, k, v, B, M, H, D)
    torch.cuda.synchronize()
    assert out.dtype == dtype and lse.shape == (B, H, M)
    for b in range(B):
        o_ref, l_ref = oa.prefix_attention(np64(q[b]), np64(k[b]), np64(v[b]))
        assert_attn_close(np64(out[b]), o_ref, what=f"b={b}")
        assert_lse_close(np64(lse[b]), l_ref, what=f"b={b}")


def test_prefix_attention_expanded_kv_and_cache_seqlens(gpu):
    B, M, H, D, N = 1, 16, 8, 128, 300
    q = rand((B, M, H, D), 4, torch.bfloat16, gpu)
    k2 = rand((B, N, 2, D), 5, torch.bfloat16, gpu)
    v2 = rand((B, N, 2, D), 6, torch.bfloat16, gpu)
    # repeat_kv-expanded form (H key heads) must equal the GQA form
    ke = k2.repeat_interleave(4, dim=2)
    ve = v2.repeat_interleave(4, dim=2)
    o1, l1 = prefix_attention_forward(q, k2, v2, B, M, H, D)
    o2, l2 = prefix_attention_forward(q, ke, ve, B, M, H, D)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    from diffspec_mi355x.runtime.attention_compat import flash_attn_with_kvcache
    o3, l3 = flash_attn_with_kvcache(q, k2, v2, causal=False, cache_seqlens=123, return_softmax_lse=True)
    o_ref, l_ref = oa.prefix_attention(np64(q[0]), np64(k2[0, :123]), np64(v2[0, :123]))
    assert_attn_close(np64(o3[0]), o_ref)
    assert_lse_close(np64(l3[0]), l_ref)
    # A scalar length is the reference's k_cache[:, :n] (attention_compat.py:113):
    # an int or 0-dim tensor beyond N keeps all N keys, a negative one drops -n
    # keys from the end, in both forms alike.
    for n, keys in [(N + 50, N), (-20, N - 20)]:
        for cs in (n, torch.tensor(n)):
            o4, l4 = flash_attn_with_kvcache(q, k2, v2, cache_seqlens=cs, return_softmax_lse=True)
            o_ref, l_ref = oa.prefix_attention(np64(q[0]), np64(k2[0, :keys]), np64(v2[0, :keys]))
            assert_attn_close(np64(o4[0]), o_ref, what=f"cache_seqlens={cs!r}")
            assert_lse_close(np64(l4[0]), l_ref, what=f"cache_seqlens={cs!r}")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("seqlen_dtype,dtype", [(torch.int32, torch.bfloat16), (torch.int64, torch.bfloat16),
                                                (torch.int64, torch.float32)])
def test_flash_attn_with_kvcache_per_batch_seqlens(gpu, causal, seqlen_dtype, dtype):
    """flash-attn's contract (runtime/attention_compat.py:103-132 stands in for
    it): per-batch cache_seqlens, and causal masking aligned to the end of each
    batch's keys; a row with no visible key has out 0 and lse -inf."""
    from diffspec_mi355x.runtime.attention_compat import flash_attn_with_kvcache
    B, M, H, Hk, D, N = 4, 16, 8, 2, 128, 700
    print(f"[flash_attn_with_kvcache] causal={causal} seqlens={seqlen_dtype} dtype={dtype}", flush=True)
    q = rand((B, M, H, D), 41, dtype, gpu)
    k, v = rand((B, N, Hk, D), 42, dtype, gpu), rand((B, N, Hk, D), 43, dtype, gpu)
    lens = [700, 123, 9, 0]
    out, lse = flash_attn_with_kvcache(q, k, v, causal=causal, cache_seqlens=torch.tensor(lens, dtype=seqlen_dtype,
                                                                                          device=gpu),
                                       return_softmax_lse=True)
    torch.cuda.synchronize()
    assert out.shape == q.shape and lse.shape == (B, H, M)
    for b, n in enumerate(lens):
        keep = np.ones((M, N), dtype=bool)
        keep[:, n:] = False
        if causal:
            keep &= np.arange(N)[None, :] <= (n - M + np.arange(M))[:, None]
        o_ref, l_ref = oa.masked_attention(np64(q[b]), np64(k[b]), np64(v[b]), keep)
        assert_attn_close(np64(out[b]), o_ref, what=f"b={b}")
        assert_lse_close(np64(lse[b]).T, l_ref, what=f"b={b}")
    # a scalar length is the reference's own form
    o1 = flash_attn_with_kvcache(q, k, v, causal=causal, cache_seqlens=321)
    o2 = flash_attn_with_kvcache(q, k, v, causal=causal, cache_seqlens=torch.full((B,), 321, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def rising_scores_case(profile, B, M, H, Hk, D, N, seed=11):
    """q, k whose scores grow along the key sequence (in nats, after the 1/sqrt(D) scale).

    saw: the scores rise from about 0 to about 60 over every 64 keys (two 32-key tiles)
    and drop back, so inside any run of keys that starts on a multiple of 64 the row
    maximum jumps by about 30 nats from the first tile to the second.
    late_spike: small scores except a few keys near the end whose scores are about 60
    nats above the rest.
    """
    g = torch.Generator().manual_seed(seed)
    G = H // Hk
    u = torch.where(torch.rand((Hk, D), generator=g) < 0.5, -1.0, 1.0)  # |u|^2 = D
    q = 0.3 * torch.randn((B, M, H, D), generator=g) + 4.0 * u.repeat_interleave(G, dim=0)[None, None]
    k = 0.3 * torch.randn((B, N, Hk, D), generator=g)
    v = torch.randn((B, N, Hk, D), generator=g)
    s = 4.0 * D / D ** 0.5  # score of k = u against q = 4u
    if profile == "saw":
        alpha = (60.0 / s) * (torch.arange(N) % 64).float() / 63.0
        k = k + alpha[None, :, None, None] * u[None, None]
    else:
        for n in (N - 40, N - 7, N - 1):
            k[:, n] += (60.0 / s) * u[None]
    return q, k, v


@pytest.mark.parametrize("profile,N", [("saw", 3000), ("saw", 20000), ("late_spike", 3000)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_prefix_attention_rising_scores(gpu, profile, N, dtype):
    """Row maxima that jump by tens of nats from one tile to the next inside a split:
    the online softmax must follow them (the accumulators hold the full range without
    overflow)."""
    B, M, H, Hk, D = 1, 24, 16, 4, 128
    print(f"[rising] profile={profile} N={N} dtype={dtype}", flush=True)
    q, k, v = (x.to(dtype).to(gpu) for x in rising_scores_case(profile, B, M, H, Hk, D, N))
    out, lse = prefix_attention_forward(q, k, v, B, M, H, D)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    o_ref, l_ref = oa.prefix_attention(np64(q[0]), np64(k[0]), np64(v[0]))
    assert l_ref.min() > 40.0  # every row's maximum lies > 40 nats above its first keys' scores
    assert_attn_close(np64(out[0]), o_ref)
    assert_lse_close(np64(lse[0]), l_ref)


@pytest.mark.parametrize("mask_kind", ["float_additive", "int8", "bool", "bf16_additive"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tree_attention_forward_matches_oracle(gpu, mask_kind, dtype):
    B, M, H, Hk, D, T = 2, 64, 32, 8, 128, 70
    print(f"[tree_attention_forward] mask={mask_kind} dtype={dtype}", flush=True)
    q = rand((B, M, H, D), 7, dtype, gpu)
    k = rand((B, M, Hk, D), 8, dtype, gpu)
    v = rand((B, M, Hk, D), 9, dtype, gpu)
    parents = [wl.make_tree(M, seed=s)[0] for s in (3, 4)]
    keep = np.stack([oa.ancestor_mask(p) for p in parents])
    full = np.zeros((B, 1, T, T), dtype=bool)
    full[:, 0, -M:, -M:] = keep
    if mask_kind == "float_additive":
        mask = torch.where(torch.from_numpy(full), 0.0, torch.finfo(torch.float32).min).to(gpu)
    elif mask_kind == "bf16_additive":
        mask = torch.where(torch.from_numpy(full), 0.0, -1e30).to(torch.bfloat16).to(gpu)
    elif mask_kind == "int8":
        mask = torch.from_numpy(full).to(torch.int8).to(gpu)
    else:
        mask = torch.from_numpy(full).to(gpu)
    plse = (torch.randn(B, H, M) * 2 + 8).to(gpu)
    cur, w, lse_t = tree_attention_forward(q, k, v, mask, 0, plse, B, M, H, D, return_lse=True)
    torch.cuda.synchronize()
    assert cur.shape == (B, M, H, D) and w.shape == (B, M, H, 1) and w.dtype == q.dtype
    for b in range(B):
        o_ref, w_ref, l_ref = oa.tree_attention(np64(q[b]), np64(k[b]), np64(v[b]), keep[b], np64(plse[b]))
        assert_attn_close(np64(cur[b]), o_ref, what=f"b={b}")
        assert_lse_close(np64(lse_t[b]), l_ref, what=f"b={b}")
        np.testing.assert_allclose(np64(w[b])[..., 0], w_ref, atol=8e-3)


def paged_case(gpu, n_prefix, M, H=32, Hk=8, D=128, seed=0, tree_seed=0, max_depth=8, max_outdeg=4):
    return wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, seed=seed, tree_seed=tree_seed,
                                      max_depth=max_depth, max_outdeg=max_outdeg, device=str(gpu))


def oracle_tree_verify(inp, heads=None):
    q = np64(inp.q[0])
    k = np64(inp.logical_kv(0, 0)[0])
    v = np64(inp.logical_kv(0, 1)[0])
    if heads is not None:
        H, Hk = q.shape[1], k.shape[1]
        G = H // Hk
        kv = sorted({h // G for h in heads})
        assert [h for h in heads] == [x for kh in kv for x in range(kh * G, kh * G + G)]
        q, k, v = q[:, heads], k[:, kv], v[:, kv]
    return oa.tree_verify(q, k, v, inp.n_prefix, inp.parent)


@pytest.mark.parametrize("n_prefix,M", [(4096, 64), (0, 64), (100, 7), (1000, 128), (16, 256), (6000, 256), (30000, 192)])
def test_tree_verify_paged_matches_oracle(gpu, n_prefix, M):
    print(f"[tree_verify paged] n_prefix={n_prefix} M={M}", flush=True)
    inp = paged_case(gpu, n_prefix, M, tree_seed=n_prefix + M)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    out, lse = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle_tree_verify(inp)
    assert_attn_close(np64(out[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(lse[0]), l_ref)


@pytest.mark.parametrize("ps,D,n_prefix,M", [(1, 128, 1000, 64), (2, 128, 1000, 64), (4, 64, 1000, 64),
                                             (8, 128, 1000, 64), (32, 128, 1000, 64), (64, 128, 1000, 64),
                                             (256, 128, 5000, 48)])
def test_tree_verify_page_sizes(gpu, ps, D, n_prefix, M):
    # Pages smaller than one DMA instruction (per-lane addresses), and pages
    # larger than a tile: bit-equal to the dense cache holding the same
    # logical tokens, and within tolerance of the oracle.
    print(f"[tree_verify page size] ps={ps} D={D} n_prefix={n_prefix} M={M}", flush=True)
    inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=8, Hk=2, D=D, page_size=ps, seed=ps, tree_seed=ps,
                                     device=str(gpu))
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    o_p, l_p = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table)
    kc, vc = inp.logical_kv(0, 0).contiguous(), inp.logical_kv(0, 1).contiguous()
    o_d, l_d = tree_verify(inp.q, kc, vc, n_prefix, par)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    o_ref, l_ref = oracle_tree_verify(inp)
    assert_attn_close(np64(o_p[0]), o_ref)
    assert_lse_close(np64(l_p[0]), l_ref)


@pytest.mark.parametrize("ps", [16, 4])
def test_tree_verify_batched_paged_f16(gpu, ps):
    # B = 2 with one int64 page-table row per batch over one shared pool, a
    # different tree per batch, f16 end to end.
    print(f"[tree_verify batched paged f16] ps={ps}", flush=True)
    B, M, H, Hk, D, n_prefix = 2, 40, 8, 2, 128, 700
    n_tok = n_prefix + M
    n_pages = (n_tok + ps - 1) // ps
    q = rand((B, M, H, D), 31, torch.float16, gpu)
    pool = rand((1, 2, B * n_pages, Hk, ps, D), 32, torch.float16, gpu)
    perm = np.random.default_rng(ps).permutation(B * n_pages).astype(np.int64).reshape(B, n_pages)
    pt = torch.from_numpy(perm).to(gpu)
    parents = [wl.make_tree(M, max_depth=6, max_outdeg=4, seed=40 + b)[0] for b in range(B)]
    par = torch.tensor(parents, dtype=torch.int64, device=gpu)
    o_p, l_p = tree_verify(q, pool[0, 0], pool[0, 1], n_prefix, par, page_table=pt)
    tok = torch.arange(n_tok, device=gpu)
    kc = torch.stack([pool[0, 0][pt[b][tok // ps], :, tok % ps] for b in range(B)]).contiguous()
    vc = torch.stack([pool[0, 1][pt[b][tok // ps], :, tok % ps] for b in range(B)]).contiguous()
    o_d, l_d = tree_verify(q, kc, vc, n_prefix, par)
    torch.cuda.synchronize()
    assert o_p.dtype == torch.float16
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    for b in range(B):
        o_ref, l_ref = oa.tree_verify(np64(q[b]), np64(kc[b]), np64(vc[b]), n_prefix, parents[b])
        assert_attn_close(np64(o_p[b]), o_ref, what=f"b={b}")
        assert_lse_close(np64(l_p[b]), l_ref, what=f"b={b}")


def test_tree_verify_random_configurations(gpu):
    """24 random (prefix length, tree size and shape, GQA grouping, head_dim,
    page size, dtype, bundle packing) configurations: paged and dense cache
    bit-equal, both within tolerance of the fp64 oracle."""
    rng = np.random.default_rng(77)
    for case in range(24):
        n_prefix = int(rng.choice([0, 1, 33, 1000, 9000]))
        M = int(rng.choice([1, 7, 33, 64, 100, 200, 256]))
        H, Hk = [(8, 8), (32, 8), (16, 4), (8, 2), (4, 1)][case % 5]
        D = int(rng.choice([64, 128]))
        ps = int(rng.choice([1, 16, 64]))
        dtype = torch.float16 if case % 3 == 0 else torch.bfloat16
        depth, outdeg = int(rng.integers(1, 13)), int(rng.integers(1, 7))
        # A tree of depth <= d and out-degree <= o holds at most 1 + o + ... + o^d nodes.
        while sum(outdeg ** k for k in range(depth + 1)) < M:
            depth, outdeg = depth + 1, min(outdeg + 1, 6)
        print(f"[tree_verify random {case}] N={n_prefix} M={M} H={H}/{Hk} D={D} ps={ps} {dtype} "
              f"depth={depth} outdeg={outdeg}", flush=True)
        inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, page_size=ps, dtype=dtype,
                                         seed=100 + case, tree_seed=200 + case, max_depth=depth, max_outdeg=outdeg,
                                         device=str(gpu))
        par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
        perm = None
        if case % 2 == 1:
            perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=int(rng.integers(1, 9))), dtype=torch.int32,
                                device=gpu)
        o_p, l_p = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par,
                               page_table=inp.page_table, row_perm=perm)
        kc, vc = inp.logical_kv(0, 0).contiguous(), inp.logical_kv(0, 1).contiguous()
        o_d, l_d = tree_verify(inp.q, kc, vc, n_prefix, par, row_perm=perm)
        torch.cuda.synchronize()
        assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d), f"case {case}: paged differs from dense"
        o_ref, l_ref = oracle_tree_verify(inp)
        assert_attn_close(np64(o_p[0]), o_ref, what=f"case {case}")
        assert_lse_close(np64(l_p[0]), l_ref, what=f"case {case}")


def test_tree_verify_wide_random_sweep(gpu):
    """60 random configurations over a wider range than the test above: prefix
    lengths at tile and page boundaries (0 .. 17000), trees of 1 to 600 nodes
    (the >256-node instantiation included), seven GQA groupings, head_dim 64
    and 128, pages of 1 to 64 tokens, bf16 / f16 / f32, with and without
    bundle packing.  Paged and dense results against the fp64 oracle; bit-equal
    to each other whenever both plan the same splits (with pages of a few
    tokens a long split is capped at the page-table slice staged in LDS, so
    the paged plan can hold more, shorter splits and round differently)."""
    from diffspec_mi355x import _ext
    lib = _ext.load()
    rng = np.random.default_rng(2026)
    for case in range(60):
        n_prefix = int(rng.choice([0, 1, 2, 31, 32, 33, 63, 64, 65, 500, 1000, 4095, 4097, 9000, 17000]))
        M = int(rng.choice([1, 2, 3, 17, 32, 33, 64, 65, 128, 200, 255, 256, 257, 300, 511, 600]))
        H, Hk = [(8, 8), (32, 8), (16, 4), (8, 2), (4, 1), (12, 4), (2, 2)][int(rng.integers(7))]
        D = int(rng.choice([64, 128]))
        ps = int(rng.choice([1, 2, 4, 16, 32, 64]))
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        depth, outdeg = int(rng.integers(1, 13)), int(rng.integers(1, 7))
        while sum(outdeg ** k for k in range(depth + 1)) < M:
            depth, outdeg = depth + 1, min(outdeg + 1, 6)
        perm_on, nb = bool(rng.integers(2)), int(rng.integers(1, 9))
        what = f"case {case}: N={n_prefix} M={M} H={H}/{Hk} D={D} ps={ps} {dtype} depth={depth} perm={perm_on}"
        print(f"[tree_verify wide] {what}", flush=True)
        inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, page_size=ps, dtype=dtype,
                                         seed=1000 + case, tree_seed=2000 + case, max_depth=depth,
                                         max_outdeg=outdeg, device=str(gpu))
        par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
        perm = None
        if perm_on:
            perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=nb), dtype=torch.int32, device=gpu)
        o_p, l_p = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par,
                               page_table=inp.page_table, row_perm=perm)
        o_d, l_d = tree_verify(inp.q, inp.logical_kv(0, 0).contiguous(), inp.logical_kv(0, 1).contiguous(), n_prefix,
                               par, row_perm=perm)
        torch.cuda.synchronize()
        if (lib.dsv_attn_workspace_bytes(1, M, H, Hk, D, n_prefix, ps, 1)
                == lib.dsv_attn_workspace_bytes(1, M, H, Hk, D, n_prefix, 0, 1)):
            assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d), f"{what}: paged differs from dense"
        o_ref, l_ref = oracle_tree_verify(inp)
        rel = 4e-3 if dtype == torch.float32 else 1e-2
        for o_, l_, kind in ((o_p, l_p, "paged"), (o_d, l_d, "dense")):
            assert_attn_close(np64(o_[0]), o_ref, rel=rel, what=f"{what} {kind}")
            assert_lse_close(np64(l_[0]), l_ref, what=f"{what} {kind}")


def test_flash_attn_random_causal_and_lengths(gpu):
    """30 random flash_attn_with_kvcache calls: batch 1-3 with a random length
    per batch (0 .. N), causal or not, bf16 / f16 / f32, against the fp64
    oracle; rows that see no key are zero with LSE -inf."""
    from diffspec_mi355x.runtime.attention_compat import flash_attn_with_kvcache
    rng = np.random.default_rng(77)
    for case in range(30):
        B = int(rng.integers(1, 4))
        N = int(rng.choice([1, 33, 200, 1000, 5000]))
        M = int(rng.choice([1, 5, 16, 48, 64, 100]))
        H, Hk = [(8, 8), (32, 8), (16, 4), (4, 1)][int(rng.integers(4))]
        D = int(rng.choice([64, 128]))
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        causal = bool(rng.integers(2))
        lens = rng.integers(0, N + 1, size=B)
        what = f"case {case}: B={B} N={N} M={M} H={H}/{Hk} D={D} {dtype} causal={causal} lens={lens.tolist()}"
        print(f"[flash_attn random] {what}", flush=True)
        q = rand((B, M, H, D), 10 + case, dtype, gpu)
        k = rand((B, N, Hk, D), 20 + case, dtype, gpu)
        v = rand((B, N, Hk, D), 30 + case, dtype, gpu)
        sl = torch.tensor(lens, dtype=torch.int32, device=gpu)
        out, lse = flash_attn_with_kvcache(q, k, v, cache_seqlens=sl, causal=causal, return_softmax_lse=True)
        torch.cuda.synchronize()
        for b in range(B):
            n = int(lens[b])
            keep = np.ones((M, n), dtype=bool)
            if causal:
                for m in range(M):
                    keep[m, max(0, n - M + m + 1):] = False
            o_ref, l_ref = oa.masked_attention(np64(q[b]), np64(k[b, :n]), np64(v[b, :n]), keep)
            got_o, got_l = np64(out[b]), np64(lse[b])
            vis = keep.any(axis=1)
            if vis.any():
                assert_attn_close(got_o[vis], o_ref[vis], rel=4e-3 if dtype == torch.float32 else 1e-2,
                                  what=f"{what} b={b}")
            assert (got_o[~vis] == 0).all(), f"{what} b={b}: rows without keys are not zero"
            assert_lse_close(got_l.T, l_ref, what=f"{what} b={b}")


def test_tree_verify_dense_equals_paged_and_perm_invariant(gpu):
    inp = paged_case(gpu, 3000, 64, tree_seed=5)
    par = torch.tensor(inp.parent, dtype=torch.int32, device=gpu)
    o_p, l_p = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 3000, par, page_table=inp.page_table)
    kc, vc = inp.logical_kv(0, 0).contiguous(), inp.logical_kv(0, 1).contiguous()
    o_d, l_d = tree_verify(inp.q, kc, vc, 3000, par)
    perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=8), dtype=torch.int32, device=gpu)
    o_b, l_b = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 3000, par, page_table=inp.page_table,
                           row_perm=perm)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    assert torch.equal(o_p, o_b) and torch.equal(l_p, l_b)


@pytest.mark.parametrize("n_prefix,M,shape,dtype,ps", [
    (2000, 300, "random", torch.bfloat16, 16), (500, 512, "random", torch.bfloat16, 16),
    (100, 1024, "random", torch.bfloat16, 16), (300, 1024, "chain", torch.bfloat16, 16),
    (1000, 700, "star", torch.float16, 4), (1000, 400, "random", torch.float32, 16),
    (64, 257, "random", torch.bfloat16, 16)])
def test_tree_verify_trees_beyond_256_nodes(gpu, n_prefix, M, shape, dtype, ps):
    """Trees of 257 to 1024 nodes.  A workgroup of the tree split owns 256
    packed query rows, whose nodes' ancestor masks it holds in one LDS table
    per block: against the fp64 oracle (chain, star and generated trees;
    bf16, f16 and f32), and the bundle row order bit-equal to the identity
    order."""
    print(f"[tree_verify large tree] n_prefix={n_prefix} M={M} shape={shape} dtype={dtype} ps={ps}", flush=True)
    inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=8, Hk=2, D=128, page_size=ps, dtype=dtype,
                                     scale=1.0, seed=M, tree_seed=M + 1, max_depth=12, max_outdeg=6,
                                     device=str(gpu))
    if shape == "chain":
        inp.parent = [-1] + list(range(M - 1))
    elif shape == "star":
        inp.parent = [-1] + [0] * (M - 1)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    out, lse = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table,
                           out_dtype=torch.float32)
    perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=8), dtype=torch.int32, device=gpu)
    o_b, l_b = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table,
                           row_perm=perm, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out, o_b) and torch.equal(lse, l_b)
    o_ref, l_ref = oracle_tree_verify(inp)
    assert_attn_close(np64(out[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(lse[0]), l_ref)


def test_tree_attention_forward_300_nodes(gpu):
    """The tree block alone with a dense [B, 1, T, T] mask over 300 nodes (the
    mask read per node slot of each 256-row block)."""
    B, M, H, Hk, D, T = 1, 300, 8, 2, 128, 310
    q = rand((B, M, H, D), 17, torch.bfloat16, gpu)
    k = rand((B, M, Hk, D), 18, torch.bfloat16, gpu)
    v = rand((B, M, Hk, D), 19, torch.bfloat16, gpu)
    keep = oa.ancestor_mask(wl.make_tree(M, seed=6, max_depth=12, max_outdeg=6)[0])
    full = np.zeros((B, 1, T, T), dtype=bool)
    full[:, 0, -M:, -M:] = keep
    mask = torch.from_numpy(full).to(torch.int8).to(gpu)
    plse = (torch.randn(B, H, M) * 2 + 8).to(gpu)
    cur, w, lse_t = tree_attention_forward(q, k, v, mask, 0, plse, B, M, H, D, return_lse=True)
    torch.cuda.synchronize()
    o_ref, w_ref, l_ref = oa.tree_attention(np64(q[0]), np64(k[0]), np64(v[0]), keep, np64(plse[0]))
    assert_attn_close(np64(cur[0]), o_ref)
    assert_lse_close(np64(lse_t[0]), l_ref)
    np.testing.assert_allclose(np64(w[0])[..., 0], w_ref, atol=8e-3)


@pytest.mark.parametrize("shape", ["chain", "star"])
def test_tree_verify_special_trees(gpu, shape):
    M, n_prefix = 32, 200
    inp = paged_case(gpu, n_prefix, M, tree_seed=1)
    inp.parent = [-1] + (list(range(M - 1)) if shape == "chain" else [0] * (M - 1))
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    out, lse = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle_tree_verify(inp)
    assert_attn_close(np64(out[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(lse[0]), l_ref)


def test_verify_bundle_reference_shapes_and_stats(gpu):
    # reference tests/test_fused_kernel.py:19-27 shapes, now with numeric parity
    ver = FusedBundleVerifier(bundle_size=3, enable_triton=True, device="cuda")
    B, M, H, D, N = 1, 10, 8, 64, 20
    q, k, v = rand((B, M, H, D), 11, torch.bfloat16, gpu), rand((B, N, H, D), 12, torch.bfloat16, gpu), \
        rand((B, N, H, D), 13, torch.bfloat16, gpu)
    mask = torch.tril(torch.ones(M, N, dtype=torch.int8, device=gpu))
    o, lse = ver.verify_bundle(q, k, v, [mask, mask], shared_prefix_len=5)
    torch.cuda.synchronize()
    assert o.shape == q.shape and lse.shape == (B, M, H)
    o_ref, l_ref = oa.masked_attention(np64(q[0]), np64(k[0]), np64(v[0]), mask.cpu().numpy() != 0)
    assert_attn_close(np64(o[0]), o_ref)
    assert_lse_close(np64(lse[0]), l_ref)
    st = ver.get_statistics()
    assert st["total_verifications"] == 2 and st["total_bundles"] == 1 and st["prefix_reuse_rate"] == 1


def test_verify_bundle_fully_masked_row_and_paged_equivalence(gpu):
    B, M, H, Hk, D, N, ps = 1, 12, 8, 2, 128, 300, 16
    q = rand((B, M, H, D), 14, torch.bfloat16, gpu)
    n_pages = (N + ps - 1) // ps
    pool = rand((2, 2, n_pages + 3, Hk, ps, D), 15, torch.bfloat16, gpu)
    pt = torch.from_numpy(np.random.default_rng(3).permutation(n_pages + 3)[:n_pages].astype(np.int64)).to(gpu)
    mask = (torch.rand(M, N, generator=torch.Generator().manual_seed(4)) < 0.5).to(torch.int8)
    mask[3] = 0  # fully masked row
    mask = mask.to(gpu)
    pv = PagedBundleVerifier(device="cuda")
    o_p, l_p = pv.verify_bundle_paged(q, pool, pt, [mask], layer_idx=1)
    tok = torch.arange(N, device=gpu)
    k = pool[1, 0][pt[tok // ps], :, tok % ps].unsqueeze(0).contiguous()
    v = pool[1, 1][pt[tok // ps], :, tok % ps].unsqueeze(0).contiguous()
    o_d, l_d = pv.verify_bundle(q, k, v, [mask])
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    assert torch.all(o_p[0, 3] == 0) and torch.all(torch.isneginf(l_p[0, 3]))
    o_ref, l_ref = oa.masked_attention(np64(q[0]), np64(k[0]), np64(v[0]), mask.cpu().numpy() != 0)
    assert_attn_close(np64(o_p[0]), o_ref)
    assert_lse_close(np64(l_p[0]), l_ref)


def test_fp32_inputs_4k_ctx_within_tolerance(gpu):
    """The 4096-token fp32 configuration (N=4096, M=64, GQA 32/8, D=128,
    N(0,1) fp32 drawn Q, K/V prefix, K/V tree, seed 0): fp32 tensors go
    straight to the fp32 kernel, compared with the float64 oracle at the
    default bars (fp32 output: relative 4e-3; LSE 2e-3)."""
    g = torch.Generator().manual_seed(0)
    M, H, Hk, D, N = 64, 32, 8, 128, 4096
    q = torch.randn(1, M, H, D, generator=g)
    kp, vp = torch.randn(1, N, Hk, D, generator=g), torch.randn(1, N, Hk, D, generator=g)
    kt, vt = torch.randn(1, M, Hk, D, generator=g), torch.randn(1, M, Hk, D, generator=g)
    parent, _ = wl.make_tree(M, seed=0)
    kc = torch.cat([kp, kt], 1).to(gpu)
    vc = torch.cat([vp, vt], 1).to(gpu)
    out, lse = tree_verify(q.to(gpu), kc, vc, N, torch.tensor(parent, device=gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = oa.tree_verify(q[0].double().numpy(), torch.cat([kp, kt], 1)[0].double().numpy(),
                                  torch.cat([vp, vt], 1)[0].double().numpy(), N, parent)
    assert_attn_close(np64(out[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(lse[0]), l_ref)


@pytest.mark.parametrize("n_prefix,M,ps,H,Hk,D,perm", [
    (4096, 64, 16, 32, 8, 128, False), (0, 64, 16, 32, 8, 128, False), (100, 7, 16, 32, 8, 128, True),
    (1000, 64, 1, 8, 2, 128, False), (1000, 64, 4, 8, 2, 64, False), (1000, 64, 64, 8, 2, 128, True),
    (6000, 256, 16, 32, 8, 128, False), (30000, 192, 16, 32, 8, 128, False)])
def test_tree_verify_f32_paged_equals_dense_and_matches_oracle(gpu, n_prefix, M, ps, H, Hk, D, perm):
    """fp32 page pools (page sizes 1 to 64) and the dense cache of the same
    tokens: bit-equal results, within the default bars of the oracle; with
    and without a row permutation."""
    print(f"[tree_verify f32] n_prefix={n_prefix} M={M} ps={ps} D={D} perm={perm}", flush=True)
    inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, page_size=ps, dtype=torch.float32,
                                     scale=1.0, seed=ps, tree_seed=M, device=str(gpu))
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    rp = torch.tensor(bundle_row_order(inp.parent, num_bundles=4), dtype=torch.int32, device=gpu) if perm else None
    o_p, l_p = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], n_prefix, par, page_table=inp.page_table,
                           row_perm=rp)
    kc, vc = inp.logical_kv(0, 0).contiguous(), inp.logical_kv(0, 1).contiguous()
    o_d, l_d = tree_verify(inp.q, kc, vc, n_prefix, par, row_perm=rp)
    torch.cuda.synchronize()
    assert o_p.dtype == torch.float32 and torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    o_ref, l_ref = oracle_tree_verify(inp)
    assert_attn_close(np64(o_p[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(l_p[0]), l_ref)


def test_verify_bundle_f32_dense_and_paged(gpu):
    """The bundle verifiers with fp32 q and K/V: a byte mask with a fully
    masked row, paged equal to dense, within the default bars."""
    B, M, H, Hk, D, N, ps = 1, 12, 8, 2, 128, 300, 16
    q = rand((B, M, H, D), 24, torch.float32, gpu)
    n_pages = (N + ps - 1) // ps
    pool = rand((2, 2, n_pages + 3, Hk, ps, D), 25, torch.float32, gpu)
    pt = torch.from_numpy(np.random.default_rng(5).permutation(n_pages + 3)[:n_pages].astype(np.int64)).to(gpu)
    mask = (torch.rand(M, N, generator=torch.Generator().manual_seed(6)) < 0.5).to(torch.int8)
    mask[5] = 0
    mask = mask.to(gpu)
    pv = PagedBundleVerifier(device="cuda")
    o_p, l_p = pv.verify_bundle_paged(q, pool, pt, [mask], layer_idx=0)
    tok = torch.arange(N, device=gpu)
    k = pool[0, 0][pt[tok // ps], :, tok % ps].unsqueeze(0).contiguous()
    v = pool[0, 1][pt[tok // ps], :, tok % ps].unsqueeze(0).contiguous()
    o_d, l_d = pv.verify_bundle(q, k, v, [mask])
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    assert torch.all(o_p[0, 5] == 0) and torch.all(torch.isneginf(l_p[0, 5]))
    o_ref, l_ref = oa.masked_attention(np64(q[0]), np64(k[0]), np64(v[0]), mask.cpu().numpy() != 0)
    assert_attn_close(np64(o_p[0]), o_ref, rel=4e-3)
    assert_lse_close(np64(l_p[0]), l_ref)


def test_64k_ctx_64_nodes_all_heads(gpu):
    """64K paged prefix, 64-node tree, bf16 N(0,1)*0.5: all 32 query heads
    (every KV head's workgroups) against the fp64 oracle."""
    print("[64k all heads] tree_verify", flush=True)
    inp = paged_case(gpu, 65536, 64)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    out, lse = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 65536, par, page_table=inp.page_table,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle_tree_verify(inp)
    for kvh in range(8):
        hs = slice(4 * kvh, 4 * kvh + 4)
        assert_attn_close(np64(out[0, :, hs]), o_ref[:, hs], rel=4e-3, what=f"kv head {kvh}")
        assert_lse_close(np64(lse[0, :, hs]), l_ref[:, hs], what=f"kv head {kvh}")
    # the tree block alone (where the mask matters) on the same data
    out_t, lse_t = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 0, par,
                               page_table=inp.page_table[4096:], out_dtype=torch.float32)
    torch.cuda.synchronize()
    kt = np64(inp.logical_kv(0, 0)[0, 65536:])
    vt = np64(inp.logical_kv(0, 1)[0, 65536:])
    o_t, l_t = oa.masked_attention(np64(inp.q[0]), kt, vt, oa.ancestor_mask(inp.parent))
    assert_attn_close(np64(out_t[0]), o_t, rel=4e-3)
    assert_lse_close(np64(lse_t[0]), l_t)


def test_128k_ctx_128_nodes_bundle_packed_all_heads(gpu):
    """128K paged prefix, 128-node tree (depth <= 12, out-degree <= 6), query
    rows packed in bundle order (8 bundles): all 32 query heads (both 256-row
    blocks of every KV head) against the fp64 oracle."""
    print("[128k all heads] tree_verify", flush=True)
    inp = paged_case(gpu, 131072, 128, seed=2, tree_seed=2, max_depth=12, max_outdeg=6)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=8), dtype=torch.int32, device=gpu)
    out, lse = tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 131072, par, page_table=inp.page_table,
                           row_perm=perm, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle_tree_verify(inp)
    for kvh in range(8):
        hs = slice(4 * kvh, 4 * kvh + 4)
        assert_attn_close(np64(out[0, :, hs]), o_ref[:, hs], rel=4e-3, what=f"kv head {kvh}")
        assert_lse_close(np64(lse[0, :, hs]), l_ref[:, hs], what=f"kv head {kvh}")


def test_verify_bundle_attention_profile_shape(gpu):
    """The reference attention microbenchmark's shape (benchmarks/attention_kernel_profile.py:155-161:
    q_len 48, prefix 32000, 32 heads, head_dim 128, fp16; K/V in the repeat_kv'd
    form with 32 heads), bundle mask = prefix plus a causal block over the last
    48 keys, against the fp64 oracle."""
    B, M, H, D, N = 1, 48, 32, 128, 32000
    print("[verify_bundle 48 x 32000]", flush=True)
    q = rand((B, M, H, D), 21, torch.float16, gpu)
    k = rand((B, N, H, D), 22, torch.float16, gpu)
    v = rand((B, N, H, D), 23, torch.float16, gpu)
    mask = torch.ones(M, N, dtype=torch.int8)
    mask[:, N - M:] = torch.tril(torch.ones(M, M, dtype=torch.int8))
    mask = mask.to(gpu)
    ver = FusedBundleVerifier(bundle_size=3, enable_triton=True, device="cuda")
    o, lse = ver.verify_bundle(q, k, v, [mask], shared_prefix_len=N - M)
    torch.cuda.synchronize()
    assert o.dtype == torch.float16 and lse.shape == (B, M, H)
    o_ref, l_ref = oa.masked_attention(np64(q[0]), np64(k[0]), np64(v[0]), mask.cpu().numpy() != 0)
    assert_attn_close(np64(o[0]), o_ref)
    assert_lse_close(np64(lse[0]), l_ref)


def test_tree_verify_rejects_a_row_perm_that_is_not_a_permutation(gpu):
    inp = paged_case(gpu, 100, 16)
    par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    bad = torch.arange(16, dtype=torch.int32, device=gpu)
    bad[3] = 5
    with pytest.raises(ValueError, match="not a permutation"):
        tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 100, par, page_table=inp.page_table, row_perm=bad)
    with pytest.raises(ValueError, match="permutation"):
        tree_verify(inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], 100, par, page_table=inp.page_table,
                    row_perm=bad[:15])

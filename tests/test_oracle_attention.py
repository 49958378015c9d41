"""Pins of the float64 attention oracle (CPU): closed forms, special cases,
brute force, split invariance, and agreement with the reference's own torch
CPU op sequence (oracle/ref_cpu_path.py)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import ref_cpu_path as rc
from diffspec_mi355x import workloads as wl


def rnd(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def brute_row(q, k, v, mask, D):
    """Per-row, per-head loop with explicit exponentials (no vectorisation)."""
    M, H, _ = q.shape
    N, Hk, _ = k.shape
    G = H // Hk
    out = np.zeros((M, H, D))
    lse = np.zeros((M, H))
    for i in range(M):
        for h in range(H):
            s = [float(np.dot(q[i, h], k[j, h // G])) / math.sqrt(D) if mask[i, j] else None for j in range(N)]
            vis = [x for x in s if x is not None]
            mx = max(vis)
            tot = sum(math.exp(x - mx) for x in vis)
            acc = np.zeros(D)
            for j in range(N):
                if s[j] is not None:
                    acc += math.exp(s[j] - mx) / tot * v[j, h // G]
            out[i, h] = acc
            lse[i, h] = mx + math.log(tot)
    return out, lse


def test_masked_attention_matches_brute_force_gqa():
    M, H, Hk, D, N = 5, 4, 2, 8, 7
    q, k, v = rnd((M, H, D), 1), rnd((N, Hk, D), 2), rnd((N, Hk, D), 3)
    mask = np.random.default_rng(4).random((M, N)) < 0.6
    mask[:, 0] = True
    o, l = oa.masked_attention(q, k, v, mask)
    ob, lb = brute_row(q, k, v, mask, D)
    np.testing.assert_allclose(o, ob, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l, lb, rtol=1e-12, atol=1e-12)


def test_constant_values_give_that_value():
    M, H, D, N = 3, 2, 16, 11
    q, k = rnd((M, H, D), 5), rnd((N, H, D), 6)
    v = np.broadcast_to(rnd((1, H, D), 7), (N, H, D))
    o, _ = oa.masked_attention(q, k, v)
    np.testing.assert_allclose(o, np.broadcast_to(v[:1], (M, H, D)), atol=1e-12)


def test_zero_query_is_mean_of_visible_values_and_lse_log_count():
    M, H, D, N = 4, 2, 8, 9
    q = np.zeros((M, H, D))
    k, v = rnd((N, H, D), 8), rnd((N, H, D), 9)
    mask = np.tril(np.ones((M, N), dtype=bool), k=2)
    o, l = oa.masked_attention(q, k, v, mask)
    for i in range(M):
        vis = mask[i]
        np.testing.assert_allclose(o[i], v[vis].mean(axis=0), atol=1e-12)
        np.testing.assert_allclose(l[i], math.log(vis.sum()), atol=1e-12)


def test_planted_key_dominates():
    M, H, D, N = 2, 2, 32, 50
    q = rnd((M, H, D), 10)
    k = rnd((N, H, D), 11) * 0.01
    v = rnd((N, H, D), 12)
    # key 17 aligned with q so that its logit is ~+30 above the rest
    k[17] = q[0] / np.linalg.norm(q[0], axis=-1, keepdims=True) * 30 * math.sqrt(D) / np.linalg.norm(
        q[0], axis=-1, keepdims=True)
    o, _ = oa.masked_attention(q[:1], k, v)
    np.testing.assert_allclose(o[0], v[17], atol=1e-9)


def test_chain_tree_is_causal_attention():
    M, H, D = 6, 2, 8
    parent = [-1] + list(range(M - 1))
    keep = oa.ancestor_mask(parent)
    assert np.array_equal(keep, np.tril(np.ones((M, M), dtype=bool)))


def test_star_tree_sees_root_and_self():
    M = 7
    keep = oa.ancestor_mask([-1] + [0] * (M - 1))
    exp = np.eye(M, dtype=bool)
    exp[:, 0] = True
    assert np.array_equal(keep, exp)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ancestor_mask_recurrence(seed):
    parent, _ = wl.make_tree(64, seed=seed)
    keep = oa.ancestor_mask(parent)
    # bitmask recurrence anc[i] = anc[parent[i]] | bit(i), valid because parent < child
    anc = [0] * 64
    for i in range(64):
        anc[i] = (anc[parent[i]] if parent[i] >= 0 else 0) | (1 << i)
    for i in range(64):
        assert [bool((anc[i] >> j) & 1) for j in range(64)] == keep[i].tolist()


def test_split_invariance_of_lse_merge():
    M, H, Hk, D, N = 4, 4, 1, 8, 40
    q, k, v = rnd((M, H, D), 20), rnd((N, Hk, D), 21), rnd((N, Hk, D), 22)
    o_full, l_full = oa.masked_attention(q, k, v)
    o_a, l_a = oa.masked_attention(q, k[:13], v[:13])
    o_b, l_b = oa.masked_attention(q, k[13:], v[13:])
    o, l = oa.merge_lse(o_a, l_a, o_b, l_b)
    np.testing.assert_allclose(o, o_full, atol=1e-12)
    np.testing.assert_allclose(l, l_full, atol=1e-12)


def test_sigmoid_merge_equals_lse_merge():
    M, H, D, N, T = 5, 2, 8, 30, 5
    q, k, v = rnd((M, H, D), 30), rnd((N + T, H, D), 31), rnd((N + T, H, D), 32)
    parent = [-1, 0, 1, 1, 0]
    o_p, lse_p_hm = oa.prefix_attention(q, k[:N], v[:N])
    keep = oa.ancestor_mask(parent)
    o_t, w, _ = oa.tree_attention(q, k[N:], v[N:], keep, lse_p_hm)
    merged = oa.hybrid_merge(o_t, w, o_p)
    full, _ = oa.tree_verify(q, k, v, N, parent)
    np.testing.assert_allclose(merged, full, atol=1e-12)


def test_fully_masked_row_is_zero_with_neg_inf_lse():
    q, k, v = rnd((2, 1, 4), 40), rnd((3, 1, 4), 41), rnd((3, 1, 4), 42)
    mask = np.array([[True, False, False], [False, False, False]])
    o, l = oa.masked_attention(q, k, v, mask)
    assert np.all(o[1] == 0) and np.isneginf(l[1, 0])


def test_tree_block_keep_conventions():
    M = 3
    add = np.zeros((1, 1, 5, 5), dtype=np.float32)
    add[..., -M:, -M:] = np.array([[0, -3e38, -3e38], [0, 0, -3e38], [0, -3e38, 0]])
    keep = oa.tree_block_keep(add, M)
    assert keep.tolist() == [[True, False, False], [True, True, False], [True, False, True]]
    i8 = np.array([[1, 0], [1, 1]], dtype=np.int8)
    assert oa.tree_block_keep(i8, 2).tolist() == [[True, False], [True, True]]


def test_paged_gather_matches_contiguous():
    P, Hk, ps, D, n = 6, 2, 4, 3, 21
    pool = rnd((P, Hk, ps, D), 50)
    pt = [3, 0, 5, 1, 4, 2]
    g = oa.paged_gather(pool, pt, n)
    for t in range(n):
        np.testing.assert_array_equal(g[t], pool[pt[t // ps], :, t % ps])


def test_bf16_round_matches_torch():
    x = rnd((1000,), 60, 3.0).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oa.bf16_round(x), want)


def test_oracle_matches_reference_cpu_op_sequence():
    """The closed form agrees with the reference's own CPU path (prefix
    fallback + naive tree + sigmoid merge) on a small fp32 case."""
    torch.manual_seed(0)
    B, M, H, Hk, D, N = 1, 16, 8, 2, 32, 200
    q = torch.randn(B, M, H, D)
    kc = torch.randn(B, Hk, N + M, D)
    vc = torch.randn(B, Hk, N + M, D)
    parent, _ = wl.make_tree(M, seed=3)
    keep = torch.from_numpy(oa.ancestor_mask(parent))
    out = rc.hybrid_verify_cpu(q, kc, vc, N, rc.additive_tree_mask(keep))
    want, _ = oa.tree_verify(q[0].numpy(), kc[0].transpose(0, 1).numpy(), vc[0].transpose(0, 1).numpy(), N, parent)
    np.testing.assert_allclose(out[0].numpy(), want, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_16bit_matches_torch_elementwise_ops(dtype):
    # The reference's op sequence on 16-bit tensors (torch CPU rounds each
    # elementwise op to the dtype, as on the GPU).
    g = torch.Generator().manual_seed(7)
    M, H, D = 9, 3, 64
    x = (torch.randn((H, M, D), generator=g) * 3).to(dtype)
    pos = torch.arange(100, 100 + M, dtype=torch.float32)
    inv = 1.0 / (5e5 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)

    def rotate_half(t):
        return torch.cat((-t[..., D // 2:], t[..., :D // 2]), dim=-1)

    want = (x * cos) + (rotate_half(x) * sin)
    got = oa.rope_16bit(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), f16=dtype == torch.float16)
    assert np.array_equal(got, want.float().numpy())
    # cos = 1, sin = 0 is the identity; cos = 0, sin = 1 is rotate_half exactly.
    one, zero = np.ones((M, D), np.float32), np.zeros((M, D), np.float32)
    xf = x.float().numpy()
    f16 = dtype == torch.float16
    assert np.array_equal(oa.rope_16bit(xf, one, zero, f16=f16), xf)
    assert np.array_equal(oa.rope_16bit(xf, zero, one, f16=f16), rotate_half(x).float().numpy())

"""GPU parity of the tree K/V append with RoPE (dsv_kv_append) against the
oracle and against torch's own op sequence (bit-exact)."""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.runtime.cache_state import append_tree_kv

pytestmark = pytest.mark.gpu


def _tables(M, D, dtype, base, gpu, theta=5e5):
    pos = torch.arange(base, base + M, dtype=torch.float32)
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], -1)
    return emb.cos().to(dtype).to(gpu), emb.sin().to(dtype).to(gpu)


def _rotate_half(t, D):
    return torch.cat((-t[..., D // 2:], t[..., :D // 2]), dim=-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_append_with_rope_matches_torch_ops(gpu, dtype):
    M, Hk, H, D, S, start = 37, 4, 16, 128, 120, 70
    g = torch.Generator().manual_seed(3)
    k = (torch.randn((M, Hk, D), generator=g) * 2).to(dtype).to(gpu)
    v = torch.randn((M, Hk, D), generator=g).to(dtype).to(gpu)
    q = (torch.randn((1, M, H, D), generator=g) * 2).to(dtype).to(gpu)
    cos, sin = _tables(M, D, dtype, 5000, gpu)
    k_cache = torch.randn((1, Hk, S, D), generator=g).to(dtype).to(gpu)
    v_cache = torch.randn((1, Hk, S, D), generator=g).to(dtype).to(gpu)
    k0, v0 = k_cache.clone(), v_cache.clone()
    q_out = append_tree_kv(k, v, k_cache, v_cache, start, cos=cos, sin=sin, q=q)
    torch.cuda.synchronize()
    # torch's op sequence on [Hk, M, D] / [H, M, D] with cos/sin [M, D]
    kt = k.permute(1, 0, 2)
    want_k = (kt * cos) + (_rotate_half(kt, D) * sin)
    qt = q[0].permute(1, 0, 2)
    want_q = ((qt * cos) + (_rotate_half(qt, D) * sin)).permute(1, 0, 2).unsqueeze(0)
    assert torch.equal(k_cache[0, :, start:start + M], want_k)
    assert torch.equal(v_cache[0, :, start:start + M], v.permute(1, 0, 2))
    assert torch.equal(q_out, want_q)
    # outside the tree's slots nothing changed
    assert torch.equal(k_cache[..., :start, :], k0[..., :start, :])
    assert torch.equal(k_cache[..., start + M:, :], k0[..., start + M:, :])
    assert torch.equal(v_cache[..., start + M:, :], v0[..., start + M:, :])
    # and the oracle agrees
    got = oa.rope_16bit(kt.float().cpu().numpy(), cos.float().cpu().numpy(), sin.float().cpu().numpy(),
                        f16=dtype == torch.float16)
    assert np.array_equal(k_cache[0, :, start:start + M].float().cpu().numpy(), got)


def test_paged_append_lands_at_the_logical_tokens(gpu):
    # Page pool behind a random permutation; the tree's tokens straddle pages.
    inp = wl.make_tree_verify_inputs(n_prefix=150, M=40, H=8, Hk=2, D=128, layers=1, device=str(gpu), seed=6)
    start, M, Hk, D = 150, 40, 2, 128
    before = [inp.logical_kv(0, h).clone() for h in range(2)]
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, M, Hk, D), generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn((1, M, Hk, D), generator=g).to(torch.bfloat16).to(gpu)
    cos, sin = _tables(M, D, torch.bfloat16, 150, gpu)
    append_tree_kv(k, v, inp.kv_pages[0, 0], inp.kv_pages[0, 1], start, cos=cos, sin=sin,
                   page_table=inp.page_table)
    torch.cuda.synchronize()
    kl, vl = inp.logical_kv(0, 0)[0], inp.logical_kv(0, 1)[0]
    kt = k[0]
    want_k = (kt.permute(1, 0, 2) * cos + _rotate_half(kt.permute(1, 0, 2), D) * sin).permute(1, 0, 2)
    assert torch.equal(kl[start:start + M], want_k)
    assert torch.equal(vl[start:start + M], v[0])
    assert torch.equal(kl[:start], before[0][0, :start])
    assert torch.equal(vl[:start], before[1][0, :start])


def test_append_without_rope_is_a_copy(gpu):
    M, Hk, D, S, start = 5, 2, 64, 16, 3
    k = torch.randn((M, Hk, D), device=gpu).to(torch.float16)
    v = torch.randn((M, Hk, D), device=gpu).to(torch.float16)
    kc = torch.zeros((Hk, S, D), device=gpu, dtype=torch.float16)
    vc = torch.zeros((Hk, S, D), device=gpu, dtype=torch.float16)
    assert append_tree_kv(k, v, kc, vc, start) is None
    torch.cuda.synchronize()
    assert torch.equal(kc[:, start:start + M], k.permute(1, 0, 2))
    assert torch.equal(vc[:, start:start + M], v.permute(1, 0, 2))
    assert int((kc[:, :start] != 0).sum()) == 0 and int((kc[:, start + M:] != 0).sum()) == 0


def test_append_random_shapes(gpu):
    """20 random appends, bit-exact against torch's op sequence: 1 to 300 tree
    tokens, 1-8 key heads, 1-32 query heads (with or without q), head_dim 16
    to 256, bf16 / f16, with or without RoPE, into dense caches or page pools
    of 1- to 64-token pages behind a random permutation."""
    rng = np.random.default_rng(45)
    for case in range(20):
        dtype = [torch.bfloat16, torch.float16][int(rng.integers(2))]
        M, Hk = int(rng.choice([1, 3, 64, 300])), int(rng.choice([1, 2, 8]))
        D = int(rng.choice([16, 64, 128, 256]))
        H = Hk * int(rng.choice([1, 4])) if rng.integers(2) else 0
        rope, paged = bool(rng.integers(2)), bool(rng.integers(2))
        start = int(rng.integers(0, 200))
        print(f"[append random] case {case}: {dtype} M={M} Hk={Hk} H={H} D={D} rope={rope} paged={paged} "
              f"start={start}", flush=True)
        g = torch.Generator().manual_seed(case)
        k = (torch.randn((M, Hk, D), generator=g) * 2).to(dtype).to(gpu)
        v = torch.randn((M, Hk, D), generator=g).to(dtype).to(gpu)
        q = (torch.randn((M, H, D), generator=g) * 2).to(dtype).to(gpu) if H else None
        cos, sin = _tables(M, D, dtype, start + 1000, gpu) if rope else (None, None)
        if paged:
            ps = int(rng.choice([1, 2, 16, 64]))
            n_pages = (start + M + ps - 1) // ps
            kp = torch.randn((n_pages + 2, Hk, ps, D), generator=g).to(dtype).to(gpu)
            vp = torch.randn((n_pages + 2, Hk, ps, D), generator=g).to(dtype).to(gpu)
            pt = torch.from_numpy(rng.permutation(n_pages + 2)[:n_pages].astype(np.int32)).to(gpu)
            tok = torch.arange(start + M, device=gpu)
            phys, slot = pt[tok // ps].long(), tok % ps
            k0, v0 = kp[phys, :, slot].clone(), vp[phys, :, slot].clone()      # logical view [n, Hk, D]
            q_out = append_tree_kv(k, v, kp, vp, start, cos=cos, sin=sin, page_table=pt, q=q)
            kl, vl = kp[phys, :, slot], vp[phys, :, slot]
        else:
            S = start + M + int(rng.integers(0, 9))
            kc = torch.randn((Hk, S, D), generator=g).to(dtype).to(gpu)
            vc = torch.randn((Hk, S, D), generator=g).to(dtype).to(gpu)
            k0, v0 = kc.permute(1, 0, 2).clone(), vc.permute(1, 0, 2).clone()
            q_out = append_tree_kv(k, v, kc, vc, start, cos=cos, sin=sin, q=q)
            kl, vl = kc.permute(1, 0, 2), vc.permute(1, 0, 2)
        torch.cuda.synchronize()
        if rope:
            kt = k.permute(1, 0, 2)
            want_k = ((kt * cos) + (_rotate_half(kt, D) * sin)).permute(1, 0, 2)
        else:
            want_k = k
        assert torch.equal(kl[start:start + M], want_k), f"case {case} k"
        assert torch.equal(vl[start:start + M], v), f"case {case} v"
        assert torch.equal(kl[:start], k0[:start]) and torch.equal(vl[:start], v0[:start]), f"case {case} prefix"
        if H:
            qt = q.permute(1, 0, 2)
            want_q = ((qt * cos) + (_rotate_half(qt, D) * sin)).permute(1, 0, 2) if rope else q
            assert torch.equal(q_out.reshape(M, H, D), want_q), f"case {case} q"

"""Dry-run address emulation of the attention kernels (CPU, no GPU needed).

Every configuration the GPU tests and the benchmark launch is planned by the
C ABI exactly as for a real launch, then every global and LDS address that
kernels 1-3 would touch is computed with the kernels' own address arithmetic
and checked against the extent of its argument.  Tensors here are fake
descriptors (pointers are compared, never dereferenced).
"""

import ctypes

import pytest

from diffspec_mi355x import _ext

BASE = 1 << 40  # fake device addresses, far apart per argument
GAP = 1 << 36


class Alloc:
    def __init__(self):
        self.next = BASE

    def take(self, nbytes):
        p = self.next
        self.next += max(GAP, ((nbytes + 4095) // 4096) * 4096 + GAP)
        return p


ES = {_ext.DSV_BF16: 2, _ext.DSV_F16: 2, _ext.DSV_F32: 4, _ext.DSV_I8: 1, _ext.DSV_U8: 1, _ext.DSV_BOOL: 1,
      _ext.DSV_I32: 4, _ext.DSV_I64: 8}


def tensor(alloc, shape, dtype=_ext.DSV_BF16):
    d = _ext.DsvTensor()
    n = 1
    for s in shape:
        n *= s
    d.data = alloc.take(n * ES[dtype])
    d.dtype = dtype
    d.ndim = len(shape)
    st = 1
    for i in reversed(range(len(shape))):
        d.shape[i] = shape[i]
        d.stride[i] = st
        st *= shape[i]
    return d


def view(base, offset_elems, shape, strides):
    d = _ext.DsvTensor()
    d.data = base.data + offset_elems * ES[base.dtype]
    d.dtype = base.dtype
    d.ndim = len(shape)
    for i, (s, st) in enumerate(zip(shape, strides)):
        d.shape[i] = s
        d.stride[i] = st
    return d


def none():
    return _ext.DsvTensor()


@pytest.fixture
def dry(dsv_lib):
    dsv_lib.dsv_set_dry_run(1)
    yield dsv_lib
    dsv_lib.dsv_set_dry_run(0)


def ok(lib, rc, what):
    assert rc == 0, f"{what}: {_ext.last_error()}"
    assert lib.dsv_dry_run_checks() > 0


@pytest.mark.parametrize("D,H,Hk,M,N,B", [(128, 32, 8, 64, 1000, 2), (64, 8, 8, 10, 20, 1), (128, 32, 8, 5, 4096, 1),
                                         (64, 16, 4, 33, 777, 1), (128, 8, 2, 16, 300, 1),
                                         (128, 16, 4, 24, 3000, 1), (128, 16, 4, 24, 20000, 1)])
@pytest.mark.parametrize("dt", [_ext.DSV_BF16, _ext.DSV_F32])
def test_prefix_attention(dry, D, H, Hk, M, N, B, dt):
    a = Alloc()
    q, k, v = tensor(a, (B, M, H, D), dt), tensor(a, (B, N, Hk, D), dt), tensor(a, (B, N, Hk, D), dt)
    out, lse = tensor(a, (B, M, H, D), dt), tensor(a, (B, H, M), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, N, 0, 0)
    wsp = a.take(ws)
    for nk in (-1, N // 3):
        rc = dry.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), nk, ctypes.byref(out),
                                              ctypes.byref(lse), wsp, ws, None)
        ok(dry, rc, f"prefix n_keys={nk}")


@pytest.mark.parametrize("mask_dtype", [_ext.DSV_F32, _ext.DSV_I8, _ext.DSV_BOOL, _ext.DSV_BF16])
@pytest.mark.parametrize("dt", [_ext.DSV_BF16, _ext.DSV_F32])
def test_tree_attention_forward(dry, mask_dtype, dt):
    a = Alloc()
    B, M, H, Hk, D, T = 2, 64, 32, 8, 128, 70
    q, k, v = tensor(a, (B, M, H, D), dt), tensor(a, (B, M, Hk, D), dt), tensor(a, (B, M, Hk, D), dt)
    mask = tensor(a, (B, 1, T, T), mask_dtype)
    plse = tensor(a, (B, H, M), _ext.DSV_F32)
    cur, w, tl = tensor(a, (B, M, H, D), dt), tensor(a, (B, M, H, 1), dt), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, 0, 0, 1)
    rc = dry.dsv_tree_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), ctypes.byref(mask),
                                        ctypes.byref(plse), ctypes.byref(cur), ctypes.byref(w), ctypes.byref(tl),
                                        a.take(ws), ws, None)
    ok(dry, rc, "tree_attention_forward")


def paged_case(a, n_tok, Hk=8, D=128, ps=16, layers=1, spare=0, dt=_ext.DSV_BF16):
    n_pages = (n_tok + ps - 1) // ps
    P = n_pages + spare
    pool = tensor(a, (layers, 2, P, Hk, ps, D), dt)
    pt = tensor(a, (n_pages,), _ext.DSV_I32)
    return pool, pt, P


def pool_half(pool, layer, kv):
    s = list(pool.stride)[:6]
    shp = list(pool.shape)[:6]
    return view(pool, layer * s[0] + kv * s[1], shp[2:], s[2:])


@pytest.mark.parametrize("n_prefix,M,ps,H,Hk,D,perm", [
    (4096, 64, 16, 32, 8, 128, False), (0, 64, 16, 32, 8, 128, False), (100, 7, 16, 32, 8, 128, False),
    (1000, 128, 16, 32, 8, 128, True), (16, 256, 16, 32, 8, 128, False), (65536, 64, 16, 32, 8, 128, False),
    # the prefix lengths of bench.py's prefix sweep
    (4096, 64, 16, 32, 8, 128, False), (16384, 64, 16, 32, 8, 128, False), (262144, 64, 16, 32, 8, 128, False),
    (524288, 64, 16, 32, 8, 128, False),
    (131072, 128, 16, 32, 8, 128, True), (3000, 64, 16, 32, 8, 128, True), (200, 32, 16, 32, 8, 128, False),
    (1000, 16, 16, 32, 8, 128, False),
    # per-lane DMA mode: pages smaller than a DMA instruction, unaligned tree start
    (1000, 64, 2, 32, 8, 128, False), (101, 33, 16, 32, 8, 128, False), (777, 20, 4, 16, 4, 64, False),
    (50, 9, 1, 8, 2, 128, False),
    # the page sizes of tests/test_gpu_attention.py::test_tree_verify_page_sizes
    (1000, 64, 1, 8, 2, 128, False), (1000, 64, 2, 8, 2, 128, False), (1000, 64, 4, 8, 2, 64, False),
    (1000, 64, 8, 8, 2, 128, False), (1000, 64, 32, 8, 2, 128, True), (1000, 64, 64, 8, 2, 128, False),
    (5000, 48, 256, 8, 2, 128, False),
    # several 256-row blocks per KV head over many splits
    (6000, 256, 16, 32, 8, 128, False), (30000, 192, 16, 32, 8, 128, False),
    # the second workload of tests/test_gpu_graphs.py
    (1000, 20, 16, 32, 8, 128, False),
    # trees beyond 256 nodes (tests/test_gpu_attention.py::test_tree_verify_trees_beyond_256_nodes)
    (2000, 300, 16, 8, 2, 128, False), (500, 512, 16, 8, 2, 128, True), (100, 1024, 16, 8, 2, 128, True),
    (300, 1024, 16, 8, 2, 128, False), (1000, 700, 4, 8, 2, 64, False), (64, 257, 16, 32, 8, 128, True)])
def test_tree_verify_paged_and_dense(dry, n_prefix, M, ps, H, Hk, D, perm):
    a = Alloc()
    B = 1
    q = tensor(a, (B, M, H, D))
    pool, pt, P = paged_case(a, n_prefix + M, Hk=Hk, D=D, ps=ps, layers=2, spare=3)
    par = tensor(a, (M,), _ext.DSV_I64)
    rp = tensor(a, (M,), _ext.DSV_I32) if perm else none()
    out, lse = tensor(a, (B, M, H, D)), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, ps, 1)
    wsp = a.take(ws)
    for layer in (0, 1):
        kh, vh = pool_half(pool, layer, 0), pool_half(pool, layer, 1)
        rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kh), ctypes.byref(vh), ctypes.byref(pt), n_prefix,
                                 ctypes.byref(par), ctypes.byref(rp), ctypes.byref(out), ctypes.byref(lse), wsp, ws,
                                 None)
        ok(dry, rc, f"tree_verify paged layer {layer}")
    kc, vc = tensor(a, (B, n_prefix + M, Hk, D)), tensor(a, (B, n_prefix + M, Hk, D))
    ws2 = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, 0, 1)
    rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(none()), n_prefix,
                             ctypes.byref(par), ctypes.byref(rp), ctypes.byref(out), ctypes.byref(lse), a.take(ws2),
                             ws2, None)
    ok(dry, rc, "tree_verify dense")


@pytest.mark.parametrize("n_prefix,M,ps,H,Hk,D,perm", [
    (4096, 64, 16, 32, 8, 128, False), (0, 64, 16, 32, 8, 128, False), (100, 7, 16, 32, 8, 128, True),
    (1000, 64, 1, 8, 2, 128, False), (1000, 64, 4, 8, 2, 64, False), (1000, 64, 64, 8, 2, 128, True),
    (6000, 256, 16, 32, 8, 128, False), (30000, 192, 16, 32, 8, 128, False),
    (1000, 400, 16, 8, 2, 128, True), (200, 1024, 16, 8, 2, 64, False)])
def test_tree_verify_paged_and_dense_f32(dry, n_prefix, M, ps, H, Hk, D, perm):
    """The fp32 kernel's loads, over the shapes the fp32 GPU tests launch."""
    a = Alloc()
    B, dt = 1, _ext.DSV_F32
    q = tensor(a, (B, M, H, D), dt)
    pool, pt, P = paged_case(a, n_prefix + M, Hk=Hk, D=D, ps=ps, layers=2, spare=3, dt=dt)
    par = tensor(a, (M,), _ext.DSV_I64)
    rp = tensor(a, (M,), _ext.DSV_I32) if perm else none()
    out, lse = tensor(a, (B, M, H, D), dt), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, ps, 1)
    wsp = a.take(ws)
    for layer in (0, 1):
        kh, vh = pool_half(pool, layer, 0), pool_half(pool, layer, 1)
        rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kh), ctypes.byref(vh), ctypes.byref(pt), n_prefix,
                                 ctypes.byref(par), ctypes.byref(rp), ctypes.byref(out), ctypes.byref(lse), wsp, ws,
                                 None)
        ok(dry, rc, f"tree_verify paged f32 layer {layer}")
    kc, vc = tensor(a, (B, n_prefix + M, Hk, D), dt), tensor(a, (B, n_prefix + M, Hk, D), dt)
    ws2 = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, 0, 1)
    rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(none()), n_prefix,
                             ctypes.byref(par), ctypes.byref(rp), ctypes.byref(out), ctypes.byref(lse), a.take(ws2),
                             ws2, None)
    ok(dry, rc, "tree_verify dense f32")


def test_bench_shape_with_rotated_layers(dry):
    a = Alloc()
    n_prefix, M, H, Hk, D = 65536, 64, 32, 8, 128
    q = tensor(a, (1, M, H, D))
    pool, pt, P = paged_case(a, n_prefix + M, layers=4)
    par = tensor(a, (M,), _ext.DSV_I64)
    out, lse = tensor(a, (1, M, H, D)), tensor(a, (1, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(1, M, H, Hk, D, n_prefix, 16, 1)
    wsp = a.take(ws)
    for layer in range(4):
        kh, vh = pool_half(pool, layer, 0), pool_half(pool, layer, 1)
        rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kh), ctypes.byref(vh), ctypes.byref(pt), n_prefix,
                                 ctypes.byref(par), ctypes.byref(none()), ctypes.byref(out), ctypes.byref(lse), wsp,
                                 ws, None)
        ok(dry, rc, f"bench layer {layer}")


@pytest.mark.parametrize("B,M,H,Hk,D,N", [(1, 10, 8, 8, 64, 20), (1, 12, 8, 2, 128, 300), (2, 40, 32, 8, 128, 1000)])
@pytest.mark.parametrize("dt", [_ext.DSV_BF16, _ext.DSV_F32])
def test_verify_bundle_dense_and_paged(dry, B, M, H, Hk, D, N, dt):
    a = Alloc()
    q, k, v = tensor(a, (B, M, H, D), dt), tensor(a, (B, N, Hk, D), dt), tensor(a, (B, N, Hk, D), dt)
    mask = tensor(a, (1, M, N), _ext.DSV_I8)
    out, lse = tensor(a, (B, M, H, D), dt), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, N, 0, 0)
    rc = dry.dsv_verify_bundle(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), ctypes.byref(mask), ctypes.byref(out),
                               ctypes.byref(lse), a.take(ws), ws, None)
    ok(dry, rc, "verify_bundle")
    pool, pt, P = paged_case(a, N, Hk=Hk, D=D, ps=16, layers=2, spare=3, dt=dt)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, N, 16, 0)
    rc = dry.dsv_verify_bundle_paged(ctypes.byref(q), ctypes.byref(pool), ctypes.byref(pt), 1, ctypes.byref(mask),
                                     ctypes.byref(out), ctypes.byref(lse), a.take(ws), ws, None)
    ok(dry, rc, "verify_bundle_paged")


def test_inconsistent_shapes_are_rejected_before_any_access(dry):
    a = Alloc()
    B, M, H, Hk, D, N = 1, 8, 8, 2, 128, 64
    q = tensor(a, (B, M, H, D))
    k, v = tensor(a, (B, N, Hk, D)), tensor(a, (B, N, Hk, D))
    out, lse = tensor(a, (B, M, H, D)), tensor(a, (B, H, M), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, N, 0, 0)
    wsp = a.take(ws)
    rc = dry.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), N + 1,
                                          ctypes.byref(out), ctypes.byref(lse), wsp, ws, None)
    assert rc == -1 and "exceeds" in _ext.last_error()
    k_short = view(k, 0, (B, N - 1, Hk, D), list(k.stride)[:4])
    rc = dry.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k_short), ctypes.byref(v), -1,
                                          ctypes.byref(out), ctypes.byref(lse), wsp, ws, None)
    assert rc == -1 and "shapes differ" in _ext.last_error()


def test_tree_verify_refuses_trees_beyond_1024_nodes(dry):
    a = Alloc()
    B, M, H, Hk, D, N = 1, 1025, 8, 2, 128, 100
    q = tensor(a, (B, M, H, D))
    kc, vc = tensor(a, (B, N + M, Hk, D)), tensor(a, (B, N + M, Hk, D))
    par = tensor(a, (M,), _ext.DSV_I64)
    out, lse = tensor(a, (B, M, H, D)), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = 1 << 30
    rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(none()), N,
                             ctypes.byref(par), ctypes.byref(none()), ctypes.byref(out), ctypes.byref(lse),
                             a.take(256), ws, None)
    assert rc == -2 and "1024" in _ext.last_error()


@pytest.mark.parametrize("ps", [16, 4])
def test_tree_verify_batched_page_table(dry, ps):
    # the shape of tests/test_gpu_attention.py::test_tree_verify_batched_paged_f16:
    # B = 2, one page-table row per batch (int64), f16, a parent row per batch
    a = Alloc()
    B, M, H, Hk, D, n_prefix = 2, 40, 8, 2, 128, 700
    n_pages = (n_prefix + M + ps - 1) // ps
    q = tensor(a, (B, M, H, D), _ext.DSV_F16)
    pool = tensor(a, (1, 2, B * n_pages, Hk, ps, D), _ext.DSV_F16)
    pt = tensor(a, (B, n_pages), _ext.DSV_I64)
    par = tensor(a, (B, M), _ext.DSV_I64)
    out, lse = tensor(a, (B, M, H, D), _ext.DSV_F16), tensor(a, (B, M, H), _ext.DSV_F32)
    ws = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, ps, 1)
    kh, vh = pool_half(pool, 0, 0), pool_half(pool, 0, 1)
    rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kh), ctypes.byref(vh), ctypes.byref(pt), n_prefix,
                             ctypes.byref(par), ctypes.byref(none()), ctypes.byref(out), ctypes.byref(lse), a.take(ws),
                             ws, None)
    ok(dry, rc, "tree_verify batched page table")
    kc, vc = tensor(a, (B, n_prefix + M, Hk, D), _ext.DSV_F16), tensor(a, (B, n_prefix + M, Hk, D), _ext.DSV_F16)
    ws2 = dry.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, 0, 1)
    rc = dry.dsv_tree_verify(ctypes.byref(q), ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(none()), n_prefix,
                             ctypes.byref(par), ctypes.byref(none()), ctypes.byref(out), ctypes.byref(lse), a.take(ws2),
                             ws2, None)
    ok(dry, rc, "tree_verify batched dense")

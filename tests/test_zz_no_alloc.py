"""The allocation-free tree verify (dsv_tree_verify_noalloc) through the C ABI:
bit-equal to dsv_tree_verify with a caller workspace, on two calls in a row
(the second with a smaller input, so stale scratch from the first cannot leak
into it), and a clear refusal of a shape whose split plan exceeds the fixed
scratch array."""

import ctypes

import pytest
import torch

from diffspec_mi355x import _ext
from diffspec_mi355x import workloads as wl

pytestmark = pytest.mark.gpu


def _verify(lib, inp, par, noalloc, stream=None):
    q = inp.q
    B, M, H, D = q.shape
    out = torch.empty((B, M, H, D), dtype=torch.float32, device=q.device)
    lse = torch.empty((B, M, H), dtype=torch.float32, device=q.device)
    k, v = inp.kv_pages[0, 0], inp.kv_pages[0, 1]
    args = [ctypes.byref(_ext.desc(x)) for x in (q, k, v, inp.page_table)]
    tail = [ctypes.byref(_ext.desc(par)), ctypes.byref(_ext.desc(None)), ctypes.byref(_ext.desc(out)),
            ctypes.byref(_ext.desc(lse))]
    stream = _ext.stream_of(q.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
    if noalloc:
        rc = lib.dsv_tree_verify_noalloc(*args, inp.n_prefix, *tail, stream)
    else:
        ws = _ext.workspace(lib.dsv_attn_workspace_bytes(B, M, H, k.shape[1], D, inp.n_prefix, k.shape[2], 1),
                            q.device)
        rc = lib.dsv_tree_verify(*args, inp.n_prefix, *tail, ws.data_ptr(), ws.numel(), stream)
    _ext.check(rc, "tree verify")
    return out, lse


def test_noalloc_tree_verify_matches_workspace_entry_point(gpu, dsv_lib):
    for n_prefix, M in [(65536, 64), (3000, 24)]:
        print(f"[noalloc] n_prefix={n_prefix} M={M}", flush=True)
        inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, device=str(gpu), seed=n_prefix % 7,
                                         tree_seed=M)
        par = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
        o_n, l_n = _verify(dsv_lib, inp, par, noalloc=True)
        o_w, l_w = _verify(dsv_lib, inp, par, noalloc=False)
        torch.cuda.synchronize()
        assert torch.equal(o_n, o_w) and torch.equal(l_n, l_w)


def test_noalloc_calls_on_two_streams_are_serialised(gpu, dsv_lib):
    """Two calls issued back to back on two streams, with no host
    synchronisation between them, share the GPU's scratch array: the library
    makes the second stream wait for the first call, so each result still
    equals dsv_tree_verify's with its own workspace."""
    cases = [(65536, 64, 1), (20000, 48, 2)]
    inps = [wl.make_tree_verify_inputs(n_prefix=n, M=M, device=str(gpu), seed=s, tree_seed=M) for n, M, s in cases]
    pars = [torch.tensor(i.parent, dtype=torch.int64, device=gpu) for i in inps]
    want = [_verify(dsv_lib, i, p, noalloc=False) for i, p in zip(inps, pars)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=gpu), torch.cuda.Stream(device=gpu)
    for rep in range(3):
        print(f"[noalloc two streams] round {rep}", flush=True)
        got = [_verify(dsv_lib, inps[0], pars[0], noalloc=True, stream=s1),
               _verify(dsv_lib, inps[1], pars[1], noalloc=True, stream=s2)]
        torch.cuda.synchronize()
        for (o, l), (ow, lw) in zip(got, want):
            assert torch.equal(o, ow) and torch.equal(l, lw)


def test_noalloc_refuses_a_plan_beyond_its_scratch(gpu, dsv_lib):
    # 64 trees x 8 KV heads x 4 row blocks: more units than workgroup slots,
    # so the split partials exceed the fixed scratch array.
    B, M, H, Hk, D, ps, n_prefix = 64, 256, 32, 8, 128, 16, 20000
    n_pages = (n_prefix + M + ps - 1) // ps
    q = torch.zeros((B, M, H, D), dtype=torch.bfloat16, device=gpu)
    pool = torch.zeros((2, n_pages, Hk, ps, D), dtype=torch.bfloat16, device=gpu)
    pt = torch.arange(n_pages, dtype=torch.int32, device=gpu)
    par = torch.full((M,), -1, dtype=torch.int64, device=gpu)
    out = torch.empty_like(q)
    need = dsv_lib.dsv_attn_workspace_bytes(B, M, H, Hk, D, n_prefix, ps, 1)
    assert need > 32 << 20
    rc = dsv_lib.dsv_tree_verify_noalloc(*[ctypes.byref(_ext.desc(x)) for x in (q, pool[0], pool[1], pt)], n_prefix,
                                         ctypes.byref(_ext.desc(par)), ctypes.byref(_ext.desc(None)),
                                         ctypes.byref(_ext.desc(out)), ctypes.byref(_ext.desc(None)),
                                         _ext.stream_of(gpu))
    assert rc == -2 and "allocation-free" in _ext.last_error()

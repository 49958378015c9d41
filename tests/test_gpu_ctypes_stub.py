"""The minimal ctypes binding a maintainer would add inside the reference
(runtime/tree_attention.py for tree verify and the bundle order,
draft/tree_verification.py:103-106 for the sampling branch), written against
include/dsv.h alone, gives the same results as the package's binding: tree
verify paged at 8K keys, the device bundle order, and a sampling acceptance."""

import ctypes

import pytest
import torch

from diffspec_mi355x import _ext, workloads as wl
from diffspec_mi355x.core.bundle_scheduler import bundle_row_order_device
from diffspec_mi355x.draft.tree_verification import tree_accept
from diffspec_mi355x.runtime.tree_attention import tree_verify

pytestmark = pytest.mark.gpu


class DsvTensor(ctypes.Structure):  # include/dsv.h: dsv_tensor
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 6), ("stride", ctypes.c_int64 * 6)]


_DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.int8: 3, torch.uint8: 4,
       torch.bool: 5, torch.int32: 6, torch.int64: 7}


def desc(t):
    d = DsvTensor()
    if t is not None:
        d.data, d.dtype, d.ndim = t.data_ptr(), _DT[t.dtype], t.dim()
        for i in range(t.dim()):
            d.shape[i], d.stride[i] = t.shape[i], t.stride(i)
    return d


@pytest.fixture(scope="module")
def lib():
    _ext.load()  # the package's own load (torch's HIP runtime first), then a second handle as a maintainer would
    lib = ctypes.CDLL(str(_ext.lib_path()))
    P = ctypes.POINTER(DsvTensor)
    lib.dsv_last_error.restype = ctypes.c_char_p
    lib.dsv_attn_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv_attn_workspace_bytes.argtypes = [ctypes.c_int64] * 7 + [ctypes.c_int]
    lib.dsv_tree_verify.argtypes = [P, P, P, P, ctypes.c_int64, P, P, P, P, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p]
    lib.dsv_bundle_order.argtypes = [P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, P, P, ctypes.c_void_p]
    lib.dsv_accept_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv_accept_workspace_bytes.argtypes = [ctypes.c_int64] * 3
    lib.dsv_tree_accept_sample.argtypes = [P, P, P, P, ctypes.c_int64, ctypes.c_float, ctypes.c_float, ctypes.c_int64,
                                           ctypes.c_uint64, P, P, P, P, ctypes.c_void_p, ctypes.c_size_t,
                                           ctypes.c_void_p]
    return lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(lib, rc):
    if rc != 0:
        raise RuntimeError(lib.dsv_last_error().decode())


def test_tree_verify_through_the_stub(gpu, lib):
    inp = wl.make_tree_verify_inputs(n_prefix=8192, M=64, H=32, Hk=8, D=128, device=str(gpu), seed=4, tree_seed=4)
    q, kp, vp, pt = inp.q, inp.kv_pages[0, 0], inp.kv_pages[0, 1], inp.page_table
    parent = torch.tensor(inp.parent, dtype=torch.int64, device=gpu)
    B, M, H, D = q.shape
    Hk, ps = kp.shape[1], kp.shape[2]
    out = torch.empty_like(q)
    lse = torch.empty(B, M, H, dtype=torch.float32, device=gpu)
    nbytes = lib.dsv_attn_workspace_bytes(B, M, H, Hk, D, 8192, ps, 1)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    _check(lib, lib.dsv_tree_verify(desc(q), desc(kp), desc(vp), desc(pt), 8192, desc(parent), desc(None), desc(out),
                                    desc(lse), ws.data_ptr(), nbytes, _stream()))
    o_ref, l_ref = tree_verify(q, kp, vp, 8192, parent, page_table=pt)
    torch.cuda.synchronize()
    assert torch.equal(out, o_ref) and torch.equal(lse, l_ref)


def test_bundle_order_through_the_stub(gpu, lib):
    parent = torch.tensor(wl.make_tree(128, max_depth=12, max_outdeg=6, seed=3)[0], dtype=torch.int64, device=gpu)
    perm = torch.empty(parent.shape, dtype=torch.int32, device=gpu)
    _check(lib, lib.dsv_bundle_order(desc(parent), 3, 8, 100, desc(perm), desc(None), _stream()))
    ref = bundle_row_order_device(parent, bundle_size=3, max_bundles=100, num_bundles=8)
    torch.cuda.synchronize()
    assert torch.equal(perm, ref)


def test_sample_accept_through_the_stub(gpu, lib):
    a = wl.make_accept_inputs(T=2, M=32, V=32000, device=str(gpu), seed=9)
    T, M, V = a.logits.shape
    path = torch.empty(T, M, dtype=torch.int64, device=gpu)
    toks = torch.empty(T, M, dtype=torch.int64, device=gpu)
    info = torch.empty(T, 4, dtype=torch.int64, device=gpu)
    nxt = torch.empty(T, M, dtype=torch.int64, device=gpu)
    nbytes = lib.dsv_accept_workspace_bytes(T, M, V)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    _check(lib, lib.dsv_tree_accept_sample(desc(a.logits), desc(a.draft), desc(a.parent_ref), desc(a.pos), 10, 0.7,
                                           0.9, 50, 1234, desc(path), desc(toks), desc(info), desc(nxt),
                                           ws.data_ptr(), nbytes, _stream()))
    ref = tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode="sample", temperature=0.7, top_p=0.9, top_k=50,
                      seed=1234, return_next=True)
    torch.cuda.synchronize()
    assert torch.equal(info, ref["info"]) and torch.equal(nxt, ref["next"])
    n = int(info[0, 3])
    assert torch.equal(path[0, :n], ref["path"][0, :n]) and torch.equal(toks[0, :n], ref["tokens"][0, :n])

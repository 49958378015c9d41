"""The C-ABI library (CPU-side checks only: no kernel is launched here).

  * libdsv.so loads and exports every function include/dsv.h declares, and a C99
    caller compiles against the header and links every declaration;
  * the ctypes signature table matches the header;
  * argument validation fails loudly with an error code and a message;
  * the Python API refuses CPU tensors (no CPU fallback exists).
"""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from diffspec_mi355x import _ext

HEADER = Path(__file__).resolve().parents[1] / "include" / "dsv.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ["dsv_prefix_attention_forward", "dsv_tree_attention_forward", "dsv_verify_bundle",
              "dsv_verify_bundle_paged", "dsv_tree_verify", "dsv_tree_accept", "dsv_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol(dsv_lib):
    for name in declared_functions():
        assert hasattr(dsv_lib, name), f"{name} declared in dsv.h but not exported"
        assert name in _ext.SIGNATURES, f"{name} has no ctypes signature"


def test_header_is_plain_c_and_links_every_declaration(dsv_lib, tmp_path):
    """A C99 caller (gcc -pedantic -Werror) compiles against dsv.h and links every
    declared function against the built library: the declarations are C, and
    each names an exported symbol with C linkage."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    names = declared_functions()
    src = tmp_path / "caller.c"
    src.write_text('#include "dsv.h"\n#include <stdio.h>\ntypedef void (*any_fn)(void);\nint main(void) {\n'
                   '  any_fn fns[] = {\n'
                   + "".join(f"    (any_fn)&{n},\n" for n in names)
                   + "  };\n  printf(\"%d %d\\n\", (int)(sizeof(fns) / sizeof(fns[0])), dsv_version());\n"
                   "  return 0;\n}\n")
    lib = Path(_ext.lib_path())
    exe = tmp_path / "caller"
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{HEADER.parent}", str(src),
           f"-L{lib.parent}", f"-l{lib.stem[3:]}", f"-Wl,-rpath,{lib.parent}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stderr
    assert run.stdout.split() == [str(len(names)), "1"]


def test_version(dsv_lib):
    assert dsv_lib.dsv_version() >= 1


def test_workspace_sizes(dsv_lib):
    # invalid arguments -> 0
    assert dsv_lib.dsv_attn_workspace_bytes(1, 64, 30, 8, 128, 1000, 16, 1) == 0
    n = dsv_lib.dsv_attn_workspace_bytes(1, 64, 32, 8, 128, 65536, 16, 1)
    rows = 8 * 256
    assert n >= 2 * rows * (128 * 2 + 8)  # bf16 partial rows + (max, sum): a prefix split + the tree split
    assert dsv_lib.dsv_accept_workspace_bytes(8, 64, 128256) >= 8 * 64 * 8 * 20


def _t(shape, dtype=_ext.DSV_BF16, ptr=0x1000):
    d = _ext.DsvTensor()
    d.data = ptr
    d.dtype = dtype
    d.ndim = len(shape)
    st = 1
    for i in reversed(range(len(shape))):
        d.shape[i] = shape[i]
        d.stride[i] = st
        st *= shape[i]
    return d


def test_validation_errors_are_reported(dsv_lib):
    q = _t((1, 4, 8, 128))
    k = _t((1, 16, 2, 128))
    out = _t((1, 4, 8, 128))
    lse_bad = _t((1, 4, 8), _ext.DSV_F32)  # should be [B, H, M] = (1, 8, 4)
    rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), -1,
                                              ctypes.byref(out), ctypes.byref(lse_bad), None, 0, None)
    assert rc == -1 and "lse" in _ext.last_error()
    q8 = _t((1, 4, 8, 128), _ext.DSV_I8)
    rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q8), ctypes.byref(k), ctypes.byref(k), -1,
                                              ctypes.byref(out), ctypes.byref(lse_bad), None, 0, None)
    assert rc == -2 and "bf16, f16 or f32" in _ext.last_error()
    q32 = _t((1, 4, 8, 128), _ext.DSV_F32)  # fp32 q with bf16 keys: the dtypes must agree
    rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q32), ctypes.byref(k), ctypes.byref(k), -1,
                                              ctypes.byref(out), ctypes.byref(lse_bad), None, 0, None)
    assert rc == -1 and "dtype" in _ext.last_error()
    q96 = _t((1, 4, 8, 96))
    rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q96), ctypes.byref(k), ctypes.byref(k), -1,
                                              ctypes.byref(q96), ctypes.byref(lse_bad), None, 0, None)
    assert rc == -2 and "head_dim" in _ext.last_error()
    lse = _t((1, 8, 4), _ext.DSV_F32)
    rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), -1,
                                              ctypes.byref(out), ctypes.byref(lse), None, 0, None)
    assert rc == -3 and "workspace" in _ext.last_error()


def test_attention_refuses_sizes_beyond_its_32_bit_counts(dsv_lib):
    # Query rows per KV head above 2^24, and batch x heads x rows above 2^30:
    # refused with a message, and no workspace is planned for them.
    for B, M in ((1, 1 << 23), (1 << 10, 1 << 20)):
        q = _t((B, M, 32, 128))
        k = _t((B, 64, 8, 128))
        lse = _t((B, 32, M), _ext.DSV_F32)
        rc = dsv_lib.dsv_prefix_attention_forward(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), -1,
                                                  ctypes.byref(q), ctypes.byref(lse), None, 0, None)
        assert rc == -2 and "range" in _ext.last_error()
        assert dsv_lib.dsv_attn_workspace_bytes(B, M, 32, 8, 128, 64, 0, 0) == 0
    assert dsv_lib.dsv_attn_workspace_bytes(1, 64, 32, 8, 128, 65536, 16, 1) > 0


def test_accept_validation(dsv_lib):
    logits = _t((2, 8, 100), _ext.DSV_BF16)
    draft = _t((2, 8), _ext.DSV_I64)
    parent_bad = _t((2, 8), _ext.DSV_I64)  # must be [T, M-1]
    pos = _t((8,), _ext.DSV_I64)
    o = _t((2, 8), _ext.DSV_I64)
    info = _t((2, 4), _ext.DSV_I64)
    none = _ext.DsvTensor()
    rc = dsv_lib.dsv_tree_accept(0, ctypes.byref(logits), ctypes.byref(draft), ctypes.byref(parent_bad),
                                 ctypes.byref(pos), 10, 1.0, 0.09, 0.3, ctypes.byref(o), ctypes.byref(o),
                                 ctypes.byref(info), ctypes.byref(none), None, 0, None)
    assert rc == -1 and "parent" in _ext.last_error()
    rc = dsv_lib.dsv_tree_accept(7, ctypes.byref(logits), ctypes.byref(draft), ctypes.byref(parent_bad),
                                 ctypes.byref(pos), 10, 1.0, 0.09, 0.3, ctypes.byref(o), ctypes.byref(o),
                                 ctypes.byref(info), ctypes.byref(none), None, 0, None)
    assert rc == -1 and "mode" in _ext.last_error()
    # no trees at all: rejected, not launched with an empty grid
    logits0, draft0 = _t((0, 8, 100), _ext.DSV_BF16), _t((0, 8), _ext.DSV_I64)
    parent0, o0, info0 = _t((0, 7), _ext.DSV_I64), _t((0, 8), _ext.DSV_I64), _t((0, 4), _ext.DSV_I64)
    rc = dsv_lib.dsv_tree_accept(0, ctypes.byref(logits0), ctypes.byref(draft0), ctypes.byref(parent0),
                                 ctypes.byref(pos), 10, 1.0, 0.09, 0.3, ctypes.byref(o0), ctypes.byref(o0),
                                 ctypes.byref(info0), ctypes.byref(none), None, 0, None)
    assert rc == -1 and "tree count" in _ext.last_error()


def test_accept_sample_validation(dsv_lib):
    """The sampling entry point checks its warper arguments and workspace
    before any launch (the fake tensors are never dereferenced)."""
    logits = _t((2, 8, 100), _ext.DSV_BF16)
    draft = _t((2, 8), _ext.DSV_I64)
    parent = _t((2, 7), _ext.DSV_I64)
    pos = _t((8,), _ext.DSV_I64)
    o = _t((2, 8), _ext.DSV_I64)
    info = _t((2, 4), _ext.DSV_I64)
    none = _ext.DsvTensor()

    def call(temperature=1.0, top_p=1.0, top_k=0, ws=None, nbytes=0, lg=logits):
        return dsv_lib.dsv_tree_accept_sample(ctypes.byref(lg), ctypes.byref(draft), ctypes.byref(parent),
                                              ctypes.byref(pos), 10, temperature, top_p, top_k, 5, ctypes.byref(o),
                                              ctypes.byref(o), ctypes.byref(info), ctypes.byref(none), ws, nbytes,
                                              None)

    assert call(temperature=0.0) == -1 and "temperature" in _ext.last_error()
    assert call(temperature=float("nan")) == -1 and "temperature" in _ext.last_error()
    # The reference samples only when temperature > 1e-5 (in double precision):
    # the float nearest 1e-5 lies below it and is refused; the next one up
    # passes the check (and fails later, on the fake workspace).
    f_1e5 = float(np.float32(1e-5))
    assert f_1e5 < 1e-5 and call(temperature=f_1e5) == -1 and "temperature" in _ext.last_error()
    above = float(np.nextafter(np.float32(1e-5), np.float32(1.0)))
    assert above > 1e-5 and call(temperature=above) == -3 and "workspace" in _ext.last_error()
    assert call(top_p=1.5) == -1 and "top_p" in _ext.last_error()
    assert call(top_p=-0.1) == -1 and "top_p" in _ext.last_error()
    assert call(top_k=-1) == -1 and "top_k" in _ext.last_error()
    assert call(lg=_t((2, 8, 100), _ext.DSV_I32)) == -1 and "logits" in _ext.last_error()
    rc = call(ws=0x1000, nbytes=16)
    assert rc == -3 and "workspace" in _ext.last_error()  # DSV_ERR_WORKSPACE
    need = dsv_lib.dsv_accept_workspace_bytes(2, 8, 100)
    rc = call(ws=0x1000 + 16, nbytes=need)
    assert rc == -3 and "aligned" in _ext.last_error()


def test_kv_commit_validation(dsv_lib):
    path = _t((1, 8), _ext.DSV_I64)
    info = _t((1, 4), _ext.DSV_I64)
    none = _ext.DsvTensor()
    kv_odd = _t((2, 2, 40, 6), _ext.DSV_BF16)  # 12-byte token rows
    rc = dsv_lib.dsv_kv_commit(ctypes.byref(kv_odd), ctypes.byref(none), 10, ctypes.byref(path), ctypes.byref(info),
                               0, None)
    assert rc == -2 and "16 bytes" in _ext.last_error()
    kv = _t((2, 2, 40, 64), _ext.DSV_BF16)
    rc = dsv_lib.dsv_kv_commit(ctypes.byref(kv), ctypes.byref(none), 35, ctypes.byref(path), ctypes.byref(info),
                               0, None)
    assert rc == -1 and "exceed the cache" in _ext.last_error()
    rc = dsv_lib.dsv_kv_commit(ctypes.byref(kv), ctypes.byref(none), 10, ctypes.byref(path), ctypes.byref(info),
                               1, None)
    assert rc == -1 and "tree" in _ext.last_error()
    pool = _t((2, 2, 6, 2, 16, 64), _ext.DSV_BF16)
    pt = _t((4,), _ext.DSV_I32)
    rc = dsv_lib.dsv_kv_commit(ctypes.byref(pool), ctypes.byref(pt), 60, ctypes.byref(path), ctypes.byref(info),
                               0, None)
    assert rc == -1 and "page table" in _ext.last_error()
    # A valid call plans without launching in dry-run mode.
    dsv_lib.dsv_set_dry_run(1)
    try:
        rc = dsv_lib.dsv_kv_commit(ctypes.byref(pool), ctypes.byref(pt), 40, ctypes.byref(path), ctypes.byref(info),
                                   0, None)
    finally:
        dsv_lib.dsv_set_dry_run(0)
    assert rc == 0


def test_kv_append_validation(dsv_lib):
    none = _ext.DsvTensor()
    k = _t((8, 2, 72))  # head_dim not a multiple of 16
    dst = _t((2, 40, 72))
    rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(none), ctypes.byref(none),
                               ctypes.byref(dst), ctypes.byref(dst), ctypes.byref(none), 0, ctypes.byref(none),
                               ctypes.byref(none), None)
    assert rc == -2 and "multiple of 16" in _ext.last_error()
    k = _t((8, 2, 64))
    dst = _t((2, 40, 64))
    rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(none), ctypes.byref(none),
                               ctypes.byref(dst), ctypes.byref(dst), ctypes.byref(none), 35, ctypes.byref(none),
                               ctypes.byref(none), None)
    assert rc == -1 and "exceed the cache" in _ext.last_error()
    cos = _t((8, 64))
    rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(cos), ctypes.byref(none),
                               ctypes.byref(dst), ctypes.byref(dst), ctypes.byref(none), 0, ctypes.byref(none),
                               ctypes.byref(none), None)
    assert rc == -1 and "together" in _ext.last_error()
    dst = _t((2, 40, 64), ptr=0x100000)
    vdst = _t((2, 40, 64), ptr=0x200000)
    dsv_lib.dsv_set_dry_run(1)
    try:
        rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(cos), ctypes.byref(cos),
                                   ctypes.byref(dst), ctypes.byref(vdst), ctypes.byref(none), 32, ctypes.byref(none),
                                   ctypes.byref(none), None)
    finally:
        dsv_lib.dsv_set_dry_run(0)
    assert rc == 0


def test_kv_append_refuses_sizes_beyond_its_32_bit_counts(dsv_lib):
    # The descriptors are never dereferenced: the sizes are refused first.
    none = _ext.DsvTensor()
    k = _t(((1 << 24) + 1, 1, 16))
    dst = _t((1, (1 << 24) + 8, 16))
    rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(none), ctypes.byref(none),
                               ctypes.byref(dst), ctypes.byref(dst), ctypes.byref(none), 0, ctypes.byref(none),
                               ctypes.byref(none), None)
    assert rc == -2 and "too large" in _ext.last_error()
    k = _t((1 << 20, 1 << 10, 64))  # 2^31 chunks of k and v
    dst = _t((1 << 10, (1 << 20) + 8, 64))
    rc = dsv_lib.dsv_kv_append(ctypes.byref(k), ctypes.byref(k), ctypes.byref(none), ctypes.byref(none),
                               ctypes.byref(dst), ctypes.byref(dst), ctypes.byref(none), 0, ctypes.byref(none),
                               ctypes.byref(none), None)
    assert rc == -2 and "2^31" in _ext.last_error()


def test_kv_append_rejects_aliasing_except_row_for_row_in_place(dsv_lib):
    # A thread reads a chunk pair of one row and writes the same pair of the
    # destination row: exact in-place rotation is safe, any other overlap of
    # an input with an output is refused before launch.
    none = _ext.DsvTensor()
    M, Hk, H, D, S = 8, 2, 4, 64, 40
    k = _t((M, Hk, D), ptr=0x10000)
    v = _t((M, Hk, D), ptr=0x20000)
    cos = _t((M, D), ptr=0x30000)
    sin = _t((M, D), ptr=0x40000)
    kd = _t((Hk, S, D), ptr=0x50000)
    vd = _t((Hk, S, D), ptr=0x60000)
    q = _t((M, H, D), ptr=0x70000)

    def call(k_, v_, q_, qo_, start=16):
        dsv_lib.dsv_set_dry_run(1)
        try:
            return dsv_lib.dsv_kv_append(ctypes.byref(k_), ctypes.byref(v_), ctypes.byref(cos), ctypes.byref(sin),
                                         ctypes.byref(kd), ctypes.byref(vd), ctypes.byref(none), start,
                                         ctypes.byref(q_), ctypes.byref(qo_), None)
        finally:
            dsv_lib.dsv_set_dry_run(0)

    assert call(k, v, q, _t((M, H, D), ptr=0x80000)) == 0
    assert call(k, v, q, q) == 0                                  # q rotated in place
    shifted = _t((M, H, D), ptr=0x70000 + 2 * D)                  # q_out one head over q
    assert call(k, v, q, shifted) == -1 and "q overlaps q_out" in _ext.last_error()
    assert call(k, v, q, _t((M, H, D), ptr=0x50000)) == -1 and "k_dst overlaps q_out" in _ext.last_error()
    # k already in k_dst's tree slots (token stride D, head stride S * D), row for row
    start = 16
    k_in = _ext.DsvTensor()
    k_in.data, k_in.dtype, k_in.ndim = 0x50000 + start * D * 2, _ext.DSV_BF16, 3
    for i, (n, st) in enumerate([(M, D), (Hk, S * D), (D, 1)]):
        k_in.shape[i], k_in.stride[i] = n, st
    assert call(k_in, v, q, _t((M, H, D), ptr=0x80000), start=start) == 0
    assert call(k_in, v, q, _t((M, H, D), ptr=0x80000), start=start + 1) == -1   # off by one token
    assert call(v, v, q, _t((M, H, D), ptr=0x80000)) == 0                        # k and v may share


def test_bundle_order_validation(dsv_lib):
    none = _ext.DsvTensor()
    par = _t((2000,), _ext.DSV_I64)
    perm = _t((2000,), _ext.DSV_I32)
    rc = dsv_lib.dsv_bundle_order(ctypes.byref(par), 3, 0, 100, ctypes.byref(perm), ctypes.byref(none), None)
    assert rc == -2 and "1..1024" in _ext.last_error()
    par = _t((2, 64), _ext.DSV_I32)
    perm = _t((2, 64), _ext.DSV_I32)
    rc = dsv_lib.dsv_bundle_order(ctypes.byref(par), 0, 0, 100, ctypes.byref(perm), ctypes.byref(none), None)
    assert rc == -1 and "bundle_size" in _ext.last_error()
    bad = _t((2, 64), _ext.DSV_I64)
    rc = dsv_lib.dsv_bundle_order(ctypes.byref(par), 3, 0, 100, ctypes.byref(bad), ctypes.byref(none), None)
    assert rc == -1 and "int32" in _ext.last_error()
    bad = _t((64,), _ext.DSV_I32)
    rc = dsv_lib.dsv_bundle_order(ctypes.byref(par), 3, 0, 100, ctypes.byref(perm), ctypes.byref(bad), None)
    assert rc == -1 and "shape of parent" in _ext.last_error()
    dsv_lib.dsv_set_dry_run(1)
    try:
        # num_bundles > 0 overrides bundle_size; max_bundles < 1 means one bundle
        rc = dsv_lib.dsv_bundle_order(ctypes.byref(par), 0, 8, 0, ctypes.byref(perm), ctypes.byref(perm), None)
    finally:
        dsv_lib.dsv_set_dry_run(0)
    assert rc == 0


def test_lmhead_accept_validation(dsv_lib):
    none = _ext.DsvTensor()
    T, M, Dm, V = 1, 8, 96, 500
    hidden = _t((T, M, Dm))
    weight = _t((V, Dm))
    draft, parent, pos = _t((T, M), _ext.DSV_I64), _t((T, M - 1), _ext.DSV_I64), _t((T, M), _ext.DSV_I64)
    outs = [_t((T, M), _ext.DSV_I64), _t((T, M), _ext.DSV_I64), _t((T, 4), _ext.DSV_I64)]

    def call(h, w, ws_bytes=1 << 20, lo=none):
        return dsv_lib.dsv_lmhead_accept(0, ctypes.byref(h), ctypes.byref(w), ctypes.byref(draft), ctypes.byref(parent),
                                         ctypes.byref(pos), 4, 1.0, 0.09, 0.3, ctypes.byref(outs[0]),
                                         ctypes.byref(outs[1]), ctypes.byref(outs[2]), ctypes.byref(none),
                                         ctypes.byref(lo), ctypes.c_void_p(0x100000), ws_bytes, None)

    rc = call(hidden, weight)  # Dm = 96 is not a multiple of 64
    assert rc == -2 and "multiple of 64" in _ext.last_error()
    Dm = 128
    hidden, weight = _t((T, M, Dm)), _t((V, Dm))
    rc = call(hidden, _t((V, 64)))
    assert rc == -1 and "weight must be" in _ext.last_error()
    rc = call(hidden, weight, ws_bytes=16)
    assert rc == -3 and "workspace" in _ext.last_error()
    rc = call(hidden, weight, lo=_t((T, M, V + 1)))
    assert rc == -1 and "logits_out" in _ext.last_error()
    need = dsv_lib.dsv_lmhead_accept_workspace_bytes(T, M, V)
    assert need > 0
    dsv_lib.dsv_set_dry_run(1)
    try:
        assert call(hidden, weight, ws_bytes=need, lo=_t((T, M, V))) == 0
        # a root-only tree: its parent tensor is empty and may have no storage
        h1 = _t((T, 1, Dm))
        d1, p1, q1 = _t((T, 1), _ext.DSV_I64), _t((T, 0), _ext.DSV_I64, ptr=0), _t((T, 1), _ext.DSV_I64)
        o1 = [_t((T, 1), _ext.DSV_I64), _t((T, 1), _ext.DSV_I64), _t((T, 4), _ext.DSV_I64)]
        rc = dsv_lib.dsv_lmhead_accept(1, ctypes.byref(h1), ctypes.byref(weight), ctypes.byref(d1), ctypes.byref(p1),
                                       ctypes.byref(q1), 2, 1.0, 0.09, 0.3, ctypes.byref(o1[0]), ctypes.byref(o1[1]),
                                       ctypes.byref(o1[2]), ctypes.byref(none), ctypes.byref(none),
                                       ctypes.c_void_p(0x100000), need, None)
        assert rc == 0, _ext.last_error()
    finally:
        dsv_lib.dsv_set_dry_run(0)


def test_python_api_refuses_cpu_tensors(dsv_lib):
    from diffspec_mi355x.runtime.tree_attention import prefix_attention_forward, tree_verify
    from diffspec_mi355x.draft.tree_verification import tree_accept

    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 16, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        prefix_attention_forward(q, k, k, 1, 4, 8, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        tree_verify(q, k, k, 12, torch.tensor([-1, 0, 0, 1]))
    with pytest.raises(RuntimeError, match="GPU only"):
        tree_accept(torch.zeros(1, 4, 10), torch.zeros(1, 4, dtype=torch.long), torch.zeros(1, 3, dtype=torch.long),
                    torch.arange(4), 4)

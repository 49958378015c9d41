"""ctypes binding of libdsv.so (the gfx950 kernels behind the C ABI in include/dsv.h).

Torch is imported first so that the HIP runtime torch ships is the one the
library binds to (both carry the soname libamdhip64.so.7); device pointers
and streams handed across the ABI therefore belong to one runtime.

There is no fallback: if the library is missing, or a call is made with
tensors that are not on a GPU, a RuntimeError is raised.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libdsv.so"
MAX_DIMS = 6

DSV_BF16, DSV_F16, DSV_F32, DSV_I8, DSV_U8, DSV_BOOL, DSV_I32, DSV_I64 = range(8)
ACCEPT_GREEDY, ACCEPT_TYPICAL = 0, 1

_DTYPES = {
    torch.bfloat16: DSV_BF16,
    torch.float16: DSV_F16,
    torch.float32: DSV_F32,
    torch.int8: DSV_I8,
    torch.uint8: DSV_U8,
    torch.bool: DSV_BOOL,
    torch.int32: DSV_I32,
    torch.int64: DSV_I64,
}


class DsvTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_DIMS),
        ("stride", ctypes.c_int64 * MAX_DIMS),
    ]


_P = ctypes.POINTER(DsvTensor)
_V = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# Exported symbols and their signatures (mirrors include/dsv.h).
SIGNATURES = {
    "dsv_version": (ctypes.c_int, []),
    "dsv_last_error": (ctypes.c_char_p, []),
    "dsv_set_timing_events": (ctypes.c_int, [_V, _V]),
    "dsv_set_dry_run": (ctypes.c_int, [ctypes.c_int]),
    "dsv_dry_run_checks": (_I64, []),
    "dsv_attn_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_int]),
    "dsv_prefix_attention_forward": (ctypes.c_int, [_P, _P, _P, _I64, _P, _P, _V, _SZ, _V]),
    "dsv_flash_attn_with_kvcache": (ctypes.c_int, [_P, _P, _P, _P, _I64, ctypes.c_int, _P, _P, _V, _SZ, _V]),
    "dsv_tree_attention_forward": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _V, _SZ, _V]),
    "dsv_verify_bundle": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _V, _SZ, _V]),
    "dsv_verify_bundle_paged": (ctypes.c_int, [_P, _P, _P, _I64, _P, _P, _P, _V, _SZ, _V]),
    "dsv_tree_verify": (ctypes.c_int, [_P, _P, _P, _P, _I64, _P, _P, _P, _P, _V, _SZ, _V]),
    "dsv_tree_verify_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _I64, _P, _P, _P, _P, _V]),
    "dsv_accept_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "dsv_tree_accept": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _I64, ctypes.c_float, ctypes.c_float, ctypes.c_float, _P, _P, _P, _P, _V,
         _SZ, _V],
    ),
    "dsv_tree_accept_sample": (
        ctypes.c_int,
        [_P, _P, _P, _P, _I64, ctypes.c_float, ctypes.c_float, _I64, ctypes.c_uint64, _P, _P, _P, _P, _V, _SZ, _V],
    ),
    "dsv_kv_commit": (ctypes.c_int, [_P, _P, _I64, _P, _P, _I64, _V]),
    "dsv_kv_append": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _V]),
    "dsv_bundle_order": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, _V]),
    "dsv_lmhead_accept_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "dsv_lmhead_accept": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _I64, ctypes.c_float, ctypes.c_float,
                                         ctypes.c_float, _P, _P, _P, _P, _P, _V, ctypes.c_size_t, _V]),
}

_lib: Optional[ctypes.CDLL] = None


def lib_path() -> Path:
    return Path(os.environ.get("DSV_LIB", str(LIB_PATH)))


def load() -> ctypes.CDLL:
    """Load libdsv.so once; raise with a clear message when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.exists():
        raise RuntimeError(
            f"libdsv.so not found at {path}: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or diffspec_mi355x/_build.py). There is no CPU fallback."
        )
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().dsv_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")


def desc(t: Optional[torch.Tensor]) -> DsvTensor:
    """Describe a tensor (or an absent optional argument when t is None)."""
    d = DsvTensor()
    if t is None:
        d.ndim = 0
        return d
    if t.dim() > MAX_DIMS:
        raise ValueError(f"tensors of more than {MAX_DIMS} dims are not supported")
    if t.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {t.dtype}")
    d.data = t.data_ptr() if t.numel() > 0 else (t.data_ptr() or 0)
    d.dtype = _DTYPES[t.dtype]
    d.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.shape[i] = s
        d.stride[i] = st
    return d


def require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All tensors must live on one GPU; the kernels have no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "diffspec_mi355x kernels run on the GPU only: got a tensor on "
                f"{t.device}. Move inputs to a ROCm device (there is no CPU fallback)."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor arguments")
    return dev


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch from torch's caching allocator (512-byte aligned)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def exported_symbols() -> Sequence[str]:
    return list(SIGNATURES)

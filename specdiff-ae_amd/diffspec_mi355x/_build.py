"""Build libdsv.so (the gfx950 kernels + C ABI) in-tree with hipcc.

The library is linked against the HIP runtime that ships with PyTorch
(``torch/lib/libamdhip64.so``) so that the process holds a single HIP
runtime: the one torch already loaded, whose streams and device pointers the
C ABI receives.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libdsv.so"
OBJ_DIR = LIB_DIR / "obj"

SOURCES = ["dsv_attn.hip", "dsv_attn_f32.hip", "dsv_merge.hip", "dsv_accept.hip", "dsv_sample.hip", "dsv_commit.hip", "dsv_append.hip", "dsv_bundle.hip", "dsv_lmhead.hip", "dsv_check.hip", "dsv_api.hip"]
HEADERS = ["dsv_internal.h", "dsv_attn_geo.h", "dsv_attn_f32_geo.h", "dsv_check.h", "dsv_stats.h", "dsv_dma.h"]

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libdsv.so)")


def _torch_lib_dir() -> str | None:
    try:
        import torch  # noqa: F401

        return str(Path(torch.__file__).resolve().parent / "lib")
    except Exception:
        return None


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every HIP source for gfx950 and link libdsv.so. Always rebuilds."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    inc = [f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}"]

    def compile_one(src: str) -> Path:
        obj = OBJ_DIR / (Path(src).stem + ".o")
        _run([hipcc, *COMMON_FLAGS, *inc, "-c", str(CSRC_DIR / src), "-o", str(obj)], verbose)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, SOURCES))

    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(LIB_PATH) + ".tmp"]
    tl = _torch_lib_dir()
    if tl:
        link += [f"-L{tl}", f"-Wl,-rpath,{tl}"]
    _run(link, verbose)
    os.replace(str(LIB_PATH) + ".tmp", LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)

"""Build librwkv7_hip.so: the HIP kernels and the C ABI of include/wkv7.h and include/w6a16.h, compiled for gfx950 with hipcc;
and librwkv7_noalloc.so (include/wkv7_noalloc.h), the allocation-free entry with its static device scratch array,
linked against librwkv7_hip.so so that only processes that load it hold that array.

The libraries are plain shared objects (no torch symbols); the Python layer loads them with ctypes after torch, so
they bind to the HIP runtime torch already loaded (same SONAME, libamdhip64.so.7).

    python -m rwkv_next_amd._build          (run from rwkv-infer-next_amd/)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJECT_DIR = os.path.dirname(PKG_DIR)
REPO_DIR = os.path.dirname(PROJECT_DIR)
CSRC = os.path.join(PROJECT_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "librwkv7_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
BUILD_DIR = os.path.join(PROJECT_DIR, "_build")

SOURCES = ("wkv7_recurrent.hip", "wkv7_chunked.hip", "wkv7_seg.hip", "wkv7_generic.hip", "wkv7_pool.hip",
           "wkv7_timemix.hip", "w6a16.hip", "wkv7_capi.hip")
NOALLOC_SOURCE = "wkv7_noalloc.hip"
NOALLOC_LIB_PATH = os.path.join(PKG_DIR, "librwkv7_noalloc.so")
HEADERS = ("wkv7_device.h", "wkv7_launch.h", "wkv7_token.h")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",  # explicit fmaf only: snapshots and re-runs execute identical arithmetic
    # packed fp32 instructions stay off: ordinary float code only, never v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def _link(path: str, inputs) -> None:
    tmp = path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *inputs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(path)} failed:\n{res.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = False) -> str:
    """Compile every source (always: this is the build check) and link both shared libraries in-tree."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = SOURCES + (NOALLOC_SOURCE,)
    with cf.ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(LIB_PATH, objs[:-1])
    # the allocation-free entry calls only the C ABI of librwkv7_hip.so, found next to it at run time
    _link(NOALLOC_LIB_PATH, [objs[-1], f"-L{PKG_DIR}", f"-l:{LIB_NAME}", "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {LIB_PATH} and {NOALLOC_LIB_PATH}")
    return LIB_PATH


def sources_newer_than_library() -> bool:
    if not os.path.exists(LIB_PATH):
        return True
    t = os.path.getmtime(LIB_PATH)
    files = [os.path.join(CSRC, f) for f in SOURCES + HEADERS + (NOALLOC_SOURCE,)] + \
        [os.path.join(INCLUDE, h) for h in ("wkv7.h", "w6a16.h", "wkv7_noalloc.h")]
    return any(os.path.getmtime(f) > t for f in files)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

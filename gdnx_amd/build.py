"""Build libgdnx.so (all HIP sources under csrc/) for gfx950, in-tree.

    python -m gdnx_amd.build            # or gdnx_amd.build.build()

hipcc compiles each translation unit to an object in parallel, then links the
shared library next to this file, where gdnx_amd._lib loads it from.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libgdnx.so")
OBJ = os.path.join(HERE, "_build")

ARCH = "gfx950"
# Packed fp32 VALU forms are disabled (they have produced silent wrong results
# on this pool); hipcc's host pass warns that it does not know the feature.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str, hipcc: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [hipcc, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = True) -> str:
    hipcc = _hipcc()
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = OUT + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


ASAN_OUT = os.path.join(OBJ, "asan", "libgdnx_asan.so")


def asan_runtime() -> str:
    """The shared AddressSanitizer runtime of hipcc's clang (to preload)."""
    clang = os.path.join(os.path.dirname(os.path.realpath(_hipcc())), "..", "lib", "llvm", "bin", "clang++")
    if not os.path.exists(clang):
        clang = "/opt/rocm/llvm/bin/clang++"
    r = subprocess.run([clang, "--print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return r.stdout.strip()


def build_asan(verbose: bool = False) -> str:
    """libgdnx with its host code built under AddressSanitizer and
    UndefinedBehaviorSanitizer (the device code is built as usual: the
    sanitizers apply to the host pass only), into _build/asan/.  A process
    that loads it must preload asan_runtime() first.  Used by
    tests/test_abi_asan.py to run the C ABI's argument checks and size
    arithmetic under the sanitizers on a machine without a GPU."""
    hipcc = _hipcc()
    odir = os.path.dirname(ASAN_OUT)
    os.makedirs(odir, exist_ok=True)
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
           "-Xarch_host", "-shared-libasan"]
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))

    def comp(src):
        obj = os.path.join(odir, os.path.basename(src) + ".o")
        if os.path.exists(obj) and os.path.getmtime(obj) >= max(os.path.getmtime(src), *(
                os.path.getmtime(os.path.join(CSRC, h)) for h in os.listdir(CSRC) if h.endswith(".hpp"))):
            return obj
        cmd = [hipcc, *FLAGS, "-O1", "-g", *san, "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc (sanitized) failed for {src}:\n{r.stderr[-6000:]}")
        return obj
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(comp, srcs))
    link_san = ["-shared-libasan", "-fsanitize=address,undefined", "-fno-gpu-sanitize"]   # host code only
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link_san, *objs, "-o", ASAN_OUT]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{r.stderr[-6000:]}")
    if verbose:
        print(f"built {ASAN_OUT}")
    return ASAN_OUT


if __name__ == "__main__":
    build()
    sys.exit(0)

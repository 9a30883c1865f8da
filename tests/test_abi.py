"""CPU checks of the C ABI: the library loads, exports every entry point
include/gdnx.h declares, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re

import pytest

from gdnx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for f in os.listdir(os.path.join(ROOT, "include")):
        if f.endswith(".h"):
            text = open(os.path.join(ROOT, "include", f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(gdnx_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 6
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "binding signatures out of sync with the header"


def test_abi_version_and_sizes():
    lib = _lib.load()
    assert lib.gdnx_abi_version() == _lib.ABI_VERSION
    assert lib.gdnx_delta_chunk_size(128, _lib.DTYPE_BF16) == 64
    assert lib.gdnx_delta_train_chunk_size(128, _lib.DTYPE_BF16) == 32
    assert lib.gdnx_delta_chunk_size(100, _lib.DTYPE_BF16) == 0
    # per chain and chunk: one d x d state and one C x d block of net writes, then
    # the chunk operands (T and Aq as C x C, four float32 factors per token)
    assert lib.gdnx_delta_chunk_states_bytes(4, 4096, 16, 4, 128, 64, _lib.DTYPE_BF16) == \
        4 * 16 * 4 * 64 * ((128 * 128 + 64 * 128) * 2 + 2 * 64 * 64 * 2 + 4 * 64 * 4)
    assert lib.gdnx_delta_chunk_states_bytes(1, 100, 1, 1, 64, 0, _lib.DTYPE_F32) == \
        4 * ((64 * 64 + 32 * 64) * 4 + 2 * 32 * 32 * 4 + 4 * 32 * 4)
    assert lib.gdnx_delta_fwd_workspace_bytes(1, 100, 1, 1, 64, 0, _lib.DTYPE_F32) == 4 * (2 * 32 * 32 * 4 + 4 * 32 * 4)
    assert lib.gdnx_delta_chunk_states_bytes(1, 100, 1, 1, 64, 48, _lib.DTYPE_F32) == -1


def _fwd(lib, **over):
    args = dict(q=16, k=16, v=16, ae=32, aw=32, g=32, s0=None, y=64, so=None, cs=None, ws=None,
                B=1, T=8, H=1, M=1, D=64, C=0, dt=_lib.DTYPE_F32)
    args.update(over)
    vp = lambda x: None if x is None else ctypes.c_void_p(x)
    return lib.gdnx_delta_chunk_fwd(vp(args["q"]), vp(args["k"]), vp(args["v"]), vp(args["ae"]),
                                    vp(args["aw"]), vp(args["g"]), vp(args["s0"]), vp(args["y"]),
                                    vp(args["so"]), vp(args["cs"]), vp(args["ws"]), args["B"], args["T"], args["H"],
                                    args["M"], args["D"], args["C"], args["dt"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(q=None), -1, "non-null"),
    (dict(k=24), -1, "aligned"),
    (dict(dt=7), -1, "dtype"),
    (dict(D=96), -2, "head_dim"),
    (dict(B=0), -2, "sizes"),
    (dict(C=48), -2, "chunk"),
    (dict(y=None), -1, "non-null"),
])
def test_forward_rejects_bad_arguments(over, code, msg):
    lib = _lib.load()
    rc = _fwd(lib, **over)
    assert rc == code
    assert msg in lib.gdnx_last_error().decode()


def test_backward_requires_stash_and_workspace():
    lib = _lib.load()
    vp = ctypes.c_void_p
    ptrs = [vp(16)] * 7 + [None, None, None] + [vp(16)] * 6 + [None]
    rc = lib.gdnx_delta_chunk_bwd(*ptrs, 1, 8, 1, 1, 64, 0, _lib.DTYPE_F32, None)
    assert rc == -3
    assert "workspace" in lib.gdnx_last_error().decode()

"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

libgdnx is rebuilt with its host pass sanitized (gdnx_amd.build.build_asan;
the device code is unchanged) and loaded in a child process that preloads
the ASan runtime.  The child calls every entry point declared in
include/gdnx.h through the binding's signature table with argument sets
that the entry points must refuse or size-check: null, misaligned and
fake aligned device pointers, zero, negative, huge and plausible sizes.
Any out-of-bounds access, overflow of signed size arithmetic or other
undefined behaviour in the argument checks, the size queries and the error
reporting aborts the child (UBSan does not recover) and fails the test.

The fake-pointer patterns may pass argument checking and reach a HIP call,
so this test runs only on a machine without a GPU (there every HIP call
fails cleanly with GDNX_ERR_HIP); the driver's CPU suite is such a machine.
"""
import os
import shutil
import subprocess
import sys
import textwrap

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = textwrap.dedent(r"""
    import ctypes, itertools, sys
    sys.path.insert(0, ROOT)
    from gdnx_amd import _lib
    lib = ctypes.CDLL(LIBPATH)
    vp = ctypes.c_void_p
    ptr_sets = {"null": None, "misaligned": vp(3), "aligned": vp(256)}
    int_sets = {"one": 1, "zero": 0, "neg": -1, "huge": 2 ** 30, "d128": 128, "d64": 64, "p16": 16}
    calls = 0
    for name, (res, args) in sorted(_lib.SIGNATURES.items()):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
        for (pn, pv), (iname, iv) in itertools.product(ptr_sets.items(), int_sets.items()):
            vals = []
            for a in args:
                if a is ctypes.c_void_p:
                    vals.append(pv)
                elif a in (ctypes.c_int, ctypes.c_longlong):
                    vals.append(iv)
                elif a is ctypes.c_float:
                    vals.append(0.97)
                else:
                    raise TypeError(f"{name}: argument type {a}")
            if name == "gdnx_set_check_finite":
                vals = [0]
            if name == "gdnx_gdn3_lane_rope_pairs" and pn == "aligned":
                vals[-1] = ctypes.cast((ctypes.c_int * 4)(), vp)   # a host array, not a device pointer
            rc = fn(*vals)
            calls += 1
            if res is ctypes.c_int and name not in ("gdnx_abi_version", "gdnx_set_check_finite",
                                                    "gdnx_delta_chunk_size", "gdnx_delta_train_chunk_size",
                                                    "gdnx_gdn3_num_compactions", "gdnx_gdn3_num_compactions_from",
                                                    "gdnx_gdn3_lane_rope_pairs"):
                # a compute entry point on invalid or device-less arguments: an error code
                assert rc in (-1, -2, -3, -4) or (rc == 0 and iname in ("zero", "neg")), (name, pn, iname, rc)
            lib.gdnx_last_error.restype = ctypes.c_char_p
            lib.gdnx_last_error()
    print("calls", calls)
""")


def test_abi_host_code_under_sanitizers(tmp_path):
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present: fake-pointer calls that pass argument checking would launch")
    if not shutil.which("hipcc") and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    from gdnx_amd import build
    libpath = build.build_asan()
    runtime = build.asan_runtime()
    assert os.path.exists(runtime), runtime
    script = tmp_path / "child.py"
    script.write_text(f"ROOT = {ROOT!r}\nLIBPATH = {libpath!r}\n" + CHILD)
    env = dict(os.environ, LD_PRELOAD=runtime, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-6000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-6000:]
    assert "calls" in r.stdout

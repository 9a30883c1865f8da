"""ctypes binding of libgdnx.so (the C ABI declared in include/gdnx.h).

torch is imported first so that the library's libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded (same soname): device
pointers and streams are then shared with torch.  There is no fallback: if
the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgdnx.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F64 = 2      # gdnx_check_finite only
ABI_VERSION = 12

_c_int, _c_ll, _vp, _c_float = ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); every entry point declared in include/gdnx.h
SIGNATURES = {
    "gdnx_abi_version": (_c_int, []),
    "gdnx_last_error": (ctypes.c_char_p, []),
    "gdnx_set_check_finite": (_c_int, [_c_int]),
    "gdnx_check_finite": (_c_int, [_vp, _c_ll, _c_int, _vp]),
    "gdnx_lane_sum": (_c_int, [_vp, _vp, _c_ll, _c_int, _c_int, _c_int, _vp]),
    "gdnx_delta_chunk_size": (_c_int, [_c_int, _c_int]),
    "gdnx_delta_train_chunk_size": (_c_int, [_c_int, _c_int]),
    "gdnx_delta_chunk_states_bytes": (_c_ll, [_c_int] * 7),
    "gdnx_delta_bwd_workspace_bytes": (_c_ll, [_c_int] * 7),
    "gdnx_delta_chunk_fwd": (_c_int, [_vp] * 11 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_chunk_fwd_scored": (_c_int, [_vp] * 12 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_fwd_workspace_bytes": (_c_ll, [_c_int] * 7),
    "gdnx_delta_chunk_prep": (_c_int, [_vp] * 6 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_chunk_bwd": (_c_int, [_vp] * 17 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_chunk_bwd_state": (_c_int, [_vp] * 9 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_chunk_bwd_grads": (_c_int, [_vp] * 15 + [_c_int] * 7 + [_vp]),
    "gdnx_delta_decode_step": (_c_int, [_vp] * 8 + [_c_int] * 5 + [_vp]),
    "gdnx_delta_decode_step_slots": (_c_int, [_vp] * 9 + [_c_int] * 6 + [_vp]),
    "gdnx_gdn3_workspace_bytes": (_c_ll, [_c_int] * 6),
    "gdnx_gdn3_num_compactions": (_c_int, [_c_int] * 3),
    "gdnx_gdn3_chunk_fwd": (_c_int, [_vp] * 3 + [_c_int] + [_vp] * 2 + [_c_int] + [_vp] * 10
                            + [_c_int] * 12 + [_c_float, _c_int, _c_int, _vp]),
    "gdnx_gdn3_num_compactions_from": (_c_int, [_c_int] * 4),
    "gdnx_gdn3_chunk_fwd_state": (_c_int, [_vp] * 3 + [_c_int] + [_vp] * 2 + [_c_int] + [_vp] * 6 + [_c_int]
                                  + [_vp] * 7 + [_c_int] * 12 + [_c_float, _c_int, _c_int, _vp]),
    "gdnx_gdn3_noalloc_scratch_bytes": (_c_ll, []),
    "gdnx_gdn3_chunk_fwd_state_noalloc": (_c_int, [_vp] * 3 + [_c_int] + [_vp] * 2 + [_c_int] + [_vp] * 6
                                          + [_c_int] + [_vp] * 6 + [_c_int] * 12 + [_c_float, _c_int, _c_int, _vp]),
    "gdnx_gdn3_decode_step": (_c_int, [_vp] * 3 + [_c_int] + [_vp] * 2 + [_c_int] + [_vp] * 10
                              + [_c_int] * 12 + [_c_float, _c_int, _c_int, _vp]),
    "gdnx_delta_decode_step_chan": (_c_int, [_vp] * 9 + [_c_int] * 6 + [_vp]),
    "gdnx_gdn3_train_states_bytes": (_c_ll, [_c_int] * 7),
    "gdnx_gdn3_chunk_bwd": (_c_int, [_vp] * 3 + [_c_int] + [_vp] * 2 + [_c_int] + [_vp] * 9
                            + [_c_int] * 13 + [_vp]),
    "gdnx_gdn3_compact": (_c_int, [_vp] * 8 + [_c_int] * 8 + [_c_float, _c_int, _vp]),
    "gdnx_kron_read": (_c_int, [_vp] * 6 + [_c_int] * 9 + [_vp]),
    "gdnx_gdn3_coeff": (_c_int, [_vp] * 3 + [_c_int] * 6 + [_vp]),
    "gdnx_delta_chan_states_bytes": (_c_ll, [_c_int] * 4),
    "gdnx_delta_chan_fwd_workspace_bytes": (_c_ll, [_c_int] * 4),
    "gdnx_delta_chan_fwd": (_c_int, [_vp] * 12 + [_c_int] * 4 + [_vp]),
    "gdnx_delta_chan_bwd": (_c_int, [_vp] * 17 + [_c_int] * 4 + [_vp]),
    "gdnx_gdn3_coeff_bwd": (_c_int, [_vp] * 6 + [_c_int] * 6 + [_vp]),
    "gdnx_gdn3_lane_rope_pairs": (_c_int, [_c_int, _c_int, _vp]),
    "gdnx_gdn3_prologue_fwd": (_c_int, [_vp] * 15 + [_c_int] * 6 + [_c_float, _c_int, _vp]),
    "gdnx_gdn3_prologue_bwd": (_c_int, [_vp] * 20 + [_c_int] * 6 + [_c_float, _c_int, _vp]),
    "gdnx_gdn3_epilogue_fwd": (_c_int, [_vp] * 4 + [_c_int] * 6 + [_vp]),
    "gdnx_gdn3_epilogue_workspace_bytes": (_c_ll, [_c_int] * 4),
    "gdnx_gdn3_epilogue_bwd": (_c_int, [_vp] * 8 + [_c_int] * 6 + [_vp]),
    "gdnx_rls_ckpt_bytes": (_c_ll, [_c_int] * 7),
    "gdnx_rls_fwd": (_c_int, [_vp] * 11 + [_c_int] * 7 + [_c_float, _c_int, _c_int, _c_float, _vp]),
    "gdnx_rls_bwd_workspace_bytes": (_c_ll, [_c_int] * 6),
    "gdnx_rls_bwd": (_c_int, [_vp] * 18 + [_c_int] * 7 + [_c_float, _c_int, _c_int, _c_float, _c_int, _vp, _vp]),
}


class GdnxError(RuntimeError):
    pass


class GdnxNonFinite(GdnxError):
    """A recurrence's outputs held NaN or infinity (GDNX_ERR_NONFINITE, only
    with set_check_finite(True)): the counterpart of the reference trainer's
    guard that drops such a step (train/train_gdn3_distill.py:329-354)."""


ERR_NONFINITE = -5


_lib = None


def load():
    """Load and bind libgdnx.so once; raises GdnxError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise GdnxError(f"{LIB_PATH} is not built; run `python -m gdnx_amd.build` "
                        "(there is no non-HIP fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.gdnx_abi_version() != ABI_VERSION:
        raise GdnxError(f"ABI version mismatch: library {lib.gdnx_abi_version()}, "
                        f"binding {ABI_VERSION}")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().gdnx_last_error().decode(errors="replace")
        cls = GdnxNonFinite if rc == ERR_NONFINITE else GdnxError
        raise cls(f"{what} failed ({rc}): {msg}")


def set_check_finite(on: bool) -> bool:
    """Turn the library's non-finite checking on or off (process-wide;
    gdnx_set_check_finite).  When on, every recurrence call scans its outputs
    and synchronises its stream, raising GdnxNonFinite on NaN or infinity.
    Returns the previous setting."""
    return bool(load().gdnx_set_check_finite(1 if on else 0))


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def dtype_code(dt) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise GdnxError(f"unsupported io dtype {dt} (bfloat16 or float32)")

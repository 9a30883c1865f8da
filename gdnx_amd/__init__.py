"""gdnx_amd -- MI355X-native (gfx950) chunked GDN3 / KMD-2 recurrence.

Hand-written HIP kernels behind a C ABI (include/gdnx.h, libgdnx.so), bound
with ctypes and wrapped as torch.autograd.Functions that keep the reference's
call signatures.  There is no CPU or Triton fallback: ops raise if the HIP
library is not built.
"""
from . import _lib, gdn3, kmd2, layer, ops, rls  # noqa: F401

__all__ = ["ops", "gdn3", "kmd2", "layer", "rls"]

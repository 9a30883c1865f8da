"""Torch-facing wrappers of the libgdnx kernels (device memory and streams
come from torch; all arithmetic runs in the HIP kernels).

Shapes follow include/gdnx.h: q, k, v [B,T,H,D] shared by the M lanes of a
head; per-lane per-token float32 scalars a_e, a_w, log_g [B,T,H,M]; outputs
y [B,T,H,M,D]; states [B,H,M,D,D] key-major.
"""
from __future__ import annotations

import torch

from . import _lib


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _check_dense(q, k, v, a_e, a_w, log_g):
    _need(q.is_cuda, "gdnx ops need CUDA (HIP) tensors")
    _need(q.dim() == 4 and q.shape == k.shape == v.shape, "q, k, v must share shape [B,T,H,D]")
    _need(q.dtype == k.dtype == v.dtype, "q, k, v must share dtype")
    B, T, H, D = q.shape
    _need(a_e.dim() == 4 and a_e.shape[:3] == (B, T, H), "a_e must be [B,T,H,M]")
    _need(a_e.shape == a_w.shape == log_g.shape, "a_e, a_w, log_g must share shape")
    for t in (a_e, a_w, log_g):
        _need(t.dtype == torch.float32, "a_e, a_w, log_g must be float32")
    for t in (q, k, v, a_e, a_w, log_g):
        _need(t.is_contiguous(), "inputs must be contiguous")
        _need(t.device == q.device, "inputs must be on one device")
    return B, T, H, a_e.shape[3], D


def chunk_size(head_dim: int, dtype) -> int:
    return _lib.load().gdnx_delta_chunk_size(head_dim, _lib.dtype_code(dtype))


def delta_chunk_fwd(q, k, v, a_e, a_w, log_g, state0=None, *, return_state=False,
                    save_states=False):
    """Forward of the lane-shared decoupled-erase delta rule.

    Returns (y, state_out or None, chunk_states or None)."""
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, v, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    if state0 is not None:
        _need(state0.shape == (B, H, M, D, D) and state0.dtype == torch.float32
              and state0.is_contiguous(), "state0 must be contiguous float32 [B,H,M,D,D]")
    dev = q.device
    y = torch.empty(B, T, H, M, D, dtype=q.dtype, device=dev)
    s_out = torch.empty(B, H, M, D, D, dtype=torch.float32, device=dev) if return_state else None
    cs = None
    if save_states:
        nbytes = lib.gdnx_delta_chunk_states_bytes(B, T, H, M, D, code)
        cs = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.gdnx_delta_chunk_fwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
            _lib.ptr(state0), _lib.ptr(y), _lib.ptr(s_out), _lib.ptr(cs),
            B, T, H, M, D, code, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chunk_fwd")
    return y, s_out, cs

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


def empty_result(shape, dtype, device, *srcs):
    """Zeros of ``shape`` for a call over an empty sequence (T = 0), attached to
    the autograd graph of ``srcs`` so that backward gives their (zero or empty)
    gradients, as the equivalent torch ops on empty tensors would."""
    z = torch.zeros(shape, dtype=dtype, device=device)
    if torch.is_grad_enabled():
        for s in srcs:
            if s is not None and s.requires_grad:
                z = z + (s.sum() * 0).to(dtype)
    return z


def _check_dense(q, k, v, a_e, a_w, log_g):
    _need(q.is_cuda, "gdnx ops need CUDA (HIP) tensors")
    _need(q.dim() == 4 and q.shape == k.shape == v.shape, "q, k, v must share shape [B,T,H,D]")
    _need(q.dtype == k.dtype == v.dtype, "q, k, v must share dtype")
    B, T, H, D = q.shape
    _need(a_e.dim() == 4 and tuple(a_e.shape[:3]) == (B, T, H), "a_e must be [B,T,H,M]")
    _need(a_e.shape == a_w.shape == log_g.shape, "a_e, a_w, log_g must share shape")
    for t in (a_e, a_w, log_g):
        _need(t.dtype == torch.float32, "a_e, a_w, log_g must be float32")
    for t in (q, k, v, a_e, a_w, log_g):
        _need(t.is_contiguous(), "inputs must be contiguous")
        _need(t.device == q.device, "inputs must be on one device")
    return B, T, H, a_e.shape[3], D


def chunk_size(head_dim: int, dtype, train: bool = False) -> int:
    lib = _lib.load()
    fn = lib.gdnx_delta_train_chunk_size if train else lib.gdnx_delta_chunk_size
    return fn(head_dim, _lib.dtype_code(dtype))


def forward_plan(head_dim: int, dtype, train: bool, scored: bool = False):
    """(chunk, two_pass) of the forward the autograd wrappers run.

    Training stashes for the backward (two-pass, the training chunk).  For
    inference with bf16 IO the two-pass form at the training chunk (32) is
    also the fastest: the config-1 forward (B=4, T=4096, H=16, d=128, 4
    lanes) measured 0.42 ms against 0.70 ms for the fused single-kernel scan
    at 64 and 0.64 ms for the two-pass form at 64.  The scored variant
    (|r_t| per token) and float32 IO keep the fused scan at the inference
    chunk."""
    if train:
        return chunk_size(head_dim, dtype, train=True), True
    if dtype == torch.bfloat16 and not scored:
        return chunk_size(head_dim, dtype, train=True), True
    return chunk_size(head_dim, dtype), False


def delta_chunk_fwd(q, k, v, a_e, a_w, log_g, state0=None, *, return_state=False,
                    save_states=False, chunk=0, r_norm=None, two_pass=False):
    """Forward of the lane-shared decoupled-erase delta rule.

    r_norm: optional float32 [B,T,H,M] output receiving |r_t| (the norm of
    each token's net write).  two_pass: without save_states, still run the
    parallel chunk-operand pass plus the value-split scan (it needs a
    workspace) rather than the fused single-kernel scan; with save_states
    the two-pass form is always used.  Returns (y, state_out or None,
    chunk_states or None)."""
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, v, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    if state0 is not None:
        _need(tuple(state0.shape) == (B, H, M, D, D) and state0.dtype == torch.float32
              and state0.is_contiguous(), "state0 must be contiguous float32 [B,H,M,D,D]")
    dev = q.device
    y = torch.empty(B, T, H, M, D, dtype=q.dtype, device=dev)
    s_out = torch.empty(B, H, M, D, D, dtype=torch.float32, device=dev) if return_state else None
    cs = None
    if save_states:
        nbytes = lib.gdnx_delta_chunk_states_bytes(B, T, H, M, D, chunk, code)
        _need(nbytes >= 0, f"invalid chunk {chunk} for {q.dtype}")
        cs = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    ws = None
    if two_pass and not save_states:   # (the stash holds the chunk operands otherwise)
        nws = lib.gdnx_delta_fwd_workspace_bytes(B, T, H, M, D, chunk, code)
        _need(nws >= 0, f"invalid chunk {chunk} for {q.dtype}")
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        if r_norm is None:
            rc = lib.gdnx_delta_chunk_fwd(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
                _lib.ptr(state0), _lib.ptr(y), _lib.ptr(s_out), _lib.ptr(cs), _lib.ptr(ws),
                B, T, H, M, D, chunk, code, _lib.stream_of(q))
        else:
            _need(tuple(r_norm.shape) == (B, T, H, M) and r_norm.dtype == torch.float32
                  and r_norm.is_contiguous(), "r_norm must be contiguous float32 [B,T,H,M]")
            rc = lib.gdnx_delta_chunk_fwd_scored(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
                _lib.ptr(state0), _lib.ptr(y), _lib.ptr(s_out), _lib.ptr(cs), _lib.ptr(r_norm), _lib.ptr(ws),
                B, T, H, M, D, chunk, code, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chunk_fwd")
    return y, s_out, cs


def delta_chunk_prep(q, k, a_e, a_w, log_g, *, chunk=0, ws=None):
    """The intra-chunk phase alone (gdnx_delta_chunk_prep): every chunk's
    state-independent operands (T = (I + L)^-1, decay-masked Q K^T, per-token
    factors) into a uint8 workspace, which is returned (pass ``ws`` to reuse
    one of gdnx_delta_fwd_workspace_bytes bytes)."""
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, k, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    nws = lib.gdnx_delta_fwd_workspace_bytes(B, T, H, M, D, chunk, code)
    _need(nws >= 0, f"invalid chunk {chunk} for {q.dtype}")
    if ws is None:
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=q.device)
    _need(ws.dtype == torch.uint8 and ws.numel() >= nws and ws.is_contiguous(), "ws too small")
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_chunk_prep(_lib.ptr(q), _lib.ptr(k), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
                                       _lib.ptr(ws), B, T, H, M, D, chunk, code, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chunk_prep")
    return ws


def delta_chunk_bwd(q, k, v, a_e, a_w, log_g, dy, chunk_states, chunk, dstate_out=None,
                    want_dstate0=False):
    """Backward; returns (dq, dk, dv, da_e, da_w, dlog_g, dstate0 or None)."""
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, v, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    dy = dy.to(q.dtype).contiguous()
    _need(tuple(dy.shape) == (B, T, H, M, D), "dy must be [B,T,H,M,D]")
    if dstate_out is not None:
        dstate_out = dstate_out.float().contiguous()
        _need(tuple(dstate_out.shape) == (B, H, M, D, D), "dstate_out must be [B,H,M,D,D]")
    dev = q.device
    ws = torch.empty(max(lib.gdnx_delta_bwd_workspace_bytes(B, T, H, M, D, chunk, code), 16), dtype=torch.uint8,
                     device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    da_e, da_w, dlg = torch.empty_like(a_e), torch.empty_like(a_w), torch.empty_like(log_g)
    ds0 = torch.empty(B, H, M, D, D, dtype=torch.float32, device=dev) if want_dstate0 else None
    with torch.cuda.device(dev):
        rc = lib.gdnx_delta_chunk_bwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
            _lib.ptr(dy), _lib.ptr(dstate_out), _lib.ptr(chunk_states), _lib.ptr(ws),
            _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(da_e), _lib.ptr(da_w), _lib.ptr(dlg),
            _lib.ptr(ds0), B, T, H, M, D, chunk, code, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chunk_bwd")
    return dq, dk, dv, da_e, da_w, dlg, ds0


class DeltaRuleFunction(torch.autograd.Function):
    """y, S_T (and, when asked, the detached net-write norms |r_t|) of the
    lane-shared decoupled-erase delta rule, differentiable in q, k, v, a_e,
    a_w, log_g and state0."""

    @staticmethod
    def forward(ctx, q, k, v, a_e, a_w, log_g, state0=None, want_rnorm=False):
        train = any(ctx.needs_input_grad)
        # an unused output's gradient arrives as None (no zero tensor is filled)
        ctx.set_materialize_grads(False)
        D = q.shape[-1]
        chunk, two_pass = forward_plan(D, q.dtype, train, scored=want_rnorm)
        rn = torch.empty(a_e.shape, dtype=torch.float32, device=q.device) if want_rnorm else None
        y, s_out, cs = delta_chunk_fwd(q, k, v, a_e, a_w, log_g, state0, return_state=True,
                                       save_states=train, chunk=chunk, r_norm=rn, two_pass=two_pass)
        if train:
            ctx.save_for_backward(q, k, v, a_e, a_w, log_g, cs)
            ctx.chunk = chunk
            ctx.has_state0 = state0 is not None
        if rn is None:
            return y, s_out
        ctx.mark_non_differentiable(rn)
        return y, s_out, rn

    @staticmethod
    def backward(ctx, dy, ds_out, *unused):
        q, k, v, a_e, a_w, log_g, cs = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros(*a_e.shape, q.shape[-1], dtype=q.dtype, device=q.device)
        dq, dk, dv, dae, daw, dlg, ds0 = delta_chunk_bwd(
            q, k, v, a_e, a_w, log_g, dy, cs, ctx.chunk, dstate_out=ds_out,
            want_dstate0=ctx.has_state0 and ctx.needs_input_grad[6])
        return dq, dk, dv, dae, daw, dlg, ds0, None


def delta_rule(q, k, v, a_e, a_w, log_g, state0=None, want_rnorm=False):
    """Differentiable lane-shared delta rule; returns (y, final_state) and,
    with want_rnorm, the detached per-token net-write norms |r_t| [B,T,H,M]."""
    args = [t.contiguous() for t in (q, k, v)] + [t.float().contiguous() for t in (a_e, a_w, log_g)]
    if state0 is not None:
        state0 = state0.float().contiguous()
    return DeltaRuleFunction.apply(*args, state0, want_rnorm)


def delta_chunk_bwd_stages(q, k, v, a_e, a_w, log_g, dy, chunk_states, chunk, ws=None, out=None):
    """The two backward stages as separate launches (for timing and
    profiling).  Returns (workspace, (dq, dk, dv, da_e, da_w, dlog_g))."""
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, v, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    st = _lib.stream_of(q)
    if ws is None:
        ws = torch.empty(max(lib.gdnx_delta_bwd_workspace_bytes(B, T, H, M, D, chunk, code), 16), dtype=torch.uint8,
                         device=q.device)
    if out is None:
        out = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
               torch.empty_like(a_e), torch.empty_like(a_w), torch.empty_like(log_g))
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_chunk_bwd_state(_lib.ptr(q), _lib.ptr(k), _lib.ptr(a_e), _lib.ptr(log_g),
                                            _lib.ptr(dy), None, _lib.ptr(chunk_states), _lib.ptr(ws), None,
                                            B, T, H, M, D, chunk, code, st)
    _lib.check(rc, "gdnx_delta_chunk_bwd_state")
    return ws, out


def delta_chunk_bwd_grads(q, k, v, a_e, a_w, log_g, dy, chunk_states, ws, chunk, out):
    lib = _lib.load()
    B, T, H, M, D = _check_dense(q, k, v, a_e, a_w, log_g)
    code = _lib.dtype_code(q.dtype)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_chunk_bwd_grads(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w), _lib.ptr(log_g),
            _lib.ptr(dy), _lib.ptr(chunk_states), _lib.ptr(ws), *(_lib.ptr(t) for t in out),
            B, T, H, M, D, chunk, code, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chunk_bwd_grads")
    return out


def _decode_out(out, shape, dtype, device):
    """The y buffer of a decode step: a new tensor, or the caller's ``out``
    after checking that the kernel can write it as [NS,H,M,D] contiguous."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _need(tuple(out.shape) == tuple(shape), f"out must be {list(shape)}, got {list(out.shape)}")
    _need(out.dtype == dtype, f"out must be {dtype}, got {out.dtype}")
    _need(out.is_contiguous(), "out must be contiguous")
    _need(out.device == device, "out must be on q's device")
    return out


def delta_decode_step(q, k, v, a_e, a_w, log_g, state, out=None):
    """One-token decode step (state updated in place).

    q, k, v [NS, H, D] (bf16/float32, shared by the M chains of a head);
    a_e, a_w, log_g [NS, H, M] float32; state [NS, H, M, D, D] float32.
    Returns y [NS, H, M, D] in q's dtype."""
    lib = _lib.load()
    _need(q.is_cuda and q.dim() == 3 and q.shape == k.shape == v.shape, "q, k, v must be [NS,H,D] on GPU")
    NS, H, D = q.shape
    _need(a_e.dim() == 3 and tuple(a_e.shape[:2]) == (NS, H), "a_e must be [NS,H,M]")
    M = a_e.shape[2]
    _need(a_e.shape == a_w.shape == log_g.shape, "a_e, a_w, log_g must share shape")
    _need(tuple(state.shape) == (NS, H, M, D, D) and state.dtype == torch.float32, "state must be fp32 [NS,H,M,D,D]")
    for t in (q, k, v, a_e, a_w, log_g, state):
        _need(t.is_contiguous(), "inputs must be contiguous")
        _need(t.device == q.device, "inputs and state must be on one device")
    for t in (a_e, a_w, log_g):
        _need(t.dtype == torch.float32, "a_e, a_w, log_g must be float32")
    _need(k.dtype == v.dtype == q.dtype, "q, k, v must share dtype")
    y = _decode_out(out, (NS, H, M, D), q.dtype, q.device)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_decode_step(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w),
                                        _lib.ptr(log_g), _lib.ptr(state), _lib.ptr(y), NS, H, M, D,
                                        _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_decode_step")
    return y


def delta_decode_step_slots(q, k, v, a_e, a_w, log_g, state_pool, slots, out=None):
    """One-token decode step on a state pool (gdnx_delta_decode_step_slots):
    row s of q, k, v [NS,H,D] and a_e, a_w, log_g [NS,H,M] updates
    state_pool[slots[s]] ([n_slots,H,M,D,D] float32) in place; slots is an
    int32 device tensor [NS] (a slot outside [0, n_slots) marks an empty row:
    y = 0, no state touched).  Returns y [NS,H,M,D] in q's dtype."""
    lib = _lib.load()
    _need(q.is_cuda and q.dim() == 3 and q.shape == k.shape == v.shape, "q, k, v must be [NS,H,D] on GPU")
    NS, H, D = q.shape
    _need(a_e.dim() == 3 and tuple(a_e.shape[:2]) == (NS, H), "a_e must be [NS,H,M]")
    M = a_e.shape[2]
    _need(a_e.shape == a_w.shape == log_g.shape, "a_e, a_w, log_g must share shape")
    _need(state_pool.dim() == 5 and tuple(state_pool.shape[1:]) == (H, M, D, D)
          and state_pool.dtype == torch.float32, "state_pool must be fp32 [n_slots,H,M,D,D]")
    _need(slots.dtype == torch.int32 and tuple(slots.shape) == (NS,) and slots.device == q.device,
          "slots must be an int32 device tensor [NS]")
    for t in (q, k, v, a_e, a_w, log_g, state_pool, slots):
        _need(t.is_contiguous(), "inputs must be contiguous")
        _need(t.device == q.device, "inputs, state_pool and slots must be on one device")
    for t in (a_e, a_w, log_g):
        _need(t.dtype == torch.float32, "a_e, a_w, log_g must be float32")
    _need(k.dtype == v.dtype == q.dtype, "q, k, v must share dtype")
    y = _decode_out(out, (NS, H, M, D), q.dtype, q.device)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_decode_step_slots(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w),
                                              _lib.ptr(log_g), _lib.ptr(state_pool), _lib.ptr(slots), _lib.ptr(y),
                                              NS, state_pool.shape[0], H, M, D, _lib.dtype_code(q.dtype),
                                              _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_decode_step_slots")
    return y


def delta_decode_step_chan(q, k, v, a_e, a_w, log_g, state_pool, slots=None, out=None):
    """One-token decode step with a log-decay per key channel
    (gdnx_delta_decode_step_chan): q, k, v [NS,H,D]; a_e, a_w [NS,H,M];
    log_g [NS,H,M,D]; state_pool [n_slots,H,M,D,D] float32 updated in place
    (row s updates slot slots[s], an int32 device tensor [NS], or state s
    when slots is None).  Returns y [NS,H,M,D] in q's dtype."""
    lib = _lib.load()
    _need(q.is_cuda and q.dim() == 3 and q.shape == k.shape == v.shape, "q, k, v must be [NS,H,D] on GPU")
    _need(k.dtype == v.dtype == q.dtype, "q, k, v must share dtype")
    NS, H, D = q.shape
    _need(a_e.dim() == 3 and tuple(a_e.shape[:2]) == (NS, H) and a_e.shape == a_w.shape, "a_e, a_w must be [NS,H,M]")
    M = a_e.shape[2]
    _need(tuple(log_g.shape) == (NS, H, M, D), "log_g must be [NS,H,M,D]")
    _need(state_pool.dim() == 5 and tuple(state_pool.shape[1:]) == (H, M, D, D)
          and state_pool.dtype == torch.float32, "state_pool must be fp32 [n_slots,H,M,D,D]")
    if slots is None:
        _need(state_pool.shape[0] == NS, "without slots the state must be [NS,H,M,D,D]")
    else:
        _need(slots.dtype == torch.int32 and tuple(slots.shape) == (NS,), "slots must be an int32 tensor [NS]")
    for t in (q, k, v, a_e, a_w, log_g, state_pool) + ((slots,) if slots is not None else ()):
        _need(t.is_contiguous(), "inputs must be contiguous")
        _need(t.device == q.device, "inputs, state_pool and slots must be on one device")
    for t in (a_e, a_w, log_g):
        _need(t.dtype == torch.float32, "a_e, a_w, log_g must be float32")
    y = _decode_out(out, (NS, H, M, D), q.dtype, q.device)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_decode_step_chan(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(a_e), _lib.ptr(a_w),
                                             _lib.ptr(log_g), _lib.ptr(state_pool), _lib.ptr(slots), _lib.ptr(y),
                                             NS, state_pool.shape[0], H, M, D, _lib.dtype_code(q.dtype),
                                             _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_decode_step_chan")
    return y


# ---------------------------------------------------------------------------
# per-key-channel decay (the general KMD-2 scan), float32, one chain per head
# ---------------------------------------------------------------------------
def _check_chan(q, k, v, beta_e, beta_w, log_g):
    _need(q.is_cuda, "gdnx ops need CUDA (HIP) tensors")
    _need(q.dim() == 4 and q.shape == k.shape == v.shape == log_g.shape, "q, k, v, log_g must be [B,T,H,D]")
    _need(beta_e.shape == beta_w.shape == q.shape[:3], "beta_e, beta_w must be [B,T,H]")
    for t in (q, k, v, beta_e, beta_w, log_g):
        _need(t.dtype == torch.float32 and t.is_contiguous() and t.device == q.device,
              "per-channel decay tensors must be contiguous float32 on one device")
    return q.shape


def delta_chan_fwd(q, k, v, beta_e, beta_w, log_g, state0=None, *, save_states=False, r_norm=None):
    """Forward with a decay per key channel (gdnx_delta_chan_fwd).  Returns
    (y [B,T,H,D], state_out [B,H,D,D], chunk_states or None)."""
    lib = _lib.load()
    B, T, H, D = _check_chan(q, k, v, beta_e, beta_w, log_g)
    if state0 is not None:
        _need(tuple(state0.shape) == (B, H, D, D) and state0.dtype == torch.float32 and state0.is_contiguous(),
              "state0 must be contiguous float32 [B,H,D,D]")
    if r_norm is not None:
        _need(r_norm.shape == q.shape[:3] and r_norm.dtype == torch.float32 and r_norm.is_contiguous(),
              "r_norm must be contiguous float32 [B,T,H]")
    y = torch.empty_like(q)
    s_out = torch.empty(B, H, D, D, dtype=torch.float32, device=q.device)
    cs = ws = None
    if save_states:
        cs = torch.empty(max(lib.gdnx_delta_chan_states_bytes(B, T, H, D), 16), dtype=torch.uint8, device=q.device)
    else:
        ws = torch.empty(max(lib.gdnx_delta_chan_fwd_workspace_bytes(B, T, H, D), 16), dtype=torch.uint8,
                         device=q.device)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_chan_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta_e), _lib.ptr(beta_w),
                                     _lib.ptr(log_g), _lib.ptr(state0), _lib.ptr(y), _lib.ptr(s_out), _lib.ptr(cs),
                                     _lib.ptr(ws), _lib.ptr(r_norm), B, T, H, D, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chan_fwd")
    return y, s_out, cs


def delta_chan_bwd(q, k, v, beta_e, beta_w, log_g, dy, chunk_states, dstate_out=None, want_dstate0=False):
    """Backward of delta_chan_fwd: (dq, dk, dv, dbeta_e, dbeta_w, dlog_g, dstate0 or None)."""
    lib = _lib.load()
    B, T, H, D = _check_chan(q, k, v, beta_e, beta_w, log_g)
    dy = dy.float().contiguous()
    if dstate_out is not None:
        dstate_out = dstate_out.float().contiguous()
    ws = torch.empty_like(chunk_states)
    dq, dk, dv, dlg = (torch.empty_like(q) for _ in range(4))
    dbe, dbw = torch.empty_like(beta_e), torch.empty_like(beta_w)
    ds0 = torch.empty(B, H, D, D, dtype=torch.float32, device=q.device) if want_dstate0 else None
    with torch.cuda.device(q.device):
        rc = lib.gdnx_delta_chan_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(beta_e), _lib.ptr(beta_w),
                                     _lib.ptr(log_g), _lib.ptr(dy), _lib.ptr(dstate_out), _lib.ptr(chunk_states),
                                     _lib.ptr(ws), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dbe),
                                     _lib.ptr(dbw), _lib.ptr(dlg), _lib.ptr(ds0), B, T, H, D, _lib.stream_of(q))
    _lib.check(rc, "gdnx_delta_chan_bwd")
    return dq, dk, dv, dbe, dbw, dlg, ds0


class ChanRuleFunction(torch.autograd.Function):
    """y, S_T (and, when asked, the detached |r_t|) of the delta rule with a
    decay per key channel, differentiable in q, k, v, beta_e, beta_w, log_g
    and state0."""

    @staticmethod
    def forward(ctx, q, k, v, beta_e, beta_w, log_g, state0=None, want_rnorm=False):
        train = any(ctx.needs_input_grad)
        # an unused output's gradient arrives as None (no zero tensor is filled)
        ctx.set_materialize_grads(False)
        rn = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device) if want_rnorm else None
        y, s_out, cs = delta_chan_fwd(q, k, v, beta_e, beta_w, log_g, state0, save_states=train, r_norm=rn)
        if train:
            ctx.save_for_backward(q, k, v, beta_e, beta_w, log_g, cs)
            ctx.has_state0 = state0 is not None
        if rn is None:
            return y, s_out
        ctx.mark_non_differentiable(rn)
        return y, s_out, rn

    @staticmethod
    def backward(ctx, dy, ds_out, *unused):
        q, k, v, be, bw, lg, cs = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(q)
        dq, dk, dv, dbe, dbw, dlg, ds0 = delta_chan_bwd(q, k, v, be, bw, lg, dy, cs, dstate_out=ds_out,
                                                        want_dstate0=ctx.has_state0 and ctx.needs_input_grad[6])
        return dq, dk, dv, dbe, dbw, dlg, ds0, None


def delta_rule_chan(q, k, v, beta_e, beta_w, log_g, state0=None, want_rnorm=False):
    """Differentiable delta rule with a per-key-channel log-decay log_g
    [B,T,H,D] (one chain per head, float32 arithmetic); returns (y, S_T) and,
    with want_rnorm, the detached |r_t| [B,T,H]."""
    args = [t.float().contiguous() for t in (q, k, v, beta_e, beta_w, log_g)]
    if state0 is not None:
        state0 = state0.float().contiguous()
    return ChanRuleFunction.apply(*args, state0, want_rnorm)


def gdn3_coeff(k, beta):
    """a = alpha(beta |k|^2) beta [B,T,H,M] float32 (gdnx_gdn3_coeff) for k
    [B,T,H,D] (bf16/float32, shared by the M lanes) and beta [B,T,H,M]."""
    lib = _lib.load()
    _need(k.is_cuda and k.dim() == 4 and k.is_contiguous(), "k must be contiguous [B,T,H,D] on the GPU")
    _need(beta.dim() == 4 and tuple(beta.shape[:3]) == tuple(k.shape[:3]) and beta.dtype == torch.float32
          and beta.is_contiguous(), "beta must be contiguous float32 [B,T,H,M]")
    B, T, H, D = k.shape
    M = beta.shape[3]
    a = torch.empty_like(beta)
    with torch.cuda.device(k.device):
        rc = lib.gdnx_gdn3_coeff(_lib.ptr(k), _lib.ptr(beta), _lib.ptr(a), B, T, H, M, D,
                                 _lib.dtype_code(k.dtype), _lib.stream_of(k))
    _lib.check(rc, "gdnx_gdn3_coeff")
    return a


def gdn3_coeff_bwd(k, beta, da_e, da_w, dk):
    """Backward of gdn3_coeff: returns dbeta; adds the key gradient into dk
    (in place)."""
    lib = _lib.load()
    B, T, H, D = k.shape
    M = beta.shape[3]
    for t in (da_e, da_w):
        _need(t is None or (t.shape == beta.shape and t.dtype == torch.float32 and t.is_contiguous()),
              "da_e / da_w must be contiguous float32 like beta")
    _need(dk.shape == k.shape and dk.dtype == k.dtype and dk.is_contiguous(), "dk must match k")
    dbeta = torch.empty_like(beta)
    with torch.cuda.device(k.device):
        rc = lib.gdnx_gdn3_coeff_bwd(_lib.ptr(k), _lib.ptr(beta), _lib.ptr(da_e), _lib.ptr(da_w), _lib.ptr(dk),
                                     _lib.ptr(dbeta), B, T, H, M, D, _lib.dtype_code(k.dtype), _lib.stream_of(k))
    _lib.check(rc, "gdnx_gdn3_coeff_bwd")
    return dbeta


# ---------------------------------------------------------------------------
# GDN3 Kronecker-residual regime
# ---------------------------------------------------------------------------
def _geom(A, Bk):
    N, R, a_v, a_k = A.shape
    b_v, b_k = Bk.shape[-2:]
    return N, R, a_v, a_k, b_v, b_k


COMPACT_MODES = {"svd": 0, "sketch": 1, "sketch_noqr": 1}


def compact_mode_code(mode) -> int:
    """The ABI's compact_mode for a reference mode name (gdn3/gdn3_upgrade.py:
    579-592 runs 'sketch' and 'sketch_noqr' through one branch), or an int."""
    if isinstance(mode, int):
        _need(mode in (0, 1), f"compact_mode {mode} must be 0 (svd) or 1 (sketch)")
        return mode
    key = str(mode).lower()
    _need(key in COMPACT_MODES, f"compact_mode {mode!r} must be one of {sorted(COMPACT_MODES)}")
    return COMPACT_MODES[key]


def sketch_width(R, m, n, mode=0):
    """Columns of the compaction sketch: min(R + 4, m, n) for svd
    (gdn3/gdn3_upgrade.py:677), R for the sketch modes (:580)."""
    return R if compact_mode_code(mode) == 1 else min(R + 4, m, n)


def kron_read(A, Bk, U, Vb, x):
    """S x for S = sum_r A_r (x) B_r + U Vb^T (gdnx_kron_read).

    A [N,R,a_v,a_k], Bk [N,R,b_v,b_k], U [N,V,P], Vb [N,K,P], x [N,K] or
    [N,C,K]; float32 on the GPU.  Returns float32 [N,V] or [N,C,V]."""
    lib = _lib.load()
    N, R, a_v, a_k, b_v, b_k = _geom(A, Bk)
    D = a_v * b_v
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(1) if squeeze else x
    C = x3.shape[1]
    P = U.shape[-1]
    for t in (A, Bk, U, Vb, x3):
        _need(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(),
              "kron_read inputs must be contiguous float32 on the GPU")
    _need(tuple(U.shape) == (N, D, P) and tuple(Vb.shape) == (N, D, P) and x3.shape[0] == N
          and x3.shape[2] == D, "inconsistent kron_read shapes")
    y = torch.empty(N, C, D, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.gdnx_kron_read(_lib.ptr(A), _lib.ptr(Bk), _lib.ptr(U), _lib.ptr(Vb), _lib.ptr(x3), _lib.ptr(y),
                                N, C, D, R, P, a_v, a_k, b_v, b_k, _lib.stream_of(x))
    _lib.check(rc, "gdnx_kron_read")
    return y[:, 0] if squeeze else y


def gdn3_compact(A, Bk, U, Vb, sketch, slow_decay=0.97, compact_mode="svd"):
    """One rearrangement-SVD compaction per chain (gdnx_gdn3_compact).

    Returns (A_new, B_new, stats [N,2] float64 = (|R_mat|^2, kept sigma^2));
    the reference's error is max(0, sum_n stats[:,0] - sum_n stats[:,1]).
    compact_mode 'sketch' / 'sketch_noqr' (sketch [N, b_v*b_k, R]): one
    sketched product, error 0 (stats = (|R_mat|^2, |R_mat|^2))."""
    cm = compact_mode_code(compact_mode)
    lib = _lib.load()
    N, R, a_v, a_k, b_v, b_k = _geom(A, Bk)
    D = a_v * b_v
    P = U.shape[-1]
    for t in (A, Bk, U, Vb, sketch):
        _need(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(),
              "compaction inputs must be contiguous float32 on the GPU")
    _need(tuple(sketch.shape) == (N, b_v * b_k, sketch_width(R, a_v * a_k, b_v * b_k, cm)), "bad sketch shape")
    A_new, B_new = torch.empty_like(A), torch.empty_like(Bk)
    stats = torch.empty(N, 2, dtype=torch.float64, device=A.device)
    with torch.cuda.device(A.device):
        rc = lib.gdnx_gdn3_compact(_lib.ptr(A), _lib.ptr(Bk), _lib.ptr(U), _lib.ptr(Vb), _lib.ptr(sketch),
                                   _lib.ptr(A_new), _lib.ptr(B_new), _lib.ptr(stats), N, D, R, P,
                                   a_v, a_k, b_v, b_k, float(slow_decay), cm, _lib.stream_of(A))
    _lib.check(rc, "gdnx_gdn3_compact")
    return A_new, B_new, stats


def _g3_state_check(state, N, R, factors, D, P, device):
    a_v, a_k, b_v, b_k = factors
    shapes = ((N, R, a_v, a_k), (N, R, b_v, b_k), (N, D, P), (N, D, P))
    _need(len(state) == 4, "state must be (A, B, U, Vb)")
    for t, shp, name in zip(state, shapes, ("A", "B", "U", "Vb")):
        _need(tuple(t.shape) == shp, f"state {name} must be {list(shp)}, got {list(t.shape)}")
        _need(t.dtype == torch.float32 and t.is_contiguous() and t.device == device,
              f"state {name} must be contiguous float32 on the inputs' device")


def gdn3_chunk_fwd(q, k, v, b_gates, w_gates, decay, sketch, *, M, R=4, P=16,
                   factors=(16, 16, 8, 8), slow_decay=0.97, compact_every=None, return_state=False,
                   save_states=False, state0=None, t0=0, compact_mode="svd"):
    """GDN3 recurrence with residual window and compaction (gdnx_gdn3_chunk_fwd).

    q, k, v: [B,T,H,D] (shared by the M lanes) or [B,T,H,M,D] (per lane),
    bf16 or float32, contiguous.  b_gates, w_gates: [B,T,H,M] (scalar per
    lane) or [B,T,H,M,D] float32.  decay [B,T,H,M] float32.  sketch
    [B*H*M, b_v*b_k, q] float32.  Returns (y [B,T,H,M,D] in q's dtype,
    stats [n_compactions, N, 2] float64, state (A, B, U, Vb) or None), and
    with save_states a fourth item: the training stash gdn3_chunk_bwd reads.

    state0 = (A, B, U, Vb) and t0 continue a sequence (gdnx_gdn3_chunk_fwd_state):
    the call's token t is global token t0 + t (slot (t0 + t) % P, compaction
    after it when (t0 + t + 1) % K_c == 0), from the state a previous call
    returned; inference only.  compact_mode: 'svd' (default) or 'sketch' /
    'sketch_noqr' (sketch [B*H*M, b_v*b_k, R])."""
    lib = _lib.load()
    cm = compact_mode_code(compact_mode)
    a_v, a_k, b_v, b_k = factors
    B, T, H = q.shape[:3]
    D = q.shape[-1]
    lanes = 1 if q.dim() == 4 else q.shape[3]
    _need(q.is_cuda and q.dtype in (torch.bfloat16, torch.float32), "q must be bf16/float32 on the GPU")
    _need(q.shape == k.shape == v.shape and q.dtype == k.dtype == v.dtype, "q, k, v must match")
    _need(lanes in (1, M), "q/k/v lane dim must be 1 or M")
    gate_ch = 1 if b_gates.dim() == 4 else b_gates.shape[-1]
    _need(b_gates.shape == w_gates.shape and tuple(b_gates.shape[:4]) == (B, T, H, M), "bad gate shapes")
    _need(tuple(decay.shape) == (B, T, H, M), "decay must be [B,T,H,M]")
    for t in (q, k, v, b_gates, w_gates, decay, sketch):
        _need(t.is_contiguous(), "inputs must be contiguous")
    for t in (b_gates, w_gates, decay, sketch):
        _need(t.dtype == torch.float32, "gates, decay and sketch must be float32")
    Kc = P if compact_every is None else int(compact_every)
    N = B * H * M
    qw = sketch_width(R, a_v * a_k, b_v * b_k, cm)
    _need(tuple(sketch.shape) == (N, b_v * b_k, qw) and sketch.is_cuda,
          f"sketch must be [B*H*M, b_v*b_k, {qw}] on the GPU")
    dt = _lib.dtype_code(q.dtype)
    carried = state0 is not None or t0 != 0
    _need(not (carried and save_states), "a carried state (state0 / t0) is inference only")
    if state0 is not None:
        _g3_state_check(state0, N, R, factors, D, P, q.device)
    y = torch.empty(B, T, H, M, D, dtype=q.dtype, device=q.device)
    nws = lib.gdnx_gdn3_workspace_bytes(B, H, M, D, P, dt)
    _need(nws > 0, f"unsupported GDN3 shape: head_dim {D}, P {P}")
    ws = torch.empty(nws, dtype=torch.uint8, device=q.device)
    n_ev = lib.gdnx_gdn3_num_compactions_from(int(t0), T, P, Kc)
    _need(n_ev >= 0, f"compact_every={Kc} must be a positive multiple of P={P} (t0={t0} >= 0)")
    stats = torch.empty(max(n_ev, 1), N, 2, dtype=torch.float64, device=q.device)
    state = None
    ptrs = [None] * 4
    if return_state:
        state = (torch.empty(N, R, a_v, a_k, device=q.device), torch.empty(N, R, b_v, b_k, device=q.device),
                 torch.empty(N, D, P, device=q.device), torch.empty(N, D, P, device=q.device))
        ptrs = [_lib.ptr(t) for t in state]
    tst = None
    if save_states:
        nts = lib.gdnx_gdn3_train_states_bytes(B, T, H, M, D, P, Kc)
        _need(nts > 0, f"unsupported GDN3 shape for training: head_dim {D}, P {P}")
        tst = torch.empty(nts, dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        if carried:
            s0 = [None] * 4 if state0 is None else [_lib.ptr(t) for t in state0]
            rc = lib.gdnx_gdn3_chunk_fwd_state(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), lanes, _lib.ptr(b_gates),
                                               _lib.ptr(w_gates), gate_ch, _lib.ptr(decay), _lib.ptr(sketch), *s0,
                                               int(t0), _lib.ptr(y), *ptrs, _lib.ptr(stats) if n_ev > 0 else None,
                                               _lib.ptr(ws), B, T, H, M, D, R, P, Kc, a_v, a_k, b_v, b_k,
                                               float(slow_decay), dt, cm, _lib.stream_of(q))
        else:
            rc = lib.gdnx_gdn3_chunk_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), lanes, _lib.ptr(b_gates),
                                         _lib.ptr(w_gates), gate_ch, _lib.ptr(decay), _lib.ptr(sketch), _lib.ptr(y),
                                         *ptrs, _lib.ptr(stats) if n_ev > 0 else None, _lib.ptr(ws), _lib.ptr(tst),
                                         B, T, H, M, D, R, P, Kc, a_v, a_k, b_v, b_k, float(slow_decay), dt,
                                         cm, _lib.stream_of(q))
    _lib.check(rc, "gdnx_gdn3_chunk_fwd")
    if save_states:
        return y, stats[:n_ev], state, tst
    return y, stats[:n_ev], state


def gdn3_decode_step(q, k, v, b_gates, w_gates, decay, sketch, state, pos, *, R=4, P=16,
                     factors=(16, 16, 8, 8), slow_decay=0.97, compact_every=None, slots=None,
                     return_stats=False, out=None, compact_mode="svd"):
    """One token of the GDN3 Kronecker-residual recurrence per row on a
    carried state (gdnx_gdn3_decode_step), updated in place.

    q, k, v [NS,H,D] (shared by the lanes) or [NS,H,M,D]; b_gates, w_gates
    [NS,H,M] or [NS,H,M,D] float32; decay [NS,H,M]; state = (A, B, U, Vb)
    with leading dims [n_slots, H, M] (n_slots = NS without slots); sketch
    [n_slots*H*M, b_v*b_k, q]; pos int32 device [NS]: each row's global token
    index (slot pos % P; compaction after it when (pos + 1) % K_c == 0);
    slots int32 device [NS] or None.  Returns y [NS,H,M,D] in q's dtype (and
    the per-chain compaction statistics [NS,H,M,2] float64).  compact_mode as
    in gdn3_chunk_fwd."""
    lib = _lib.load()
    cm = compact_mode_code(compact_mode)
    a_v, a_k, b_v, b_k = factors
    _need(q.is_cuda and q.dim() in (3, 4) and q.shape == k.shape == v.shape, "q, k, v must be [NS,H,(M,)D] on GPU")
    _need(q.dtype in (torch.bfloat16, torch.float32) and q.dtype == k.dtype == v.dtype, "q, k, v: bf16 or float32")
    NS, H = q.shape[:2]
    D = q.shape[-1]
    _need(decay.dim() == 3 and tuple(decay.shape[:2]) == (NS, H), "decay must be [NS,H,M]")
    M = decay.shape[2]
    lanes = 1 if q.dim() == 3 else q.shape[2]
    _need(lanes in (1, M), "q/k/v lane dim must be 1 or M")
    gate_ch = 1 if b_gates.dim() == 3 else b_gates.shape[-1]
    _need(b_gates.shape == w_gates.shape and tuple(b_gates.shape[:3]) == (NS, H, M), "bad gate shapes")
    A, Bf, U, Vb = state
    n_slots = A.shape[0]
    _need(slots is not None or n_slots == NS, "without slots the state's leading dim must be NS")
    N = n_slots * H * M
    _g3_state_check([t.view(N, *t.shape[3:]) for t in state], N, R, factors, D, P, q.device)
    _need(tuple(A.shape[:3]) == (n_slots, H, M), "state leading dims must be [n_slots, H, M]")
    _need(tuple(sketch.shape) == (N, b_v * b_k, sketch_width(R, a_v * a_k, b_v * b_k, cm)), "bad sketch shape")
    _need(pos.dtype == torch.int32 and tuple(pos.shape) == (NS,), "pos must be an int32 tensor [NS]")
    if slots is not None:
        _need(slots.dtype == torch.int32 and tuple(slots.shape) == (NS,), "slots must be an int32 tensor [NS]")
    for t in (q, k, v, b_gates, w_gates, decay, sketch, pos) + ((slots,) if slots is not None else ()):
        _need(t.is_contiguous() and t.device == q.device, "inputs must be contiguous on one device")
    for t in (b_gates, w_gates, decay, sketch):
        _need(t.dtype == torch.float32, "gates, decay and sketch must be float32")
    Kc = P if compact_every is None else int(compact_every)
    y = _decode_out(out, (NS, H, M, D), q.dtype, q.device)
    stats = torch.empty(NS, H, M, 2, dtype=torch.float64, device=q.device) if return_stats else None
    with torch.cuda.device(q.device):
        rc = lib.gdnx_gdn3_decode_step(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), lanes, _lib.ptr(b_gates),
                                       _lib.ptr(w_gates), gate_ch, _lib.ptr(decay), _lib.ptr(sketch),
                                       *(_lib.ptr(t) for t in state), _lib.ptr(slots), _lib.ptr(pos), _lib.ptr(y),
                                       _lib.ptr(stats), NS, n_slots, H, M, D, R, P, Kc, a_v, a_k, b_v, b_k,
                                       float(slow_decay), _lib.dtype_code(q.dtype), cm, _lib.stream_of(q))
    _lib.check(rc, "gdnx_gdn3_decode_step")
    return (y, stats) if return_stats else y


def gdn3_chunk_bwd(q, k, v, b_gates, w_gates, decay, dy, train_states, *, M, R=4, P=16,
                   factors=(16, 16, 8, 8), compact_every=None):
    """Backward of gdn3_chunk_fwd (gdnx_gdn3_chunk_bwd) from the stash its
    save_states call returned.  Returns float32 (dq, dk, dv [B,T,H,M,D] per
    lane, db_gates, dw_gates in the gates' layout, ddecay [B,T,H,M])."""
    lib = _lib.load()
    a_v, a_k, b_v, b_k = factors
    B, T, H = q.shape[:3]
    D = q.shape[-1]
    lanes = 1 if q.dim() == 4 else q.shape[3]
    gate_ch = 1 if b_gates.dim() == 4 else b_gates.shape[-1]
    Kc = P if compact_every is None else int(compact_every)
    dy = dy.to(q.dtype).contiguous()
    _need(tuple(dy.shape) == (B, T, H, M, D), "dy must be [B,T,H,M,D]")
    dq, dk, dv = (torch.empty(B, T, H, M, D, dtype=torch.float32, device=q.device) for _ in range(3))
    db, dw = torch.empty_like(b_gates), torch.empty_like(w_gates)
    ddec = torch.empty_like(decay)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_gdn3_chunk_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), lanes, _lib.ptr(b_gates),
                                     _lib.ptr(w_gates), gate_ch, _lib.ptr(decay), _lib.ptr(dy),
                                     _lib.ptr(train_states), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(db),
                                     _lib.ptr(dw), _lib.ptr(ddec), B, T, H, M, D, R, P, Kc, a_v, a_k, b_v, b_k,
                                     _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(rc, "gdnx_gdn3_chunk_bwd")
    return dq, dk, dv, db, dw, ddec


def lane_sum(x, dtype):
    """gdnx_lane_sum: x float32 [..., M, D] (contiguous) summed over the lane
    dim M in lane order, returned as [..., D] in dtype (bfloat16 or float32):
    the gradient of a q, k or v its head's lanes share."""
    lib = _lib.load()
    _need(x.dtype == torch.float32 and x.is_contiguous() and x.dim() >= 2, "x must be contiguous float32 [..., M, D]")
    _need(dtype in (torch.float32, torch.bfloat16), "dtype must be float32 or bfloat16")
    M, D = x.shape[-2:]
    out = torch.empty(*x.shape[:-2], D, dtype=dtype, device=x.device)
    rows = out.numel() // D if D else 0
    with torch.cuda.device(x.device):
        rc = lib.gdnx_lane_sum(_lib.ptr(x), _lib.ptr(out), rows, M, D, _lib.dtype_code(dtype), _lib.stream_of(x))
    _lib.check(rc, "gdnx_lane_sum")
    return out


# ---------------------------------------------------------------------------
# GDN3 layer boundary (gdnx_gdn3_prologue_* / gdnx_gdn3_epilogue_*)
# ---------------------------------------------------------------------------
def gdn3_lane_rope_pairs(M: int, key_dim: int):
    """Lane RoPE pair counts d_m (0: identity lane), by the library's rule."""
    import ctypes
    lib = _lib.load()
    out = (ctypes.c_int * 4)()
    _lib.check(lib.gdnx_gdn3_lane_rope_pairs(M, key_dim, ctypes.cast(out, ctypes.c_void_p)),
               "gdnx_gdn3_lane_rope_pairs")
    return [out[m] for m in range(M)]


def _row_io(t, shape, dt, name):
    _need(tuple(t.shape) == tuple(shape), f"{name} must be {list(shape)}, got {list(t.shape)}")
    return t.to(dt).contiguous()


def gdn3_prologue_fwd(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, rates, rope_cos, rope_sin,
                      decay_clamp=0.999):
    """q, k [B,T,H,K] (bf16/float32; the other IO inputs are cast to it);
    b_proj [B,T,H,M,K]; w_proj [B,T,H,M,V]; proj_a, proj_b [B,T,H];
    decay_proj [B,T,H,M,4]; rates [4]; rope tables [M,T,K//2] float32.
    Returns (q_rope, k_rope [B,T,H,M,K] in q's dtype, b_gates, w_gates,
    decay float32)."""
    lib = _lib.load()
    _need(q.is_cuda and q.dim() == 4 and q.shape == k.shape, "q, k must be [B,T,H,K] on the GPU")
    B, T, H, K = q.shape
    _need(b_proj.dim() == 5, "b_proj must be [B,T,H,M,K]")
    M, V = b_proj.shape[3], w_proj.shape[-1]
    dt = q.dtype
    if B * T * H == 0:
        return (torch.empty(B, T, H, M, K, dtype=dt, device=q.device), torch.empty(B, T, H, M, K, dtype=dt, device=q.device),
                torch.empty(B, T, H, M, K, device=q.device), torch.empty(B, T, H, M, V, device=q.device),
                torch.empty(B, T, H, M, device=q.device))
    q, k = q.contiguous(), k.to(dt).contiguous()
    bp = _row_io(b_proj, (B, T, H, M, K), dt, "b_proj")
    wp = _row_io(w_proj, (B, T, H, M, V), dt, "w_proj")
    pa = _row_io(proj_a, (B, T, H), dt, "proj_a")
    pb = _row_io(proj_b, (B, T, H), dt, "proj_b")
    dp = _row_io(decay_proj, (B, T, H, M, 4), dt, "decay_proj")
    rates = _row_io(rates, (4,), torch.float32, "rates")
    _need(tuple(rope_cos.shape) == tuple(rope_sin.shape) == (M, T, K // 2) and rope_cos.dtype == torch.float32,
          "rope tables must be float32 [M, T, K//2]")
    qr = torch.empty(B, T, H, M, K, dtype=dt, device=q.device)
    kr = torch.empty_like(qr)
    bg = torch.empty(B, T, H, M, K, dtype=torch.float32, device=q.device)
    wg = torch.empty(B, T, H, M, V, dtype=torch.float32, device=q.device)
    dec = torch.empty(B, T, H, M, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        rc = lib.gdnx_gdn3_prologue_fwd(*map(_lib.ptr, (q, k, bp, pa, wp, pb, dp, rates, rope_cos.contiguous(),
                                                        rope_sin.contiguous(), qr, kr, bg, wg, dec)),
                                        B, T, H, M, K, V, float(decay_clamp), _lib.dtype_code(dt),
                                        _lib.stream_of(q))
    _lib.check(rc, "gdnx_gdn3_prologue_fwd")
    return qr, kr, bg, wg, dec


def gdn3_prologue_bwd(b_proj, proj_a, w_proj, proj_b, decay_proj, rates, rope_cos, rope_sin,
                      d_q_rope, d_k_rope, d_b_gates, d_w_gates, d_decay, decay_clamp=0.999):
    """Backward of gdn3_prologue_fwd; the IO inputs in the forward's compute
    dtype.  Returns float32 (dq, dk [B,T,H,K], d_b_proj, d_proj_a, d_w_proj,
    d_proj_b, d_decay_proj)."""
    lib = _lib.load()
    B, T, H, M, K = b_proj.shape
    V = w_proj.shape[-1]
    dev = b_proj.device
    f32 = [t.float().contiguous() for t in (d_q_rope, d_k_rope, d_b_gates, d_w_gates, d_decay)]
    _need(tuple(f32[0].shape) == tuple(f32[1].shape) == (B, T, H, M, K), "d_q_rope / d_k_rope must be [B,T,H,M,K]")
    _need(tuple(f32[2].shape) == (B, T, H, M, K) and tuple(f32[3].shape) == (B, T, H, M, V)
          and tuple(f32[4].shape) == (B, T, H, M), "bad gate / decay gradient shapes")
    dq = torch.empty(B, T, H, K, dtype=torch.float32, device=dev)
    dk = torch.empty_like(dq)
    dbp = torch.empty(B, T, H, M, K, dtype=torch.float32, device=dev)
    dwp = torch.empty(B, T, H, M, V, dtype=torch.float32, device=dev)
    dpa = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    dpb = torch.empty_like(dpa)
    ddp = torch.empty(B, T, H, M, 4, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.gdnx_gdn3_prologue_bwd(*map(_lib.ptr, (b_proj, proj_a, w_proj, proj_b, decay_proj, rates, rope_cos,
                                                        rope_sin, *f32, dq, dk, dbp, dpa, dwp, dpb, ddp)),
                                        B, T, H, M, K, V, float(decay_clamp), _lib.dtype_code(b_proj.dtype),
                                        _lib.stream_of(b_proj))
    _lib.check(rc, "gdnx_gdn3_prologue_bwd")
    return dq, dk, dbp, dpa, dwp, dpb, ddp


def gdn3_epilogue_fwd(y, router_logits, norm):
    """y [B,T,H,M,V] (bf16/float32), router_logits [B,T,H,M], norm [V] ->
    [B,T,H,V] in y's dtype."""
    lib = _lib.load()
    _need(y.is_cuda and y.dim() == 5, "y must be [B,T,H,M,V] on the GPU")
    B, T, H, M, V = y.shape
    y = y.contiguous()
    lg = _row_io(router_logits, (B, T, H, M), y.dtype, "router_logits")
    nm = _row_io(norm, (V,), torch.float32, "norm")
    out = torch.empty(B, T, H, V, dtype=y.dtype, device=y.device)
    with torch.cuda.device(y.device):
        rc = lib.gdnx_gdn3_epilogue_fwd(_lib.ptr(y), _lib.ptr(lg), _lib.ptr(nm), _lib.ptr(out), B, T, H, M, V,
                                        _lib.dtype_code(y.dtype), _lib.stream_of(y))
    _lib.check(rc, "gdnx_gdn3_epilogue_fwd")
    return out


def gdn3_epilogue_bwd(y, router_logits, norm, d_out):
    """Backward of gdn3_epilogue_fwd: (d_y [B,T,H,M,V] in y's dtype,
    d_router_logits [B,T,H,M], d_norm [V] float32)."""
    lib = _lib.load()
    B, T, H, M, V = y.shape
    dout = _row_io(d_out, (B, T, H, V), y.dtype, "d_out")
    dy = torch.empty_like(y)
    dlg = torch.empty(B, T, H, M, dtype=torch.float32, device=y.device)
    dnm = torch.empty(V, dtype=torch.float32, device=y.device)
    ws = torch.empty(max(lib.gdnx_gdn3_epilogue_workspace_bytes(B, T, H, V), 16), dtype=torch.uint8,
                     device=y.device)
    with torch.cuda.device(y.device):
        rc = lib.gdnx_gdn3_epilogue_bwd(*map(_lib.ptr, (y, router_logits, norm, dout, dy, dlg, dnm, ws)),
                                        B, T, H, M, V, _lib.dtype_code(y.dtype), _lib.stream_of(y))
    _lib.check(rc, "gdnx_gdn3_epilogue_bwd")
    return dy, dlg, dnm

"""Rank-r block-Householder delta rule with the RLS T-factor on the GPU
(gdnx_rls_fwd / gdnx_rls_bwd).

The recurrence of KMD2LinearAttn._scan (gdn3/kmd2.py:166-214) and of the
testbed mixer (research/testbed_mqar.py:226-262): per chain (b, h), state
S [dv, dk], per token with r write slots

    S <- S diag(a);   Kt = Bg * K;   S <- S - (S Kt^T)(eps I + Kt Kt^T)^-1 Kt
    S <- S + (Wg * V)^T K;           y = sum_o mix_o S q_o

With ``compact_P`` > 0 it is also the testbed mixer's scan with its
dense-state compaction (research/testbed_mqar.py:245-260): after the write
of every compact_P-th token S <- s S_lr + (1 - s) S, S_lr the best
rank-compact_R approximation of S (exact, in-kernel Jacobi eigensolver); the
gradient treats S_lr as a constant (the testbed's no_grad SVD), or passes
straight through with ``straight_through=True`` (its compact_ste).

``rls_scan(q, K, V, Bg, Wg, a)`` takes the reference method's arguments
(q [B,T,H,r_out,dk]; K, Bg [B,T,H,r,dk]; V, Wg [B,T,H,r,dv]; a [B,T,H,dk])
plus its two attributes ``eps`` (rls_eps) and ``out_mix`` [H, r_out], and
returns y [B,T,H,dv] in float32 like the reference.  It is differentiable in
all inputs and out_mix: the forward keeps a state every few tokens, the
backward kernel recomputes between them.  Head dims are zero-padded to the
kernel's sizes (key dim 32 / 64 / 128, value dim a multiple of 16): zero key
and value columns with a = 1 leave the scan unchanged, exactly.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib, ops


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _kdim(dk):
    for d in (32, 64, 128):
        if dk <= d:
            return d
    raise ValueError(f"key dim {dk} > 128 is not supported")


def _vdim(dv):
    _need(dv <= 128, f"value dim {dv} > 128 is not supported")
    return max(16, (dv + 15) // 16 * 16)


def _pad(x, n, value=0.0):
    return x if x.shape[-1] == n else F.pad(x, (0, n - x.shape[-1]), value=value)


def _prep(q, K, V, Bg, Wg, a):
    dk, dv = K.shape[-1], V.shape[-1]
    kd, vd = _kdim(dk), _vdim(dv)
    f = [t.float() for t in (q, K, V, Bg, Wg, a)]
    q_, K_, Bg_ = (_pad(t, kd).contiguous() for t in (f[0], f[1], f[3]))
    V_, Wg_ = (_pad(t, vd).contiguous() for t in (f[2], f[4]))
    a_ = _pad(f[5], kd, 1.0).contiguous()
    return q_, K_, V_, Bg_, Wg_, a_, kd, vd


def rls_fwd(q, K, V, Bg, Wg, a, eps=0.5, out_mix=None, state0=None, *, return_state=False, checkpoint=False,
            compact_P=0, compact_R=0, slow_decay=0.97):
    """Raw forward on padded float32 tensors (see rls_scan).  Returns
    (y, state or None, ckpt or None) at the padded dims."""
    lib = _lib.load()
    B, T, H, RO, kd = q.shape
    R, vd = V.shape[3], V.shape[4]
    dev = q.device
    _need(q.is_cuda, "rls: tensors must be on the GPU")
    mix = None
    if RO > 1:
        _need(out_mix is not None and tuple(out_mix.shape) == (H, RO), "out_mix must be [H, r_out]")
        mix = out_mix.float().contiguous()
    y = torch.empty(B, T, H, vd, dtype=torch.float32, device=dev)
    st = torch.empty(B, H, vd, kd, dtype=torch.float32, device=dev) if return_state else None
    ck = None
    if checkpoint:
        n = lib.gdnx_rls_ckpt_bytes(B, T, H, R, kd, vd, int(compact_P))
        _need(n >= 0, "rls: unsupported shape")
        ck = torch.empty(max(n // 4, 4), dtype=torch.float32, device=dev)
    s0 = None if state0 is None else state0.float().contiguous()
    with torch.cuda.device(dev):
        rc = lib.gdnx_rls_fwd(*map(_lib.ptr, (q, K, V, Bg, Wg, a, mix, s0, y, st, ck)), B, T, H, R, RO, kd, vd,
                              float(eps), int(compact_P), int(compact_R), float(slow_decay), _lib.stream_of(q))
    _lib.check(rc, "gdnx_rls_fwd")
    return y, st, ck


class _RLSScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, K, V, Bg, Wg, a, out_mix, state0, eps, want_state, compact):
        dk, dv = K.shape[-1], V.shape[-1]
        q_, K_, V_, Bg_, Wg_, a_, kd, vd = _prep(q, K, V, Bg, Wg, a)
        s0 = None if state0 is None else _pad(_pad(state0.float(), kd).transpose(-1, -2), vd).transpose(-1, -2)
        cP, cR, sd, ste = compact
        y, st, ck = rls_fwd(q_, K_, V_, Bg_, Wg_, a_, eps, out_mix, s0, return_state=want_state, checkpoint=True,
                            compact_P=cP, compact_R=cR, slow_decay=sd)
        ctx.save_for_backward(q_, K_, V_, Bg_, Wg_, a_, out_mix, ck)
        ctx.meta = (dk, dv, float(eps), state0 is not None, compact)
        y = y[..., :dv]
        if want_state:
            return y, st[..., :dv, :dk]
        return y

    @staticmethod
    def backward(ctx, dy, *rest):
        q_, K_, V_, Bg_, Wg_, a_, out_mix, ck = ctx.saved_tensors
        dk, dv, eps, has_s0, (cP, cR, sd, ste) = ctx.meta
        lib = _lib.load()
        B, T, H, RO, kd = q_.shape
        R, vd = V_.shape[3], V_.shape[4]
        dev = q_.device
        dy_ = _pad(dy.float(), vd).contiguous()
        dst = None
        if rest and rest[0] is not None:
            dst = _pad(_pad(rest[0].float(), kd).transpose(-1, -2), vd).transpose(-1, -2).contiguous()
        outs = [torch.empty_like(t) for t in (q_, K_, V_, Bg_, Wg_, a_)]
        dmix = torch.empty(B, H, RO, dtype=torch.float32, device=dev)
        ds0 = torch.empty(B, H, vd, kd, dtype=torch.float32, device=dev) if has_s0 else None
        mix = out_mix.float().contiguous() if RO > 1 else None
        ws = None
        if not cP:   # value rows spread over workgroups, column sums reduced by a second kernel
            n = lib.gdnx_rls_bwd_workspace_bytes(B, T, H, R, kd, vd)
            ws = torch.empty(max(n, 16), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = lib.gdnx_rls_bwd(*map(_lib.ptr, (q_, K_, V_, Bg_, Wg_, a_, mix, ck, dy_, dst, *outs, dmix, ds0)),
                                  B, T, H, R, RO, kd, vd, eps, int(cP), int(cR), float(sd), int(bool(ste)),
                                  _lib.ptr(ws), _lib.stream_of(q_))
        _lib.check(rc, "gdnx_rls_bwd")
        dq, dK, dV, dBg, dWg, da = outs
        dq, dK, dBg, da = (t[..., :dk] for t in (dq, dK, dBg, da))
        dV, dWg = dV[..., :dv], dWg[..., :dv]
        dm = dmix.sum(0) if (RO > 1 and ctx.needs_input_grad[6]) else None
        d0 = ds0[..., :dv, :dk] if has_s0 else None
        return dq, dK, dV, dBg, dWg, da, dm, d0, None, None, None


def rls_scan(q, K, V, Bg, Wg, a, eps=0.5, out_mix=None, state0=None, return_state=False, *, compact_P=0,
             compact_R=0, slow_decay=0.97, straight_through=False):
    """KMD2LinearAttn._scan on the GPU (gdn3/kmd2.py:166-214).

    q [B,T,H,r_out,dk]; K, Bg [B,T,H,r,dk]; V, Wg [B,T,H,r,dv];
    a [B,T,H,dk]; out_mix [H, r_out] (read when r_out > 1); state0
    [B,H,dv,dk] or None (zeros, as the reference).  r, r_out <= 4, dk, dv
    <= 128.  Returns y [B,T,H,dv] float32 (and the final state [B,H,dv,dk]
    when return_state); differentiable in every tensor argument.
    compact_P / compact_R / slow_decay / straight_through: the testbed's
    compaction (compact_P = 0: none); compact_R <= min(dk, dv) <= 64."""
    _need(q.dim() == 5 and K.dim() == 5 and V.dim() == 5, "q, K, V must be 5-d ([B,T,H,slots,dim])")
    B, T, H, RO, dk = q.shape
    R, dv = K.shape[3], V.shape[4]
    _need(K.shape == Bg.shape and tuple(K.shape[:3]) == (B, T, H), "K and Bg must be [B,T,H,r,dk]")
    _need(V.shape == Wg.shape and tuple(V.shape[:4]) == (B, T, H, R), "V and Wg must be [B,T,H,r,dv]")
    _need(tuple(a.shape) == (B, T, H, dk), "a must be [B,T,H,dk]")
    if T == 0:   # empty sequence: no output, the state is the initial one
        y = ops.empty_result((B, 0, H, dv), torch.float32, q.device, q, K, V, Bg, Wg, a, out_mix)
        if not return_state:
            return y
        st = state0.float() + 0 if state0 is not None else torch.zeros(B, H, dv, dk, device=q.device)
        return y, st
    compact = (int(compact_P), int(compact_R), float(slow_decay), bool(straight_through))
    out = _RLSScan.apply(q, K, V, Bg, Wg, a, out_mix if RO > 1 else None, state0, float(eps), bool(return_state),
                         compact)
    return out

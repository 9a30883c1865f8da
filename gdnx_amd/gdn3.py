"""GDN3-facing entry points (the reference's recurrence interface).

``gdn3_scan`` is GDN3LinearAttn's recurrence (gdn3/gdn3_upgrade.py:403-531,
frozen oracle gdn3/_reference_recurrence.py:33-94) in the dense-state regime
with lane-shared q/k/v and scalar per-lane gates b = w = beta: per chain
(b, h, lane)

    gamma = clamp(exp(log_g), 0, 1);  S <- gamma S
    r = beta v - S (beta k);  alpha = (1 - exp(-beta |k|^2)) / (beta |k|^2)
    S <- S + alpha r k^T;     y = S q

i.e. the chunked delta rule with erase = write coefficient
a = alpha(beta |k|^2) * beta (the exact-alpha write of
gdn3/gdn3_upgrade.py:641-648).  The coefficient, the recurrence and both
backwards are HIP kernels of libgdnx.

``gdn3_recurrent_state`` is the same method in its general regime: a
P-slot residual window and periodic rearrangement-SVD compaction of the
Kronecker factors, differentiable with the frozen oracle's gradient
semantics (the factors a compaction leaves carry no gradient: it runs under
no_grad, gdn3/_reference_recurrence.py:86-88; the residual slots keep
theirs), through the gdnx_gdn3_chunk_bwd kernel.
"""
from __future__ import annotations

import collections

import torch

from . import ops


def gdn3_coeff(k, beta):
    """a = alpha(beta |k|^2) beta for k [B,T,H,D] shared by beta's M lanes,
    alpha(c) = (1 - exp(-c))/c with the Taylor branch 1 - c/2 + c^2/6 for
    |c| < 1e-6 (gdn3/gdn3_upgrade.py:641-648); the gdnx_gdn3_coeff kernel
    (not differentiable; gdn3_scan carries its gradient)."""
    return ops.gdn3_coeff(k.contiguous(), beta.float().contiguous())


class GDN3ScanFunction(torch.autograd.Function):
    """Dense-regime GDN3 recurrence, differentiable in q, k, v, beta, log_g
    and state0: the coefficient kernel, then the delta-rule forward; the
    backward runs the delta-rule backward and folds the coefficient's
    gradient into dk and dbeta in one kernel (no elementwise torch ops)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, log_g, state0):
        train = any(ctx.needs_input_grad)
        # an unused output's gradient arrives as None (no zero tensor is filled)
        ctx.set_materialize_grads(False)
        D = q.shape[-1]
        a = ops.gdn3_coeff(k, beta)
        chunk, two_pass = ops.forward_plan(D, q.dtype, train)
        y, s_out, cs = ops.delta_chunk_fwd(q, k, v, a, a, log_g, state0, return_state=True,
                                           save_states=train, chunk=chunk, two_pass=two_pass)
        if train:
            ctx.save_for_backward(q, k, v, beta, a, log_g, cs)
            ctx.chunk = chunk
            ctx.has_state0 = state0 is not None
        return y, s_out

    @staticmethod
    def backward(ctx, dy, ds_out):
        q, k, v, beta, a, log_g, cs = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros(*a.shape, q.shape[-1], dtype=q.dtype, device=q.device)
        dq, dk, dv, dae, daw, dlg, ds0 = ops.delta_chunk_bwd(
            q, k, v, a, a, log_g, dy, cs, ctx.chunk, dstate_out=ds_out,
            want_dstate0=ctx.has_state0 and ctx.needs_input_grad[5])
        dbeta = ops.gdn3_coeff_bwd(k, beta, dae, daw, dk)
        return dq, dk, dv, dbeta, dlg, ds0


def gdn3_scan(q, k, v, beta, log_g, state0=None, return_state=False):
    """Differentiable GDN3 dense-regime recurrence.

    q, k, v: [B,T,H,D] (bf16 or float32, shared by the lanes); beta, log_g:
    [B,T,H,M] float32 (log_g > 0 is clamped, i.e. gamma <= 1).  Returns
    y [B,T,H,M,D] in q's dtype (and the final state [B,H,M,D,D] fp32).
    """
    if q.shape[1] == 0:
        B, _, H, D = q.shape
        M = beta.shape[3]
        y = ops.empty_result((B, 0, H, M, D), q.dtype, q.device, q, k, v, beta, log_g)
        if not return_state:
            return y
        s = state0.float() + 0 if state0 is not None else torch.zeros(B, H, M, D, D, device=q.device)
        return y, s
    args = [t.contiguous() for t in (q, k, v)] + [t.float().contiguous() for t in (beta, log_g)]
    if state0 is not None:
        state0 = state0.float().contiguous()
    y, s = GDN3ScanFunction.apply(*args, state0)
    return (y, s) if return_state else y


_SKETCHES = collections.OrderedDict()
_SKETCH_CACHE = 8


def default_sketch(N, n, q, device):
    """The compaction sketch: randn(N, n, q) float32 from a CPU generator
    seeded 1234 (the reference draws randn(N, n, q) from a generator seeded
    1234 on R_mat's device, gdn3/gdn3_upgrade.py:681-682; the CPU stream is
    the one its CPU runs use, so this matches the reference on the CPU, not
    its GPU runs).  Row n depends only on n, not on N.  The last few
    (device, shape) draws are kept (least recently used dropped first)."""
    key = (str(device), N, n, q)
    if key in _SKETCHES:
        _SKETCHES.move_to_end(key)
        return _SKETCHES[key]
    gen = torch.Generator(device="cpu").manual_seed(1234)
    G = torch.randn(N, n, q, dtype=torch.float32, generator=gen).to(device)
    _SKETCHES[key] = G
    while len(_SKETCHES) > _SKETCH_CACHE:
        _SKETCHES.popitem(last=False)
    return G


def _lane_shared(x):
    """[B,T,H,M,D] with a stride-0 lane dim (an expand) -> its [B,T,H,D] view."""
    return x.dim() == 5 and x.stride(3) == 0


def _scalar_gate(g):
    return g.dim() == 5 and g.stride(-1) == 0


class _GDN3Chunk(torch.autograd.Function):
    """gdnx_gdn3_chunk_fwd / _bwd on normalised inputs: q, k, v [B,T,H,D]
    (shared) or [B,T,H,M,D] in the compute dtype, gates [B,T,H,M] or
    [B,T,H,M,D] float32, decay [B,T,H,M] float32.  Returns y, the compaction
    statistics and, with want_state, the final (A, B, U, Vb); only y is
    differentiable."""

    @staticmethod
    def forward(ctx, q, k, v, bg, wg, dec, sketch, cfg, want_state):
        # the statistics' and states' (non-differentiable) gradients arrive as None
        ctx.set_materialize_grads(False)
        M, R, P, factors, slow_decay, Kc, cmode = cfg
        y, stats, state, tst = ops.gdn3_chunk_fwd(q, k, v, bg, wg, dec, sketch, M=M, R=R, P=P, factors=factors,
                                                  slow_decay=slow_decay, compact_every=Kc,
                                                  return_state=want_state, save_states=True, compact_mode=cmode)
        ctx.save_for_backward(q, k, v, bg, wg, dec, tst)
        ctx.cfg = cfg
        extra = (stats,) + (tuple(state) if want_state else ())
        ctx.mark_non_differentiable(*extra)
        return (y,) + extra

    @staticmethod
    def backward(ctx, dy, *unused):
        q, k, v, bg, wg, dec, tst = ctx.saved_tensors
        M, R, P, factors, _, Kc, _ = ctx.cfg
        if dy is None:
            return (None,) * 9
        dq, dk, dv, db, dw, ddec = ops.gdn3_chunk_bwd(q, k, v, bg, wg, dec, dy, tst, M=M, R=R, P=P,
                                                      factors=factors, compact_every=Kc)
        if q.dim() == 4:   # q, k, v shared by the lanes: their lane sums, in the IO dtype
            return (ops.lane_sum(dq, q.dtype), ops.lane_sum(dk, k.dtype), ops.lane_sum(dv, v.dtype), db, dw,
                    ddec, None, None, None)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), db, dw, ddec, None, None, None


def gdn3_recurrent_state(q, k, v, b_gates, w_gates, decay_factors, *, R=4, P=16,
                         factors=(16, 16, 8, 8), slow_decay=0.97, compact_every=None,
                         sketch=None, return_state=False, state0=None, t0=0, compact_mode="svd"):
    """GDN3LinearAttn._gdn3_recurrent_state on the GPU.

    Reference: gdn3/gdn3_upgrade.py:403-531 with the semantics of its frozen
    oracle gdn3/_reference_recurrence.py:33-94 (the chunked reference departs
    from that oracle after the second compaction window).  q, k, b_gates:
    [B,T,H,M,K]; v, w_gates: [B,T,H,M,V]; decay_factors [B,T,H,M]
    (q/k/v may also be [B,T,H,D], shared by the lanes, and the gates
    [B,T,H,M], one scalar per lane)
    (multiplicative, clamped to [0, 1]).  Lane-expanded q/k/v (stride 0 over
    M) are read once per head; gates expanded over the channel dim are read
    as one scalar per lane.  bf16 q/k/v compute on bf16 MFMA operands with
    fp32 state; other float dtypes run in float32.  compact_every defaults to
    P (the reference layer compacts every P tokens).  Returns y
    [B,T,H,M,V] in the compute dtype, plus ((A, B, U, Vb), comp_err) when
    return_state (comp_err is the reference's summed discarded energy, a
    device tensor).  When an input requires grad, y is differentiable in q,
    k, v, the gates and the decay (P = 16, 32 or 64); the state and comp_err
    are not.

    state0 = (A, B, U, Vb) and t0 continue a sequence from the state a
    previous call returned after t0 tokens (inference only: no gradient flows
    into or through a carried state); two calls over [0, T1) and [T1, T)
    equal one over [0, T).

    compact_mode: the layer's mode (gdn3/gdn3_upgrade.py:579-592): 'svd'
    (default) or 'sketch' / 'sketch_noqr', one sketched product per
    compaction with a sketch [N, b_v*b_k, R] and a compaction error of 0.
    """
    cm = ops.compact_mode_code(compact_mode)
    B, T, H, M = decay_factors.shape
    cdt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    D = q.shape[-1]
    a_v, a_k, b_v, b_k = factors
    N = B * H * M
    carried = state0 is not None or t0 != 0
    if state0 is not None:
        state0 = tuple(t.float().contiguous() for t in state0)
    if T == 0:   # empty sequence: zero output, the initial state passes through, no compaction
        y = ops.empty_result((B, 0, H, M, D), cdt, q.device, q, k, v, b_gates, w_gates, decay_factors)
        if not return_state:
            return y
        dev = q.device
        if state0 is not None:
            state = tuple(t.clone() for t in state0)
        else:
            state = (torch.zeros(N, R, a_v, a_k, device=dev), torch.zeros(N, R, b_v, b_k, device=dev),
                     torch.zeros(N, D, P, device=dev), torch.zeros(N, D, P, device=dev))
        return y, state, torch.zeros((), dtype=torch.float64, device=dev)

    def lanes5(x):
        return x.unsqueeze(3) if x.dim() == 4 else x
    if all(x.dim() == 4 or _lane_shared(x) for x in (q, k, v)):
        q4, k4, v4 = (x.to(cdt).contiguous() if x.dim() == 4 else x.select(3, 0).to(cdt).contiguous()
                      for x in (q, k, v))
    else:
        q4, k4, v4 = (lanes5(x).to(cdt).expand(B, T, H, M, D).contiguous() for x in (q, k, v))

    def chan5(g):
        return g.unsqueeze(-1) if g.dim() == 4 else g
    if all(g.dim() == 4 or _scalar_gate(g) for g in (b_gates, w_gates)):
        bg, wg = (g.float().contiguous() if g.dim() == 4 else g.select(-1, 0).float().contiguous()
                  for g in (b_gates, w_gates))
    else:
        bg = chan5(b_gates).float().expand(B, T, H, M, D).contiguous()
        wg = chan5(w_gates).float().expand(B, T, H, M, D).contiguous()
    dec = decay_factors.float().contiguous()
    qw = ops.sketch_width(R, a_v * a_k, b_v * b_k, cm)
    G = default_sketch(N, b_v * b_k, qw, q.device) if sketch is None else sketch.float().contiguous()
    train = torch.is_grad_enabled() and any(t.requires_grad for t in (q4, k4, v4, bg, wg, dec))
    if train and carried:
        raise ValueError("gdn3_recurrent_state: a carried state (state0 / t0) is inference only; "
                         "run under torch.no_grad() or without state0")
    if carried:
        y, stats, state = ops.gdn3_chunk_fwd(q4, k4, v4, bg, wg, dec, G, M=M, R=R, P=P, factors=factors,
                                             slow_decay=slow_decay, compact_every=compact_every,
                                             return_state=return_state, state0=state0, t0=t0, compact_mode=cm)
    elif train:
        out = _GDN3Chunk.apply(q4, k4, v4, bg, wg, dec, G, (M, R, P, factors, slow_decay, compact_every, cm),
                               return_state)
        y, stats, state = out[0], out[1], (tuple(out[2:]) if return_state else None)
    else:
        y, stats, state = ops.gdn3_chunk_fwd(q4, k4, v4, bg, wg, dec, G, M=M, R=R, P=P, factors=factors,
                                             slow_decay=slow_decay, compact_every=compact_every,
                                             return_state=return_state, compact_mode=cm)
    if not return_state:
        return y
    err = (stats[:, :, 0].sum(1) - stats[:, :, 1].sum(1)).clamp(min=0.0).sum()
    return y, state, err


class GDN3RecurrentState:
    """Autograd entry with the argument order of the reference method
    (q, k, v, b_gates, w_gates, decay_factors): ``GDN3RecurrentState.apply``
    returns y, differentiable through the gdnx_gdn3_chunk_bwd kernel."""

    @staticmethod
    def apply(q, k, v, b_gates, w_gates, decay_factors, R=4, P=16, factors=(16, 16, 8, 8),
              slow_decay=0.97, compact_every=None, compact_mode="svd"):
        return gdn3_recurrent_state(q, k, v, b_gates, w_gates, decay_factors, R=R, P=P, factors=factors,
                                    slow_decay=slow_decay, compact_every=compact_every, compact_mode=compact_mode)


def gdn3_decode_step(q, k, v, b_gates, w_gates, decay_factors, state, pos, *, R=4, P=16,
                     factors=(16, 16, 8, 8), slow_decay=0.97, compact_every=None, sketch=None,
                     slots=None, return_stats=False, compact_mode="svd"):
    """One token of the GDN3 recurrence per row, on a carried state updated in
    place: one iteration of the frozen oracle's loop
    (gdn3/_reference_recurrence.py:60-90) with the compaction after tokens
    whose (pos + 1) % compact_every == 0 (the reference has no decode path).

    q, k, v [NS,H,M,D] (a stride-0 lane dim is read once per head) or
    [NS,H,D]; b_gates, w_gates [NS,H,M,K] / [NS,H,M,V] (an expand over the
    channels is read as one scalar per lane) or [NS,H,M]; decay_factors
    [NS,H,M].  state = (A, B, U, Vb) as gdn3_recurrent_state returns it
    ([N, ...] with N = rows*H*M, rows = NS without slots) or with leading
    dims [n_slots, H, M]; updated in place.  pos: each row's global token
    index (int, sequence or int32 tensor [NS]); slots: int32 device tensor
    [NS] of state rows (None: row s is state row s).  The sketch defaults to
    the rows gdn3_recurrent_state draws for the same chains.  Returns y
    [NS,H,M,V] in the compute dtype (and the compaction statistics [NS,H,M,2]).
    compact_mode as in gdn3_recurrent_state."""
    cm = ops.compact_mode_code(compact_mode)
    NS, H, M = decay_factors.shape
    D = q.shape[-1]
    dev = q.device
    cdt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    a_v, a_k, b_v, b_k = factors

    def shared(x):
        return x.dim() == 3 or (x.dim() == 4 and x.stride(2) == 0)
    if all(shared(x) for x in (q, k, v)):
        q3, k3, v3 = (x if x.dim() == 3 else x.select(2, 0) for x in (q, k, v))
    else:
        q3, k3, v3 = (x.expand(NS, H, M, D) if x.dim() == 4 else x.unsqueeze(2).expand(NS, H, M, D)
                      for x in (q, k, v))
    q3, k3, v3 = (x.to(cdt).contiguous() for x in (q3, k3, v3))

    def scalar(g):
        return g.dim() == 3 or g.stride(-1) == 0
    if all(scalar(g) for g in (b_gates, w_gates)):
        bg, wg = (g if g.dim() == 3 else g.select(-1, 0) for g in (b_gates, w_gates))
    else:
        bg, wg = (g.unsqueeze(-1).expand(NS, H, M, D) if g.dim() == 3 else g for g in (b_gates, w_gates))
    bg, wg = bg.float().contiguous(), wg.float().contiguous()
    dec = decay_factors.float().contiguous()

    A, Bf, U, Vb = state
    if A.dim() == 4:   # [N, R, a_v, a_k]: view as [rows, H, M, ...] (same storage)
        n_rows = A.shape[0] // (H * M)
        A, Bf, U, Vb = (t.view(n_rows, H, M, *t.shape[1:]) for t in (A, Bf, U, Vb))
    n_slots = A.shape[0]
    if not isinstance(pos, torch.Tensor):
        pos = [int(pos)] * NS if isinstance(pos, int) else [int(x) for x in pos]
        if any(x < 0 for x in pos):
            raise ValueError("gdn3_decode_step: token positions must be >= 0")
        pos = torch.tensor(pos, dtype=torch.int32)
    pos = pos.to(device=dev, dtype=torch.int32).contiguous()
    if slots is not None and not isinstance(slots, torch.Tensor):
        slots = torch.tensor([int(x) for x in slots], dtype=torch.int32)
    if slots is not None:
        slots = slots.to(device=dev, dtype=torch.int32).contiguous()
    qw = ops.sketch_width(R, a_v * a_k, b_v * b_k, cm)
    G = default_sketch(n_slots * H * M, b_v * b_k, qw, dev) if sketch is None else sketch.float().contiguous()
    return ops.gdn3_decode_step(q3, k3, v3, bg, wg, dec, G, (A, Bf, U, Vb), pos, R=R, P=P, factors=factors,
                                slow_decay=slow_decay, compact_every=compact_every, slots=slots,
                                return_stats=return_stats, compact_mode=cm)

"""KMD-2 scan entry points with the reference's call signatures.

``scan(q, k, v, g, beta_e, beta_w, out_mix=None)`` and
``scan_with_update_norm(...)`` replace gdn3/kmd2_fast_scan.py:281-282 (the
torch.compile'd chunked scan) and, through them, the slow loop of
KMD2NativeAttn._scan (gdn3/kmd2_native.py:109-132); their exact semantics are
the frozen reference research/kernel_ab/ref_scan.py:24-48:

    S <- diag(g_t) S;  m = S^T k_t;  S <- S + k_t (beta_w v_t - beta_e m)^T
    y_t = sum_r out_mix[h, r] q_{t,r}^T S

i.e. the decoupled-erase delta rule with a_e = beta_e, a_w = beta_w and the
query slots mixed linearly into one query (y is linear in q).  The update
score of scan_with_update_norm is |k_t| |beta_w v_t - beta_e m_t|
(gdn3/kmd2_fast_scan.py:229-230), returned detached.

Shapes: q [B,T,H,r_out,dk], k [B,T,H,dk], v [B,T,H,dv], g [B,T,H,dk]
(multiplicative decay in (0, 1]), beta_e / beta_w [B,T,H], out_mix [H,r_out]
(used when r_out > 1).  dk, dv <= 128: the kernels run at D = 64 or 128
and narrower dims are zero-padded, which is exact (a zero key channel never
enters the state, a zero value column stays zero; padded outputs are sliced
off, so their gradients are zero too).

Two kernel paths: a decay constant over dk (a per-token scalar, e.g. an
expand over dk, or the layer at initialisation where decay_chan = 0) runs
the scalar-decay kernels in the input dtype (bf16 or float32); a decay that
varies over the key channels (gdn3/kmd2_native.py:163-164, g =
exp(g_head + decay_chan)) runs the per-channel kernels (libgdnx
gdnx_delta_chan_*), in float32.
"""
from __future__ import annotations

import torch

from . import ops


def _mixed_query(q, out_mix):
    r_out = q.shape[3]
    if r_out == 1:
        return q[:, :, :, 0]
    if out_mix is None:
        raise ValueError("out_mix [H, r_out] is required when r_out > 1")
    w = out_mix.float().view(1, 1, out_mix.shape[0], r_out, 1)
    return (q.float() * w).sum(3).to(q.dtype)


def _scalar_decay(g):
    """True when g [B,T,H,dk] carries one decay per token, so the scalar-decay
    kernels give the same values and gradients: g broadcast over dk (stride
    0), or a no-grad g whose channels are equal.  A full g that requires grad
    takes the per-channel path without looking at its values (no host sync):
    its channels get gradients of their own."""
    if g.shape[-1] == 1 or g.stride(-1) == 0:
        return True
    if g.requires_grad:
        return False
    return bool((g.amax(-1) == g.amin(-1)).all())


def _kernel_dim(dk, dv):
    D = max(dk, dv)
    if D > 128:
        raise NotImplementedError(f"dk={dk}, dv={dv}: the kernels carry head dims up to 128")
    return 64 if D <= 64 else 128


def _pad_last(x, D, value=0.0):
    n = x.shape[-1]
    return x if n == D else torch.nn.functional.pad(x, (0, D - n), value=value)


def _pad_state(state0, D):
    """[B,H,dk,dv] -> the kernels' [B,H,D,D] (zero rows / columns are exact)."""
    dk, dv = state0.shape[-2:]
    s = state0.float()
    if dk != D or dv != D:
        s = torch.nn.functional.pad(s, (0, D - dv, 0, D - dk))
    return s.contiguous()


def _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores, state0=None, want_state=False):
    B, T, H, r_out, dk = q.shape
    dv = v.shape[-1]
    if T == 0:
        y = ops.empty_result((B, 0, H, dv), q.dtype if q.dtype == torch.bfloat16 else torch.float32, q.device,
                             q, k, v, g, beta_e, beta_w, out_mix)
        out = (y, torch.zeros(B, 0, H, device=q.device)) if want_scores else y
        if want_state:
            st = state0.float().clone() if state0 is not None else torch.zeros(B, H, dk, dv, device=q.device)
            return out, st
        return out
    D = _kernel_dim(dk, dv)
    scalar = _scalar_decay(g)
    qe = _mixed_query(q if scalar else q.float(), out_mix)
    qe, kp, vp = _pad_last(qe, D), _pad_last(k, D), _pad_last(v, D)
    s0 = None if state0 is None else _pad_state(state0, D)
    if scalar:
        # one decay per token: the scalar-decay kernels (exact gradients also
        # for an expand over dk, which autograd sums back into the token decay)
        dt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
        log_g = torch.log(g[..., 0].float().clamp(min=1e-30)).unsqueeze(-1)
        out = ops.delta_rule(qe.to(dt), kp.to(dt), vp.to(dt), beta_e.float().unsqueeze(-1),
                             beta_w.float().unsqueeze(-1), log_g,
                             None if s0 is None else s0.unsqueeze(2), want_rnorm=want_scores)
        y = out[0][:, :, :, 0]
        st = out[1][:, :, 0]
        rn = out[2][..., 0] if want_scores else None
    else:
        # a padded key channel has no key, so its decay (1) never matters
        log_g = _pad_last(torch.log(g.float().clamp(min=1e-30)), D)
        out = ops.delta_rule_chan(qe, kp, vp, beta_e, beta_w, log_g, s0, want_rnorm=want_scores)
        y = out[0].to(q.dtype) if q.dtype == torch.bfloat16 else out[0]
        st = out[1]
        rn = out[2] if want_scores else None
    y = y[..., :dv] if dv != D else y
    if want_scores:
        scores = (k.float().norm(dim=-1) * rn).detach()
        res = (y, scores)
    else:
        res = y
    if want_state:
        return res, (st[..., :dk, :dv] if (dk, dv) != (D, D) else st)
    return res


def scan(q, k, v, g, beta_e, beta_w, out_mix=None):
    """y [B,T,H,dv] of the KMD-2 recurrence (differentiable in q, k, v, g,
    beta_e, beta_w and out_mix)."""
    return _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores=False)


def scan_with_update_norm(q, k, v, g, beta_e, beta_w, out_mix=None):
    """(y [B,T,H,dv], scores [B,T,H] float32 detached), scores = |k| |update|."""
    return _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores=True)


def scan_with_state(q, k, v, g, beta_e, beta_w, out_mix=None, state0=None):
    """scan from an initial state: (y [B,T,H,dv], final state [B,H,dk,dv]
    float32), differentiable in the inputs and state0.  The state is the
    reference's S [B,H,dk,dv] (research/kernel_ab/ref_scan.py:24-48 starts it
    at zero); a prefill whose state decode_step then carries."""
    return _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores=False, state0=state0, want_state=True)


def decode_step(q, k, v, g, beta_e, beta_w, state, out_mix=None):
    """One token of the KMD-2 recurrence per sequence on a carried state,
    updated in place (one iteration of research/kernel_ab/ref_scan.py:40-47;
    the reference has no decode path): q [B,H,r_out,dk], k [B,H,dk],
    v [B,H,dv], g [B,H,dk] (multiplicative decay per key channel), beta_e,
    beta_w [B,H], state [B,H,dk,dv] float32.  Returns y [B,H,dv] (float32, or
    bf16 for bf16 q).  Per-channel decay on the gdnx_delta_decode_step_chan
    kernel; the query slots enter mixed (the read is linear in q)."""
    B, H, r_out, dk = q.shape
    dv = v.shape[-1]
    if tuple(state.shape) != (B, H, dk, dv) or state.dtype != torch.float32:
        raise ValueError(f"state must be float32 [B,H,dk,dv] = {[B, H, dk, dv]}")
    D = _kernel_dim(dk, dv)
    dt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    qe = _mixed_query(q.unsqueeze(1), out_mix)[:, 0]
    qe, kp, vp = (_pad_last(x, D).to(dt).contiguous() for x in (qe, k, v))
    log_g = _pad_last(torch.log(g.float().clamp(min=1e-30)), D).unsqueeze(2).contiguous()
    padded = (dk, dv) != (D, D) or not state.is_contiguous()
    pool = _pad_state(state, D).unsqueeze(2) if padded else state.unsqueeze(2)
    y = ops.delta_decode_step_chan(qe, kp, vp, beta_e.float().unsqueeze(-1).contiguous(),
                                   beta_w.float().unsqueeze(-1).contiguous(), log_g, pool)
    if padded:
        state.copy_(pool[:, :, 0, :dk, :dv])
    return y[:, :, 0, :dv]

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
(used when r_out > 1).  dk = dv in {64, 128}.  The HIP kernels carry one
decay per token and head: g must be constant over dk (as in the GDN3 dense
regime, where the lane decay is broadcast); a per-channel decay raises
NotImplementedError rather than being approximated.
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


def _scalar_log_decay(g, check):
    """log of the per-token decay, from g [B,T,H,dk] constant over dk.

    Gradients are exact for a decay expanded over dk (stride 0, e.g.
    g = gamma[..., None].expand(...)): autograd sums them into gamma.  A
    materialised per-channel g has per-channel gradients these kernels do
    not form, so it is refused when it requires grad."""
    if g.requires_grad and g.shape[-1] > 1 and g.stride(-1) != 0:
        raise NotImplementedError("gradients of a materialised per-channel decay are not implemented; "
                                  "pass g as an expand over dk of a per-token decay")
    g0 = g[..., 0]
    if check and g.shape[-1] > 1 and g.stride(-1) != 0:
        if not bool((g.amax(-1) == g.amin(-1)).all()):
            raise NotImplementedError("per-channel decay (g varying over dk) is not implemented in gdnx_amd; "
                                      "pass g constant over dk")
    return torch.log(g0.float().clamp(min=1e-30))


def _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores, check_decay=True):
    B, T, H, r_out, dk = q.shape
    dv = v.shape[-1]
    if dk != dv:
        raise NotImplementedError(f"dk ({dk}) != dv ({dv}) is not supported")
    dt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    qe = _mixed_query(q, out_mix).to(dt)
    log_g = _scalar_log_decay(g, check_decay).unsqueeze(-1)
    a_e = beta_e.float().unsqueeze(-1)
    a_w = beta_w.float().unsqueeze(-1)
    out = ops.delta_rule(qe, k.to(dt), v.to(dt), a_e, a_w, log_g, want_rnorm=want_scores)
    y = out[0][:, :, :, 0]
    if not want_scores:
        return y
    rn = out[2][..., 0]
    scores = (k.float().norm(dim=-1) * rn).detach()
    return y, scores


def scan(q, k, v, g, beta_e, beta_w, out_mix=None):
    """y [B,T,H,dv] of the KMD-2 recurrence (differentiable in q, k, v, g,
    beta_e, beta_w and out_mix)."""
    return _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores=False)


def scan_with_update_norm(q, k, v, g, beta_e, beta_w, out_mix=None):
    """(y [B,T,H,dv], scores [B,T,H] float32 detached), scores = |k| |update|."""
    return _scan(q, k, v, g, beta_e, beta_w, out_mix, want_scores=True)

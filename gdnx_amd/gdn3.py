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
gdn3/gdn3_upgrade.py:641-648).  The elementwise prologue runs in torch
(autograd carries its gradient into beta and k); the recurrence and its
backward are the HIP kernels of libgdnx.
"""
from __future__ import annotations

import torch

from . import ops


def stable_alpha(c, eps: float = 1e-6):
    """alpha(c) = -expm1(-c)/c with the Taylor branch 1 - c/2 + c^2/6 for
    |c| < eps (gdn3/gdn3_upgrade.py:641-648)."""
    small = c.abs() < eps
    safe = torch.where(small, torch.ones_like(c), c)
    return torch.where(small, 1.0 - c / 2.0 + c * c / 6.0, -torch.expm1(-safe) / safe)


def gdn3_coeff(k, beta):
    """a = alpha(beta |k|^2) beta for k [B,T,H,D] shared by beta's M lanes."""
    c = beta.float() * k.float().square().sum(-1, keepdim=True)
    return stable_alpha(c) * beta.float()


def gdn3_scan(q, k, v, beta, log_g, state0=None, return_state=False):
    """Differentiable GDN3 dense-regime recurrence.

    q, k, v: [B,T,H,D] (bf16 or float32, shared by the lanes); beta, log_g:
    [B,T,H,M] float32 (log_g > 0 is clamped, i.e. gamma <= 1).  Returns
    y [B,T,H,M,D] in q's dtype (and the final state [B,H,M,D,D] fp32).
    """
    a = gdn3_coeff(k, beta)
    y, s = ops.delta_rule(q, k, v, a, a, log_g.float(), state0)
    return (y, s) if return_state else y

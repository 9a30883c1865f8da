"""Rank-r block-Householder delta rule with the RLS T-factor -- CPU oracle
(TEST INFRASTRUCTURE ONLY).

Only tests/ and bench.py's cpu_baseline leg use this module, as the checker;
the HIP product path never imports it.

KMD2LinearAttn._scan (gdn3/kmd2.py:166-214) and the testbed mixer's scan
(research/testbed_mqar.py:214-262), per chain (b, h) with the state S
[d_v, d_k] (value-major, as the reference), per token t with r write slots:

    S   <- S diag(a_t)                                  channel decay (key axis)
    Kt   = Bg_t * K_t                                   [r, d_k] gated erase keys
    S   <- S - (S Kt^T) (eps I + Kt Kt^T)^-1 Kt         block erase (RLS T-factor)
    S   <- S + (Wg_t * V_t)^T K_t                       rank-r gated write
    (testbed, every P tokens) compaction, below
    y_t  = sum_o mix_o S q_{t,o}                        r_out query slots

with mix = out_mix[h] when r_out > 1 (otherwise the single read).  For r = 1
the reference's fast path divides by eps + |Kt|^2, which is the same T-factor.

Testbed compaction (research/testbed_mqar.py:245-260), when (t+1) % P == 0:
    S_lr = best rank-R approximation of S (truncated SVD, no gradient)
    plain:            S <- s S_lr + (1 - s) S
    straight-through: S takes the value s S_lr + (1 - s) S, its gradient is
                      the identity

Pinning (tests/test_oracle_rls.py): golden vectors from the reference's own
``_scan`` and the testbed mixer's forward (tests/golden/make_golden_rls.py),
outputs and every input gradient; plus what the mathematics fixes: r = 1
with a scalar erase gate reduces to the delta rule of oracle.delta, a full-rank
compaction is the identity, the straight-through gradient equals the
uncompacted scan's, and the truncation is the Eckart-Young optimum.
"""
from __future__ import annotations

import torch

__all__ = ["rls_scan", "truncate_rank"]


def truncate_rank(S, R):
    """Best rank-R approximation of each [d_v, d_k] matrix of S (no gradient)."""
    with torch.no_grad():
        U, sg, Vh = torch.linalg.svd(S, full_matrices=False)
        return (U[..., :R] * sg[..., None, :R]) @ Vh[..., :R, :]


def rls_scan(q, K, V, Bg, Wg, a, eps=0.5, out_mix=None, *, compact_P=0, compact_R=0, slow_decay=0.97,
             ste=False, state0=None, dtype=torch.float64, return_state=False):
    """q [B,T,H,r_out,dk]; K, Bg [B,T,H,r,dk]; V, Wg [B,T,H,r,dv];
    a [B,T,H,dk]; out_mix [H, r_out] (used when r_out > 1); state0
    [B,H,dv,dk] or None.  Returns y [B,T,H,dv] in ``dtype`` (and the final
    state [B,H,dv,dk] when return_state); differentiable by autograd."""
    B, T, H, r_out, dk = q.shape
    r, dv = V.shape[3], V.shape[4]
    S = (torch.zeros(B, H, dv, dk, dtype=dtype) if state0 is None else state0.to(dtype))
    eye = torch.eye(r, dtype=dtype)
    mix = None if out_mix is None or r_out == 1 else out_mix.to(dtype)
    q, K, V, Bg, Wg, a = (x.to(dtype) for x in (q, K, V, Bg, Wg, a))
    ys = []
    for t in range(T):
        S = S * a[:, t].unsqueeze(2)                               # [B,H,1,dk]
        Kt = Bg[:, t] * K[:, t]                                    # [B,H,r,dk]
        SK = S @ Kt.transpose(-1, -2)                              # [B,H,dv,r]
        Tf = torch.linalg.inv(eps * eye + Kt @ Kt.transpose(-1, -2))
        S = S - SK @ Tf @ Kt
        S = S + (Wg[:, t] * V[:, t]).transpose(-1, -2) @ K[:, t]
        if compact_P and (t + 1) % compact_P == 0:
            S_lr = truncate_rank(S, compact_R)
            if ste:
                S = S + (slow_decay * S_lr + (1 - slow_decay) * S.detach() - S).detach()
            else:
                S = slow_decay * S_lr + (1 - slow_decay) * S
        yt = S @ q[:, t].transpose(-1, -2)                         # [B,H,dv,r_out]
        yt = (yt * mix[None, :, None, :]).sum(-1) if mix is not None else yt[..., 0]
        ys.append(yt)
    y = torch.stack(ys, 1)
    return (y, S) if return_state else y

"""Dense decoupled-erase delta rule -- CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker.  The HIP product path never imports it.

Semantics, with the state S in the key-major layout [d_k, d_v] used by the
reference's KMD-2 scan (research/kernel_ab/ref_scan.py:37-47):

    S_bar = gamma_t * S_{t-1}          gamma scalar per chain, or per key row
    r_t   = w_t - S_bar^T e_t          net write (e = erase key, w = write value)
    S_t   = S_bar + k_t r_t^T
    y_t   = S_t^T q_t                  post-update read

* KMD-2 native (``ref_scan.scan``, research/kernel_ab/ref_scan.py:24-48, and
  ``reference_scan_with_scores``, research/kmd2_ablation/exact_cache.py:1231-1295):
  e = beta_e k, w = beta_w v, gamma per key channel, r_out query slots mixed
  by ``out_mix``; score_t = |k_t| * |beta_w v_t - beta_e k_t^T S_bar|.
* GDN3 in its dense regime (gdn3/_reference_recurrence.py:60-84 with the
  residual buffer never overwritten and never compacted, P >= T) with scalar
  gates b = w = beta: e = a k, w = a v, a = alpha(beta |k|^2) beta, with
  alpha(c) = (1 - exp(-c)) / c (gdn3/gdn3_upgrade.py:641-648) and the decay
  clamped to [0, 1] (gdn3/_reference_recurrence.py:61).

Pinning (see tests/test_oracle_delta.py):
  delta_rule_sequential -- reference known-answer tests
      (tests/ablation/test_exact_cache_math.py:563-597: y=12, score=4; zero
      and sub-epsilon keys), an independent scalar-loop restatement on tiny
      shapes (the pattern of test_exact_cache_math.py:387-494), invariants
      (v=0 => y=0, gamma=0 resets, beta=0 => pure decay).
  kmd2_scan             -- same, plus the r_out mixing identity.
  delta_rule_chunked    -- equals delta_rule_sequential in float64 to 1e-12.
  delta_rule_chunked_chan -- per-key-channel decay; equals
                           delta_rule_sequential (per-channel gamma) in float64.
  stable_alpha          -- closed form, Taylor branch and branch continuity.
"""
from __future__ import annotations

import math

import torch

__all__ = [
    "lane_delta",
    "stable_alpha",
    "delta_rule_sequential",
    "delta_rule_chunked",
    "delta_rule_chunked_chan",
    "kmd2_scan",
    "gdn3_dense_coeffs",
    "gdn3_dense_layer",
]


def stable_alpha(c: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """alpha(c) = (1 - exp(-c)) / c, second-order Taylor series for |c| < eps.

    Follows ``GDN3LinearAttn._stable_alpha_vec`` (gdn3/gdn3_upgrade.py:641-648).
    """
    small = c.abs() < eps
    safe = torch.where(small, torch.ones_like(c), c)
    exact = -torch.expm1(-safe) / safe
    series = 1.0 - c / 2.0 + c * c / 6.0
    return torch.where(small, series, exact)


def delta_rule_sequential(q, k, e, w, gamma, state0=None):
    """Token-by-token decoupled-erase delta rule.

    q, k, e: [N, T, dk]; w: [N, T, dv]; gamma: [N, T] (scalar per chain) or
    [N, T, dk] (per key channel), multiplicative decay.  state0: [N, dk, dv]
    or None (zeros).  Returns (y [N, T, dv], S_T [N, dk, dv]).

    The loop body restates research/kernel_ab/ref_scan.py:40-45 with the erase
    key e and the write key k decoupled (they coincide up to beta_e there).
    """
    N, T, dk = k.shape
    dv = w.shape[-1]
    S = k.new_zeros(N, dk, dv) if state0 is None else state0
    ys = []
    for t in range(T):
        g = gamma[:, t]
        S = S * (g.view(N, 1, 1) if g.dim() == 1 else g.unsqueeze(-1))
        r = w[:, t] - torch.einsum("nkv,nk->nv", S, e[:, t])
        S = S + k[:, t].unsqueeze(-1) * r.unsqueeze(-2)
        ys.append(torch.einsum("nkv,nk->nv", S, q[:, t]))
    return torch.stack(ys, 1), S


def delta_rule_chunked(q, k, e, w, log_gamma, chunk: int = 64, state0=None,
                       log_floor: float = -200.0):
    """Chunk-parallel form of ``delta_rule_sequential`` for scalar decay.

    log_gamma: [N, T] natural log of the per-token decay (<= 0).  Within a
    chunk with carried state S0 and inclusive prefix G_i = sum_{s<=i} log g_s:

        D_ij  = exp(G_i - G_j) [j <= i]        (never a ratio of products)
        (I + L) R = W - diag(exp G) E S0,      L_ij = D_ij (e_i . k_j), j < i
        Y     = diag(exp G) Q S0 + (D o Q K^T) R
        S_C   = exp(G_last) S0 + (diag(D_last,:) K)^T R

    This is the algebra the HIP kernels implement (the reference's chunked
    KMD-2 path, gdn3/kmd2_fast_scan.py:1-18, uses the ratio k/gcumF instead,
    which underflows at chunk 64).  Differentiable with torch autograd.
    ``log_floor`` bounds log-decays so that a zero decay stays finite.
    """
    N, T, dk = k.shape
    dv = w.shape[-1]
    S = k.new_zeros(N, dk, dv) if state0 is None else state0
    lg = log_gamma.clamp(min=log_floor)
    ys = []
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        c = t1 - t0
        Q, K, E, W = q[:, t0:t1], k[:, t0:t1], e[:, t0:t1], w[:, t0:t1]
        G = lg[:, t0:t1].cumsum(1)
        idx = torch.arange(c)
        incl = idx.view(c, 1) >= idx.view(1, c)
        strict = idx.view(c, 1) > idx.view(1, c)
        diff = G.unsqueeze(2) - G.unsqueeze(1)
        D = torch.where(incl, diff, torch.full_like(diff, -math.inf)).exp()
        gam = G.exp()
        L = torch.where(strict, D * (E @ K.transpose(1, 2)), torch.zeros_like(D))
        rhs = W - gam.unsqueeze(-1) * (E @ S)
        eye = torch.eye(c, dtype=k.dtype).expand(N, c, c)
        R = torch.linalg.solve_triangular(eye + L, rhs, upper=False, unitriangular=True)
        Aq = D * (Q @ K.transpose(1, 2))
        ys.append(gam.unsqueeze(-1) * (Q @ S) + Aq @ R)
        dec = (G[:, -1:] - G).exp()
        S = G[:, -1].exp().view(N, 1, 1) * S + (K * dec.unsqueeze(-1)).transpose(1, 2) @ R
    return torch.cat(ys, 1), S


def delta_rule_chunked_chan(q, k, a_e, w, log_gamma, chunk: int = 16, state0=None,
                            log_floor: float = -60.0):
    """Chunk form of ``delta_rule_sequential`` with a decay per key channel.

    q, k: [N, T, dk]; a_e: [N, T] erase coefficient (e_t = a_e,t k_t);
    w: [N, T, dv]; log_gamma: [N, T, dk] natural log of the decay (clamped
    to [log_floor, 0]).  Within a chunk with carried state S0 and per-channel
    inclusive prefix G_i = sum_{s<=i} log g_s ([dk] per token):

        M_ij  = sum_d x_id k_jd exp(G_id - G_jd), j <= i  (every exponent <= 0)
        (I + L) R = W - diag(a_e) (K o e^G) S0,   L_ij = a_e,i M_ij[x=k], j < i
        Y     = (Q o e^G) S0 + Aq R,              Aq_ij = M_ij[x=q], j <= i
        S_C   = diag(e^{G_last}) S0 + (K o e^{G_last - G})^T R

    (gdn3/kmd2_native.py:109-132 restated per chunk; the reference's chunked
    path gdn3/kmd2_fast_scan.py:198-214 divides by the cumulative product
    instead).  The decay-weighted grams are formed per channel, so no factor
    ever exceeds 1.  Differentiable with torch autograd.
    """
    N, T, dk = k.shape
    dv = w.shape[-1]
    S = k.new_zeros(N, dk, dv) if state0 is None else state0
    lg = log_gamma.clamp(min=log_floor, max=0.0)
    ys = []
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        c = t1 - t0
        Q, K, ae, W = q[:, t0:t1], k[:, t0:t1], a_e[:, t0:t1], w[:, t0:t1]
        G = lg[:, t0:t1].cumsum(1)                                   # [N, c, dk]
        idx = torch.arange(c)
        incl = (idx.view(c, 1) >= idx.view(1, c)).view(1, c, c, 1)
        diff = G.unsqueeze(2) - G.unsqueeze(1)                       # [N, i, j, dk]
        Dx = torch.where(incl, diff, torch.full_like(diff, -math.inf)).exp()
        Mk = torch.einsum("nid,njd,nijd->nij", K, K, Dx)
        Mq = torch.einsum("nid,njd,nijd->nij", Q, K, Dx)
        strict = idx.view(c, 1) > idx.view(1, c)
        L = torch.where(strict, ae.unsqueeze(-1) * Mk, torch.zeros_like(Mk))
        E = G.exp()
        rhs = W - ae.unsqueeze(-1) * ((K * E) @ S)
        eye = torch.eye(c, dtype=k.dtype).expand(N, c, c)
        R = torch.linalg.solve_triangular(eye + L, rhs, upper=False, unitriangular=True)
        ys.append((Q * E) @ S + Mq @ R)
        F = (G[:, -1:] - G).exp()
        S = G[:, -1].exp().unsqueeze(-1) * S + (K * F).transpose(1, 2) @ R
    return torch.cat(ys, 1), S


def kmd2_scan(q, k, v, g, beta_e, beta_w, out_mix=None, return_scores=False,
              dtype=torch.float64, state0=None, return_state=False):
    """KMD-2 native scan: ``scan(q, k, v, g, beta_e, beta_w, out_mix)``.

    Restates research/kernel_ab/ref_scan.py:24-48 (identical maths to
    gdn3/kmd2_native.py:109-132) and the update score of
    research/kmd2_ablation/exact_cache.py:1276-1293.
    q [B,T,H,r_out,dk], k [B,T,H,dk], v [B,T,H,dv], g [B,T,H,dk]
    (multiplicative per-channel decay), beta_e/beta_w [B,T,H],
    out_mix [H,r_out] (required iff r_out > 1).  Returns y [B,T,H,dv]
    (and scores [B,T,H], detached, when return_scores).  state0
    [B,H,dk,dv] starts the loop from a carried state instead of zero (the
    reference always starts at zero); return_state appends the final state.
    """
    B, T, H, r_out, dk = q.shape
    dv = v.shape[-1]
    q, k, v, g, be, bw = (x.to(dtype) for x in (q, k, v, g, beta_e, beta_w))
    mix = None if out_mix is None else out_mix.to(dtype)
    S = torch.zeros(B, H, dk, dv, dtype=dtype) if state0 is None else state0.to(dtype)
    ys, scores = [], []
    for t in range(T):
        Sb = g[:, t].unsqueeze(-1) * S
        key = k[:, t]
        m = torch.einsum("bhk,bhkv->bhv", key, Sb)
        upd = bw[:, t].unsqueeze(-1) * v[:, t] - be[:, t].unsqueeze(-1) * m
        S = Sb + key.unsqueeze(-1) * upd.unsqueeze(-2)
        reads = torch.einsum("bhrk,bhkv->bhrv", q[:, t], S)
        if r_out == 1:
            ys.append(reads[:, :, 0])
        else:
            ys.append((reads * mix.view(1, H, r_out, 1)).sum(2))
        scores.append(key.norm(dim=-1) * upd.norm(dim=-1))
    y = torch.stack(ys, 1) if T > 0 else torch.zeros(B, 0, H, dv, dtype=dtype)
    out = (y, torch.stack(scores, 1).detach()) if return_scores else y
    if return_state:
        return (*out, S) if return_scores else (out, S)
    return out


def gdn3_dense_coeffs(k, beta):
    """Effective erase/write coefficient a = alpha(beta |k|^2) * beta.

    k: [..., dk] (shared by the lanes), beta: [..., M] scalar gate per lane.
    With b_gate = w_gate = beta (scalar), h = beta k and c = k.h = beta |k|^2
    (gdn3/_reference_recurrence.py:67-74); the net write stored in the buffer
    is alpha r with r = beta v - S_bar (beta k), so e = w-coefficient = alpha beta.
    """
    c = beta * (k * k).sum(-1, keepdim=True)
    return stable_alpha(c) * beta


def gdn3_dense_layer(q, k, v, beta, log_g, chunk=None, dtype=torch.float64):
    """GDN3 layer recurrence in the dense regime with lanes sharing q/k/v.

    q, k: [B,T,H,dk], v: [B,T,H,dv] (shared by all M lanes), beta: [B,T,H,M],
    log_g: [B,T,H,M] log-decay (clamped to <= 0, i.e. gamma clamped to 1).
    Returns y [B,T,H,M,dv].  chunk=None runs the sequential loop, otherwise
    the chunked algebra (same maths).
    """
    B, T, H, dk = k.shape
    M = beta.shape[-1]
    dv = v.shape[-1]
    q, k, v, beta, log_g = (x.to(dtype) for x in (q, k, v, beta, log_g))
    a = gdn3_dense_coeffs(k, beta)                                 # [B,T,H,M]

    def chains(x):                                                 # [B,T,H,d] -> [N,T,d]
        x = x.unsqueeze(3).expand(B, T, H, M, x.shape[-1])
        return x.permute(0, 2, 3, 1, 4).reshape(B * H * M, T, x.shape[-1])

    qc, kc, vc = chains(q), chains(k), chains(v)
    ac = a.permute(0, 2, 3, 1).reshape(B * H * M, T)
    lg = log_g.clamp(max=0.0).permute(0, 2, 3, 1).reshape(B * H * M, T)
    ec = kc * ac.unsqueeze(-1)
    wc = vc * ac.unsqueeze(-1)
    if chunk is None:
        y, _ = delta_rule_sequential(qc, kc, ec, wc, lg.exp())
    else:
        y, _ = delta_rule_chunked(qc, kc, ec, wc, lg, chunk=chunk)
    return y.reshape(B, H, M, T, dv).permute(0, 3, 1, 2, 4)


def lane_delta(q, k, v, a_e, a_w, log_g, state0=None, chunk=None, dtype=torch.float64):
    """Lane-shared delta rule with explicit per-lane coefficients (the HIP
    op's interface): q, k, v [B,T,H,D], a_e, a_w, log_g [B,T,H,M], state0
    [B,H,M,D,D] or None.  e = a_e k, w = a_w v, gamma = exp(min(log_g, 0)).
    Returns (y [B,T,H,M,D], S_T [B,H,M,D,D]); differentiable."""
    B, T, H, D = k.shape
    M = a_e.shape[-1]
    q, k, v, a_e, a_w, log_g = (x.to(dtype) for x in (q, k, v, a_e, a_w, log_g))

    def chains(x):
        x = x.unsqueeze(3).expand(B, T, H, M, D)
        return x.permute(0, 2, 3, 1, 4).reshape(B * H * M, T, D)

    qc, kc, vc = chains(q), chains(k), chains(v)
    ae = a_e.permute(0, 2, 3, 1).reshape(B * H * M, T, 1)
    aw = a_w.permute(0, 2, 3, 1).reshape(B * H * M, T, 1)
    lg = log_g.clamp(max=0.0).permute(0, 2, 3, 1).reshape(B * H * M, T)
    s0 = None if state0 is None else state0.to(dtype).reshape(B * H * M, D, D)
    if chunk is None:
        y, S = delta_rule_sequential(qc, kc, kc * ae, vc * aw, lg.exp(), s0)
    else:
        y, S = delta_rule_chunked(qc, kc, kc * ae, vc * aw, lg, chunk=chunk, state0=s0)
    return y.reshape(B, H, M, T, D).permute(0, 3, 1, 2, 4), S.reshape(B, H, M, D, D)

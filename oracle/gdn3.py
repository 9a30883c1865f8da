"""GDN3 Kronecker-residual recurrence -- CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker.  The HIP product path never imports it.

State per chain n (N = B*H*M chains, GDN3 layout [d_v, d_k]):
    S = sum_r A_r (x) B_r + U Vb^T,  A [R,a_v,a_k], B [R,b_v,b_k], U [V,P], Vb [K,P]
Per token (gdn3/_reference_recurrence.py:60-90):
    gamma = clamp(dec, 0, 1);  A, B, Vb *= gamma   (A(x)B decays by gamma^2)
    h = b (.) k;  u = w (.) v;  r = u - S h;  alpha = alpha(k.h)
    y = S q + alpha (k.q) r                         (post-update read)
    U[:, p] = alpha r;  Vb[:, p] = k;  p = t mod P  (circular, always full)
    compaction after token t when (t+1) mod K_c == 0, under no_grad; U, Vb kept.
With K_c = P this is the reference loop exactly (its slot counter resets to 0 at
each compaction, _reference_recurrence.py:84-90); K_c must be a multiple of P.

Compaction (gdn3/gdn3_upgrade.py:650-719 ``_compact_vec``; on the CPU the same
computation as ``_compact_fast`` in 'svd' mode, :565-624):
    R_mat = sum_r vec(A_r) vec(B_r)^T + rearrange(U Vb^T)        [a_v a_k, b_v b_k]
    randomized range finder with sketch G [N, n, q], q = min(R+4, m, n), two
    power iterations, QR, SVD of the q x n projection; top-R singular triplets
    give A_svd_r = sigma_r u_r, B_svd_r = v_r;  A <- s A + (1-s) A_svd,
    B <- s B + (1-s) B_svd;  err = max(0, |R_mat|^2 - sum_{r<R} sigma_r^2)
    summed over the batch.
The sketch is an explicit input; ``reference_sketch`` reproduces the
reference's Generator(cpu).manual_seed(1234) float32 draw.  ``sign_mode``:
'lapack' keeps torch.linalg.svd's signs (what the reference does on the CPU);
'canonical' flips each (u_r, v_r) pair so that the largest-magnitude entry of
v_r is positive (first index on ties) -- the convention the HIP kernel uses.

Pinning (tests/test_oracle_gdn3.py):
  kron_read        -- brute force against torch.kron materialisation.
  compact          -- golden vectors written from the reference's own
                      _compact_vec / _compact_fast (tests/golden/), plus
                      invariants (s=1 keeps A,B; exact rank-R recovery; err>=0).
  gdn3_recurrence  -- golden vectors from reference_recurrent_state, and the
                      bridge identity to delta.gdn3_dense_layer for P >= T.
"""
from __future__ import annotations

import torch

from .delta import stable_alpha

__all__ = ["kron_read", "reference_sketch", "sketch_width", "compact", "compact_sketch", "gdn3_recurrence"]


def kron_read(A, Bk, U, Vb, x):
    """S x for S = sum_r A_r (x) B_r + U Vb^T without forming S.

    (A (x) B) x = vec(A X B^T), X = x.reshape(a_k, b_k) (gdn3/kernels.py:7-16);
    follows ``_kron_read_vec`` (gdn3/gdn3_upgrade.py:626-639).
    A [N,R,a_v,a_k], Bk [N,R,b_v,b_k], U [N,V,P], Vb [N,K,P], x [N,K] -> [N,V].
    """
    N, R, a_v, a_k = A.shape
    b_v, b_k = Bk.shape[-2:]
    X = x.reshape(N, a_k, b_k)
    AX = torch.einsum("nrvk,nkb->nrvb", A, X)
    AXB = torch.einsum("nrvb,nrwb->nvw", AX, Bk)
    y = AXB.reshape(N, a_v * b_v)
    coeff = torch.einsum("nkp,nk->np", Vb, x)
    return y + torch.einsum("nvp,np->nv", U, coeff)


def reference_sketch(N, n, q):
    """The reference's compaction sketch, drawn as it does on the CPU:
    torch.Generator(cpu).manual_seed(1234); randn(N, n, q) in float32
    (gdn3/gdn3_upgrade.py:681-682 and :552-563)."""
    gen = torch.Generator(device="cpu").manual_seed(1234)
    return torch.randn(N, n, q, dtype=torch.float32, generator=gen)


def _canonical_signs(Us, Vs):
    # flip (u_r, v_r) so the largest-|.| entry of v_r is positive (first on ties)
    idx = Vs.abs().argmax(dim=1, keepdim=True)                  # [N,1,q]
    sgn = torch.sign(torch.gather(Vs, 1, idx))
    sgn = torch.where(sgn == 0, torch.ones_like(sgn), sgn)
    return Us * sgn, Vs * sgn


def sketch_width(R, m, n, mode="svd"):
    """Columns of the compaction sketch: min(R + 4, m, n) for 'svd'
    (gdn3/gdn3_upgrade.py:677), R for 'sketch' / 'sketch_noqr' (:580)."""
    return R if mode in ("sketch", "sketch_noqr") else min(R + 4, m, n)


def _rearranged(A, Bk, U, Vb):
    N, R, a_v, a_k = A.shape
    b_v, b_k = Bk.shape[-2:]
    vecA = A.reshape(N, R, a_v * a_k)
    vecB = Bk.reshape(N, R, b_v * b_k)
    Rm = torch.einsum("nra,nrb->nab", vecA, vecB)
    Sres = torch.einsum("nvp,nkp->nvk", U, Vb)
    Sres = (Sres.reshape(N, a_v, b_v, a_k, b_k).permute(0, 1, 3, 2, 4)
            .reshape(N, a_v * a_k, b_v * b_k))
    return Rm + Sres


def compact_sketch(A, Bk, U, Vb, slow_decay, sketch):
    """The 'sketch' and 'sketch_noqr' compaction modes (one branch in the
    reference, gdn3/gdn3_upgrade.py:579-592): no range finder, no SVD.  With
    the sketch G [N, n, R]: Y = R_mat G; Q = Y with unit columns (norms
    clamped at 1e-12); Bm = Q^T R_mat; A_svd_r = |Bm_r| Q_r,
    B_svd_r = Bm_r / |Bm_r|; the blend as in ``compact``; error 0."""
    N, R, a_v, a_k = A.shape
    b_v, b_k = Bk.shape[-2:]
    Rm = _rearranged(A, Bk, U, Vb)
    G = sketch.to(Rm.dtype)
    assert G.shape == (N, b_v * b_k, R), (G.shape, (N, b_v * b_k, R))
    Y = Rm @ G
    Q = Y / Y.square().sum(1).sqrt().clamp_min(1e-12)[:, None, :]
    Bm = Q.transpose(-2, -1) @ Rm
    b_scale = Bm.square().sum(-1).sqrt().clamp_min(1e-12)
    A_svd = (Q * b_scale[:, None, :]).permute(0, 2, 1).reshape(N, R, a_v, a_k)
    B_svd = (Bm / b_scale[:, :, None]).reshape(N, R, b_v, b_k)
    s = slow_decay
    return s * A + (1 - s) * A_svd, s * Bk + (1 - s) * B_svd, torch.zeros((), dtype=Rm.dtype)


def compact(A, Bk, U, Vb, slow_decay, sketch, sign_mode="lapack", mode="svd"):
    """Rearrangement-SVD compaction with two-timescale blend.

    Restates gdn3/gdn3_upgrade.py:650-719.  Returns (A_new, B_new, err); the
    residual buffer U, Vb is left unchanged by the reference (:719).  mode
    'sketch' / 'sketch_noqr' runs ``compact_sketch`` instead.
    """
    if mode in ("sketch", "sketch_noqr"):
        return compact_sketch(A, Bk, U, Vb, slow_decay, sketch)
    if mode != "svd":
        raise ValueError(f"unknown compaction mode {mode!r}")
    N, R, a_v, a_k = A.shape
    b_v, b_k = Bk.shape[-2:]
    Rm = _rearranged(A, Bk, U, Vb)
    energy = (Rm ** 2).sum()
    m, n = Rm.shape[-2:]
    qr = min(R + 4, m, n)
    G = sketch.to(Rm.dtype)
    assert G.shape == (N, n, qr), (G.shape, (N, n, qr))
    Y = Rm @ G
    for _ in range(2):
        Y = Rm @ (Rm.transpose(-2, -1) @ Y)
    Q, _ = torch.linalg.qr(Y)
    Bm = Q.transpose(-2, -1) @ Rm
    Ub, Ss, Vh = torch.linalg.svd(Bm, full_matrices=False)
    Us = Q @ Ub
    Vs = Vh.transpose(-2, -1)
    if sign_mode == "canonical":
        Us, Vs = _canonical_signs(Us, Vs)
    elif sign_mode != "lapack":
        raise ValueError(f"unknown sign_mode {sign_mode!r}")
    kept = (Ss[:, :R] ** 2).sum()
    err = (energy - kept).clamp(min=0.0)
    A_svd = (Us[:, :, :R] * Ss[:, None, :R]).permute(0, 2, 1).reshape(N, R, a_v, a_k)
    B_svd = Vs[:, :, :R].permute(0, 2, 1).reshape(N, R, b_v, b_k)
    s = slow_decay
    return s * A + (1 - s) * A_svd, s * Bk + (1 - s) * B_svd, err


def gdn3_recurrence(q, k, v, b_gates, w_gates, dec, *, R=4, P=16,
                    factors=(16, 16, 8, 8), slow_decay=0.97, compact_every=None,
                    sketch=None, sign_mode="lapack", dtype=torch.float64,
                    return_state=False, state0=None, t0=0, compact_mode="svd"):
    """Sequential GDN3 recurrence, ``reference_recurrent_state`` generalised.

    Restates gdn3/_reference_recurrence.py:33-94.  q,k,b_gates [B,T,H,M,K],
    v,w_gates [B,T,H,M,V], dec [B,T,H,M] (multiplicative decay, clamped to
    [0,1]).  factors = (a_v, a_k, b_v, b_k) with a_v*b_v = V, a_k*b_k = K.
    compact_every = K_c (default P).  Returns y [B,T,H,M,V] (and the final
    state (A, Bk, U, Vb) plus the summed compaction error when return_state).

    Carried state (no counterpart in the reference, whose loop always starts
    from zero at p = 0): state0 = (A, Bk, U, Vb) in the layouts above, as a
    previous call returned them, and t0 = the number of tokens that call had
    processed.  Token t of this call is then global token t0 + t: it writes
    slot (t0 + t) mod P and a compaction follows it when (t0 + t + 1) mod K_c
    == 0, so running [0, T1) and then [T1, T) from the returned state equals
    one run over [0, T).
    """
    B, T, H, M, K = q.shape
    V = v.shape[-1]
    a_v, a_k, b_v, b_k = factors
    assert a_v * b_v == V and a_k * b_k == K
    Kc = P if compact_every is None else compact_every
    assert Kc % P == 0, "compaction interval must be a multiple of P"
    N = B * H * M

    def flat(x, d):
        return x.permute(1, 0, 2, 3, 4).reshape(T, N, d).to(dtype)

    qf, kf, vf = flat(q, K), flat(k, K), flat(v, V)
    bg, wg = flat(b_gates, K), flat(w_gates, V)
    dc = dec.permute(1, 0, 2, 3).reshape(T, N).to(dtype)
    qrank = sketch_width(R, a_v * a_k, b_v * b_k, compact_mode)
    G = reference_sketch(N, b_v * b_k, qrank) if sketch is None else sketch

    if state0 is None:
        A = torch.zeros(N, R, a_v, a_k, dtype=dtype)
        Bk = torch.zeros(N, R, b_v, b_k, dtype=dtype)
        U = torch.zeros(N, V, P, dtype=dtype)
        Vb = torch.zeros(N, K, P, dtype=dtype)
    else:
        A, Bk, U, Vb = (x.to(dtype) for x in state0)
        assert A.shape == (N, R, a_v, a_k) and Bk.shape == (N, R, b_v, b_k)
        assert U.shape == (N, V, P) and Vb.shape == (N, K, P)
    ys = []
    err_total = torch.zeros((), dtype=dtype)
    for tl in range(T):
        t = t0 + tl
        gam = dc[tl].clamp(0.0, 1.0)
        A = A * gam.view(N, 1, 1, 1)
        Bk = Bk * gam.view(N, 1, 1, 1)
        Vb = Vb * gam.view(N, 1, 1)
        kt, qt = kf[tl], qf[tl]
        h = bg[tl] * kt
        u = wg[tl] * vf[tl]
        r = u - kron_read(A, Bk, U, Vb, h)
        alpha = stable_alpha((kt * h).sum(-1))
        s_q = kron_read(A, Bk, U, Vb, qt)
        ys.append(s_q + (alpha * (kt * qt).sum(-1)).unsqueeze(-1) * r)
        slot = torch.tensor([t % P])
        U = U.index_copy(2, slot, (alpha.unsqueeze(-1) * r).unsqueeze(-1))
        Vb = Vb.index_copy(2, slot, kt.unsqueeze(-1))
        if (t + 1) % Kc == 0:
            with torch.no_grad():
                A, Bk, err = compact(A.detach(), Bk.detach(), U, Vb, slow_decay, G,
                                     sign_mode, mode=compact_mode)
            err_total = err_total + err
    Y = torch.stack(ys, 0).reshape(T, B, H, M, V).permute(1, 0, 2, 3, 4)
    if return_state:
        return Y, (A, Bk, U, Vb), err_total
    return Y

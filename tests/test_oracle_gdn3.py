"""Pins the GDN3 Kronecker-residual oracle (CPU only).

Golden vectors in tests/golden/gdn3_golden.npz were written by
tests/golden/make_golden.py from the reference's own _compact_vec,
_compact_fast, reference_recurrent_state and chunked _gdn3_recurrent_state.
"""
import os

import numpy as np
import pytest
import torch

from oracle import delta, gdn3

GOLD = os.path.join(os.path.dirname(__file__), "golden", "gdn3_golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def test_kron_read_matches_dense_materialisation():
    gen = torch.Generator().manual_seed(3)
    d = torch.float64
    N, R = 2, 3
    A = torch.randn(N, R, 4, 2, generator=gen, dtype=d)
    Bk = torch.randn(N, R, 3, 5, generator=gen, dtype=d)
    U = torch.randn(N, 12, 7, generator=gen, dtype=d)
    Vb = torch.randn(N, 10, 7, generator=gen, dtype=d)
    x = torch.randn(N, 10, generator=gen, dtype=d)
    S = torch.stack([sum(torch.kron(A[n, r], Bk[n, r]) for r in range(R)) + U[n] @ Vb[n].T
                     for n in range(N)])
    torch.testing.assert_close(gdn3.kron_read(A, Bk, U, Vb, x), torch.einsum("nvk,nk->nv", S, x),
                               atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("which", ["vec", "fast"])
def test_compact_matches_reference_golden(gold, which):
    A, Bk, U, Vb = gold["compact_A"], gold["compact_Bk"], gold["compact_U"], gold["compact_Vb"]
    G = gdn3.reference_sketch(3, 64, 8)
    A1, B1, err = gdn3.compact(A, Bk, U, Vb, 0.97, G, "lapack")
    torch.testing.assert_close(A1, gold[f"compact_{which}_A"], atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(B1, gold[f"compact_{which}_B"], atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(err.reshape(1), gold[f"compact_{which}_err"], atol=1e-2, rtol=1e-4)
    # the float64 restatement agrees too (same signs on this input)
    A2, B2, _ = gdn3.compact(A.double(), Bk.double(), U.double(), Vb.double(), 0.97, G, "lapack")
    torch.testing.assert_close(A2.float(), gold[f"compact_{which}_A"], atol=5e-5, rtol=1e-3)


def _kron_sum(A, Bk):
    N, R = A.shape[:2]
    return torch.stack([sum(torch.kron(A[n, r], Bk[n, r]) for r in range(R)) for n in range(N)])


@pytest.mark.parametrize("sign_mode", ["lapack", "canonical"])
def test_compact_recovers_exact_rank_R_state(sign_mode):
    gen = torch.Generator().manual_seed(11)
    d = torch.float64
    N, R = 2, 4
    A = torch.randn(N, R, 16, 16, generator=gen, dtype=d)
    Bk = torch.randn(N, R, 8, 8, generator=gen, dtype=d)
    zero = torch.zeros(N, 128, 16, dtype=d)
    G = gdn3.reference_sketch(N, 64, 8)
    A1, B1, err = gdn3.compact(A, Bk, zero, zero, 0.0, G, sign_mode)
    torch.testing.assert_close(_kron_sum(A1, B1), _kron_sum(A, Bk), atol=1e-9, rtol=1e-9)
    assert abs(err.item()) < 1e-8 * (_kron_sum(A, Bk) ** 2).sum().item()
    # s = 1 keeps the factors
    A2, B2, err2 = gdn3.compact(A, Bk, zero, zero, 1.0, G, sign_mode)
    assert torch.equal(A2, A) and torch.equal(B2, Bk) and err2.item() >= 0


def test_canonical_signs_are_a_pair_flip_of_lapack():
    gen = torch.Generator().manual_seed(12)
    d = torch.float64
    N = 3
    A = torch.randn(N, 4, 16, 16, generator=gen, dtype=d) * 0.2
    Bk = torch.randn(N, 4, 8, 8, generator=gen, dtype=d) * 0.2
    U = torch.randn(N, 128, 16, generator=gen, dtype=d)
    Vb = torch.randn(N, 128, 16, generator=gen, dtype=d)
    G = gdn3.reference_sketch(N, 64, 8)
    Al, Bl, el = gdn3.compact(A, Bk, U, Vb, 0.0, G, "lapack")
    Ac, Bc, ec = gdn3.compact(A, Bk, U, Vb, 0.0, G, "canonical")
    torch.testing.assert_close(_kron_sum(Ac, Bc), _kron_sum(Al, Bl), atol=1e-10, rtol=1e-10)
    assert el.item() == pytest.approx(ec.item())
    for n in range(N):
        for r in range(4):
            v = Bc[n, r].flatten()
            assert v[v.abs().argmax()] > 0


def _seqA_inputs(gold):
    return [gold["seqA_" + n] for n in ("q", "k", "v", "bg", "wg", "dec")]


def test_recurrence_matches_reference_loop_fp32(gold):
    y = gdn3.gdn3_recurrence(*_seqA_inputs(gold), dtype=torch.float32)
    torch.testing.assert_close(y, gold["seqA_y"], atol=2e-5, rtol=1e-4)


def test_recurrence_fp64_matches_reference_loop(gold):
    y = gdn3.gdn3_recurrence(*_seqA_inputs(gold), dtype=torch.float64)
    rel = ((y.float() - gold["seqA_y"]).norm() / gold["seqA_y"].norm()).item()
    assert rel < 2e-4      # the reference runs its SVDs in float32


def test_recurrence_gradients_match_reference(gold):
    ins = [t.double().requires_grad_(True) for t in _seqA_inputs(gold)]
    y = gdn3.gdn3_recurrence(*ins, dtype=torch.float64)
    grads = torch.autograd.grad(y.pow(2).mean(), ins)
    for name, g in zip(["q", "k", "v", "bg", "wg", "dec"], grads):
        ref = gold["seqA_grad_" + name]
        rel = ((g.float() - ref).norm() / ref.norm()).item()
        assert rel < 1e-4, (name, rel)


def test_canonical_sign_divergence_is_bounded(gold):
    """Finding F2 quantified.  The GPU kernels fix the sign of each right
    singular vector canonically (largest-|.| entry positive); the reference
    keeps whatever its SVD backend returns (gdn3/gdn3_upgrade.py:605,696).
    Both are exact compactions, so the gap is rounding amplified by the
    singular-value gaps, carried forward by the 0.97 blend.  Measured (fp64
    oracle, same inputs): golden case A 8.4e-5 rel-L2 from the reference's own
    y overall, 1.4e-4 from the third window on; 8.0e-5 / 1.3e-4 between the
    two sign modes; a 1024-token run with a compaction every 16 tokens (64
    compactions) 4.5e-4 to 5.2e-4 per 256-token block.  The bands below move
    if either convention or the blend changes."""
    ins = _seqA_inputs(gold)
    yc = gdn3.gdn3_recurrence(*ins, sign_mode="canonical")
    yl = gdn3.gdn3_recurrence(*ins, sign_mode="lapack")
    ref = gold["seqA_y"].double()

    def rel(a, b):
        return ((a - b).norm() / b.norm()).item()
    assert 4e-5 <= rel(yc, ref) <= 2e-4
    assert 7e-5 <= rel(yc[:, 32:], ref[:, 32:]) <= 3e-4
    assert 4e-5 <= rel(yc, yl) <= 2e-4
    # long horizon at the layer default (P = K_c = 16)
    g = torch.Generator().manual_seed(81)
    B, T, H, M, D = 1, 1024, 1, 1, 128
    q = torch.nn.functional.normalize(torch.randn(B, T, H, M, D, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, M, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, M, D, generator=g)
    bg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    wg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    dec = torch.exp(torch.log1p(-torch.tensor(0.02)) + 0.01 * torch.randn(B, T, H, M, generator=g)).clamp(max=1)
    yc = gdn3.gdn3_recurrence(q, k, v, bg, wg, dec, sign_mode="canonical")
    yl = gdn3.gdn3_recurrence(q, k, v, bg, wg, dec, sign_mode="lapack")
    blocks = [rel(yc[:, i:i + 256], yl[:, i:i + 256]) for i in range(0, T, 256)]
    assert all(2e-4 <= b <= 1e-3 for b in blocks), blocks


def test_reference_chunked_path_departs_from_its_oracle(gold):
    """Finding F1: the reference's chunked path never decays A, B between
    compactions, so from the third window on it differs from the frozen
    sequential loop by more than its own parity tolerance (atol 1e-4)."""
    diff = (gold["seqA_ychunk"] - gold["seqA_y"]).abs()
    assert diff[:, :32].max() < 1e-4          # first two windows agree
    assert diff[:, 32:].max() > 1e-4          # from the third window on they do not


def test_config0_gdn3_mode_matches_reference(gold):
    from oracle import inputs
    x = inputs.config0()
    beta = x["beta"]
    bg = beta.unsqueeze(-1).expand(*beta.shape, 64)
    y = gdn3.gdn3_recurrence(x["q"].unsqueeze(3), x["k"].unsqueeze(3), x["v"].unsqueeze(3), bg, bg,
                             x["g"].exp(), R=4, P=64, factors=(8, 8, 8, 8), dtype=torch.float64)
    rel = ((y.float() - gold["seqB_y"]).norm() / gold["seqB_y"].norm()).item()
    assert rel < 1e-5


def test_bridge_gdn3_without_compaction_is_the_dense_rule():
    """P >= T (buffer never overwritten, compaction only after the last token)
    and scalar gates b = w = beta: GDN3 equals the dense rule with
    beta_e = beta_w = alpha(beta |k|^2) beta."""
    from oracle import inputs
    x = inputs.dense_inputs(1, 24, 2, 16, M=2, seed=9, decay="tau", taus=(0.05, 0.001))
    beta = x["beta"]
    B, T, H, M = beta.shape
    q5 = x["q"].unsqueeze(3).expand(B, T, H, M, 16)
    k5 = x["k"].unsqueeze(3).expand(B, T, H, M, 16)
    v5 = x["v"].unsqueeze(3).expand(B, T, H, M, 16)
    gate = beta.unsqueeze(-1).expand(B, T, H, M, 16)
    y1 = gdn3.gdn3_recurrence(q5, k5, v5, gate, gate, x["g"].double().exp(), R=2, P=T,
                              factors=(4, 4, 4, 4))
    y2 = delta.gdn3_dense_layer(x["q"], x["k"], x["v"], beta, x["g"])
    torch.testing.assert_close(y1, y2, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("P,Kc,splits", [(16, 16, (7, 33)), (16, 48, (16, 50)), (32, 32, (31, 32, 65))])
def test_carried_state_split_equals_whole_run(P, Kc, splits):
    """The oracle's carried state (state0, t0) continues the whole-run loop
    exactly: runs over [0, s1), [s1, s2), ... from each returned state equal
    one run, through slot wrap-arounds and compactions (mid-window splits
    included).  The whole run itself is pinned by the golden vectors above."""
    g = torch.Generator().manual_seed(5)
    B, T, H, M, D = 1, 80, 1, 2, 64
    q, k = (torch.nn.functional.normalize(torch.randn(B, T, H, M, D, generator=g), dim=-1) for _ in range(2))
    v = torch.randn(B, T, H, M, D, generator=g)
    bg, wg = (torch.sigmoid(torch.randn(B, T, H, M, D, generator=g)) for _ in range(2))
    dec = torch.rand(B, T, H, M, generator=g) * 0.1 + 0.9
    kw = dict(R=4, P=P, factors=(8, 8, 8, 8), compact_every=Kc, return_state=True)
    y, st, err = gdn3.gdn3_recurrence(q, k, v, bg, wg, dec, **kw)
    bounds = (0,) + splits + (T,)
    ys, s, e_tot = [], None, 0.0
    for a, b in zip(bounds[:-1], bounds[1:]):
        yy, s, e = gdn3.gdn3_recurrence(q[:, a:b], k[:, a:b], v[:, a:b], bg[:, a:b], wg[:, a:b], dec[:, a:b],
                                      state0=s, t0=a, **kw)
        ys.append(yy)
        e_tot += e.item()
    assert torch.allclose(torch.cat(ys, 1), y, rtol=0, atol=1e-12)
    for x1, x2 in zip(s, st):
        assert torch.allclose(x1, x2, rtol=0, atol=1e-12)
    assert abs(e_tot - err.item()) <= 1e-9 * max(1.0, err.item())


def _rearrange_loops(S, a_v, a_k, b_v, b_k):
    """R_mat[(i, j), (k, l)] = S[i*b_v + k, j*b_k + l], by explicit loops (the
    Van Loan-Pitsianis rearrangement: sum_r kron(A_r, B_r) <-> sum_r vec(A_r) vec(B_r)^T)."""
    Rm = torch.empty(a_v * a_k, b_v * b_k, dtype=S.dtype)
    for i in range(a_v):
        for j in range(a_k):
            for kk in range(b_v):
                for ll in range(b_k):
                    Rm[i * a_k + j, kk * b_k + ll] = S[i * b_v + kk, j * b_k + ll]
    return Rm


def test_compact_sketch_closed_form():
    """slow_decay 0: the new Kronecker sum is Q Q^T R_mat, Q = the columns of
    R_mat G normalised to unit length; B rows have unit norm; error 0; the
    blend is linear in slow_decay."""
    gen = torch.Generator().manual_seed(5)
    d = torch.float64
    N, R, a_v, a_k, b_v, b_k, P = 2, 3, 4, 2, 3, 5, 6
    A = torch.randn(N, R, a_v, a_k, generator=gen, dtype=d)
    Bk = torch.randn(N, R, b_v, b_k, generator=gen, dtype=d)
    U = torch.randn(N, a_v * b_v, P, generator=gen, dtype=d)
    Vb = torch.randn(N, a_k * b_k, P, generator=gen, dtype=d)
    G = torch.randn(N, b_v * b_k, R, generator=gen, dtype=d)
    A0, B0, err = gdn3.compact(A, Bk, U, Vb, 0.0, G, mode="sketch")
    assert err.item() == 0.0
    S = _kron_sum(A, Bk) + U @ Vb.transpose(1, 2)
    S_new = _kron_sum(A0, B0)
    for n in range(N):
        Rm = _rearrange_loops(S[n], a_v, a_k, b_v, b_k).numpy()
        Y = Rm @ G[n].numpy()
        Q = Y / np.linalg.norm(Y, axis=0, keepdims=True)
        np.testing.assert_allclose(_rearrange_loops(S_new[n], a_v, a_k, b_v, b_k).numpy(), Q @ Q.T @ Rm,
                                   rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(B0.reshape(N, R, -1).norm(dim=-1).numpy(), 1.0, rtol=1e-12)
    A1, B1, _ = gdn3.compact(A, Bk, U, Vb, 0.9, G, mode="sketch_noqr")
    torch.testing.assert_close(A1, 0.9 * A + 0.1 * A0, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(B1, 0.9 * Bk + 0.1 * B0, atol=1e-12, rtol=1e-12)
    with pytest.raises(ValueError):
        gdn3.compact(A, Bk, U, Vb, 0.9, G, mode="qr")


def test_compact_sketch_rank_one_known_answers():
    """A rank-one R_mat = a b^T: one sketch column recovers it exactly; R
    columns, all parallel to a, give R a b^T (the sketch modes skip the
    orthogonalisation)."""
    gen = torch.Generator().manual_seed(9)
    d = torch.float64
    a = torch.randn(1, 1, 4, 2, generator=gen, dtype=d)
    b = torch.randn(1, 1, 3, 5, generator=gen, dtype=d)
    zU, zV = torch.zeros(1, 12, 4, dtype=d), torch.zeros(1, 10, 4, dtype=d)
    A1, B1, _ = gdn3.compact(a, b, zU, zV, 0.0, torch.randn(1, 15, 1, generator=gen, dtype=d), mode="sketch")
    torch.testing.assert_close(_kron_sum(A1, B1), _kron_sum(a, b), atol=1e-12, rtol=1e-12)
    for R in (2, 3):
        A = torch.cat([a, torch.zeros(1, R - 1, 4, 2, dtype=d)], 1)
        Bk = torch.cat([b, torch.zeros(1, R - 1, 3, 5, dtype=d)], 1)
        A1, B1, _ = gdn3.compact(A, Bk, zU, zV, 0.0, torch.randn(1, 15, R, generator=gen, dtype=d),
                                 mode="sketch")
        torch.testing.assert_close(_kron_sum(A1, B1), R * _kron_sum(a, b), atol=1e-12, rtol=1e-12)


def test_recurrence_sketch_mode_width():
    """The recurrence draws a width-R sketch in the sketch modes and a
    width-min(R+4, m, n) one for svd."""
    assert gdn3.sketch_width(4, 256, 64, "sketch") == 4
    assert gdn3.sketch_width(4, 256, 64, "svd") == 8
    assert gdn3.sketch_width(4, 6, 64, "svd") == 6

"""The rank-r RLS T-factor scan oracle (oracle/rls.py) against the reference's
own scan and testbed mixer (golden vectors from tests/golden/make_golden_rls.py:
outputs and every input gradient), and against what the mathematics fixes."""
import os

import numpy as np
import pytest
import torch

from oracle import delta as od
from oracle import rls

GOLD = os.path.join(os.path.dirname(__file__), "golden", "rls_golden.npz")


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()


@pytest.fixture(scope="module")
def gold():
    z = np.load(GOLD, allow_pickle=False)
    out = {}
    for key in z.files:
        case, name = key.split("/")
        out.setdefault(case, {})[name] = torch.from_numpy(z[key])
    return out


@pytest.mark.parametrize("case", ["r1", "r2o2"])
def test_scan_matches_reference(gold, case):
    g = gold[case]
    names = ["q", "K", "V", "Bg", "Wg", "a"]
    r_out = g["q"].shape[3]
    leaves = [g[n].double().requires_grad_(True) for n in names]
    mix = g["out_mix"].double().requires_grad_(True)
    y = rls.rls_scan(*leaves, eps=float(g["eps"][0]), out_mix=mix)
    assert rel(y, g["y"]) <= 1e-5
    params = leaves + ([mix] if r_out > 1 else [])
    grads = torch.autograd.grad(y, params, g["dy"].double())
    for n, d in zip(names + ["out_mix"], grads):
        assert rel(d, g["d" + n]) <= 1e-4, n


@pytest.mark.parametrize("case,ste", [("tb_plain", False), ("tb_ste", True)])
def test_testbed_compaction_matches_reference(gold, case, ste):
    g = gold[case]
    leaves = {n: g[n].double().requires_grad_(True)
              for n in ("q", "K", "V", "bg_logit", "wg_logit", "dec_logit")}
    Bg = torch.sigmoid(leaves["bg_logit"])
    Wg = torch.sigmoid(leaves["wg_logit"])
    a = torch.sigmoid(leaves["dec_logit"]).clamp(max=0.9995)     # testbed_mqar.py:212
    y = rls.rls_scan(leaves["q"], leaves["K"], leaves["V"], Bg, Wg, a, eps=float(g["eps"][0]),
                     compact_P=int(g["P"][0]), compact_R=int(g["R"][0]), slow_decay=0.97, ste=ste)
    assert rel(y, g["y"]) <= 1e-5
    grads = torch.autograd.grad(y, list(leaves.values()), g["dy"].double())
    for n, d in zip(leaves, grads):
        assert rel(d, g["d" + n]) <= 1e-4, n


def _rand(B, T, H, r, r_out, dk, dv, seed, scalar_gate=False):
    gen = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, r_out, dk, generator=gen, dtype=torch.float64), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, T, H, r, dk, generator=gen, dtype=torch.float64), dim=-1)
    V = torch.randn(B, T, H, r, dv, generator=gen, dtype=torch.float64)
    if scalar_gate:
        Bg = torch.rand(B, T, H, r, 1, generator=gen, dtype=torch.float64).expand(B, T, H, r, dk)
    else:
        Bg = torch.rand(B, T, H, r, dk, generator=gen, dtype=torch.float64)
    Wg = torch.rand(B, T, H, r, dv, generator=gen, dtype=torch.float64)
    a = 0.9 + 0.099 * torch.rand(B, T, H, dk, generator=gen, dtype=torch.float64)
    return q, K, V, Bg, Wg, a


def test_rank_one_scalar_gate_is_the_delta_rule():
    """r = 1 with an erase gate constant over channels: k~ = b k, so the erase
    is (b^2 / (eps + b^2 |k|^2)) (S k) k^T -- the decoupled-erase delta rule
    (oracle.delta, key-major state) with e = b^2 T k and w = Wg * v."""
    B, T, H, dk, dv, eps = 1, 15, 2, 8, 6, 0.5
    q, K, V, Bg, Wg, a = _rand(B, T, H, 1, 1, dk, dv, seed=3, scalar_gate=True)
    y = rls.rls_scan(q, K, V, Bg, Wg, a, eps=eps)
    b = Bg[:, :, :, 0, 0]
    k = K[:, :, :, 0]
    Tf = 1.0 / (eps + b * b * (k * k).sum(-1))
    e = (b * b * Tf).unsqueeze(-1) * k

    def nt(x):
        return x.permute(0, 2, 1, *range(3, x.dim())).reshape(B * H, T, *x.shape[3:])
    y2, _ = od.delta_rule_sequential(nt(q[:, :, :, 0]), nt(k), nt(e), nt(Wg[:, :, :, 0] * V[:, :, :, 0]), nt(a))
    assert torch.allclose(y, y2.view(B, H, T, dv).permute(0, 2, 1, 3), atol=1e-12)


def test_rank_r_erase_is_the_projection_limit():
    """eps -> 0 with r slots: the erase projects the state onto the orthogonal
    complement of the erase keys' span, S Kt^T = 0 after the erase."""
    B, T, H, r, dk, dv = 1, 1, 1, 3, 8, 5
    q, K, V, Bg, Wg, a = _rand(B, T, H, r, 1, dk, dv, seed=4)
    S0 = torch.randn(B, H, dv, dk, dtype=torch.float64)
    _, S = rls.rls_scan(q, K, torch.zeros_like(V), Bg, Wg, torch.ones_like(a), eps=1e-12, state0=S0,
                        return_state=True)
    Kt = (Bg * K)[:, 0]
    assert (S @ Kt.transpose(-1, -2)).abs().max() < 1e-9


def test_full_rank_compaction_is_identity_and_ste_gradient_is_uncompacted():
    B, T, H, r, dk, dv = 1, 16, 2, 2, 6, 5
    xs = [x.requires_grad_(True) for x in _rand(B, T, H, r, 1, dk, dv, seed=5)]
    dy = torch.randn(B, T, H, dv, dtype=torch.float64)
    y0 = rls.rls_scan(*xs)
    g0 = torch.autograd.grad(y0, xs, dy)
    y1 = rls.rls_scan(*xs, compact_P=4, compact_R=min(dk, dv), ste=True)
    g1 = torch.autograd.grad(y1, xs, dy)
    assert torch.allclose(y0, y1, atol=1e-12)
    for a, b in zip(g0, g1):
        assert torch.allclose(a, b, atol=1e-12)
    y2 = rls.rls_scan(*xs, compact_P=4, compact_R=min(dk, dv), ste=False)
    assert torch.allclose(y0, y2, atol=1e-12)


def test_truncation_is_the_eckart_young_optimum():
    gen = torch.Generator().manual_seed(6)
    S = torch.randn(3, 7, 9, generator=gen, dtype=torch.float64)
    R = 2
    L = rls.truncate_rank(S, R)
    sg = torch.linalg.svdvals(S)
    assert torch.allclose((S - L).norm(dim=(-2, -1)), sg[:, R:].square().sum(-1).sqrt())
    assert int(torch.linalg.matrix_rank(L[0])) == R
    # a rank-R matrix is kept as it is
    low = torch.randn(7, R, dtype=torch.float64) @ torch.randn(R, 9, dtype=torch.float64)
    assert torch.allclose(rls.truncate_rank(low, R), low, atol=1e-10)

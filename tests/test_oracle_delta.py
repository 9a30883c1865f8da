"""Pins the dense delta-rule oracle (CPU only).

Known-answer tests restate tests/ablation/test_exact_cache_math.py:563-597 of
the reference; the scalar oracle follows the pattern of its _scalar_oracle
(:387-494) and input distribution _random_inputs (:496-520).
"""
import math

import pytest
import torch

from oracle import delta


def _scalar_scan(q, k, v, g, be, bw, mix):
    """Independent pure-Python restatement (lists of floats, no batched ops)."""
    B, T, H, R, dk = q.shape
    dv = v.shape[-1]
    S = [[[[0.0] * dv for _ in range(dk)] for _ in range(H)] for _ in range(B)]
    Y = torch.zeros(B, T, H, dv, dtype=torch.float64)
    SC = torch.zeros(B, T, H, dtype=torch.float64)
    for t in range(T):
        for b in range(B):
            for h in range(H):
                Sb = [[float(g[b, t, h, i]) * S[b][h][i][j] for j in range(dv)] for i in range(dk)]
                m = [sum(float(k[b, t, h, i]) * Sb[i][j] for i in range(dk)) for j in range(dv)]
                upd = [float(bw[b, t, h]) * float(v[b, t, h, j]) - float(be[b, t, h]) * m[j]
                       for j in range(dv)]
                S[b][h] = [[Sb[i][j] + float(k[b, t, h, i]) * upd[j] for j in range(dv)]
                           for i in range(dk)]
                reads = [[sum(float(q[b, t, h, r, i]) * S[b][h][i][j] for i in range(dk))
                          for j in range(dv)] for r in range(R)]
                for j in range(dv):
                    if R == 1:
                        Y[b, t, h, j] = reads[0][j]
                    else:
                        Y[b, t, h, j] = sum(float(mix[h, r]) * reads[r][j] for r in range(R))
                SC[b, t, h] = math.sqrt(sum(float(k[b, t, h, i]) ** 2 for i in range(dk))) * \
                    math.sqrt(sum(u * u for u in upd))
    return Y, SC


def _random_inputs(slots, dtype=torch.float64):
    gen = torch.Generator().manual_seed(2718 + slots)
    B, T, H, dk, dv = 2, 3, 2, 2, 3
    q = torch.randn(B, T, H, slots, dk, generator=gen, dtype=dtype)
    k = torch.randn(B, T, H, dk, generator=gen, dtype=dtype)
    v = torch.randn(B, T, H, dv, generator=gen, dtype=dtype)
    g = 0.55 + 0.4 * torch.rand(B, T, H, dk, generator=gen, dtype=dtype)
    be = 0.1 + 0.75 * torch.rand(B, T, H, generator=gen, dtype=dtype)
    bw = 0.1 + 0.75 * torch.rand(B, T, H, generator=gen, dtype=dtype)
    mix = torch.tensor([[0.1, 0.2, 0.3, 0.4], [-0.3, 0.7, 0.15, 0.45]], dtype=dtype)
    return q, k, v, g, be, bw, (mix if slots > 1 else None)


def test_known_answer_reads_updated_state():
    # q=3, k=2, v=5, decay=0.25, beta_e=0.7, beta_w=0.4 => y=12, score=4
    one = lambda x, *s: torch.tensor(x, dtype=torch.float64).reshape(*s)
    y, sc = delta.kmd2_scan(one(3.0, 1, 1, 1, 1, 1), one(2.0, 1, 1, 1, 1), one(5.0, 1, 1, 1, 1),
                            one(0.25, 1, 1, 1, 1), one(0.7, 1, 1, 1), one(0.4, 1, 1, 1),
                            return_scores=True)
    assert y.item() == pytest.approx(12.0, abs=1e-12)
    assert sc.item() == pytest.approx(4.0, abs=1e-12)


@pytest.mark.parametrize("key,expected", [([0.0, 0.0], 0.0), ([1.0e-12, 0.0], 2.5e-12)])
def test_known_answer_zero_and_subepsilon_key(key, expected):
    q = torch.ones(1, 1, 1, 1, 2, dtype=torch.float64)
    k = torch.tensor([[[key]]], dtype=torch.float64)
    v = torch.tensor([[[[3.0, 4.0]]]], dtype=torch.float64)
    g = torch.ones(1, 1, 1, 2, dtype=torch.float64)
    _, sc = delta.kmd2_scan(q, k, v, g, torch.ones(1, 1, 1, dtype=torch.float64),
                            torch.full((1, 1, 1), 0.5, dtype=torch.float64), return_scores=True)
    assert sc.item() == pytest.approx(expected, rel=1e-12, abs=0.0)


@pytest.mark.parametrize("slots", [1, 4])
def test_kmd2_scan_matches_scalar_loop(slots):
    q, k, v, g, be, bw, mix = _random_inputs(slots)
    y, sc = delta.kmd2_scan(q, k, v, g, be, bw, mix, return_scores=True)
    y2, sc2 = _scalar_scan(q, k, v, g, be, bw, mix)
    torch.testing.assert_close(y, y2, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(sc, sc2, atol=1e-12, rtol=1e-10)


def test_out_mix_is_linear_in_query_slots():
    q, k, v, g, be, bw, mix = _random_inputs(4)
    y = delta.kmd2_scan(q, k, v, g, be, bw, mix)
    q_eff = (q * mix.view(1, 1, 2, 4, 1)).sum(3, keepdim=True)
    y1 = delta.kmd2_scan(q_eff, k, v, g, be, bw, None)
    torch.testing.assert_close(y, y1, atol=1e-12, rtol=1e-10)


def _chain_inputs(N=3, T=37, dk=5, dv=4, seed=0, zero_at=None):
    gen = torch.Generator().manual_seed(seed)
    d = torch.float64
    q = torch.randn(N, T, dk, generator=gen, dtype=d)
    k = torch.nn.functional.normalize(torch.randn(N, T, dk, generator=gen, dtype=d), dim=-1)
    e = k * torch.rand(N, T, 1, generator=gen, dtype=d)
    w = torch.randn(N, T, dv, generator=gen, dtype=d)
    lg = -torch.nn.functional.softplus(1.2 * torch.randn(N, T, generator=gen, dtype=d) - 0.6)
    if zero_at is not None:
        lg[:, zero_at] = -math.inf
    return q, k, e, w, lg


def test_sequential_matches_kmd2_mapping():
    """delta_rule_sequential with e = beta_e k, w = beta_w v is the KMD-2 scan."""
    q, k, v, g, be, bw, _ = _random_inputs(1)
    B, T, H, _, dk = q.shape
    y = delta.kmd2_scan(q, k, v, g, be, bw)
    fl = lambda x: x.permute(0, 2, 1, *range(3, x.dim())).reshape(B * H, T, *x.shape[3:])
    kk = fl(k)
    ys, _ = delta.delta_rule_sequential(fl(q[:, :, :, 0]), kk, kk * fl(be).unsqueeze(-1),
                                        fl(v) * fl(bw).unsqueeze(-1), fl(g))
    torch.testing.assert_close(ys.reshape(B, H, T, -1).transpose(1, 2), y, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("chunk", [1, 4, 16, 64])
def test_chunked_equals_sequential_fp64(chunk):
    q, k, e, w, lg = _chain_inputs(zero_at=20)
    y0, s0 = delta.delta_rule_sequential(q, k, e, w, lg.exp())
    y1, s1 = delta.delta_rule_chunked(q, k, e, w, lg, chunk=chunk)
    torch.testing.assert_close(y1, y0, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(s1, s0, atol=1e-11, rtol=1e-10)


def test_chunked_gradients_equal_sequential():
    ins = [t.requires_grad_(True) for t in _chain_inputs(T=21)]
    y0, _ = delta.delta_rule_sequential(*ins[:4], ins[4].exp())
    up = torch.randn_like(y0)
    g0 = torch.autograd.grad((y0 * up).sum(), ins)
    y1, _ = delta.delta_rule_chunked(*ins, chunk=8)
    g1 = torch.autograd.grad((y1 * up).sum(), ins)
    for a, b in zip(g0, g1):
        torch.testing.assert_close(a, b, atol=1e-10, rtol=1e-9)


def _chan_inputs(N=3, T=45, dk=8, dv=6, seed=5, strong=False):
    gen = torch.Generator().manual_seed(seed)
    d = torch.float64
    q = torch.randn(N, T, dk, generator=gen, dtype=d)
    k = torch.nn.functional.normalize(torch.randn(N, T, dk, generator=gen, dtype=d), dim=-1)
    ae = torch.sigmoid(torch.randn(N, T, generator=gen, dtype=d))
    w = torch.randn(N, T, dv, generator=gen, dtype=d)
    scale = 6.0 if strong else 1.2
    lg = -torch.nn.functional.softplus(scale * torch.randn(N, T, dk, generator=gen, dtype=d) - 0.6)
    return q, k, ae, w, lg


@pytest.mark.parametrize("chunk,strong", [(1, False), (16, False), (16, True), (7, True)])
def test_chunked_chan_equals_sequential_fp64(chunk, strong):
    """Per-key-channel decay: the chunk algebra (decay-weighted grams formed
    per channel) equals the token loop, also with decays down to e^-40 per
    token, where a cumulative-product ratio would under/overflow."""
    q, k, ae, w, lg = _chan_inputs(strong=strong)
    y0, s0 = delta.delta_rule_sequential(q, k, k * ae.unsqueeze(-1), w, lg.exp())
    y1, s1 = delta.delta_rule_chunked_chan(q, k, ae, w, lg, chunk=chunk)
    torch.testing.assert_close(y1, y0, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(s1, s0, atol=1e-11, rtol=1e-10)


def test_chunked_chan_reduces_to_scalar_decay():
    """A decay constant over the channels gives the scalar-decay chunk form."""
    q, k, ae, w, lg = _chan_inputs()
    lg1 = lg[..., :1]
    y0, s0 = delta.delta_rule_chunked(q, k, k * ae.unsqueeze(-1), w, lg1[..., 0], chunk=16)
    y1, s1 = delta.delta_rule_chunked_chan(q, k, ae, w, lg1.expand_as(lg), chunk=16)
    torch.testing.assert_close(y1, y0, atol=1e-11, rtol=1e-10)


def test_chunked_chan_gradients_equal_sequential():
    ins = [t.requires_grad_(True) for t in _chan_inputs(T=21)]
    q, k, ae, w, lg = ins
    y0, _ = delta.delta_rule_sequential(q, k, k * ae.unsqueeze(-1), w, lg.exp())
    up = torch.randn_like(y0)
    g0 = torch.autograd.grad((y0 * up).sum(), ins)
    y1, _ = delta.delta_rule_chunked_chan(*ins, chunk=8)
    g1 = torch.autograd.grad((y1 * up).sum(), ins)
    for a, b in zip(g0, g1):
        torch.testing.assert_close(a, b, atol=1e-10, rtol=1e-9)


def test_invariants_zero_value_zero_decay_zero_beta():
    q, k, e, w, lg = _chain_inputs()
    y, _ = delta.delta_rule_sequential(q, k, e, torch.zeros_like(w), lg.exp())
    assert y.abs().max() == 0
    # a zero decay at t=20 makes every later output independent of earlier inputs
    q, k, e, w, lg = _chain_inputs(zero_at=20)
    w2 = w.clone()
    w2[:, :20] = torch.randn_like(w2[:, :20])
    ya, _ = delta.delta_rule_sequential(q, k, e, w, lg.exp())
    yb, _ = delta.delta_rule_sequential(q, k, e, w2, lg.exp())
    torch.testing.assert_close(ya[:, 20:], yb[:, 20:], atol=1e-13, rtol=0)
    assert (ya[:, :20] - yb[:, :20]).abs().max() > 1e-3
    # beta = 0 (no erase, no write) after t=10 => y_t = gamma-decayed S_10^T q_t
    e0, w0 = e.clone(), w.clone()
    e0[:, 10:] = 0
    w0[:, 10:] = 0
    lg2 = lg.clone()
    lg2[:, 20] = -0.5
    y, _ = delta.delta_rule_sequential(q, k, e0, w0, lg2.exp())
    _, S10 = delta.delta_rule_sequential(q[:, :10], k[:, :10], e[:, :10], w[:, :10], lg2[:, :10].exp())
    cum = lg2[:, 10:].cumsum(1).exp()
    expect = cum.unsqueeze(-1) * torch.einsum("nkv,ntk->ntv", S10, q[:, 10:])
    torch.testing.assert_close(y[:, 10:], expect, atol=1e-12, rtol=1e-10)


def test_stable_alpha_closed_form_series_and_continuity():
    c = torch.tensor([0.0, 1e-9, -1e-9, 0.3, 1.0, 5.0, -0.2], dtype=torch.float64)
    a = delta.stable_alpha(c)
    exact = torch.tensor([1.0 if x == 0 else
                          (1 - x / 2 + x * x / 6 - x ** 3 / 24 if abs(x) < 1e-4 else -math.expm1(-x) / x)
                          for x in c.tolist()], dtype=torch.float64)
    torch.testing.assert_close(a, exact, atol=1e-12, rtol=1e-12)
    lo = delta.stable_alpha(torch.tensor([1e-6 * (1 - 1e-9)], dtype=torch.float64))
    hi = delta.stable_alpha(torch.tensor([1e-6 * (1 + 1e-9)], dtype=torch.float64))
    assert abs(lo.item() - hi.item()) < 1e-12
    assert delta.stable_alpha(torch.tensor([1.0], dtype=torch.float64)).item() == pytest.approx(1 - math.exp(-1))


def test_gdn3_dense_layer_chunked_equals_sequential():
    from oracle import inputs
    x = inputs.dense_inputs(1, 40, 2, 8, M=3, seed=5, decay="tau", taus=(0.05, 0.02, 0.001), rope=False)
    y0 = delta.gdn3_dense_layer(x["q"], x["k"], x["v"], x["beta"], x["g"])
    y1 = delta.gdn3_dense_layer(x["q"], x["k"], x["v"], x["beta"], x["g"], chunk=16)
    assert y0.shape == (1, 40, 2, 3, 8)
    torch.testing.assert_close(y1, y0, atol=1e-11, rtol=1e-10)

"""The GDN3 layer pre-ops / post-ops oracle (oracle/gdn3_layer.py) against the
reference layer's own forward (golden vectors written by
tests/golden/make_golden_layer.py) and the properties each step has."""
import os

import numpy as np
import pytest
import torch

from oracle import gdn3_layer as gl

GOLD = os.path.join(os.path.dirname(__file__), "golden", "gdn3_layer_golden.npz")


@pytest.fixture(scope="module")
def gold():
    z = np.load(GOLD, allow_pickle=False)
    return {k: torch.from_numpy(z[k]) for k in z.files}


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()


def test_prologue_matches_reference_layer(gold):
    g = gold
    out = gl.prologue(g["pro_q"], g["pro_k"], g["pro_b_proj"], g["pro_proj_a"], g["pro_w_proj"], g["pro_proj_b"],
                      g["pro_decay_proj"], g["pro_rates"], float(g["decay_clamp"][0]))
    for name, a in zip(("q_rope", "k_rope", "b_gates", "w_gates", "decay"), out):
        assert rel(a, g["pro_" + name]) <= 2e-6, name


def test_epilogue_matches_reference_layer(gold):
    g = gold
    out = gl.epilogue(g["epi_y"], g["epi_router_logits"], g["epi_norm"])
    assert rel(out, g["epi_out"]) <= 2e-6


def test_rope_quirks_are_exercised(gold):
    """The golden case covers what no closed form pins: lane 0 (scale 1,
    32 pairs > the table's 16) left unchanged, lanes 1-3 transformed, and
    the second half built from the updated first half (a rotation would
    preserve the pair norms, this does not)."""
    q, qr = gold["pro_q"].double(), gold["pro_q_rope"].double()
    params = gl.lane_rope_params(4, 128)
    assert params[0][3] and not any(p[3] for p in params[1:])
    assert [p[0] for p in params] == [32, 16, 32, 32] and [p[2] for p in params] == [31, 15, 15, 15]
    assert torch.equal(qr[:, :, :, 0].float(), q.float())
    for m in (1, 2, 3):
        assert rel(qr[:, :, :, m], q) > 1e-3
    d = 16   # lane 1
    a, b = q[..., :d], q[..., d:2 * d]
    n_in = (a ** 2 + b ** 2)[:, 1:]
    n_out = (qr[:, :, :, 1, :d] ** 2 + qr[:, :, :, 1, d:2 * d] ** 2)[:, 1:]
    assert rel(n_out, n_in) > 1e-3


def test_prologue_properties():
    g = torch.Generator().manual_seed(3)
    B, T, H, M, K = 1, 9, 2, 4, 64
    q = torch.randn(B, T, H, K, generator=g)
    xs = [torch.randn(B, T, H, M, K, generator=g) for _ in range(2)]
    pa, pb = torch.randn(B, T, H, generator=g), torch.randn(B, T, H, generator=g)
    dp = torch.randn(B, T, H, M, 4, generator=g) * 5
    rates = torch.tensor([0.05, 0.02, 0.005, 0.001])
    qr, _, bg, wg, dec = gl.prologue(q, q, xs[0], pa, xs[1], pb, dp, rates, 0.999)
    # position 0: every lane unchanged; past the pairs: unchanged
    assert torch.allclose(qr[:, 0], q[:, 0].double().unsqueeze(2).expand(B, H, M, K))
    for m, (d, _, _, _) in enumerate(gl.lane_rope_params(M, K)):
        assert torch.equal(qr[:, :, :, m, 2 * d:], q[..., 2 * d:].double())
    # the lane transform inverts as a triangular map
    cos, sin = gl.lane_rope_tables(M, T, K, torch.float64)
    for m, (d, _, _, ident) in enumerate(gl.lane_rope_params(M, K)):
        if ident:
            continue
        c, s = cos[m, :, :d].view(1, T, 1, d), sin[m, :, :d].view(1, T, 1, d)
        x1n, x2n = qr[:, :, :, m, :d], qr[:, :, :, m, d:2 * d]
        x2 = (x2n - x1n * s) / c
        x1 = (x1n + x2 * s) / c
        assert torch.allclose(torch.cat([x1, x2], -1), q[..., :2 * d].double(), atol=1e-9)
    assert bool(((bg > 0) & (bg < 1)).all()) and bool(((wg > 0) & (wg < 1)).all())
    assert bool(((dec > 0) & (dec <= 0.999)).all())
    # softplus clamped at 5: a huge projection decays by the clamped rate only
    big = torch.full((1, 1, 1, 1, 4), 100.0)
    _, _, _, _, d1 = gl.prologue(q[:, :1, :1], q[:, :1, :1], xs[0][:, :1, :1, :1], pa[:, :1, :1], xs[1][:, :1, :1, :1],
                                 pb[:, :1, :1], big, rates, 0.999)
    assert torch.allclose(d1, torch.exp(-5.0 * rates.double()).mean().view(1, 1, 1, 1))


def test_epilogue_properties():
    g = torch.Generator().manual_seed(4)
    B, T, H, M, V = 2, 5, 3, 4, 32
    y = torch.randn(B, T, H, M, V, generator=g)
    logits = torch.randn(B, T, H, M, generator=g)
    norm = torch.ones(V)
    out = gl.epilogue(y, logits, norm)
    assert torch.allclose(out.norm(dim=-1), torch.full((B, T, H), V ** 0.5, dtype=torch.float64))
    # equal logits: the plain mean of the lanes, normalised
    out2 = gl.epilogue(y, torch.zeros_like(logits), norm)
    ref = torch.nn.functional.normalize(y.double().mean(3), dim=-1) * V ** 0.5
    assert torch.allclose(out2, ref)

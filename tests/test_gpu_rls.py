"""Rank-r RLS T-factor scan on the GPU (gdnx_amd.rls: gdnx_rls_fwd / _bwd)
against the reference's own scan (golden vectors, tests/golden/rls_golden.npz)
and the float64 oracle (oracle/rls.py, pinned by those vectors in
tests/test_oracle_rls.py), output and every input gradient.

Tolerance (rel-L2): 1e-5 -- a float32 sequential recurrence against float64
over up to a few hundred tokens (measured 1e-7 .. 6e-7, also against the
golden vectors, which are the reference's float32 values)."""
import os

import numpy as np
import pytest
import torch

from oracle import rls as orls

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "rls_golden.npz")


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _inputs(B, T, H, r, r_out, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, r_out, dk, generator=g), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, T, H, r, dk, generator=g), dim=-1)
    V = torch.randn(B, T, H, r, dv, generator=g)
    Bg = torch.sigmoid(torch.randn(B, T, H, r, dk, generator=g))
    Wg = torch.sigmoid(torch.randn(B, T, H, r, dv, generator=g))
    a = torch.sigmoid(torch.randn(B, T, H, dk, generator=g) + 4.0).clamp(max=0.999)
    mix = torch.rand(H, r_out, generator=g) + 0.2
    return [q, K, V, Bg, Wg, a], mix


@pytest.mark.parametrize("case", ["r1", "r2o2"])
def test_rls_matches_reference_golden(gpu_lib, case):
    """The reference's _scan on its own (small) dims: key dim 16 and value
    dims 8 / 12 run zero-padded to the kernel's 32 / 16."""
    from gdnx_amd import rls
    print(f"case: rls golden {case}", flush=True)
    z = np.load(GOLD, allow_pickle=False)
    t = {k.split("/")[1]: torch.from_numpy(z[k]) for k in z.files if k.startswith(case + "/")}
    names = ["q", "K", "V", "Bg", "Wg", "a"]
    leaves = [t[n].to(DEV).requires_grad_(True) for n in names]
    r_out = t["q"].shape[3]
    mix = t["out_mix"].to(DEV).requires_grad_(True)
    y = rls.rls_scan(*leaves, eps=float(t["eps"][0]), out_mix=mix)
    params = leaves + ([mix] if r_out > 1 else [])
    grads = torch.autograd.grad(y, params, t["dy"].to(DEV))
    torch.cuda.synchronize()
    assert rel_l2(y, t["y"]) <= 1e-5
    for n, d in zip(names + ["out_mix"], grads):
        err = rel_l2(d, t["d" + n])
        print(f"  d{n} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-5, n


CASES = [
    # (B, T, H, r, r_out, dk, dv, eps)
    (2, 40, 2, 1, 1, 64, 64, 0.5),
    (1, 77, 2, 4, 1, 32, 32, 0.5),
    (1, 50, 1, 2, 2, 32, 48, 0.25),
    (1, 33, 2, 1, 4, 128, 64, 0.5),
    (1, 21, 1, 3, 1, 64, 16, 1.0),
    (1, 19, 1, 4, 4, 128, 128, 0.5),
    (2, 300, 1, 1, 1, 64, 64, 0.5),
    (1, 45, 2, 2, 1, 40, 24, 0.5),
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_rls_forward_backward_match_oracle(gpu_lib, case):
    from gdnx_amd import rls
    B, T, H, r, r_out, dk, dv, eps = case
    print(f"case: rls {case}", flush=True)
    xs, mix = _inputs(B, T, H, r, r_out, dk, dv, seed=11)
    dy = torch.randn(B, T, H, dv, generator=torch.Generator().manual_seed(12))
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    mixd = mix.to(DEV).requires_grad_(True)
    y = rls.rls_scan(*leaves, eps=eps, out_mix=mixd)
    params = leaves + ([mixd] if r_out > 1 else [])
    grads = torch.autograd.grad(y, params, dy.to(DEV))
    torch.cuda.synchronize()
    ref_leaves = [x.double().requires_grad_(True) for x in xs]
    mixr = mix.double().requires_grad_(True)
    yr = orls.rls_scan(*ref_leaves, eps=eps, out_mix=mixr)
    gref = torch.autograd.grad(yr, ref_leaves + ([mixr] if r_out > 1 else []), dy.double())
    err = rel_l2(y, yr)
    print(f"  y rel-L2 {err:.2e}", flush=True)
    assert y.shape == yr.shape and err <= 1e-5
    for n, a, b in zip(["dq", "dK", "dV", "dBg", "dWg", "da", "dout_mix"], grads, gref):
        err = rel_l2(a, b)
        print(f"  {n} rel-L2 {err:.2e}", flush=True)
        assert a.shape == b.shape and err <= 1e-5, n


def test_rls_state_in_and_out(gpu_lib):
    """Initial and final state (continuation): two calls over T1 + T2 tokens
    equal one call over T1 + T2; gradients reach state0 and flow back
    through a returned state."""
    from gdnx_amd import rls
    print("case: rls state continuation", flush=True)
    B, T1, T2, H, r, dk, dv = 1, 23, 18, 2, 2, 64, 32
    xs, _ = _inputs(B, T1 + T2, H, r, 1, dk, dv, seed=21)
    dev = [x.to(DEV) for x in xs]
    y_full, s_full = rls.rls_scan(*dev, return_state=True)
    y1, s1 = rls.rls_scan(*(x[:, :T1] for x in dev), return_state=True)
    y2, s2 = rls.rls_scan(*(x[:, T1:] for x in dev), state0=s1, return_state=True)
    torch.cuda.synchronize()
    assert rel_l2(torch.cat([y1, y2], 1), y_full) <= 1e-5
    assert rel_l2(s2, s_full) <= 1e-5
    # gradients through the state against the oracle
    s0 = torch.randn(B, H, dv, dk, generator=torch.Generator().manual_seed(22)) * 0.3
    dy = torch.randn(B, T1, H, dv, generator=torch.Generator().manual_seed(23))
    ds = torch.randn(B, H, dv, dk, generator=torch.Generator().manual_seed(24))
    leaves = [x[:, :T1].contiguous().requires_grad_(True) for x in dev] + [s0.to(DEV).requires_grad_(True)]
    y, s = rls.rls_scan(*leaves[:6], state0=leaves[6], return_state=True)
    grads = torch.autograd.grad([y, s], leaves, [dy.to(DEV), ds.to(DEV)])
    rl = [x[:, :T1].double().requires_grad_(True) for x in xs] + [s0.double().requires_grad_(True)]
    yr, sr = orls.rls_scan(*rl[:6], state0=rl[6], return_state=True)
    gr = torch.autograd.grad([yr, sr], rl, [dy.double(), ds.double()])
    assert rel_l2(y, yr) <= 1e-5 and rel_l2(s, sr) <= 1e-5
    for a, b in zip(grads, gr):
        assert rel_l2(a, b) <= 1e-5


def test_rls_backward_is_deterministic(gpu_lib):
    from gdnx_amd import rls
    print("case: rls determinism", flush=True)
    xs, _ = _inputs(2, 64, 2, 1, 1, 64, 64, seed=31)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    dy = torch.randn(2, 64, 2, 64, device=DEV)
    g1 = torch.autograd.grad(rls.rls_scan(*leaves), leaves, dy)
    g2 = torch.autograd.grad(rls.rls_scan(*leaves), leaves, dy)
    torch.cuda.synchronize()
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case,ste", [("tb_plain", False), ("tb_ste", True)])
def test_rls_compaction_matches_testbed_golden(gpu_lib, case, ste):
    """The testbed mixer's scan with SVD compaction every P tokens (its own
    forward, research/testbed_mqar.py:245-260), gates and decay through the
    mixer's sigmoids (torch, outside the kernel); key dim 16 / value dim 16
    run zero-padded."""
    from gdnx_amd import rls
    print(f"case: rls compaction golden {case}", flush=True)
    z = np.load(GOLD, allow_pickle=False)
    t = {k.split("/")[1]: torch.from_numpy(z[k]) for k in z.files if k.startswith(case + "/")}
    names = ["q", "K", "V", "bg_logit", "wg_logit", "dec_logit"]
    lv = {n: t[n].to(DEV).requires_grad_(True) for n in names}
    y = rls.rls_scan(lv["q"], lv["K"], lv["V"], torch.sigmoid(lv["bg_logit"]), torch.sigmoid(lv["wg_logit"]),
                     torch.sigmoid(lv["dec_logit"]).clamp(max=0.9995), eps=float(t["eps"][0]),
                     compact_P=int(t["P"][0]), compact_R=int(t["R"][0]), slow_decay=0.97, straight_through=ste)
    grads = torch.autograd.grad(y, list(lv.values()), t["dy"].to(DEV))
    torch.cuda.synchronize()
    err = rel_l2(y, t["y"])
    print(f"  y rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-4
    for n, d in zip(names, grads):
        err = rel_l2(d, t["d" + n])
        print(f"  d{n} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-4, n


COMPACT_CASES = [
    # (B, T, H, r, dk, dv, P, R, ste)
    (1, 40, 2, 2, 32, 32, 8, 3, False),
    (1, 40, 2, 2, 32, 32, 8, 3, True),
    (1, 48, 1, 1, 64, 64, 16, 8, False),
    (2, 30, 1, 2, 32, 48, 10, 5, False),
    (1, 36, 1, 1, 64, 32, 12, 4, True),
]


@pytest.mark.parametrize("case", COMPACT_CASES, ids=[f"k{i}" for i in range(len(COMPACT_CASES))])
def test_rls_compaction_matches_oracle(gpu_lib, case):
    """In-kernel truncated SVD (Jacobi on the smaller Gram of S) and the
    compaction's gradient (no-grad truncation, or straight-through) against
    the float64 oracle.  Bound 1e-4: the truncation moves with the state's
    float32 error amplified by sigma_1 / (sigma_R - sigma_{R+1})."""
    from gdnx_amd import rls
    B, T, H, r, dk, dv, P, R, ste = case
    print(f"case: rls compaction {case}", flush=True)
    xs, _ = _inputs(B, T, H, r, 1, dk, dv, seed=51)
    dy = torch.randn(B, T, H, dv, generator=torch.Generator().manual_seed(52))
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y = rls.rls_scan(*leaves, compact_P=P, compact_R=R, slow_decay=0.97, straight_through=ste)
    grads = torch.autograd.grad(y, leaves, dy.to(DEV))
    torch.cuda.synchronize()
    rl = [x.double().requires_grad_(True) for x in xs]
    yr = orls.rls_scan(*rl, compact_P=P, compact_R=R, slow_decay=0.97, ste=ste)
    gr = torch.autograd.grad(yr, rl, dy.double())
    err = rel_l2(y, yr)
    print(f"  y rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-4
    for n, a, b in zip(["dq", "dK", "dV", "dBg", "dWg", "da"], grads, gr):
        err = rel_l2(a, b)
        print(f"  {n} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-4, n

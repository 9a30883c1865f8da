"""Edge shapes on every GPU path: a single token (T = 1), a length that is not
a multiple of the chunk or window, and an empty sequence (T = 0, which must
return empty outputs and zero-size gradients without a launch error).
Checked against the float64 oracles at the float32 bound of each path."""
import pytest
import torch
import torch.nn.functional as F

from oracle import delta
from oracle import gdn3 as og
from oracle import gdn3_layer as gl
from oracle import rls as orls

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    if b.numel() == 0:
        return 0.0 if a.numel() == 0 else float("inf")
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _dense(B, T, H, M, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, M, generator=g))
    lg = -0.05 * torch.rand(B, T, H, M, generator=g)
    return [q, k, v, beta, lg]


@pytest.mark.parametrize("T", [1, 45, 0])
def test_gdn3_scan_edge_lengths(gpu_lib, T):
    from gdnx_amd import gdn3
    print(f"case: gdn3_scan T={T}", flush=True)
    B, H, M, D = 1, 2, 2, 128
    xs = _dense(B, T, H, M, D, seed=1)
    dy = torch.randn(B, T, H, M, D, generator=torch.Generator().manual_seed(2))
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y = gdn3.gdn3_scan(*leaves)
    grads = torch.autograd.grad(y, leaves, dy.to(DEV), allow_unused=True)
    torch.cuda.synchronize()
    assert y.shape == (B, T, H, M, D)
    if T == 0:   # (the oracles' token loops need T >= 1)
        assert all(g is None or g.numel() == 0 for g in grads)
        return
    ref = [x.double().requires_grad_(True) for x in xs]
    a = delta.gdn3_dense_coeffs(ref[1], ref[3])
    yr, _ = delta.lane_delta(ref[0], ref[1], ref[2], a, a, ref[4])
    assert rel_l2(y, yr) <= 1e-4
    gr = torch.autograd.grad(yr, ref, dy.double())
    for a_, b_ in zip(grads, gr):
        assert rel_l2(a_, b_) <= 1e-4


@pytest.mark.parametrize("T", [1, 17, 0])
def test_gdn3_recurrent_state_edge_lengths(gpu_lib, T):
    """General regime (window P = 16, compaction every 16): one token, a
    length past one window, and empty."""
    from gdnx_amd import gdn3
    print(f"case: gdn3_recurrent_state T={T}", flush=True)
    B, H, M, D = 1, 1, 2, 128
    g = torch.Generator().manual_seed(3)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    bg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    wg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    dec = 0.95 + 0.04 * torch.rand(B, T, H, M, generator=g)
    dy = torch.randn(B, T, H, M, D, generator=g)
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v, bg, wg, dec)]
    G = og.reference_sketch(B * H * M, 64, 8)
    y = gdn3.gdn3_recurrent_state(*leaves, sketch=G.to(DEV))
    grads = torch.autograd.grad(y, leaves, dy.to(DEV), allow_unused=True)
    torch.cuda.synchronize()
    assert y.shape == (B, T, H, M, D)
    if T == 0:
        assert all(g_ is None or g_.numel() == 0 for g_ in grads)
        _, state, err = gdn3.gdn3_recurrent_state(*leaves, sketch=G.to(DEV), return_state=True)
        assert all(torch.count_nonzero(t) == 0 for t in state) and float(err) == 0.0
        return
    ref = [x.double().requires_grad_(True) for x in (q, k, v, bg, wg, dec)]

    def lanes(x):
        return x.unsqueeze(3).expand(B, T, H, M, D)
    yr = og.gdn3_recurrence(lanes(ref[0]), lanes(ref[1]), lanes(ref[2]), ref[3], ref[4], ref[5], R=4, P=16,
                            factors=(16, 16, 8, 8), compact_every=16, sketch=G, sign_mode="canonical",
                            slow_decay=0.97)
    assert rel_l2(y, yr) <= 1e-4
    gr = torch.autograd.grad(yr, ref, dy.double())
    for a_, b_ in zip(grads, gr):
        assert rel_l2(a_, b_) <= 1e-4


@pytest.mark.parametrize("T", [1, 0])
@pytest.mark.parametrize("chan", [False, True])
def test_kmd2_scan_edge_lengths(gpu_lib, T, chan):
    from gdnx_amd import kmd2
    print(f"case: kmd2 T={T} chan={chan}", flush=True)
    B, H, d = 2, 2, 64
    g = torch.Generator().manual_seed(5)
    q = F.normalize(torch.randn(B, T, H, 1, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, d, generator=g), dim=-1)
    v = torch.randn(B, T, H, d, generator=g)
    if chan:
        gam = torch.exp(-0.1 * torch.rand(B, T, H, d, generator=g))
    else:
        gam = torch.exp(-0.1 * torch.rand(B, T, H, 1, generator=g)).expand(B, T, H, d)
    be = torch.sigmoid(torch.randn(B, T, H, generator=g))
    bw = torch.sigmoid(torch.randn(B, T, H, generator=g))
    y = kmd2.scan(*(x.to(DEV) for x in (q, k, v, gam, be, bw)))
    torch.cuda.synchronize()
    assert y.shape == (B, T, H, d)
    if T == 0:
        return
    yr = delta.kmd2_scan(q, k, v, gam, be, bw, None)
    assert rel_l2(y, yr) <= 1e-4


@pytest.mark.parametrize("T", [1, 0])
def test_rls_scan_edge_lengths(gpu_lib, T):
    from gdnx_amd import rls
    print(f"case: rls T={T}", flush=True)
    B, H, r, dk, dv = 1, 2, 2, 64, 32
    g = torch.Generator().manual_seed(6)
    xs = [F.normalize(torch.randn(B, T, H, 1, dk, generator=g), dim=-1),
          F.normalize(torch.randn(B, T, H, r, dk, generator=g), dim=-1),
          torch.randn(B, T, H, r, dv, generator=g), torch.rand(B, T, H, r, dk, generator=g),
          torch.rand(B, T, H, r, dv, generator=g), 0.9 + 0.09 * torch.rand(B, T, H, dk, generator=g)]
    dy = torch.randn(B, T, H, dv, generator=g)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y, s = rls.rls_scan(*leaves, return_state=True)
    grads = torch.autograd.grad(y, leaves, dy.to(DEV), allow_unused=True)
    torch.cuda.synchronize()
    assert y.shape == (B, T, H, dv) and s.shape == (B, H, dv, dk)
    if T == 0:
        assert torch.count_nonzero(s) == 0
        assert all(g_ is None or g_.numel() == 0 for g_ in grads)
        return
    yr, sr = orls.rls_scan(*[x.double() for x in xs], return_state=True)
    assert rel_l2(y, yr) <= 1e-5 and rel_l2(s, sr) <= 1e-5


@pytest.mark.parametrize("T", [1, 0])
def test_layer_boundary_edge_lengths(gpu_lib, T):
    from gdnx_amd import layer
    print(f"case: layer boundary T={T}", flush=True)
    B, H, M, K = 2, 2, 4, 128
    g = torch.Generator().manual_seed(7)
    xs = [torch.randn(B, T, H, K, generator=g), torch.randn(B, T, H, K, generator=g),
          torch.randn(B, T, H, M, K, generator=g), torch.randn(B, T, H, generator=g),
          torch.randn(B, T, H, M, K, generator=g), torch.randn(B, T, H, generator=g),
          torch.randn(B, T, H, M, 4, generator=g)]
    rates = torch.tensor([0.05, 0.02, 0.005, 0.001])
    outs = layer.gdn3_prologue(*(x.to(DEV) for x in xs), rates.to(DEV))
    y = torch.randn(B, T, H, M, K, generator=g)
    lg = torch.randn(B, T, H, M, generator=g)
    nm = 0.5 + torch.rand(K, generator=g)
    yl = [t.to(DEV).requires_grad_(True) for t in (y, lg, nm)]
    out = layer.gdn3_epilogue(*yl)
    grads = torch.autograd.grad(out, yl, torch.ones_like(out))
    torch.cuda.synchronize()
    ref = gl.prologue(*xs, rates)
    for a_, b_ in zip(outs, ref):
        assert a_.shape == b_.shape and rel_l2(a_, b_) <= 1e-6
    assert out.shape == (B, T, H, K) and rel_l2(out, gl.epilogue(y, lg, nm)) <= 1e-6
    if T == 0:
        assert torch.count_nonzero(grads[2]) == 0     # d norm over no rows

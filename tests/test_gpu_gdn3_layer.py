"""GDN3 layer boundary on the GPU (gdnx_amd.layer: gdnx_gdn3_prologue_* and
gdnx_gdn3_epilogue_*), against the float64 CPU oracle oracle/gdn3_layer.py
(pinned by golden vectors from the reference layer's own forward in
tests/test_oracle_gdn3_layer.py) and against those golden vectors directly.

Forward and every input gradient, through torch autograd on the oracle.
Tolerances (rel-L2): 1e-6 for float32 IO on the element-wise pre-/post-ops
(float32 exp / sigmoid / softplus and the device-built RoPE tables; measured
~1e-7), also against the golden vectors (float32 values of the reference's
CPU run); 1e-2 for bf16 IO (outputs, gradients and the in-place RoPE
intermediate rounded to bf16).  The layer core is bounded by its recurrence
(1e-4 in test_gpu_gdn3_bwd.py); the routing-logit gradient is a difference
of two dot products, w_m (du.y_m - du.u), which roughly doubles that relative
error, so the core's float32 bound is 2e-4."""
import os

import numpy as np
import pytest
import torch

from oracle import gdn3 as og
from oracle import gdn3_layer as gl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "gdn3_layer_golden.npz")
RATES = torch.tensor([0.05, 0.02, 0.005, 0.001])


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _pro_inputs(B, T, H, M, K, V, seed, spread=6.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    bp = torch.randn(B, T, H, M, K, generator=g)
    pa = torch.randn(B, T, H, generator=g)
    wp = torch.randn(B, T, H, M, V, generator=g)
    pb = torch.randn(B, T, H, generator=g)
    # decay_proj spread over softplus's clamp at 5 and below the decay clamp
    dp = torch.randn(B, T, H, M, 4, generator=g) * spread
    dp[..., 0, 0, :] = -40.0      # softplus -> 0: decay 1 -> clamped (zero gradient)
    return [q, k, bp, pa, wp, pb, dp]


def _oracle_prologue(xs, clamp, grads_out=None):
    leaves = [x.double().requires_grad_(True) for x in xs]
    outs = gl.prologue(*leaves, RATES, clamp)
    if grads_out is None:
        return outs, None
    grads = torch.autograd.grad(outs, leaves, [g.double() for g in grads_out])
    return outs, grads


def _out_grads(B, T, H, M, K, V, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, T, H, M, K, generator=g), torch.randn(B, T, H, M, K, generator=g),
            torch.randn(B, T, H, M, K, generator=g), torch.randn(B, T, H, M, V, generator=g),
            torch.randn(B, T, H, M, generator=g)]


def test_prologue_matches_reference_golden(gpu_lib):
    """The reference layer's own recurrence inputs (float32, K = 128: lane 0
    is the identity, lanes 1-3 use 16 / 32 / 32 pairs)."""
    from gdnx_amd import layer
    print("case: prologue golden", flush=True)
    z = np.load(GOLD, allow_pickle=False)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    names = ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj")
    xs = [t["pro_" + n].to(DEV) for n in names]
    outs = layer.gdn3_prologue(*xs, t["pro_rates"].to(DEV), float(t["decay_clamp"][0]))
    torch.cuda.synchronize()
    for name, a in zip(("q_rope", "k_rope", "b_gates", "w_gates", "decay"), outs):
        err = rel_l2(a, t["pro_" + name])
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-6, name


def test_epilogue_matches_reference_golden(gpu_lib):
    from gdnx_amd import layer
    print("case: epilogue golden", flush=True)
    z = np.load(GOLD, allow_pickle=False)
    y, lg, nm = (torch.from_numpy(z[k]).to(DEV) for k in ("epi_y", "epi_router_logits", "epi_norm"))
    out = layer.gdn3_epilogue(y, lg, nm)
    torch.cuda.synchronize()
    assert rel_l2(out, torch.from_numpy(z["epi_out"])) <= 1e-6


PRO_CASES = [
    # (B, T, H, M, K, V, io)
    (1, 40, 2, 4, 128, 128, torch.float32),
    (2, 33, 3, 4, 64, 64, torch.float32),
    (1, 17, 2, 3, 96, 32, torch.float32),
    (1, 40, 2, 4, 128, 128, torch.bfloat16),
    (1, 5, 1, 2, 256, 256, torch.bfloat16),
]


@pytest.mark.parametrize("case", PRO_CASES, ids=[f"p{i}" for i in range(len(PRO_CASES))])
def test_prologue_forward_and_backward_match_oracle(gpu_lib, case):
    from gdnx_amd import layer
    B, T, H, M, K, V, io = case
    print(f"case: prologue {case}", flush=True)
    clamp = 0.999
    xs = _pro_inputs(B, T, H, M, K, V, seed=5)
    gos = _out_grads(B, T, H, M, K, V, seed=6)
    xio = [x.to(io) for x in xs]
    ref, gref = _oracle_prologue(xio, clamp, gos)
    leaves = [x.to(DEV).requires_grad_(True) for x in xio]
    outs = layer.gdn3_prologue(*leaves, RATES.to(DEV), clamp)
    grads = torch.autograd.grad(outs, leaves, [g.to(DEV) for g in gos])
    torch.cuda.synchronize()
    tol = 1e-2 if io == torch.bfloat16 else 1e-6
    for name, a, r in zip(("q_rope", "k_rope", "b_gates", "w_gates", "decay"), outs, ref):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert a.shape == r.shape and err <= tol, name
    assert outs[0].dtype == io and outs[2].dtype == torch.float32
    for name, a, r, x in zip(("dq", "dk", "d_b_proj", "d_proj_a", "d_w_proj", "d_proj_b", "d_decay_proj"),
                             grads, gref, xio):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert a.shape == x.shape and a.dtype == x.dtype and err <= tol, name
    # the clamped decays pass no gradient (torch's clamp convention)
    assert torch.count_nonzero(grads[6][..., 0, 0, :]) == 0


EPI_CASES = [
    # (B, T, H, M, V, io)
    (1, 40, 2, 4, 128, torch.float32),
    (2, 19, 3, 3, 64, torch.float32),
    (1, 7, 2, 4, 256, torch.float32),
    (1, 40, 2, 4, 128, torch.bfloat16),
    (1, 9, 2, 1, 36, torch.float32),
]


@pytest.mark.parametrize("case", EPI_CASES, ids=[f"e{i}" for i in range(len(EPI_CASES))])
def test_epilogue_forward_and_backward_match_oracle(gpu_lib, case):
    from gdnx_amd import layer
    B, T, H, M, V, io = case
    print(f"case: epilogue {case}", flush=True)
    g = torch.Generator().manual_seed(8)
    y = torch.randn(B, T, H, M, V, generator=g).to(io)
    lg = (torch.randn(B, T, H, M, generator=g) * 2).to(io)
    nm = 0.5 + torch.rand(V, generator=g)
    dout = torch.randn(B, T, H, V, generator=g).to(io)
    leaves = [t.double().requires_grad_(True) for t in (y, lg, nm)]
    ref = gl.epilogue(*leaves)
    gref = torch.autograd.grad(ref, leaves, dout.double())
    dl = [t.to(DEV).requires_grad_(True) for t in (y, lg, nm)]
    out = layer.gdn3_epilogue(*dl)
    grads = torch.autograd.grad(out, dl, dout.to(DEV))
    torch.cuda.synchronize()
    tol = 1e-2 if io == torch.bfloat16 else 1e-6
    assert out.dtype == io and rel_l2(out, ref) <= tol
    for name, a, r, x in zip(("dy", "d_router_logits", "d_norm"), grads, gref, (y, lg, nm)):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert a.shape == x.shape and a.dtype == x.dtype and err <= tol, name


def test_epilogue_zero_row_takes_the_eps_branch(gpu_lib):
    """A row whose routed vector is 0 divides by eps = 1e-6 (F.normalize):
    output 0 there and gradient d_out * norm * sqrt(V) / eps (no |u| term)."""
    from gdnx_amd import layer
    print("case: epilogue eps branch", flush=True)
    B, T, H, M, V = 1, 6, 2, 4, 128
    g = torch.Generator().manual_seed(12)
    y = torch.randn(B, T, H, M, V, generator=g)
    y[0, 2, 1] = 0.0
    lg, nm = torch.randn(B, T, H, M, generator=g), 0.5 + torch.rand(V, generator=g)
    dout = torch.randn(B, T, H, V, generator=g)
    leaves = [t.double().requires_grad_(True) for t in (y, lg, nm)]
    ref = gl.epilogue(*leaves)
    gref = torch.autograd.grad(ref, leaves, dout.double())
    dl = [t.to(DEV).requires_grad_(True) for t in (y, lg, nm)]
    out = layer.gdn3_epilogue(*dl)
    grads = torch.autograd.grad(out, dl, dout.to(DEV))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0, 2, 1]) == 0
    assert rel_l2(out, ref) <= 1e-6
    for a, r in zip(grads, gref):
        assert rel_l2(a, r) <= 1e-6


def test_epilogue_d_norm_is_deterministic(gpu_lib):
    """d_norm sums per-workgroup partials in a fixed order: two calls agree
    bitwise (rows beyond one workgroup per row block)."""
    from gdnx_amd import ops
    print("case: epilogue d_norm determinism", flush=True)
    B, T, H, M, V = 2, 2100, 4, 4, 128
    g = torch.Generator().manual_seed(13)
    y = torch.randn(B, T, H, M, V, generator=g).to(DEV)
    lg = torch.randn(B, T, H, M, generator=g).to(DEV)
    nm = (0.5 + torch.rand(V, generator=g)).to(DEV)
    dout = torch.randn(B, T, H, V, generator=g).to(DEV)
    a = ops.gdn3_epilogue_bwd(y, lg, nm, dout)
    b = ops.gdn3_epilogue_bwd(y, lg, nm, dout)
    torch.cuda.synchronize()
    for x, z in zip(a, b):
        assert torch.equal(x, z)
    leaves = [t.double().cpu().requires_grad_(True) for t in (y, lg, nm)]
    ref = gl.epilogue(*leaves)
    gn = torch.autograd.grad(ref, leaves[2], dout.double().cpu())[0]
    assert rel_l2(a[2], gn) <= 1e-6


CORE_CASES = [
    # (B, T, H, M, D, io)
    (1, 48, 2, 4, 128, torch.float32),
    (1, 40, 1, 4, 64, torch.float32),
    (1, 48, 2, 4, 128, torch.bfloat16),
]


@pytest.mark.parametrize("case", CORE_CASES, ids=[f"c{i}" for i in range(len(CORE_CASES))])
def test_layer_core_matches_oracle_composition(gpu_lib, case):
    """prologue -> recurrence (compaction every 16) -> epilogue against the
    oracle's prologue -> gdn3_recurrence -> epilogue in float64, output and
    the gradients of all eleven inputs that carry one."""
    from gdnx_amd import layer
    B, T, H, M, D, io = case
    print(f"case: layer core {case}", flush=True)
    xs = _pro_inputs(B, T, H, M, D, D, seed=21, spread=2.0)
    g = torch.Generator().manual_seed(22)
    xs[0] = torch.nn.functional.normalize(xs[0], dim=-1)
    xs[1] = torch.nn.functional.normalize(xs[1], dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    lg = torch.randn(B, T, H, M, generator=g)
    nm = 0.5 + torch.rand(D, generator=g)
    dout = torch.randn(B, T, H, D, generator=g)
    factors = (16, 16, 8, 8) if D == 128 else (8, 8, 8, 8)
    N = B * H * M
    G = og.reference_sketch(N, factors[2] * factors[3], min(8, factors[0] * factors[1], factors[2] * factors[3]))
    ins = [x.to(io) for x in xs[:2]] + [x for x in xs[2:]] + [v.to(io), lg, nm]

    dl = [t.to(DEV).requires_grad_(True) for t in ins]
    q, k, bp, pa, wp, pb, dp, vv, lgd, nmd = dl
    out = layer.gdn3_layer_core(q, k, vv, bp, pa, wp, pb, dp, RATES.to(DEV), lgd, nmd, factors=factors,
                                sketch=G.to(DEV))
    grads = torch.autograd.grad(out, dl, dout.to(DEV).to(out.dtype))
    torch.cuda.synchronize()

    leaves = [t.double().requires_grad_(True) for t in ins]
    q, k, bp, pa, wp, pb, dp, vv, lgd, nmd = leaves
    qr, kr, bg, wg, dec = gl.prologue(q, k, bp, pa, wp, pb, dp, RATES, 0.999)
    ve = vv.unsqueeze(3).expand(B, T, H, M, D)
    y = og.gdn3_recurrence(qr, kr, ve, bg, wg, dec, R=4, P=16, factors=factors, compact_every=16, sketch=G,
                           sign_mode="canonical", slow_decay=0.97)
    ref = gl.epilogue(y, lgd, nmd)
    gref = torch.autograd.grad(ref, leaves, dout.double())
    tol = 1e-2 if io == torch.bfloat16 else 2e-4
    err = rel_l2(out, ref)
    print(f"  out rel-L2 {err:.2e}", flush=True)
    assert err <= tol
    names = ("dq", "dk", "d_b_proj", "d_proj_a", "d_w_proj", "d_proj_b", "d_decay_proj", "dv",
             "d_router_logits", "d_norm")
    for name, a, r in zip(names, grads, gref):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= tol, name

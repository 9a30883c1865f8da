"""GDN3 dense-regime layer recurrence (gdnx_amd.gdn3.gdn3_scan) on the GPU:
the exact-alpha coefficient kernel and its backward, and the whole scan's
outputs and gradients (q, k, v, beta, log_g) against torch autograd through
the float64 CPU oracle (rel-L2 <= 1e-4 for float32 IO, <= 1e-2 for bf16)."""
import pytest
import torch

from oracle import delta, inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [128, 64])
def test_coeff_kernel_matches_oracle(gpu_lib, dtype, D):
    """a = alpha(beta |k|^2) beta and its gradients across the three branches
    of the kernel: |c| < 1e-6 (Taylor value), c < 0.05 (series derivative)
    and the closed forms; zero keys give c = 0 exactly."""
    from gdnx_amd import ops
    print(f"case: gdn3 coeff D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(21)
    B, T, H, M = 2, 37, 3, 4
    k = torch.randn(B, T, H, D, generator=g)
    scale = torch.tensor([1.0, 1e-2, 1e-4, 3.0])[torch.randint(0, 4, (B, T, H, 1), generator=g)]
    k = (k * scale / D ** 0.5).to(dtype)
    k[0, 3] = 0
    beta = torch.sigmoid(torch.randn(B, T, H, M, generator=g)) * torch.tensor([1.0, 1e-3, 0.3, 2.0])
    da_e, da_w = torch.randn(B, T, H, M, generator=g), torch.randn(B, T, H, M, generator=g)
    kd = k.double().requires_grad_(True)
    bd = beta.double().requires_grad_(True)
    a_ref = delta.gdn3_dense_coeffs(kd, bd)
    a = ops.gdn3_coeff(k.to(DEV), beta.to(DEV))
    assert rel_l2(a, a_ref) <= 1e-6
    dk_ref, db_ref = torch.autograd.grad(a_ref, (kd, bd), grad_outputs=(da_e + da_w).double())
    dk = torch.zeros(B, T, H, D, dtype=dtype, device=DEV)
    db = ops.gdn3_coeff_bwd(k.to(DEV), beta.to(DEV), da_e.to(DEV), da_w.to(DEV), dk)
    torch.cuda.synchronize()
    assert rel_l2(db, db_ref) <= 1e-5
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_l2(dk, dk_ref) <= tol
    # the key gradient is added into dk in place
    ops.gdn3_coeff_bwd(k.to(DEV), beta.to(DEV), da_e.to(DEV), da_w.to(DEV), dk)
    assert rel_l2(dk, 2 * dk_ref) <= tol


def _oracle_grads(x, dtype, dO):
    ins = [(x[n].to(dtype) if n in "qkv" else x[n]).double().requires_grad_(True)
           for n in ("q", "k", "v", "beta", "g")]
    a = delta.gdn3_dense_coeffs(ins[1], ins[3])
    y, _ = delta.lane_delta(ins[0], ins[1], ins[2], a, a, ins[4], chunk=32)
    return y, torch.autograd.grad(y, ins, grad_outputs=dO.to(dtype).double())


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("D,T", [(128, 200), (64, 77)])
def test_gdn3_scan_gradients(gpu_lib, dtype, tol, D, T):
    from gdnx_amd import gdn3
    print(f"case: gdn3_scan grads D={D} T={T} {dtype}", flush=True)
    x = inputs.dense_inputs(2, T, 2, D, M=4, seed=31, decay="tau", rope=True, with_grad_out=True)
    ins = [(x[n].to(dtype) if n in "qkv" else x[n]).to(DEV).requires_grad_(True)
           for n in ("q", "k", "v", "beta", "g")]
    y = gdn3.gdn3_scan(*ins)
    grads = torch.autograd.grad(y, ins, grad_outputs=x["dO"].to(dtype).to(DEV))
    torch.cuda.synchronize()
    y_ref, g_ref = _oracle_grads(x, dtype, x["dO"])
    assert rel_l2(y, y_ref) <= tol
    for name, gg, rr in zip(("dq", "dk", "dv", "dbeta", "dg"), grads, g_ref):
        err = rel_l2(gg, rr)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= tol, name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gdn3_scan_bitwise_repeatable(gpu_lib, dtype):
    """gdn3_scan forward and backward run twice on the same inputs in one
    process give bitwise equal outputs and gradients (fixed summation orders,
    no atomics; the reference pins its two scan paths bitwise,
    tests/ablation/test_fast_scan_api.py:272,317)."""
    from gdnx_amd import gdn3
    print(f"case: gdn3_scan bitwise repeat {dtype}", flush=True)
    x = inputs.dense_inputs(2, 300, 2, 128, M=4, seed=61, decay="tau", rope=True, with_grad_out=True)
    runs = []
    for _ in range(2):
        ins = [(x[n].to(dtype) if n in "qkv" else x[n]).to(DEV).requires_grad_(True)
               for n in ("q", "k", "v", "beta", "g")]
        y = gdn3.gdn3_scan(*ins)
        g = torch.autograd.grad(y, ins, grad_outputs=x["dO"].to(dtype).to(DEV))
        runs.append([y.detach()] + list(g))
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("P,Kc", [(16, 16), (32, 64)], ids=["layer-default", "p32"])
def test_gdn3_recurrent_state_bitwise_repeatable(gpu_lib, P, Kc):
    """The Kronecker-residual regime (window, compaction, backward) run twice
    in one process: bitwise equal y, final state and gradients."""
    import torch.nn.functional as F
    from gdnx_amd import gdn3
    from oracle import gdn3 as og
    print(f"case: gdn3_recurrent_state bitwise repeat P={P} Kc={Kc}", flush=True)
    g = torch.Generator().manual_seed(62)
    B, T, H, M, D = 1, 200, 2, 2, 128
    q = F.normalize(torch.randn(B, T, H, M, D, generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, T, H, M, D, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, T, H, M, D, generator=g).bfloat16()
    bg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    wg = torch.sigmoid(torch.randn(B, T, H, M, D, generator=g))
    dec = torch.exp(-torch.rand(B, T, H, M, generator=g) * 0.05)
    dy = torch.randn(B, T, H, M, D, generator=g).bfloat16()
    G = og.reference_sketch(B * H * M, 64, 8).to(DEV)
    runs = []
    for _ in range(2):
        leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bg, wg, dec)]
        y, st, _ = gdn3.gdn3_recurrent_state(*leaves, P=P, compact_every=Kc, sketch=G, return_state=True)
        grads = torch.autograd.grad(y, leaves, dy.to(DEV))
        runs.append([y.detach()] + [s.detach() for s in st] + list(grads))
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)

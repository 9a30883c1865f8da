"""Backward parity of the HIP chunked delta rule against torch autograd
through the float64 CPU oracle (tolerances: rel-L2 <= 1e-4 for float32 IO,
<= 1e-2 for bf16 IO, for outputs and every gradient)."""
import pytest
import torch

from oracle import delta, inputs

pytestmark = pytest.mark.gpu
NAMES = ["q", "k", "v", "a_e", "a_w", "log_g"]


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _case(B, T, H, D, M, seed, dtype, decay="tau"):
    if decay == "tau" and M > 4:
        decay = "softplus"
    taus = (0.05, 0.02, 0.005, 0.001)[:M] if decay == "tau" else None
    x = inputs.dense_inputs(B, T, H, D, M=M, seed=seed, decay=decay, taus=taus, rope=True,
                            with_grad_out=True)
    a = delta.gdn3_dense_coeffs(x["k"].double(), x["beta"].double()).float()
    gen = torch.Generator().manual_seed(seed + 1)
    aw = (a * (0.5 + torch.rand(a.shape, generator=gen))).float()   # decoupled write coefficient
    vals = [x["q"].to(dtype), x["k"].to(dtype), x["v"].to(dtype), a, aw, x["g"].float()]
    return vals, x["dO"].to(dtype)


def _grads_gpu(vals, dO, state0=None, dstate=None):
    from gdnx_amd import ops
    dev = "cuda:0"
    ins = [t.to(dev).clone().requires_grad_(True) for t in vals]
    s0 = None if state0 is None else state0.to(dev).clone().requires_grad_(True)
    y, sT = ops.delta_rule(*ins, state0=s0)
    loss = (y.float() * dO.to(dev).float()).sum()
    if dstate is not None:
        loss = loss + (sT * dstate.to(dev)).sum()
    wrt = ins + ([s0] if s0 is not None else [])
    g = torch.autograd.grad(loss, wrt)
    torch.cuda.synchronize()
    return y.detach(), [t.cpu() for t in g]


def _grads_oracle(vals, dO, state0=None, dstate=None):
    ins = [t.double().clone().requires_grad_(True) for t in vals]
    s0 = None if state0 is None else state0.double().clone().requires_grad_(True)
    y, sT = delta.lane_delta(*ins, state0=s0, chunk=16)
    loss = (y * dO.double()).sum()
    if dstate is not None:
        loss = loss + (sT * dstate.double()).sum()
    wrt = ins + ([s0] if s0 is not None else [])
    return y.detach(), list(torch.autograd.grad(loss, wrt))


def _check(vals, dO, tol, **kw):
    yg, gg = _grads_gpu(vals, dO, **kw)
    yo, go = _grads_oracle(vals, dO, **kw)
    errs = {"y": rel_l2(yg, yo)}
    for n, a, b in zip(NAMES + ["state0"], gg, go):
        errs[n] = rel_l2(a, b)
    print(errs, flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


@pytest.mark.parametrize("D,T,M", [(64, 256, 1), (128, 100, 2), (64, 45, 3)])
def test_fp32_gradients(gpu_lib, D, T, M):
    print(f"case: fp32 grads D={D} T={T} M={M}", flush=True)
    vals, dO = _case(1, T, 2, D, M, seed=21, dtype=torch.float32)
    _check(vals, dO, 1e-4)


def test_config0_gradients(gpu_lib):
    print("case: config0 grads", flush=True)
    vals, dO = _case(1, 256, 2, 64, 1, seed=1000, dtype=torch.float32, decay="softplus")
    _check(vals, dO, 1e-4)


@pytest.mark.parametrize("D,T", [(128, 200), (64, 96)])
def test_bf16_gradients(gpu_lib, D, T):
    print(f"case: bf16 grads D={D} T={T}", flush=True)
    vals, dO = _case(2, T, 2, D, 4, seed=22, dtype=torch.bfloat16)
    _check(vals, dO, 1e-2)


@pytest.mark.parametrize("T", [31, 64, 97, 330])
def test_bf16_state_gradients_ragged(gpu_lib, T):
    """bf16 at head dim 128 (the training configuration): a single partial
    chunk, whole chunks and ragged tails, with initial and final state
    gradients."""
    print(f"case: bf16 state grads T={T}", flush=True)
    vals, dO = _case(1, T, 3, 128, 4, seed=24, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(25)
    s0 = torch.randn(1, 3, 4, 128, 128, generator=gen) * 0.05
    ds = torch.randn(1, 3, 4, 128, 128, generator=gen) * 0.1
    _check(vals, dO, 1e-2, state0=s0, dstate=ds)


@pytest.mark.parametrize("D,T,M", [(128, 600, 3), (64, 520, 1), (128, 513, 2), (128, 300, 5)],
                         ids=["d128-3seg-M3", "d64-3seg-M1", "d128-3seg-M2", "d128-M5"])
def test_bf16_checkpointed_segments(gpu_lib, D, T, M):
    """The bf16 training default (32-token chunks): the forward keeps one state
    per 256-token segment, the reverse scan forms P3 = R dS^T at every chunk
    end, and the gradient kernel rebuilds the states forward inside each
    segment.  Several segments with ragged tails (T = 513 leaves a one-token
    segment), three lanes, one lane, and M = 5 (more lanes than the
    checkpointed kernel takes: the per-chunk stash), with initial and final
    state gradients."""
    print(f"case: bf16 checkpointed D={D} T={T} M={M}", flush=True)
    vals, dO = _case(1, T, 2, D, M, seed=26, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(27)
    s0 = torch.randn(1, 2, M, D, D, generator=gen) * 0.05
    ds = torch.randn(1, 2, M, D, D, generator=gen) * 0.1
    _check(vals, dO, 1e-2, state0=s0, dstate=ds)


@pytest.mark.parametrize("chunk", [32, 64])
def test_bf16_backward_bitwise_repeatable(gpu_lib, chunk):
    """Two runs of the training forward + backward on the same inputs in one
    process give bitwise equal outputs and gradients (fixed summation orders,
    no atomics), as the reference pins its two scan paths bitwise
    (tests/ablation/test_fast_scan_api.py:272,317)."""
    from gdnx_amd import ops
    print(f"case: bitwise repeat chunk={chunk}", flush=True)
    vals, dO = _case(2, 400, 3, 128, 4, seed=28, dtype=torch.bfloat16)
    dev = "cuda:0"
    q, k, v, ae, aw, lg = (t.to(dev).contiguous() for t in vals)
    runs = []
    for _ in range(2):
        y, s, cs = ops.delta_chunk_fwd(q, k, v, ae, aw, lg, return_state=True, save_states=True, chunk=chunk)
        g = ops.delta_chunk_bwd(q, k, v, ae, aw, lg, dO.to(dev), cs, chunk)[:6]
        runs.append([y, s] + list(g))
    torch.cuda.synchronize()
    for a_, b_ in zip(*runs):
        assert torch.equal(a_, b_)


def test_state_gradients_fp32(gpu_lib):
    print("case: state0/dstate grads", flush=True)
    vals, dO = _case(1, 70, 2, 64, 2, seed=23, dtype=torch.float32)
    gen = torch.Generator().manual_seed(9)
    s0 = torch.randn(1, 2, 2, 64, 64, generator=gen) * 0.1
    ds = torch.randn(1, 2, 2, 64, 64, generator=gen)
    _check(vals, dO, 1e-4, state0=s0, dstate=ds)


def test_unused_output_gradients(gpu_lib):
    """An output the loss does not use reaches the backward as None (no zero
    tensor filled): a loss of y alone gives the gradients of y plus a zero
    state gradient, and a loss of the final state alone those of the state
    plus a zero dy, bit for bit."""
    from gdnx_amd import ops
    print("case: unused output gradients", flush=True)
    dev = "cuda:0"
    vals, dO = _case(1, 70, 2, 64, 2, seed=29, dtype=torch.float32)
    ds = torch.randn(1, 2, 2, 64, 64, generator=torch.Generator().manual_seed(5)).to(dev)
    dO = dO.to(dev).float()

    def grads(use_y, use_s, zero_other):
        ins = [t.to(dev).clone().requires_grad_(True) for t in vals]
        y, sT = ops.delta_rule(*ins)
        loss = (y.float() * (dO if use_y else 0 * dO)).sum() if use_y or zero_other else 0
        if use_s or zero_other:
            loss = loss + (sT * (ds if use_s else 0 * ds)).sum()
        g = torch.autograd.grad(loss, ins)
        torch.cuda.synchronize()
        return [t.cpu() for t in g]

    for use_y, use_s in ((True, False), (False, True)):
        for a_, b_ in zip(grads(use_y, use_s, False), grads(use_y, use_s, True)):
            assert torch.equal(a_, b_)


def test_config2_full_size_gradients(gpu_lib):
    """Config 2 (B=4, T=4096, H=16, D=128, 4 lanes, bf16) end to end on the
    GPU; the float64 oracle checks batch 0 / head 0 (heads are independent,
    so their q/k/v gradients are exact sub-blocks)."""
    print("case: config2 full size", flush=True)
    from gdnx_amd import ops
    x = inputs.config2()
    dev = "cuda:0"
    a = delta.gdn3_dense_coeffs(x["k"].double(), x["beta"].double()).float()
    vals = [x["q"], x["k"], x["v"], a, a.clone(), x["g"].float()]
    ins = [t.to(dev).requires_grad_(True) for t in vals]
    y, _ = ops.delta_rule(*ins)
    g = torch.autograd.grad((y.float() * x["dO"].to(dev).float()).sum(), ins)
    torch.cuda.synchronize()
    for t in g:
        assert torch.isfinite(t.float()).all()
    sub = [t[:1, :, :1] for t in vals]
    yo, go = _grads_oracle(sub, x["dO"][:1, :, :1])
    errs = {"y": rel_l2(y[:1, :, :1], yo)}
    for n, a_, b_ in zip(NAMES, g, go):
        errs[n] = rel_l2(a_[:1, :, :1], b_)
    print(errs, flush=True)
    assert all(v <= 1e-2 for v in errs.values()), errs


@pytest.mark.parametrize("chunk", [32, 64])
def test_bf16_gradients_explicit_chunk(gpu_lib, chunk):
    """The bf16 training forward and backward at both stash chunks (32, the
    default: one state per 256-token segment, recomputed by the checkpointed
    gradient kernel; 64: every chunk's state stashed, one gradient workgroup
    per chunk), through the ops layer."""
    from gdnx_amd import ops
    print(f"case: bf16 grads chunk={chunk}", flush=True)
    vals, dO = _case(2, 150, 3, 128, 4, seed=24, dtype=torch.bfloat16)
    dev = "cuda:0"
    q, k, v, ae, aw, lg = (t.to(dev).contiguous() for t in vals)
    y, _, cs = ops.delta_chunk_fwd(q, k, v, ae, aw, lg, save_states=True, chunk=chunk)
    grads = ops.delta_chunk_bwd(q, k, v, ae, aw, lg, dO.to(dev), cs, chunk)[:6]
    torch.cuda.synchronize()
    yo, go = _grads_oracle(vals, dO)
    errs = {"y": rel_l2(y, yo)}
    errs.update({n: rel_l2(a_, b_) for n, a_, b_ in zip(NAMES, grads, go)})
    print(errs, flush=True)
    assert all(v_ <= 1e-2 for v_ in errs.values()), errs


def test_config2_full_size_gdn3_scan(gpu_lib):
    """Config 2 end to end through gdn3.gdn3_scan, the op the headline bench
    times (coefficient kernel, prep, scans, gradient kernels, coefficient
    backward), differentiated in q, k, v, beta and log_g; the float64 oracle
    (exact-alpha coefficient + chunked delta rule) checks batch 0 / head 0."""
    print("case: config2 full size gdn3_scan", flush=True)
    from gdnx_amd import gdn3
    x = inputs.config2()
    dev = "cuda:0"
    ins = [x[n].to(dev).requires_grad_(True) for n in ("q", "k", "v", "beta", "g")]
    y = gdn3.gdn3_scan(*ins)
    g = torch.autograd.grad(y, ins, grad_outputs=x["dO"].to(dev))
    torch.cuda.synchronize()
    for t in g:
        assert torch.isfinite(t.float()).all()
    sub = [x[n][:1, :, :1].double().requires_grad_(True) for n in ("q", "k", "v", "beta", "g")]
    a = delta.gdn3_dense_coeffs(sub[1], sub[3])
    yo, _ = delta.lane_delta(sub[0], sub[1], sub[2], a, a, sub[4], chunk=16)
    go = torch.autograd.grad(yo, sub, grad_outputs=x["dO"][:1, :, :1].double())
    errs = {"y": rel_l2(y[:1, :, :1], yo)}
    errs.update({n: rel_l2(a_[:1, :, :1], b_) for n, a_, b_ in zip(("dq", "dk", "dv", "dbeta", "dg"), g, go)})
    print(errs, flush=True)
    assert all(v_ <= 1e-2 for v_ in errs.values()), errs

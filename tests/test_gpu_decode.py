"""Decode step parity: the HIP one-token step against the CPU oracle's
sequential recurrence on the same carried state, and against the chunked
forward (T decode steps equal one T-token chunked scan)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import delta, inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _coeffs(k, beta, n_tau):
    """Config 4 chains: every lane's a = alpha(beta |k|^2) beta is shared by
    its n_tau decay chains."""
    a = delta.gdn3_dense_coeffs(k.double(), beta.double()).float()
    return a.repeat_interleave(n_tau, dim=-1).contiguous()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [128, 64])
def test_decode_steps_match_oracle(gpu_lib, dtype, D):
    from gdnx_amd import ops
    print(f"case: decode 4 steps D={D} {dtype}", flush=True)
    NS, H, M, NT, steps = 3, 2, 2, 2, 4
    x = inputs.decode_inputs(S=NS, H=H, M=M, n_tau=NT, d=D, steps=steps, seed=41)
    state = x["state0"].reshape(NS, H, M * NT, D, D).contiguous()
    st_gpu = state.to(DEV).clone()
    ref_state = state.double()
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-4
    for t in range(steps):
        q, k, v = (x[n][t].to(dtype) for n in ("q", "k", "v"))
        a = _coeffs(k, x["beta"][t], NT)
        lg = x["g"][t].reshape(NS, H, M * NT).contiguous()
        y = ops.delta_decode_step(q.to(DEV), k.to(DEV), v.to(DEV), a.to(DEV), a.to(DEV), lg.to(DEV), st_gpu)
        yo, ref_state = delta.lane_delta(q[:, None], k[:, None], v[:, None], a[:, None], a[:, None],
                                         lg[:, None], state0=ref_state)
        torch.cuda.synchronize()
        assert y.dtype == dtype and y.shape == (NS, H, M * NT, D)
        assert rel_l2(y, yo[:, 0]) <= tol, t
    assert rel_l2(st_gpu, ref_state) <= 1e-5


def test_decode_equals_chunked_forward(gpu_lib):
    """T decode steps from a carried state == one chunked forward over T tokens."""
    from gdnx_amd import ops
    print("case: decode vs chunked forward", flush=True)
    B, T, H, M, D = 2, 5, 3, 4, 128
    x = inputs.dense_inputs(B, T, H, D, M=M, seed=42, decay="tau", rope=True)
    a = delta.gdn3_dense_coeffs(x["k"].double(), x["beta"].double()).float()
    s0 = torch.randn(B, H, M, D, D, generator=torch.Generator().manual_seed(3)) * 0.02
    q, k, v = (x[n].to(DEV) for n in ("q", "k", "v"))
    a, g = a.to(DEV), x["g"].to(DEV)
    y_chunk, s_chunk, _ = ops.delta_chunk_fwd(q, k, v, a, a, g, state0=s0.to(DEV), return_state=True)
    st = s0.to(DEV).clone()
    ys = [ops.delta_decode_step(q[:, t].contiguous(), k[:, t].contiguous(), v[:, t].contiguous(),
                                a[:, t].contiguous(), a[:, t].contiguous(), g[:, t].contiguous(), st)
          for t in range(T)]
    torch.cuda.synchronize()
    assert rel_l2(torch.stack(ys, 1), y_chunk) <= 1e-4
    assert rel_l2(st, s_chunk) <= 1e-4


def test_decode_config4_full_size(gpu_lib):
    """Config 4 width: 256 sequences x 16 heads x (4 lanes x 4 decays) chains
    of 128x128 fp32 state (4.3 GB), bf16 IO.  One step on the GPU, checked on
    a 2x2-head subset by the oracle; the rest must stay finite."""
    from gdnx_amd import ops
    print("case: decode config4 full size", flush=True)
    NS, H, M, NT, D = 256, 16, 4, 4, 128
    state = torch.randn(NS, H, M * NT, D, D, device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(1004)) * 0.02
    gen = torch.Generator().manual_seed(1005)
    q = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
    v = torch.randn(NS, H, D, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(NS, H, M, generator=gen))
    a = _coeffs(k, beta, NT)
    base = torch.log1p(-torch.tensor(inputs.TAUS)).repeat(M)
    lg = (base.view(1, 1, M * NT) + 0.01 * torch.randn(NS, H, M * NT, generator=gen)).contiguous()
    sub = state[:2, :2].double().cpu()
    y = ops.delta_decode_step(q.to(DEV), k.to(DEV), v.to(DEV), a.to(DEV), a.to(DEV), lg.to(DEV), state)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    yo, so = delta.lane_delta(q[:2, None, :2], k[:2, None, :2], v[:2, None, :2], a[:2, None, :2],
                              a[:2, None, :2], lg[:2, None, :2], state0=sub)
    assert rel_l2(y[:2, :2], yo[:, 0]) <= 1e-2
    assert rel_l2(state[:2, :2], so) <= 1e-5

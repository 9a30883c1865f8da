"""Forward parity of the HIP chunked delta-rule kernel against the CPU oracle."""
import pytest
import torch

from oracle import delta, inputs

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _coeffs(x):
    a = delta.gdn3_dense_coeffs(x["k"].double(), x["beta"].double()).float()
    return a


def _run(gpu_lib, x, dtype):
    from gdnx_amd import ops
    dev = "cuda:0"
    a = _coeffs(x).to(dev)
    y, _, _ = ops.delta_chunk_fwd(x["q"].to(dev, dtype).contiguous(), x["k"].to(dev, dtype).contiguous(),
                                  x["v"].to(dev, dtype).contiguous(), a, a.clone(),
                                  x["g"].to(dev).contiguous())
    torch.cuda.synchronize()
    return y


def _oracle(x, dtype):
    # oracle sees the same (rounded) inputs as the kernel
    q, k, v = (x[n].to(dtype).double() for n in ("q", "k", "v"))
    return delta.gdn3_dense_layer(q, k, v, x["beta"].double(), x["g"].double(), chunk=64)


def test_config0_fp32(gpu_lib):
    print("case: config0 fp32 B=1 T=256 H=2 D=64", flush=True)
    x = inputs.config0()
    y = _run(gpu_lib, x, torch.float32)
    ref = _oracle(x, torch.float32)
    assert y.shape == ref.shape
    assert rel_l2(y, ref) <= 1e-4


@pytest.mark.parametrize("D,T,M", [(128, 100, 2), (64, 77, 3), (128, 256, 4)])
def test_fp32_shapes(gpu_lib, D, T, M):
    print(f"case: fp32 D={D} T={T} M={M}", flush=True)
    taus = (0.05, 0.02, 0.005, 0.001)[:M]
    x = inputs.dense_inputs(2, T, 3, D, M=M, seed=11, decay="tau", taus=taus, rope=True)
    y = _run(gpu_lib, x, torch.float32)
    assert rel_l2(y, _oracle(x, torch.float32)) <= 1e-4


@pytest.mark.parametrize("D,T", [(128, 300), (64, 130), (128, 64)])
def test_bf16_shapes(gpu_lib, D, T):
    print(f"case: bf16 D={D} T={T}", flush=True)
    x = inputs.dense_inputs(2, T, 2, D, M=4, seed=12, decay="tau", rope=True)
    y = _run(gpu_lib, x, torch.bfloat16)
    assert y.dtype == torch.bfloat16
    assert rel_l2(y, _oracle(x, torch.bfloat16)) <= 1e-2


def test_realistic_decay_fp32(gpu_lib):
    """Decays spanning (0, 1] (the reference bench's distribution,
    research/kernel_ab/bench_scan.py:46-51), including exact zeros."""
    print("case: realistic decay fp32", flush=True)
    x = inputs.dense_inputs(1, 200, 2, 64, M=1, seed=13)
    gen = torch.Generator().manual_seed(5)
    x["g"] = -torch.nn.functional.softplus(1.2 * torch.randn(x["g"].shape, generator=gen) - 0.6)
    x["g"][0, 70, 0, 0] = -float("inf")
    y = _run(gpu_lib, x, torch.float32)
    assert rel_l2(y, _oracle(x, torch.float32)) <= 1e-4


def test_state_carry_split_equals_whole(gpu_lib):
    from gdnx_amd import ops
    print("case: split-run state carry", flush=True)
    dev = "cuda:0"
    x = inputs.dense_inputs(1, 192, 2, 128, M=2, seed=14, decay="tau", taus=(0.05, 0.001))
    q, k, v = (x[n].to(dev).contiguous() for n in ("q", "k", "v"))
    a = _coeffs(x).to(dev)
    g = x["g"].to(dev)
    y, s, _ = ops.delta_chunk_fwd(q, k, v, a, a, g, return_state=True)
    y1, s1, _ = ops.delta_chunk_fwd(q[:, :96].contiguous(), k[:, :96].contiguous(), v[:, :96].contiguous(),
                                    a[:, :96].contiguous(), a[:, :96].contiguous(), g[:, :96].contiguous(),
                                    return_state=True)
    y2, s2, _ = ops.delta_chunk_fwd(q[:, 96:].contiguous(), k[:, 96:].contiguous(), v[:, 96:].contiguous(),
                                    a[:, 96:].contiguous(), a[:, 96:].contiguous(), g[:, 96:].contiguous(),
                                    state0=s1, return_state=True)
    assert rel_l2(torch.cat([y1, y2], 1), y) <= 1e-5
    assert rel_l2(s2, s) <= 1e-5


def test_config1_full_size_against_oracle_subset(gpu_lib):
    """Config 1 at full size (B=4, T=4096, H=16, D=128, 4 lanes, bf16): the
    kernel runs on all 256 chains; the chunked float64 oracle checks batch 0,
    heads 0-1 (chains are independent)."""
    print("case: config1 full size", flush=True)
    x = inputs.config1()
    y = _run(gpu_lib, x, torch.bfloat16)
    assert torch.isfinite(y.float()).all()
    sub = {n: x[n][:1, :, :2] for n in ("q", "k", "v", "beta", "g")}
    ref = _oracle(sub, torch.bfloat16)
    assert rel_l2(y[:1, :, :2], ref) <= 1e-2

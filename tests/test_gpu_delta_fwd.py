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


def _run(gpu_lib, x, dtype, two_pass=False):
    """two_pass False: the fused single-kernel scan; True: the parallel
    chunk-operand pass plus the value-split scan (the training path)."""
    from gdnx_amd import ops
    dev = "cuda:0"
    a = _coeffs(x).to(dev)
    y, _, _ = ops.delta_chunk_fwd(x["q"].to(dev, dtype).contiguous(), x["k"].to(dev, dtype).contiguous(),
                                  x["v"].to(dev, dtype).contiguous(), a, a.clone(),
                                  x["g"].to(dev).contiguous(), two_pass=two_pass)
    torch.cuda.synchronize()
    return y


def _oracle(x, dtype):
    # oracle sees the same (rounded) inputs as the kernel
    q, k, v = (x[n].to(dtype).double() for n in ("q", "k", "v"))
    return delta.gdn3_dense_layer(q, k, v, x["beta"].double(), x["g"].double(), chunk=64)


@pytest.mark.parametrize("two_pass", [False, True])
def test_config0_fp32(gpu_lib, two_pass):
    print(f"case: config0 fp32 B=1 T=256 H=2 D=64 two_pass={two_pass}", flush=True)
    x = inputs.config0()
    y = _run(gpu_lib, x, torch.float32, two_pass)
    ref = _oracle(x, torch.float32)
    assert y.shape == ref.shape
    assert rel_l2(y, ref) <= 1e-4


@pytest.mark.parametrize("two_pass", [False, True])
@pytest.mark.parametrize("D,T,M", [(128, 100, 2), (64, 77, 3), (128, 256, 4)])
def test_fp32_shapes(gpu_lib, D, T, M, two_pass):
    print(f"case: fp32 D={D} T={T} M={M} two_pass={two_pass}", flush=True)
    taus = (0.05, 0.02, 0.005, 0.001)[:M]
    x = inputs.dense_inputs(2, T, 3, D, M=M, seed=11, decay="tau", taus=taus, rope=True)
    y = _run(gpu_lib, x, torch.float32, two_pass)
    assert rel_l2(y, _oracle(x, torch.float32)) <= 1e-4


@pytest.mark.parametrize("two_pass", [False, True])
@pytest.mark.parametrize("D,T", [(128, 300), (64, 130), (128, 64)])
def test_bf16_shapes(gpu_lib, D, T, two_pass):
    print(f"case: bf16 D={D} T={T} two_pass={two_pass}", flush=True)
    x = inputs.dense_inputs(2, T, 2, D, M=4, seed=12, decay="tau", rope=True)
    y = _run(gpu_lib, x, torch.bfloat16, two_pass)
    assert y.dtype == torch.bfloat16
    assert rel_l2(y, _oracle(x, torch.bfloat16)) <= 1e-2


@pytest.mark.parametrize("two_pass", [False, True])
def test_realistic_decay_fp32(gpu_lib, two_pass):
    """Decays spanning (0, 1] (the reference bench's distribution,
    research/kernel_ab/bench_scan.py:46-51), including exact zeros."""
    print(f"case: realistic decay fp32 two_pass={two_pass}", flush=True)
    x = inputs.dense_inputs(1, 200, 2, 64, M=1, seed=13)
    gen = torch.Generator().manual_seed(5)
    x["g"] = -torch.nn.functional.softplus(1.2 * torch.randn(x["g"].shape, generator=gen) - 0.6)
    x["g"][0, 70, 0, 0] = -float("inf")
    y = _run(gpu_lib, x, torch.float32, two_pass)
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


@pytest.mark.parametrize("two_pass", [False, True])
def test_config1_full_size_against_oracle_subset(gpu_lib, two_pass):
    """Config 1 at full size (B=4, T=4096, H=16, D=128, 4 lanes, bf16): the
    kernel runs on all 256 chains; the chunked float64 oracle checks batch 0,
    heads 0-1 (chains are independent)."""
    print(f"case: config1 full size two_pass={two_pass}", flush=True)
    x = inputs.config1()
    y = _run(gpu_lib, x, torch.bfloat16, two_pass)
    assert torch.isfinite(y.float()).all()
    sub = {n: x[n][:1, :, :2] for n in ("q", "k", "v", "beta", "g")}
    ref = _oracle(sub, torch.bfloat16)
    assert rel_l2(y[:1, :, :2], ref) <= 1e-2


@pytest.mark.parametrize("dtype,chunk", [(torch.bfloat16, 64), (torch.bfloat16, 32), (torch.float32, 32),
                                         (torch.float32, 16)])
def test_two_pass_equals_single_pass(gpu_lib, dtype, chunk):
    """The parallel operand pass + value-split scan gives the fused
    single-kernel result, and both write the same backward stash: states,
    net writes and chunk operands.  Same arithmetic; in bf16 the two-pass
    form rounds T to bf16 before scaling its columns by a_w / a_e exp(G)
    (the fused form rounds once after), so the two differ by up to about
    one bf16 rounding (each is checked against the oracle separately)."""
    from gdnx_amd import ops
    print(f"case: two-pass vs single-pass {dtype} C={chunk}", flush=True)
    x = inputs.dense_inputs(2, 200, 3, 128, M=4, seed=77, decay="tau", rope=True, io_dtype=dtype)
    a = delta.gdn3_dense_coeffs(x["k"].double(), x["beta"].double()).float()
    s0 = torch.randn(2, 3, 4, 128, 128, generator=torch.Generator().manual_seed(1)) * 0.02
    args = [t.to("cuda:0") for t in (x["q"], x["k"], x["v"], a, a, x["g"])]
    rn = torch.empty(2, 200, 3, 4, device="cuda:0")
    # two-pass, with and without a stash; fused single kernel (the scored variant), with a stash
    y1, s1, c1 = ops.delta_chunk_fwd(*args, s0.to("cuda:0"), return_state=True, save_states=True, chunk=chunk)
    y3, s3, _ = ops.delta_chunk_fwd(*args, s0.to("cuda:0"), return_state=True, chunk=chunk, two_pass=True)
    y2, s2, c2 = ops.delta_chunk_fwd(*args, s0.to("cuda:0"), return_state=True, save_states=True, chunk=chunk,
                                     r_norm=rn)
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 5e-3
    assert rel_l2(y1, y2) <= tol
    assert rel_l2(s1, s2) <= tol
    assert torch.equal(y1, y3) and torch.equal(s1, s3)
    # states and net writes (compute dtype) agree to rounding; the chunk
    # operands come from the same prep kernel on both paths: bitwise equal
    # the stash precedes the chunk operands: its size is the whole buffer's
    # less the operand records' (bf16 C = 32 keeps one record per chunk pair)
    lib = gpu_lib
    code = 1 if dtype == torch.bfloat16 else 0
    nst = (lib.gdnx_delta_chunk_states_bytes(2, 200, 3, 4, 128, chunk, code)
           - lib.gdnx_delta_fwd_workspace_bytes(2, 200, 3, 4, 128, chunk, code))
    ct = torch.float32 if dtype == torch.float32 else torch.bfloat16
    assert rel_l2(c1[:nst].view(ct).float(), c2[:nst].view(ct).float()) <= tol
    assert torch.equal(c1[nst:], c2[nst:])
    # the intra-chunk phase alone (gdnx_delta_chunk_prep) writes the same records
    pw = ops.delta_chunk_prep(args[0], args[1], args[3], args[4], args[5], chunk=chunk)
    torch.cuda.synchronize()
    assert torch.equal(pw[:c1.numel() - nst], c1[nst:])

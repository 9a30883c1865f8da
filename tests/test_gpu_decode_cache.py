"""Decode-state cache (gdnx_amd.decode_cache, gdnx_delta_decode_step_slots)
on the GPU.  No reference counterpart (the reference keeps no recurrent
cache); checked against the library's other paths on the same inputs:
  * a slot-indexed step equals the contiguous step on the gathered states
    (bitwise), leaves other slots untouched and gives zeros for empty rows;
  * prefill over T0 tokens followed by T1 single-token steps equals one
    chunked forward over T0 + T1 tokens (outputs and final state; the
    chunked path itself is pinned against the float64 oracle in
    test_gpu_delta_fwd.py) -- rel-L2 1e-5 for float32 IO, 1e-2 for bf16
    (the chunked path rounds its MFMA operands to bf16, the step does not)."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _seq_inputs(B, T, H, M, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    a_e = torch.sigmoid(torch.randn(B, T, H, M, generator=g))
    a_w = torch.sigmoid(torch.randn(B, T, H, M, generator=g))
    log_g = -0.05 * torch.rand(B, T, H, M, generator=g) * torch.arange(1, M + 1).view(1, 1, 1, M)
    return [t.to(DEV) for t in (q.to(dtype), k.to(dtype), v.to(dtype), a_e, a_w, log_g)]


@pytest.mark.parametrize("D", [128, 64])
def test_slot_step_equals_contiguous_step(gpu_lib, D):
    from gdnx_amd import ops
    print(f"case: decode slots D={D}", flush=True)
    n_slots, NS, H, M = 6, 4, 2, 3
    g = torch.Generator().manual_seed(3)
    pool = (torch.randn(n_slots, H, M, D, D, generator=g) * 0.05).to(DEV)
    slots = torch.tensor([4, 1, -1, 2], dtype=torch.int32, device=DEV)
    q, k, v, a_e, a_w, log_g = (t[:, 0] for t in _seq_inputs(NS, 1, H, M, D, seed=4, dtype=torch.bfloat16))
    before = pool.clone()
    live = [0, 1, 3]
    ref_state = before[slots[live].long()].contiguous()
    y_ref = ops.delta_decode_step(*(t[live].contiguous() for t in (q, k, v, a_e, a_w, log_g)), ref_state)
    y = ops.delta_decode_step_slots(q, k, v, a_e, a_w, log_g, pool, slots)
    torch.cuda.synchronize()
    assert torch.equal(y[live], y_ref)
    assert torch.count_nonzero(y[2]) == 0
    for r, s in zip(live, slots[live].tolist()):
        assert torch.equal(pool[s], ref_state[live.index(r)])
    for s in (0, 3, 5):
        assert torch.equal(pool[s], before[s])


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_prefill_then_steps_equal_chunked_forward(gpu_lib, dtype, tol):
    from gdnx_amd import ops
    from gdnx_amd.decode_cache import DecodeStateCache
    print(f"case: prefill + decode vs chunked {dtype}", flush=True)
    B, T0, T1, H, M, D = 2, 37, 5, 2, 2, 128
    xs = _seq_inputs(B, T0 + T1, H, M, D, seed=7, dtype=dtype)
    y_full, s_full, _ = ops.delta_chunk_fwd(*xs, return_state=True)
    cache = DecodeStateCache(n_slots=5, H=H, M=M, D=D, device=DEV)
    other = cache.alloc(1)                      # an unrelated sequence stays untouched
    slots = cache.alloc(B)
    y_pre = cache.prefill(slots, *(t[:, :T0] for t in xs))
    ys = [cache.step(slots, *(t[:, T0 + i].contiguous() for t in xs)) for i in range(T1)]
    torch.cuda.synchronize()
    assert rel_l2(y_pre, y_full[:, :T0]) <= tol
    assert rel_l2(torch.stack(ys, 1), y_full[:, T0:]) <= tol
    assert rel_l2(cache.pool[slots], s_full) <= tol
    assert torch.count_nonzero(cache.pool[other]) == 0


def test_slot_reuse_starts_from_zero(gpu_lib):
    """A freed slot handed out again starts from a zero state: its step
    equals a step from zero; the batch mixes it with a live sequence and an
    empty row."""
    from gdnx_amd import ops
    from gdnx_amd.decode_cache import DecodeStateCache
    print("case: decode cache slot reuse", flush=True)
    H, M, D = 2, 2, 64
    cache = DecodeStateCache(n_slots=3, H=H, M=M, D=D, device=DEV)
    a, b = cache.alloc(2)
    cache.prefill([a, b], *_seq_inputs(2, 20, H, M, D, seed=9, dtype=torch.float32))
    kept = cache.pool[b].clone()
    cache.free([a])
    with pytest.raises(ValueError):
        cache.free([a])
    (c,) = cache.alloc(1)
    assert c == a and torch.count_nonzero(cache.pool[c]) == 0
    xs = [t[:, 0] for t in _seq_inputs(3, 1, H, M, D, seed=10, dtype=torch.float32)]
    y = cache.step([c, b, -1], *xs)
    s0 = torch.zeros(1, H, M, D, D, device=DEV)       # updated in place by the steps below
    s1 = kept.unsqueeze(0).clone()
    y0 = ops.delta_decode_step(*(t[:1].contiguous() for t in xs), s0)
    y1 = ops.delta_decode_step(*(t[1:2].contiguous() for t in xs), s1)
    torch.cuda.synchronize()
    assert torch.equal(y[0:1], y0) and torch.equal(cache.pool[c], s0[0])
    assert torch.equal(y[1:2], y1) and torch.equal(cache.pool[b], s1[0])
    assert torch.count_nonzero(y[2]) == 0

"""The allocation-free GDN3 forward (gdnx_gdn3_chunk_fwd_state_noalloc)
against the same forward with a caller workspace (gdnx_gdn3_chunk_fwd_state),
through the C ABI: two calls in a row, the second smaller, each bitwise equal
to the workspace entry point's results (same kernels, same order).  Its
static scratch keeps the previous call's contents, so the second call also
shows that nothing stale leaks into a call.  Beyond the scratch's size the
entry point refuses before any launch (tested on the CPU, in test_abi.py,
where no kernel can run on the fake pointers such a test passes).  The
layer's default regime (K_c = P = 16) runs as one fused launch that needs
no scratch, so it is taken whatever the chain count."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn3 as og

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, T, H, M, D, seed, io, P=16):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(io)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(io)
    v = torch.randn(B, T, H, D, generator=g).to(io)
    bg = torch.sigmoid(torch.randn(B, T, H, M, generator=g))
    wg = torch.sigmoid(torch.randn(B, T, H, M, generator=g))
    dec = torch.exp(-torch.rand(B, T, H, M, generator=g) * 0.05)
    N = B * H * M
    state = (torch.randn(N, 4, 16, 16, generator=g) * 0.1, torch.randn(N, 4, 8, 8, generator=g) * 0.3,
             torch.randn(N, D, P, generator=g) * 0.05, F.normalize(torch.randn(N, D, P, generator=g), dim=1))
    return [t.to(DEV).contiguous() for t in (q, k, v, bg, wg, dec)], [t.to(DEV).contiguous() for t in state]


def _run(lib, noalloc, x, st0, t0, B, T, H, M, D, io, P=16, Kc=32):
    from gdnx_amd import _lib
    N = B * H * M
    q, k, v, bg, wg, dec = x
    G = og.reference_sketch(N, 64, 8).to(DEV)
    y = torch.empty(B, T, H, M, D, dtype=io, device=DEV)
    out = [torch.empty_like(t) for t in st0]
    n_ev = lib.gdnx_gdn3_num_compactions_from(t0, T, P, Kc)
    stats = torch.empty(max(n_ev, 1), N, 2, dtype=torch.float64, device=DEV)
    p = _lib.ptr
    dt = _lib.dtype_code(io)
    stream = _lib.stream_of(q)
    common = [p(q), p(k), p(v), 1, p(bg), p(wg), 1, p(dec), p(G), *(p(t) for t in st0), t0, p(y),
              *(p(t) for t in out), p(stats)]
    dims = [B, T, H, M, D, 4, P, Kc, 16, 16, 8, 8, ctypes.c_float(0.97), dt, 0, stream]
    if noalloc:
        rc = lib.gdnx_gdn3_chunk_fwd_state_noalloc(*common, *dims)
    else:
        ws = torch.empty(lib.gdnx_gdn3_workspace_bytes(B, H, M, D, P, dt), dtype=torch.uint8, device=DEV)
        rc = lib.gdnx_gdn3_chunk_fwd_state(*common, p(ws), *dims)
    assert rc == 0, lib.gdnx_last_error().decode()
    torch.cuda.synchronize()
    return y, out, stats[:n_ev]


@pytest.mark.parametrize("P,Kc", [(16, 32), (16, 16), (32, 64)], ids=["window", "fused", "P32"])
@pytest.mark.parametrize("io", [torch.bfloat16, torch.float32])
def test_noalloc_forward_equals_workspace_forward(gpu_lib, io, P, Kc):
    lib = gpu_lib
    print(f"case: gdn3 no-alloc forward {io} P={P} Kc={Kc}", flush=True)
    # first a larger call, then a smaller one (fewer chains, other start slot)
    for (B, T, H, M, t0, seed) in ((2, 100, 4, 4, 37, 1), (1, 23, 2, 2, 5, 2)):
        x, st0 = _inputs(B, T, H, M, 128, seed, io, P)
        y_ref, s_ref, c_ref = _run(lib, False, x, st0, t0, B, T, H, M, 128, io, P, Kc)
        y, s, c = _run(lib, True, x, st0, t0, B, T, H, M, 128, io, P, Kc)
        assert torch.equal(y, y_ref), (B, T)
        for a, b in zip(s, s_ref):
            assert torch.equal(a, b), (B, T)
        assert torch.equal(c, c_ref)

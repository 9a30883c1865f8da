"""GDN3 compaction modes, the layer-method adapter, long horizons and the
non-finite status, on the GPU against the CPU oracle.

* 'sketch' / 'sketch_noqr' compaction (gdn3/gdn3_upgrade.py:579-592, one
  branch for both names): the oracle's compact_sketch is pinned by its closed
  form and rank-one known answers in tests/test_oracle_gdn3.py; the GPU's
  compaction kernel, forward, backward and decode step in that mode are held
  to it here.
* gdnx_amd.adapter: the drop-in GDN3LinearAttn._gdn3_recurrent_state on an
  object carrying the layer's attributes; y and _last_comp_err against the
  oracle (which restates gdn3/_reference_recurrence.py and the compaction).
* Long horizons: T = 1024 with a compaction every 16 tokens (64 compactions)
  forward and backward, and T = 512 at float32 with M = 2, against autograd
  through the float64 oracle.
* GDNX_ERR_NONFINITE: with checking on, a NaN input makes the recurrence
  entry points raise GdnxNonFinite; gdnx_check_finite scans one buffer.

Tolerances (rel-L2) as in the other GDN3 tests: 1e-4 for float32 IO, 1e-2
for bf16; 1e-3 for the compacted factors at float32.  The long-horizon cases
are held to the same 1e-4 for y and the gradients (measured on MI355X: 1.2e-5
to 7.7e-5); each compaction's SVD moves its singular vectors by (perturbation
of R_mat) / (singular-value gap), and 64 of them carry the fp32 rounding
forward, which is what the margin to 1e-4 covers.
"""
import ctypes
import types

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn3 as og
from oracle import inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _inputs(B, T, H, M, D, seed, io, gate, per_lane):
    g = torch.Generator().manual_seed(seed)
    shape_qkv = (B, T, H, M, D) if per_lane else (B, T, H, D)
    q = F.normalize(torch.randn(*shape_qkv, generator=g), dim=-1)
    k = F.normalize(torch.randn(*shape_qkv, generator=g), dim=-1)
    v = torch.randn(*shape_qkv, generator=g)
    gshape = (B, T, H, M, D) if gate == "channel" else (B, T, H, M)
    bg = torch.sigmoid(torch.randn(*gshape, generator=g))
    wg = torch.sigmoid(torch.randn(*gshape, generator=g))
    taus = torch.tensor([inputs.TAUS[m % 4] for m in range(M)])
    dec = torch.exp(torch.log1p(-taus).view(1, 1, 1, M) + 0.01 * torch.randn(B, T, H, M, generator=g))
    dy = torch.randn(B, T, H, M, D, generator=g)
    return [q.to(io), k.to(io), v.to(io), bg, wg, dec.clamp(max=1.0)], dy


def _oracle(xs, M, P, Kc, factors, G, mode="svd", slow_decay=0.97, dy=None):
    """y (and with dy the gradients of the six inputs) of the float64 oracle."""
    leaves = [x.double().requires_grad_(dy is not None) for x in xs]
    q, k, v, bg, wg, dec = leaves
    D = q.shape[-1]

    def lanes(x):
        return x if x.dim() == 5 else x.unsqueeze(3).expand(*x.shape[:3], M, x.shape[-1])

    def gates(x):
        return x if x.dim() == 5 else x.unsqueeze(-1).expand(*x.shape, D)
    with torch.set_grad_enabled(dy is not None):
        y, state, err = og.gdn3_recurrence(lanes(q), lanes(k), lanes(v), gates(bg), gates(wg), dec, R=4, P=P,
                                           factors=factors, compact_every=Kc, sketch=G, sign_mode="canonical",
                                           slow_decay=slow_decay, return_state=True, compact_mode=mode)
    if dy is None:
        return y, state, err
    return y, torch.autograd.grad(y, leaves, dy.double())


# ---------------------------------------------------------------------------
# sketch compaction mode
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("factors,P", [((16, 16, 8, 8), 16), ((8, 8, 8, 8), 32)])
def test_sketch_compact_matches_oracle(gpu_lib, factors, P):
    from gdnx_amd import ops
    print(f"case: sketch compact factors={factors} P={P}", flush=True)
    N, R = 6, 4
    a_v, a_k, b_v, b_k = factors
    g = torch.Generator().manual_seed(12)
    A = torch.randn(N, R, a_v, a_k, generator=g)
    Bk = torch.randn(N, R, b_v, b_k, generator=g)
    U = torch.randn(N, a_v * b_v, P, generator=g)
    Vb = torch.randn(N, a_k * b_k, P, generator=g)
    G = og.reference_sketch(N, b_v * b_k, R)
    An, Bn, st = ops.gdn3_compact(*(t.to(DEV) for t in (A, Bk, U, Vb, G)), slow_decay=0.9,
                                  compact_mode="sketch")
    Ar, Br, err = og.compact(A.double(), Bk.double(), U.double(), Vb.double(), 0.9, G, mode="sketch")
    assert rel_l2(An, Ar) <= 1e-5
    assert rel_l2(Bn, Br) <= 1e-5
    assert err.item() == 0.0
    assert (st[:, 0] - st[:, 1]).abs().max().item() == 0.0   # error 0: kept = energy
    with pytest.raises(Exception):   # a width-(R+4) sketch is the svd mode's, not this one's
        ops.gdn3_compact(*(t.to(DEV) for t in (A, Bk, U, Vb)), og.reference_sketch(N, b_v * b_k, R + 4).to(DEV),
                         compact_mode="sketch")


SKETCH_CASES = [
    # (B, T, H, M, D, factors, P, Kc, io, gate, per_lane)
    (1, 80, 2, 2, 128, (16, 16, 8, 8), 16, 16, torch.float32, "channel", False),
    (2, 64, 1, 2, 128, (16, 16, 8, 8), 16, 32, torch.bfloat16, "lane", False),
    (1, 96, 1, 2, 64, (8, 8, 8, 8), 32, 32, torch.float32, "lane", True),
]


@pytest.mark.parametrize("case", SKETCH_CASES, ids=[f"c{i}" for i in range(len(SKETCH_CASES))])
def test_sketch_forward_matches_oracle(gpu_lib, case):
    from gdnx_amd import gdn3
    B, T, H, M, D, factors, P, Kc, io, gate, per_lane = case
    print(f"case: sketch fwd {case}", flush=True)
    xs, _ = _inputs(B, T, H, M, D, seed=51, io=io, gate=gate, per_lane=per_lane)
    N = B * H * M
    G = og.reference_sketch(N, factors[2] * factors[3], 4)
    with torch.no_grad():
        y, (A, Bk, U, Vb), err = gdn3.gdn3_recurrent_state(*(t.to(DEV) for t in xs), R=4, P=P, factors=factors,
                                                           compact_every=Kc, sketch=G.to(DEV), return_state=True,
                                                           compact_mode="sketch_noqr")
    torch.cuda.synchronize()
    yr, (Ar, Br, Ur, Vr), err_r = _oracle(xs, M, P, Kc, factors, G, mode="sketch")
    tol = 1e-2 if io == torch.bfloat16 else 1e-4
    assert rel_l2(y, yr) <= tol
    assert rel_l2(U, Ur) <= tol and rel_l2(Vb, Vr) <= tol
    state_tol = 1e-2 if io == torch.bfloat16 else 1e-3
    assert rel_l2(A, Ar) <= state_tol and rel_l2(Bk, Br) <= state_tol
    assert err.item() == 0.0 and err_r.item() == 0.0


def test_sketch_default_sketch_is_the_reference_draw(gpu_lib):
    """Without an explicit sketch the sketch mode draws randn(N, b_v*b_k, R)
    seeded 1234 on the CPU (the reference's _gdn3_sketch_matrix shape in this
    mode, gdn3/gdn3_upgrade.py:580)."""
    from gdnx_amd import gdn3
    print("case: sketch default draw", flush=True)
    xs, _ = _inputs(1, 48, 1, 2, 128, seed=52, io=torch.float32, gate="lane", per_lane=False)
    with torch.no_grad():
        y = gdn3.gdn3_recurrent_state(*(t.to(DEV) for t in xs), compact_mode="sketch")
    yr, _, _ = _oracle(xs, 2, 16, 16, (16, 16, 8, 8), og.reference_sketch(2, 64, 4), mode="sketch")
    assert rel_l2(y, yr) <= 1e-4


def test_sketch_backward_matches_oracle(gpu_lib):
    from gdnx_amd import gdn3
    print("case: sketch bwd", flush=True)
    B, T, H, M, D = 1, 64, 1, 2, 128
    factors = (16, 16, 8, 8)
    xs, dy = _inputs(B, T, H, M, D, seed=53, io=torch.float32, gate="channel", per_lane=False)
    G = og.reference_sketch(B * H * M, 64, 4)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y = gdn3.gdn3_recurrent_state(*leaves, factors=factors, compact_every=16, sketch=G.to(DEV),
                                  compact_mode="sketch")
    grads = torch.autograd.grad(y, leaves, dy.to(DEV))
    torch.cuda.synchronize()
    yr, gref = _oracle(xs, M, 16, 16, factors, G, mode="sketch", dy=dy)
    assert rel_l2(y, yr) <= 1e-4
    for name, a, r in zip(("dq", "dk", "dv", "db_gates", "dw_gates", "ddecay"), grads, gref):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-4, name


def test_sketch_decode_after_prefill_matches_oracle(gpu_lib):
    from gdnx_amd import gdn3
    print("case: sketch decode", flush=True)
    B, H, M, D, P, Kc, T1, steps = 2, 1, 2, 128, 16, 16, 21, 40
    factors = (16, 16, 8, 8)
    T = T1 + steps
    xs, _ = _inputs(B, T, H, M, D, seed=54, io=torch.float32, gate="lane", per_lane=False)
    G = og.reference_sketch(B * H * M, 64, 4)
    yr, (Ar, Br, Ur, Vr), _ = _oracle(xs, M, P, Kc, factors, G, mode="sketch")
    xd = [t.to(DEV) for t in xs]
    with torch.no_grad():
        y0, state, _ = gdn3.gdn3_recurrent_state(*(t[:, :T1] for t in xd), P=P, factors=factors, compact_every=Kc,
                                                 sketch=G.to(DEV), return_state=True, compact_mode="sketch")
        ys = [y0]
        for t in range(T1, T):
            ys.append(gdn3.gdn3_decode_step(*(u[:, t] for u in xd), state, t, P=P, factors=factors,
                                            compact_every=Kc, sketch=G.to(DEV), compact_mode="sketch").unsqueeze(1))
    torch.cuda.synchronize()
    assert rel_l2(torch.cat(ys, 1), yr) <= 1e-4
    A, Bk, U, Vb = state
    assert rel_l2(U, Ur) <= 1e-4 and rel_l2(A, Ar) <= 1e-3 and rel_l2(Bk, Br) <= 1e-3


# ---------------------------------------------------------------------------
# long horizons (svd mode)
# ---------------------------------------------------------------------------
LONG_CASES = [
    # (T, M, D, factors, Kc, gate)
    (1024, 1, 128, (16, 16, 8, 8), 16, "channel"),
    (1024, 2, 64, (8, 8, 8, 8), 16, "lane"),
    (512, 2, 128, (16, 16, 8, 8), 16, "channel"),
]


@pytest.mark.parametrize("case", LONG_CASES, ids=[f"T{c[0]}M{c[1]}D{c[2]}" for c in LONG_CASES])
def test_long_horizon_forward_backward(gpu_lib, case):
    from gdnx_amd import gdn3
    T, M, D, factors, Kc, gate = case
    print(f"case: long horizon {case} ({T // Kc} compactions)", flush=True)
    xs, dy = _inputs(1, T, 1, M, D, seed=55, io=torch.float32, gate=gate, per_lane=False)
    G = og.reference_sketch(M, factors[2] * factors[3], 8)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y = gdn3.gdn3_recurrent_state(*leaves, factors=factors, compact_every=Kc, sketch=G.to(DEV))
    grads = torch.autograd.grad(y, leaves, dy.to(DEV))
    torch.cuda.synchronize()
    yr, gref = _oracle(xs, M, 16, Kc, factors, G, dy=dy)
    err = rel_l2(y, yr)
    print(f"  y rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-4
    for name, a, r in zip(("dq", "dk", "dv", "db_gates", "dw_gates", "ddecay"), grads, gref):
        err = rel_l2(a, r)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-4, name


# ---------------------------------------------------------------------------
# the layer-method adapter
# ---------------------------------------------------------------------------
class _Layer:
    """The attributes GDN3LinearAttn._gdn3_recurrent_state reads
    (gdn3/gdn3_upgrade.py:403-531)."""

    def __init__(self, mode="svd", P=16):
        self.R, self.P, self.a_v, self.a_k, self.b_v, self.b_k = 4, P, 16, 16, 8, 8
        self.slow_decay, self.compact_mode = 0.97, mode


@pytest.mark.parametrize("mode", ["svd", "sketch"])
@pytest.mark.parametrize("sync", ["0", "1"])
def test_adapter_method_matches_oracle(gpu_lib, monkeypatch, mode, sync):
    from gdnx_amd import adapter
    print(f"case: adapter mode={mode} sync={sync}", flush=True)
    monkeypatch.setenv("GDN3_SYNC_COMP_ERR", sync)
    adapter.install(_Layer)
    layer = _Layer(mode)
    B, T, H, M, D = 1, 64, 2, 2, 128
    xs, _ = _inputs(B, T, H, M, D, seed=56, io=torch.float32, gate="channel", per_lane=False)
    q, k, v, bg, wg, dec = (t.to(DEV) for t in xs)
    qe, ke, ve = (t.unsqueeze(3).expand(B, T, H, M, D) for t in (q, k, v))   # as forward builds them
    y = layer._gdn3_recurrent_state(qe, ke, ve, bg, wg, dec)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and y.shape == (B, T, H, M, D)
    G = og.reference_sketch(B * H * M, 64, 4 if mode == "sketch" else 8)
    yr, _, err_r = _oracle(xs, M, 16, 16, (16, 16, 8, 8), G, mode=mode)
    assert rel_l2(y, yr) <= 1e-4
    err = layer._last_comp_err
    if sync == "1":
        assert isinstance(err, float)
    else:
        assert isinstance(err, torch.Tensor) and not err.requires_grad
        err = err.item()
    assert abs(err - err_r.item()) <= 1e-4 * max(1.0, abs(err_r.item()))


def test_adapter_method_is_differentiable(gpu_lib):
    from gdnx_amd import adapter
    print("case: adapter gradients", flush=True)
    layer = types.SimpleNamespace(R=4, P=16, a_v=16, a_k=16, b_v=8, b_k=8, slow_decay=0.97)
    B, T, H, M, D = 1, 48, 1, 2, 128
    xs, dy = _inputs(B, T, H, M, D, seed=57, io=torch.float32, gate="lane", per_lane=True)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    y = adapter.gdn3_recurrent_state_method(layer, *leaves)
    grads = torch.autograd.grad(y, leaves, dy.to(DEV))
    yr, gref = _oracle(xs, M, 16, 16, (16, 16, 8, 8), og.reference_sketch(B * H * M, 64, 8), dy=dy)
    assert rel_l2(y, yr) <= 1e-4
    for a, r in zip(grads, gref):
        assert rel_l2(a, r) <= 1e-4


# ---------------------------------------------------------------------------
# non-finite status
# ---------------------------------------------------------------------------
def test_nonfinite_status(gpu_lib):
    from gdnx_amd import _lib, gdn3, ops
    print("case: non-finite status", flush=True)
    lib = _lib.load()
    x = torch.ones(1000, device=DEV)
    assert lib.gdnx_check_finite(_lib.ptr(x), x.numel(), _lib.DTYPE_F32, _lib.stream_of(x)) == 0
    x[777] = float("inf")
    assert lib.gdnx_check_finite(_lib.ptr(x), x.numel(), _lib.DTYPE_F32, _lib.stream_of(x)) == _lib.ERR_NONFINITE
    xd = torch.zeros(300, dtype=torch.float64, device=DEV)
    xd[5] = float("nan")
    assert lib.gdnx_check_finite(_lib.ptr(xd), 300, _lib.DTYPE_F64, _lib.stream_of(xd)) == _lib.ERR_NONFINITE
    xb = torch.zeros(64, dtype=torch.bfloat16, device=DEV)
    assert lib.gdnx_check_finite(_lib.ptr(xb), 64, _lib.DTYPE_BF16, _lib.stream_of(xb)) == 0

    xs, _ = _inputs(1, 32, 1, 2, 128, seed=58, io=torch.float32, gate="lane", per_lane=False)
    xd6 = [t.to(DEV) for t in xs]
    bad = [t.clone() for t in xd6]
    bad[2][0, 5, 0, 3] = float("nan")
    dense = inputs.dense_inputs(1, 64, 1, 128, M=2, seed=2, taus=list(inputs.TAUS[:2]), decay="tau")
    dq, dk, dv = (dense[n].to(DEV) for n in ("q", "k", "v"))
    dbeta, dg = dense["beta"].to(DEV), dense["g"].to(DEV)
    dv_bad = dv.clone()
    dv_bad[0, 9, 0, 1] = float("inf")
    with torch.no_grad():
        prev = _lib.set_check_finite(True)
        try:
            gdn3.gdn3_recurrent_state(*xd6)                       # finite: no error
            with pytest.raises(_lib.GdnxNonFinite):
                gdn3.gdn3_recurrent_state(*bad)
            ops.delta_chunk_fwd(dq, dk, dv, dbeta, dbeta, dg)
            with pytest.raises(_lib.GdnxNonFinite):
                ops.delta_chunk_fwd(dq, dk, dv_bad, dbeta, dbeta, dg)
        finally:
            _lib.set_check_finite(prev)
        gdn3.gdn3_recurrent_state(*bad)                           # checking off: no status
    torch.cuda.synchronize()

"""Carried state on the GPU against the CPU oracle: continuation and decode.

The reference has no decode path and no carried state (its recurrences start
from zero at slot 0, gdn3/_reference_recurrence.py:52-56); what these tests
pin is that splitting a sequence changes nothing.  The GDN3 Kronecker-residual
state (A, B, U, Vb, and the token count that fixes the slot and the
compaction schedule) continued over several calls, or advanced one token at a
time by the decode step after a chunked prefill, must give the oracle's
single whole-sequence run (oracle/gdn3.py, golden-pinned in
tests/test_oracle_gdn3.py; sign_mode 'canonical', the compaction's sign
convention on the GPU).  The KMD-2 per-channel decode step after a prefill
must give the oracle's whole-sequence scan (oracle/delta.py kmd2_scan).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import delta as od
from oracle import gdn3 as og
from oracle import inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _g3_inputs(B, T, H, M, D, seed, io, gate, per_lane):
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
    return q.to(io), k.to(io), v.to(io), bg, wg, dec.clamp(max=1.0)


def _oracle_run(x, M, factors, P, Kc, G):
    q, k, v, bg, wg, dec = x
    D = q.shape[-1]

    def lanes(t):
        return t.double() if t.dim() == 5 else t.double().unsqueeze(3).expand(*t.shape[:3], M, D)

    def gates(t):
        return t.double() if t.dim() == 5 else t.double().unsqueeze(-1).expand(*t.shape, D)
    return og.gdn3_recurrence(lanes(q), lanes(k), lanes(v), gates(bg), gates(wg), dec.double(), R=4, P=P,
                              factors=factors, compact_every=Kc, sketch=G, sign_mode="canonical",
                              return_state=True)


def _seg(x, t0, t1):
    return [t[:, t0:t1] for t in x]


G3_CASES = [
    # (D, factors, P, Kc, io, gate, per_lane)
    (128, (16, 16, 8, 8), 16, 32, torch.float32, "lane", False),
    (128, (16, 16, 8, 8), 16, 16, torch.bfloat16, "channel", False),
    (64, (8, 8, 8, 8), 32, 32, torch.float32, "channel", True),
    (64, (8, 8, 8, 8), 16, 48, torch.bfloat16, "lane", True),
    (128, (16, 16, 8, 8), 64, 64, torch.float32, "lane", False),
    (128, (16, 16, 8, 8), 32, 32, torch.bfloat16, "lane", True),
    (64, (8, 8, 8, 8), 64, 64, torch.bfloat16, "channel", False),
]
G3_IDS = [f"d{c[0]}p{c[2]}k{c[3]}{'bf' if c[4] == torch.bfloat16 else 'f'}{c[5][0]}{'L' if c[6] else ''}"
          for c in G3_CASES]


@pytest.mark.parametrize("case", G3_CASES, ids=G3_IDS)
@pytest.mark.parametrize("splits", [(37,), (64,), (5, 40, 77, 96)], ids=["mid", "boundary", "many"])
def test_gdn3_split_run_equals_whole_run(gpu_lib, case, splits):
    """Continuation calls from the returned state (t0 = tokens so far) give
    the whole run: outputs, the final state and the compaction error."""
    from gdnx_amd import gdn3
    D, factors, P, Kc, io, gate, per_lane = case
    print(f"case: gdn3 split {case} splits={splits}", flush=True)
    B, T, H, M = 1, 100, 2, 2
    N = B * H * M
    a_v, a_k, b_v, b_k = factors
    x = _g3_inputs(B, T, H, M, D, seed=31, io=io, gate=gate, per_lane=per_lane)
    G = og.reference_sketch(N, b_v * b_k, min(8, a_v * a_k, b_v * b_k))
    yr, (Ar, Br, Ur, Vr), err_r = _oracle_run(x, M, factors, P, Kc, G)
    bounds = (0,) + tuple(splits) + (T,)
    ys, state, err = [], None, 0.0
    with torch.no_grad():
        for t0, t1 in zip(bounds[:-1], bounds[1:]):
            y, state, e = gdn3.gdn3_recurrent_state(*(t.to(DEV) for t in _seg(x, t0, t1)), R=4, P=P,
                                                    factors=factors, compact_every=Kc, sketch=G.to(DEV),
                                                    return_state=True, state0=state, t0=t0)
            ys.append(y)
            err += e.item()
    torch.cuda.synchronize()
    tol = 1e-2 if io == torch.bfloat16 else 1e-4
    y = torch.cat(ys, 1)
    assert y.shape == (B, T, H, M, D)
    assert rel_l2(y, yr) <= tol
    A, Bk, U, Vb = state
    # the net writes U = alpha (u - S h) are differences of nearly equal
    # terms, so their fp32 rounding is relatively larger than y's (about 1e-4
    # over these 100 tokens for the whole run as for the split one, with or
    # without compactions); the compacted factors: see test_gpu_gdn3
    # (singular vectors amplify rounding)
    state_tol = 1e-2 if io == torch.bfloat16 else 1e-3
    assert rel_l2(U, Ur) <= state_tol
    assert rel_l2(Vb, Vr) <= tol
    assert rel_l2(A, Ar) <= state_tol
    assert rel_l2(Bk, Br) <= state_tol
    assert abs(err - err_r.item()) <= tol * max(1.0, abs(err_r.item()))


@pytest.mark.parametrize("case", G3_CASES, ids=G3_IDS)
def test_gdn3_decode_after_prefill_matches_oracle(gpu_lib, case):
    """A 37-token chunked prefill, then 2P + 9 one-token decode steps (each
    crossing slot wrap-arounds and at least one compaction), against the
    oracle's whole run."""
    from gdnx_amd import gdn3
    D, factors, P, Kc, io, gate, per_lane = case
    print(f"case: gdn3 decode {case}", flush=True)
    B, H, M, T1 = 2, 2, 2, 37
    steps = 2 * P + 9
    T = T1 + steps
    N = B * H * M
    a_v, a_k, b_v, b_k = factors
    x = _g3_inputs(B, T, H, M, D, seed=32, io=io, gate=gate, per_lane=per_lane)
    G = og.reference_sketch(N, b_v * b_k, min(8, a_v * a_k, b_v * b_k))
    yr, (Ar, Br, Ur, Vr), _ = _oracle_run(x, M, factors, P, Kc, G)
    xd = [t.to(DEV) for t in x]
    Gd = G.to(DEV)
    with torch.no_grad():
        y0, state, _ = gdn3.gdn3_recurrent_state(*_seg(xd, 0, T1), R=4, P=P, factors=factors, compact_every=Kc,
                                                 sketch=Gd, return_state=True)
        ys = [y0]
        for t in range(T1, T):
            yt = gdn3.gdn3_decode_step(*(u[:, t] for u in xd), state, t, R=4, P=P, factors=factors,
                                       compact_every=Kc, sketch=Gd)
            ys.append(yt.unsqueeze(1))
    torch.cuda.synchronize()
    tol = 1e-2 if io == torch.bfloat16 else 1e-4
    y = torch.cat(ys, 1)
    assert rel_l2(y[:, :T1], yr[:, :T1]) <= tol
    assert rel_l2(y[:, T1:], yr[:, T1:]) <= tol
    A, Bk, U, Vb = state
    assert rel_l2(U, Ur) <= tol
    assert rel_l2(Vb, Vr) <= tol
    state_tol = 1e-2 if io == torch.bfloat16 else 1e-3
    assert rel_l2(A, Ar) <= state_tol
    assert rel_l2(Bk, Br) <= state_tol


def test_gdn3_decode_cache_slots(gpu_lib):
    """DecodeStateCache (gdn3 kind): sequences prefilled separately to
    different lengths, then stepped together with an empty row; each equals
    its own oracle run with its slot's sketch rows."""
    from gdnx_amd.decode_cache import DecodeStateCache
    print("case: gdn3 decode cache", flush=True)
    H, M, D, P, Kc, n_slots = 2, 2, 128, 16, 16, 4
    factors = (16, 16, 8, 8)
    cache = DecodeStateCache(n_slots, H, M, D, DEV, kind="gdn3", P=P, compact_every=Kc)
    sa, sb = cache.alloc(2)
    lens = {sa: 21, sb: 40}
    steps = 20
    seqs = {s: _g3_inputs(1, lens[s] + steps, H, M, D, seed=40 + s, io=torch.float32, gate="lane",
                          per_lane=False) for s in (sa, sb)}
    ys = {}
    with torch.no_grad():
        for s in (sa, sb):
            ys[s] = [cache.prefill([s], *(t[:, :lens[s]].to(DEV) for t in seqs[s]))]
        for j in range(steps):
            rows = [sb, -1, sa]
            xs = [torch.cat([seqs[s][i][:, lens[s] + j] if s >= 0 else torch.zeros_like(seqs[sa][i][:, 0])
                             for s in rows]).to(DEV) for i in range(6)]
            y = cache.step(rows, *xs)
            assert (y[1] == 0).all()
            ys[sb].append(y[0:1].unsqueeze(1))
            ys[sa].append(y[2:3].unsqueeze(1))
    torch.cuda.synchronize()
    HM = H * M
    for s in (sa, sb):
        G = cache.sketch.view(n_slots, HM, *cache.sketch.shape[1:])[s].cpu()
        yr, (Ar, Br, Ur, Vr), _ = _oracle_run(seqs[s], M, factors, P, Kc, G)
        assert rel_l2(torch.cat(ys[s], 1), yr) <= 1e-4, s
        A, Bk, U, Vb = cache.state(s)
        assert rel_l2(U.reshape(HM, D, P), Ur) <= 1e-4
        assert rel_l2(A.reshape(HM, 4, 16, 16), Ar) <= 1e-3
        assert cache.pos[s] == lens[s] + steps


def test_gdn3_decode_config4_width(gpu_lib):
    """The GDN3 step at config-4 width: 256 sequences x 16 heads x 16 chains
    (4 lanes x 4 decay timescales), bf16 IO, fp32 Kronecker-residual state
    (5.6 GB).  Two steps, the second closing a compaction interval on every
    row; a 2-sequence x 2-head subset is checked against the oracle."""
    from gdnx_amd import gdn3
    print("case: gdn3 decode config4 width", flush=True)
    NS, H, M, D, P = 256, 16, 16, 128, 16
    factors = (16, 16, 8, 8)
    gen = torch.Generator().manual_seed(1004)
    N = NS * H * M
    # Kronecker terms of decreasing weight, so the kept rank-4 part is well
    # separated from the residual's directions (a small singular-value gap
    # would amplify fp32 rounding in the refitted factors)
    A = torch.randn(NS, H, M, 4, 16, 16, generator=gen) * torch.tensor([0.4, 0.2, 0.1, 0.05]).view(4, 1, 1)
    Bk = torch.randn(NS, H, M, 4, 8, 8, generator=gen) * 0.5
    U = torch.randn(NS, H, M, D, P, generator=gen) * 0.02
    Vb = F.normalize(torch.randn(NS, H, M, D, P, generator=gen), dim=-2)
    state = tuple(t.to(DEV) for t in (A, Bk, U, Vb))
    sub = tuple(t[:2, :2].reshape(2 * 2 * M, *t.shape[3:]).double() for t in (A, Bk, U, Vb))
    G = og.reference_sketch(N, 64, 8)
    Gd = G.to(DEV)
    Gsub = G.view(NS, H, M, 64, 8)[:2, :2].reshape(2 * 2 * M, 64, 8)
    ys, xs = [], []
    for step in range(2):
        q = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
        k = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
        v = torch.randn(NS, H, D, generator=gen).bfloat16()
        bg = torch.sigmoid(torch.randn(NS, H, M, generator=gen))
        wg = torch.sigmoid(torch.randn(NS, H, M, generator=gen))
        base = torch.log1p(-torch.tensor(inputs.TAUS)).repeat(4)
        dec = torch.exp(base.view(1, 1, M) + 0.01 * torch.randn(NS, H, M, generator=gen)).clamp(max=1.0)
        xs.append((q, k, v, bg, wg, dec))
        pos = 30 + step   # the second step's token closes the interval (31 + 1) % 16 == 0
        with torch.no_grad():
            ys.append(gdn3.gdn3_decode_step(*(t.to(DEV) for t in (q, k, v, bg, wg, dec)), state, pos, R=4, P=P,
                                            factors=factors, compact_every=P, sketch=Gd))
    torch.cuda.synchronize()
    assert all(torch.isfinite(y.float()).all() for y in ys)
    # oracle: the subset's chains from the same state, global tokens 30, 31
    xo = [torch.stack([x[i][:2, :2] for x in xs], 1) for i in range(6)]   # [2, 2(steps), 2, ...]
    q, k, v = (t.double().unsqueeze(3).expand(2, 2, 2, M, D) for t in xo[:3])
    bg, wg = (t.double().unsqueeze(-1).expand(2, 2, 2, M, D) for t in xo[3:5])
    yr, (Ar, Br, Ur, Vr), _ = og.gdn3_recurrence(q, k, v, bg, wg, xo[5].double(), R=4, P=P, factors=factors,
                                                 compact_every=P, sketch=Gsub, sign_mode="canonical",
                                                 return_state=True, state0=sub, t0=30)
    y = torch.stack([t[:2, :2] for t in ys], 1)
    assert rel_l2(y, yr) <= 1e-2
    assert rel_l2(state[2][:2, :2].reshape(2 * 2 * M, D, P), Ur) <= 1e-2
    assert rel_l2(state[0][:2, :2].reshape(2 * 2 * M, 4, 16, 16), Ar) <= 1e-2


def test_gdn3_decode_negative_position_is_an_empty_row(gpu_lib):
    """A row whose device-side position is negative has no residual slot: the
    step writes y = 0 for it and leaves its state bitwise unchanged, and no
    compaction runs on it (for pos = -1, (pos + 1) % K_c would be 0).  The
    other row, whose token closes a compaction interval, still advances."""
    from gdnx_amd import gdn3
    print("case: gdn3 decode pos = -1", flush=True)
    NS, H, M, D, P = 2, 1, 2, 64, 16
    gen = torch.Generator().manual_seed(77)
    N = NS * H * M
    state = tuple(t.to(DEV) for t in (torch.randn(N, 4, 8, 8, generator=gen) * 0.3,
                                      torch.randn(N, 4, 8, 8, generator=gen) * 0.3,
                                      torch.randn(N, D, P, generator=gen) * 0.05,
                                      F.normalize(torch.randn(N, D, P, generator=gen), dim=1)))
    before = tuple(t.clone() for t in state)
    q, k, v = (F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).to(DEV) for _ in range(3))
    bg = torch.sigmoid(torch.randn(NS, H, M, generator=gen)).to(DEV)
    wg = torch.sigmoid(torch.randn(NS, H, M, generator=gen)).to(DEV)
    dec = torch.full((NS, H, M), 0.97, device=DEV)
    pos = torch.tensor([P - 1, -1], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        y = gdn3.gdn3_decode_step(q, k, v, bg, wg, dec, state, pos, R=4, P=P, factors=(8, 8, 8, 8),
                                  compact_every=P)
    torch.cuda.synchronize()
    assert torch.equal(y[1], torch.zeros_like(y[1]))
    for t, t0 in zip(state, before):
        assert torch.equal(t[H * M:], t0[H * M:])      # row 1's chains untouched
        assert not torch.equal(t[:H * M], t0[:H * M])  # row 0's chains advanced


KMD2_CASES = [(128, 128, 1, torch.float32), (64, 64, 4, torch.float32), (8, 64, 4, torch.float32),
              (128, 128, 2, torch.bfloat16)]


def _kmd2_inputs(B, T, H, r_out, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, r_out, dk, generator=g)
    k = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1)
    v = torch.randn(B, T, H, dv, generator=g)
    gd = torch.exp(-torch.rand(B, T, H, dk, generator=g) * 0.2)       # per-channel decay in (0.82, 1]
    be = torch.sigmoid(torch.randn(B, T, H, generator=g))
    bw = torch.sigmoid(torch.randn(B, T, H, generator=g))
    mix = torch.softmax(torch.randn(H, r_out, generator=g), -1)
    return q, k, v, gd, be, bw, mix


@pytest.mark.parametrize("dk,dv,r_out,io", KMD2_CASES, ids=[f"{a}x{b}r{c}{str(d)[6:]}" for a, b, c, d in KMD2_CASES])
def test_kmd2_decode_after_prefill_matches_oracle(gpu_lib, dk, dv, r_out, io):
    """KMD-2 per-channel decay: scan_with_state over a prefill, then 12
    decode steps, against the oracle's whole-sequence scan and final state."""
    from gdnx_amd import kmd2
    print(f"case: kmd2 decode dk={dk} dv={dv} r_out={r_out} {io}", flush=True)
    B, H, T1, steps = 2, 3, 19, 12
    T = T1 + steps
    q, k, v, gd, be, bw, mix = _kmd2_inputs(B, T, H, r_out, dk, dv, seed=51)
    q, k, v = q.to(io), k.to(io), v.to(io)
    yr, Sr = od.kmd2_scan(q.double(), k.double(), v.double(), gd, be, bw, mix, return_state=True)
    d = [t.to(DEV) for t in (q, k, v, gd, be, bw, mix)]
    with torch.no_grad():
        y0, S = kmd2.scan_with_state(*(t[:, :T1] for t in d[:6]), out_mix=d[6])
        ys = [y0.float()]
        for t in range(T1, T):
            ys.append(kmd2.decode_step(*(u[:, t] for u in d[:6]), S, out_mix=d[6]).float().unsqueeze(1))
    torch.cuda.synchronize()
    tol = 1e-2 if io == torch.bfloat16 else 1e-4
    y = torch.cat(ys, 1)
    assert S.shape == (B, H, dk, dv)
    assert rel_l2(y[:, :T1], yr[:, :T1]) <= tol
    assert rel_l2(y[:, T1:], yr[:, T1:]) <= tol
    assert rel_l2(S, Sr) <= tol


def test_kmd2_decode_cache_slots(gpu_lib):
    """DecodeStateCache (chan kind): two sequences prefilled to different
    lengths, stepped together with an empty row, against the oracle."""
    from gdnx_amd.decode_cache import DecodeStateCache
    print("case: kmd2 decode cache", flush=True)
    H, D, steps = 2, 128, 9
    cache = DecodeStateCache(3, H, 1, D, DEV, kind="chan")
    sa, sb = cache.alloc(2)
    lens = {sa: 7, sb: 33}
    seqs = {s: _kmd2_inputs(1, lens[s] + steps, H, 1, D, D, seed=60 + s) for s in (sa, sb)}
    ys = {}
    with torch.no_grad():
        for s in (sa, sb):
            q, k, v, gd, be, bw, _ = (t[:, :lens[s]].to(DEV) if t.dim() > 2 else t for t in seqs[s])
            ys[s] = [cache.prefill([s], q[:, :, :, 0], k, v, be, bw, torch.log(gd))]
        for j in range(steps):
            rows = [sa, -1, sb]

            def row(s, i):
                t = seqs[s][i][:, lens[s] + j]
                return t[:, :, 0] if i == 0 else t
            q, k, v, gd, be, bw = (torch.cat([row(s, i) if s >= 0 else torch.zeros_like(row(sa, i)) for s in rows])
                                   for i in range(6))
            y = cache.step(rows, q.to(DEV), k.to(DEV), v.to(DEV), be.unsqueeze(-1).to(DEV), bw.unsqueeze(-1).to(DEV),
                           torch.log(gd).unsqueeze(2).to(DEV))
            assert (y[1] == 0).all()
            ys[sa].append(y[0:1, :, 0].unsqueeze(1))
            ys[sb].append(y[2:3, :, 0].unsqueeze(1))
    torch.cuda.synchronize()
    for s in (sa, sb):
        q, k, v, gd, be, bw, mix = seqs[s]
        yr, Sr = od.kmd2_scan(q, k, v, gd, be, bw, None, return_state=True)
        assert rel_l2(torch.cat(ys[s], 1), yr) <= 1e-4, s
        assert rel_l2(cache.state(s)[:, 0], Sr[0]) <= 1e-4


def test_decode_config4_16_consecutive_steps(gpu_lib):
    """Config 4 (dense state): 16 consecutive one-token steps at full width
    (256 x 16 heads x 16 chains, 4.3 GB of fp32 state, bf16 IO); a 2x2-head
    subset is carried by the oracle through all 16 steps."""
    from gdnx_amd import ops
    from oracle import delta
    print("case: decode config4 16 steps", flush=True)
    NS, H, M, NT, D, steps = 256, 16, 4, 4, 128, 16
    state = torch.randn(NS, H, M * NT, D, D, device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(1004)) * 0.02
    ref = state[:2, :2].double().cpu()
    gen = torch.Generator().manual_seed(1006)
    base = torch.log1p(-torch.tensor(inputs.TAUS)).repeat(M)
    for t in range(steps):
        q = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
        k = F.normalize(torch.randn(NS, H, D, generator=gen), dim=-1).bfloat16()
        v = torch.randn(NS, H, D, generator=gen).bfloat16()
        beta = torch.sigmoid(torch.randn(NS, H, M, generator=gen))
        a = delta.gdn3_dense_coeffs(k.double(), beta.double()).float().repeat_interleave(NT, dim=-1).contiguous()
        lg = (base.view(1, 1, M * NT) + 0.01 * torch.randn(NS, H, M * NT, generator=gen)).contiguous()
        y = ops.delta_decode_step(q.to(DEV), k.to(DEV), v.to(DEV), a.to(DEV), a.to(DEV), lg.to(DEV), state)
        yo, ref = delta.lane_delta(q[:2, None, :2], k[:2, None, :2], v[:2, None, :2], a[:2, None, :2],
                                   a[:2, None, :2], lg[:2, None, :2], state0=ref)
        torch.cuda.synchronize()
        assert torch.isfinite(y.float()).all(), t
        assert rel_l2(y[:2, :2], yo[:, 0]) <= 1e-2, t
    assert rel_l2(state[:2, :2], ref) <= 1e-5

"""Delta rule with a decay per key channel (gdnx_delta_chan_fwd / _bwd, the
general KMD-2 decay of gdn3/kmd2_native.py:163-164) on the GPU, against the
float64 CPU oracle delta.delta_rule_chunked_chan (pinned against the token
loop in tests/test_oracle_delta.py) and torch autograd through it.  The
kernels compute in float32; the bar is rel-L2 <= 1e-4 on outputs, final
state and every gradient."""
import pytest
import torch
import torch.nn.functional as F

from oracle import delta

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _inputs(B, T, H, D, seed, strong=False, with_state=False):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    be = torch.sigmoid(torch.randn(B, T, H, generator=g))
    bw = torch.sigmoid(torch.randn(B, T, H, generator=g))
    # per-channel log decay: slow channels near 0, a few fast ones
    lg = -torch.rand(B, T, H, D, generator=g) * torch.logspace(-3, 0, D).view(1, 1, 1, D)
    if strong:
        # decays down to e^-40 per token, and values outside [-60, 0] that
        # the kernels clamp (their gradient is zero)
        lg = lg * 40.0
        lg[:, 3, :, :4] = 0.5
        lg[:, 5, :, 4:8] = -75.0
    s0 = torch.randn(B, H, D, D, generator=g) * 0.1 if with_state else None
    return q, k, v, be, bw, lg, s0


def _flat(x):
    """[B,T,H,...] -> [B*H, T, ...]"""
    return x.transpose(1, 2).reshape(x.shape[0] * x.shape[2], x.shape[1], *x.shape[3:])


def _oracle(q, k, v, be, bw, lg, s0):
    B, T, H, D = q.shape
    st = None if s0 is None else s0.reshape(B * H, D, D)
    w = (bw.unsqueeze(-1) * v)
    y, s = delta.delta_rule_chunked_chan(_flat(q), _flat(k), _flat(be), _flat(w), _flat(lg), chunk=16,
                                         state0=st)
    return y.reshape(B, H, T, D).transpose(1, 2), s.reshape(B, H, D, D)


@pytest.mark.parametrize("D,T,strong,with_state", [(128, 100, False, True), (64, 77, True, False),
                                                   (128, 64, True, True), (64, 5, False, False)])
def test_chan_forward_matches_oracle(gpu_lib, D, T, strong, with_state):
    from gdnx_amd import ops
    print(f"case: chan fwd D={D} T={T} strong={strong} state={with_state}", flush=True)
    x = _inputs(2, T, 3, D, seed=D + T, strong=strong, with_state=with_state)
    yr, sr = _oracle(*(t.double() if t is not None else None for t in x))
    dev = [t.to(DEV) if t is not None else None for t in x]
    y, s, _ = ops.delta_chan_fwd(*dev)
    torch.cuda.synchronize()
    assert rel_l2(y, yr) <= 1e-4
    assert rel_l2(s, sr) <= 1e-4
    # the training forward (state stash) gives the same outputs
    y2, s2, cs = ops.delta_chan_fwd(*dev, save_states=True)
    torch.cuda.synchronize()
    assert cs is not None
    assert torch.equal(y2, y) and torch.equal(s2, s)


@pytest.mark.parametrize("D,T,strong,with_state", [(128, 100, False, True), (64, 77, True, True),
                                                   (64, 48, False, False)])
def test_chan_gradients_match_oracle(gpu_lib, D, T, strong, with_state):
    from gdnx_amd import ops
    print(f"case: chan grads D={D} T={T} strong={strong} state={with_state}", flush=True)
    B, H = 2, 2
    x = _inputs(B, T, H, D, seed=3 * D + T, strong=strong, with_state=with_state)
    gen = torch.Generator().manual_seed(7)
    dy = torch.randn(B, T, H, D, generator=gen)
    dS = torch.randn(B, H, D, D, generator=gen) * 0.1
    ref = [t.double().requires_grad_(True) if t is not None else None for t in x]
    yr, sr = _oracle(*ref)
    leaves_r = [t for t in ref if t is not None]
    g_ref = torch.autograd.grad((yr, sr), leaves_r, (dy.double(), dS.double()))
    dev = [t.to(DEV).requires_grad_(True) if t is not None else None for t in x]
    y, s = ops.delta_rule_chan(*dev)
    leaves = [t for t in dev if t is not None]
    grads = torch.autograd.grad((y, s), leaves, (dy.to(DEV), dS.to(DEV)))
    torch.cuda.synchronize()
    assert rel_l2(y, yr) <= 1e-4
    assert rel_l2(s, sr) <= 1e-4
    names = ("dq", "dk", "dv", "dbeta_e", "dbeta_w", "dlog_g", "dstate0")
    for name, a, b in zip(names, grads, g_ref):
        err = rel_l2(a, b)
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-4, name
    if strong:
        # clamped decays carry no gradient
        dlg = grads[5].cpu()
        assert torch.all(dlg[:, 3, :, :4] == 0) and torch.all(dlg[:, 5, :, 4:8] == 0)


def test_chan_update_norm_matches_token_loop(gpu_lib):
    """|r_t| of the forward (r_norm) equals |beta_w v_t - beta_e S_t^T k_t|
    of the token loop."""
    from gdnx_amd import ops
    print("case: chan r_norm", flush=True)
    B, T, H, D = 1, 40, 2, 64
    q, k, v, be, bw, lg, _ = _inputs(B, T, H, D, seed=11)
    S = torch.zeros(B, H, D, D, dtype=torch.float64)
    rn_ref = []
    for t in range(T):
        S = S * lg[:, t].double().exp().unsqueeze(-1)
        m = torch.einsum("bhk,bhkv->bhv", k[:, t].double(), S)
        r = bw[:, t].double().unsqueeze(-1) * v[:, t].double() - be[:, t].double().unsqueeze(-1) * m
        S = S + k[:, t].double().unsqueeze(-1) * r.unsqueeze(-2)
        rn_ref.append(r.norm(dim=-1))
    rn_ref = torch.stack(rn_ref, 1)
    y, s, rn = ops.delta_rule_chan(*(t.to(DEV) for t in (q, k, v, be, bw, lg)), want_rnorm=True)
    torch.cuda.synchronize()
    assert rn.shape == (B, T, H) and not rn.requires_grad
    assert rel_l2(rn, rn_ref) <= 1e-4

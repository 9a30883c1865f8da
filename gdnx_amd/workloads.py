"""Seeded synthetic workloads of the benchmark / parity configurations.

Data generation only (no recurrence maths): bench.py builds its timed
workloads from these, and the parity tests (through oracle.inputs, which
re-exports them) their inputs.

Every generator draws from ``torch.Generator('cpu').manual_seed(seed)`` in a
fixed order and returns CPU tensors; config k uses seed 1000 + k by default.

  config 0: B=1, H=2, T=256, d=64, one lane, one decay, float32
            q, k ~ N(0,1) then L2-normalised, v ~ N(0,1), beta = sigmoid(N(0,1)),
            log-decay g = -softplus(N(0,1)) * 0.1
  config 1: B=4, T=4096, H=16, d=128, M=4 lanes sharing q/k/v (bf16),
            beta [B,T,H,M] = sigmoid(N(0,1)), lane m decays with
            tau_m in {0.05, 0.02, 0.005, 0.001}: g = log(1 - tau_m) + N(0, 0.01^2),
            clamped <= 0 inside the op; partial RoPE on dims 0..31 of q, k
            (16 half-split pairs x[i] <-> x[16+i], theta_i = t * 1e4^(-i/15)).
  config 2: config 1 plus dO ~ N(0,1) [B,T,H,M,d] in bf16.
  config 3: long context, B=1, T=32768, H=16, d=128, M=4 lanes sharing q/k/v
            (bf16, partial RoPE as config 1); per-lane scalar erase / write
            gates b, w = sigmoid(N(0,1)); multiplicative decay
            exp(log(1 - tau_m) + N(0, 0.01^2)); 64 key/value pairs (k
            L2-normalised, v ~ N(0,1)) written at distinct random positions
            in [0, 4096) and queried (q = k_i) at the last 64 positions.
  config 4: batched decode, 256 sequences x H=16 x 4 lanes x 4 decays.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

TAUS = (0.05, 0.02, 0.005, 0.001)


def partial_rope(x, n_pairs=16, base=1e4):
    """Half-split partial rotary embedding on the first 2*n_pairs channels.

    x: [B,T,H,d].  Pairs (i, n_pairs + i), angle t * base^(-i/(n_pairs-1)):
    the pairing of gdn3/gdn3_upgrade.py:390-398 and the inverse-frequency
    denominator d_pairs-1 of :369-373, identical for every lane.
    """
    B, T, H, d = x.shape
    i = torch.arange(n_pairs, dtype=torch.float64)
    inv = base ** (-i / max(1, n_pairs - 1))
    ang = torch.arange(T, dtype=torch.float64).view(T, 1) * inv.view(1, n_pairs)
    cos = ang.cos().to(x.dtype).view(1, T, 1, n_pairs)
    sin = ang.sin().to(x.dtype).view(1, T, 1, n_pairs)
    x1 = x[..., :n_pairs]
    x2 = x[..., n_pairs:2 * n_pairs]
    out = x.clone()
    out[..., :n_pairs] = x1 * cos - x2 * sin
    out[..., n_pairs:2 * n_pairs] = x1 * sin + x2 * cos
    return out


def dense_inputs(B, T, H, d, M=1, seed=1000, taus=None, rope=False,
                 decay="softplus", io_dtype=torch.float32, with_grad_out=False):
    """Inputs of the lane-shared dense GDN3 regime.

    Returns dict(q, k, v [B,T,H,d] in io_dtype; beta, g [B,T,H,M] float32;
    dO [B,T,H,M,d] io_dtype when with_grad_out).  decay='softplus' draws
    g = -softplus(N(0,1)) * 0.1 (config 0); decay='tau' uses the lane
    timescales ``taus`` (configs 1-2).
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, d, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, H, d, generator=gen), dim=-1)
    v = torch.randn(B, T, H, d, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, M, generator=gen))
    if decay == "softplus":
        g = -F.softplus(torch.randn(B, T, H, M, generator=gen)) * 0.1
    elif decay == "tau":
        taus = TAUS if taus is None else taus
        assert len(taus) == M
        base = torch.tensor([math.log(1.0 - t) for t in taus], dtype=torch.float32)
        g = base.view(1, 1, 1, M) + 0.01 * torch.randn(B, T, H, M, generator=gen)
    else:
        raise ValueError(decay)
    if rope:
        q = partial_rope(q)
        k = partial_rope(k)
    out = dict(q=q.to(io_dtype), k=k.to(io_dtype), v=v.to(io_dtype),
               beta=beta, g=g)
    if with_grad_out:
        out["dO"] = torch.randn(B, T, H, M, d, generator=gen).to(io_dtype)
    return out


def config0(seed=1000):
    return dense_inputs(1, 256, 2, 64, M=1, seed=seed, decay="softplus")


def config1(seed=1001, T=4096, B=4, H=16, d=128, io_dtype=torch.bfloat16):
    return dense_inputs(B, T, H, d, M=4, seed=seed, decay="tau", rope=True,
                        io_dtype=io_dtype)


def config3(seed=1003, T=32768, B=1, H=16, d=128, M=4, n_pairs=64, span=4096,
            io_dtype=torch.bfloat16):
    """Config 3 (GDN3 long context with compaction).  Returns dict(q, k, v
    [B,T,H,d] io_dtype; b, w, dec [B,T,H,M] float32; pos [n_pairs] insert
    positions; qpos [n_pairs] query positions)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, d, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, H, d, generator=gen), dim=-1)
    v = torch.randn(B, T, H, d, generator=gen)
    b = torch.sigmoid(torch.randn(B, T, H, M, generator=gen))
    w = torch.sigmoid(torch.randn(B, T, H, M, generator=gen))
    base = torch.tensor([math.log(1.0 - t) for t in TAUS[:M]], dtype=torch.float32)
    g = base.view(1, 1, 1, M) + 0.01 * torch.randn(B, T, H, M, generator=gen)
    dec = torch.exp(g.clamp(max=0.0))
    n_pairs = min(n_pairs, span, T // 2)
    pos = torch.randperm(min(span, T), generator=gen)[:n_pairs]
    kp = F.normalize(torch.randn(n_pairs, B, H, d, generator=gen), dim=-1)
    vp = torch.randn(n_pairs, B, H, d, generator=gen)
    qpos = torch.arange(T - n_pairs, T)
    q, k = partial_rope(q), partial_rope(k)
    for i in range(n_pairs):
        k[:, pos[i]] = kp[i]
        v[:, pos[i]] = vp[i]
        q[:, qpos[i]] = kp[i]
    return dict(q=q.to(io_dtype), k=k.to(io_dtype), v=v.to(io_dtype), b=b, w=w, dec=dec,
                pos=pos, qpos=qpos)


def config2(seed=1002, T=4096, B=4, H=16, d=128, io_dtype=torch.bfloat16):
    return dense_inputs(B, T, H, d, M=4, seed=seed, decay="tau", rope=True,
                        io_dtype=io_dtype, with_grad_out=True)


def decode_inputs(S=256, H=16, M=4, n_tau=4, d=128, steps=1, seed=1004,
                  state_std=0.02):
    """Config 4: batched one-token decode.  Chains are (seq, head, lane, tau).

    state0 [S,H,M,n_tau,d,d] float32 ~ N(0, state_std^2) (key-major [dk, dv]);
    per step: q, k (L2-normalised), v [steps,S,H,d] bf16 shared by lanes and
    decays; beta [steps,S,H,M] = sigmoid(N(0,1)); g [steps,S,H,M,n_tau] =
    log(1 - tau) + N(0, 0.01^2).
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    state0 = torch.randn(S, H, M, n_tau, d, d, generator=gen) * state_std
    q = F.normalize(torch.randn(steps, S, H, d, generator=gen), dim=-1)
    k = F.normalize(torch.randn(steps, S, H, d, generator=gen), dim=-1)
    v = torch.randn(steps, S, H, d, generator=gen)
    beta = torch.sigmoid(torch.randn(steps, S, H, M, generator=gen))
    base = torch.tensor([math.log(1.0 - t) for t in TAUS[:n_tau]], dtype=torch.float32)
    g = base.view(1, 1, 1, 1, n_tau) + 0.01 * torch.randn(steps, S, H, M, n_tau, generator=gen)
    return dict(state0=state0, q=q.bfloat16(), k=k.bfloat16(), v=v.bfloat16(),
                beta=beta, g=g)

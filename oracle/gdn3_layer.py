"""GDN3 layer boundary pre-ops and post-ops -- CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/ use this module, as the checker; the HIP product path never
imports it.  Restates the element-wise steps of GDN3LinearAttn.forward that
surround the recurrence (gdn3/gdn3_upgrade.py:785-858), in torch (float64 by
default, differentiable with autograd):

prologue (the recurrence inputs, :796-828 and the lane RoPE :342-401)
    b_gates = sigmoid(b_proj + 0.1 proj_a)          [B,T,H,M,K]   (:799-802)
    w_gates = sigmoid(w_proj + 0.1 proj_b)          [B,T,H,M,V]   (:804-807)
    decay   = clamp(mean_tau exp(-min(softplus(x), 5) rate_tau), max=clamp)
                                                    [B,T,H,M]     (:811-822)
    q_m, k_m = lane RoPE of the lane-shared q, k    [B,T,H,M,K]   (:827-828)
      lane m transforms the half-split pairs (x_i, x_{d+i}), i < d = int(K f_m // 2),
      with the angle a = t s_m / 10000^(i / n_m), (f_m, s_m) = ([.5, .25, .5, .5],
      [1, .3, .5, .2])[m], n_m = max(1, int(K/4)//2 - 1) when s_m != 1; when
      s_m == 1 the denominator is max(1, d - 1), and the lane is left unchanged
      when d exceeds the layer's RoPE table width int(K/4)//2 (:355-372).  The
      reference writes the first half in place before it computes the second
      (:396-398, x1 and x2 are views of the tensor being written), so
          x_i' = x_i cos a - x_{d+i} sin a,   x_{d+i}' = x_i' sin a + x_{d+i} cos a
      (not a rotation: the second half reads the updated first half).
epilogue (the lane routing and head norm, :842-856)
    routed = sum_m softmax_m(router_logits) y_m;
    out = routed / max(|routed|, 1e-6) * sqrt(V) * norm

Pinning (tests/test_oracle_gdn3_layer.py): golden vectors captured from the
reference layer's own forward (tests/golden/make_golden_layer.py), and the
properties each step has (lane 0 at K = 128 and t = 0 are the identity, the
lane transform inverts as a triangular map, decay in (0, clamp], the routed
output has norm sqrt(V) |norm|, routing weights sum to one).
"""
from __future__ import annotations

import math

import torch

__all__ = ["LANE_ROPE_FRACTIONS", "LANE_ROPE_SCALES", "lane_rope_params", "lane_rope_tables", "prologue",
           "epilogue"]

LANE_ROPE_FRACTIONS = (0.50, 0.25, 0.50, 0.50)   # gdn3/gdn3_upgrade.py:181
LANE_ROPE_SCALES = (1.0, 0.3, 0.5, 0.2)          # gdn3/gdn3_upgrade.py:182


def lane_rope_params(M, K):
    """Per lane (d_pairs, scale, denominator, identity) following
    _lane_rope_factors (gdn3/gdn3_upgrade.py:342-376)."""
    table_width = int(K * 0.25) // 2          # cos_pe columns (:166-170)
    out = []
    for m in range(M):
        frac, scale = LANE_ROPE_FRACTIONS[m], LANE_ROPE_SCALES[m]
        d = int(K * frac // 2)
        if d < 1:
            out.append((0, scale, 1, True))
        elif scale != 1.0:
            out.append((d, scale, max(1, int(K * 0.25) // 2 - 1), False))
        else:
            out.append((d, scale, max(1, d - 1), d > table_width))
    return out


def lane_rope_tables(M, T, K, dtype=torch.float32):
    """(cos, sin) [M, T, K//2] per lane, zero-padded past each lane's pairs
    (cos 1, sin 0 there and for identity lanes): the angles of
    _lane_rope_factors in float32."""
    half = K // 2
    cos = torch.ones(M, T, half, dtype=dtype)
    sin = torch.zeros(M, T, half, dtype=dtype)
    for m, (d, scale, den, ident) in enumerate(lane_rope_params(M, K)):
        if d < 1 or ident:
            continue
        inv_freq = 1.0 / (10000.0 ** (torch.arange(0, d, dtype=torch.float32) / den))
        ang = (torch.arange(T, dtype=torch.float32) * scale)[:, None] * inv_freq[None, :]
        cos[m, :, :d] = torch.cos(ang).to(dtype)
        sin[m, :, :d] = torch.sin(ang).to(dtype)
    return cos, sin


def _rope(x, M, dtype):
    """x [B,T,H,K] shared by the lanes -> [B,T,H,M,K] rotated per lane."""
    B, T, H, K = x.shape
    cos, sin = lane_rope_tables(M, T, K, dtype)
    xe = x.to(dtype).unsqueeze(3).expand(B, T, H, M, K)
    outs = []
    for m, (d, _, _, ident) in enumerate(lane_rope_params(M, K)):
        xm = xe[:, :, :, m]
        if d < 1 or ident:
            outs.append(xm)
            continue
        c = cos[m, :, :d].view(1, T, 1, d)
        s = sin[m, :, :d].view(1, T, 1, d)
        x1, x2 = xm[..., :d], xm[..., d:2 * d]
        x1n = x1 * c - x2 * s
        outs.append(torch.cat([x1n, x1n * s + x2 * c, xm[..., 2 * d:]], -1))
    return torch.stack(outs, 3)


def prologue(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, rates, decay_clamp=0.999,
             dtype=torch.float64):
    """q, k [B,T,H,K] (lane-shared, after the convolution); b_proj [B,T,H,M,K],
    w_proj [B,T,H,M,V], proj_a, proj_b [B,T,H], decay_proj [B,T,H,M,4],
    rates [4].  Returns (q_rope, k_rope [B,T,H,M,K], b_gates, w_gates, decay)."""
    M = b_proj.shape[3]
    b_gates = torch.sigmoid(b_proj.to(dtype) + proj_a.to(dtype)[..., None, None] * 0.1)
    w_gates = torch.sigmoid(w_proj.to(dtype) + proj_b.to(dtype)[..., None, None] * 0.1)
    g_raw = torch.nn.functional.softplus(decay_proj.to(dtype)).clamp(max=5.0)
    decay = torch.exp(-g_raw * rates.to(dtype)).mean(dim=-1).clamp(max=decay_clamp)
    return _rope(q, M, dtype), _rope(k, M, dtype), b_gates, w_gates, decay


def epilogue(y, router_logits, norm, dtype=torch.float64):
    """y [B,T,H,M,V] (the recurrence output), router_logits [B,T,H,M],
    norm [V] -> [B,T,H,V]."""
    V = y.shape[-1]
    w = torch.softmax(router_logits.to(dtype), dim=-1)
    routed = (w.unsqueeze(-1) * y.to(dtype)).sum(dim=3)
    routed = torch.nn.functional.normalize(routed, p=2, dim=-1, eps=1e-6) * math.sqrt(V)
    return routed * norm.to(dtype)

"""GDN3 layer boundary on the GPU: the fused pre-ops and post-ops around the
recurrence, and the layer core that chains them.

GDN3LinearAttn.forward (gdn3/gdn3_upgrade.py:785-856) builds the recurrence
inputs and consumes its output with element-wise torch ops:

* ``gdn3_prologue`` replaces lines 796-828: the sigmoid erase / write gates
  (b_proj + 0.1 proj_a, w_proj + 0.1 proj_b), the braided multi-timescale
  decay (softplus clamped at 5, four base rates, mean, clamp at
  ``decay_clamp``) and the per-lane partial RoPE of the lane-shared q and k
  (_apply_partial_rope :378-401, with its in-place update: the second half
  of each pair reads the already-rotated first half).  One HIP kernel per
  direction (gdnx_gdn3_prologue_fwd / _bwd).
* ``gdn3_epilogue`` replaces lines 842-851: softmax lane routing, the
  per-head L2 normalisation (eps 1e-6), sqrt(V) and the learned ``norm``
  scale.  One HIP kernel per direction (gdnx_gdn3_epilogue_fwd / _bwd; the
  d_norm reduction over rows is deterministic).
* ``gdn3_layer_core`` runs prologue -> gdn3_recurrent_state -> epilogue,
  i.e. lines 785-851 from the projections to the tensor _agg_proj receives.

All three are differentiable (torch.autograd.Function over the HIP kernels);
gradients follow torch's conventions at the clamps (the gradient passes where
the clamp's input is <= its bound).  The RoPE angle tables are computed the
way the reference computes its cached tables (_lane_rope_factors
:342-376, float32 torch ops on the tensor's device) and cached per
(M, T, K, device).
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from . import gdn3, ops

LANE_ROPE_SCALES = (1.0, 0.3, 0.5, 0.2)   # gdn3/gdn3_upgrade.py:182
DEFAULT_DECAY_CLAMP = 0.999               # gdn3/gdn3_upgrade.py:80 (env GDN3_DECAY_CLAMP)

_TABLES: "OrderedDict[tuple, tuple]" = OrderedDict()
_TABLE_CACHE_SIZE = 16


def lane_rope_tables(M: int, T: int, K: int, device):
    """(cos, sin) float32 [M, T, K//2] on ``device``: lane m's angles
    t * scale_m / 10000^(i / den_m) in its first d_m columns (d_m from
    gdnx_gdn3_lane_rope_pairs; den_m = max(1, floor(K/4)/2 - 1) for scale !=
    1, max(1, d_m - 1) otherwise, gdn3/gdn3_upgrade.py:355-373); cos 1 / sin 0
    elsewhere."""
    key = (M, T, K, str(torch.device(device)))
    hit = _TABLES.get(key)
    if hit is not None:
        _TABLES.move_to_end(key)
        return hit
    cos = torch.ones(M, T, K // 2, dtype=torch.float32, device=device)
    sin = torch.zeros(M, T, K // 2, dtype=torch.float32, device=device)
    pos = torch.arange(T, device=device, dtype=torch.float32)
    for m, d in enumerate(ops.gdn3_lane_rope_pairs(M, K)):
        if d == 0:
            continue
        scale = LANE_ROPE_SCALES[m]
        den = max(1, int(K * 0.25) // 2 - 1) if scale != 1.0 else max(1, d - 1)
        inv_freq = 1.0 / (10000.0 ** (torch.arange(0, d, device=device, dtype=torch.float32) / den))
        ang = (pos * scale)[:, None] * inv_freq[None, :]
        cos[m, :, :d] = torch.cos(ang)
        sin[m, :, :d] = torch.sin(ang)
    _TABLES[key] = (cos, sin)
    while len(_TABLES) > _TABLE_CACHE_SIZE:
        _TABLES.popitem(last=False)
    return cos, sin


class _Prologue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, rates, decay_clamp):
        B, T, H, K = q.shape
        M = b_proj.shape[3]
        cos, sin = lane_rope_tables(M, T, K, q.device)
        qr, kr, bg, wg, dec = ops.gdn3_prologue_fwd(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, rates,
                                                    cos, sin, decay_clamp)
        dt = qr.dtype
        saved = [t.to(dt).contiguous() for t in (b_proj, proj_a, w_proj, proj_b, decay_proj)]
        ctx.save_for_backward(*saved, rates.float().contiguous(), cos, sin)
        ctx.decay_clamp = decay_clamp
        ctx.in_dtypes = tuple(t.dtype for t in (q, k, b_proj, proj_a, w_proj, proj_b, decay_proj))
        return qr, kr, bg, wg, dec

    @staticmethod
    def backward(ctx, dqr, dkr, dbg, dwg, ddec):
        bp, pa, wp, pb, dp, rates, cos, sin = ctx.saved_tensors
        B, T, H, M, K = bp.shape
        V = wp.shape[-1]

        def g(t, shape):
            return torch.zeros(shape, dtype=torch.float32, device=bp.device) if t is None else t
        grads = ops.gdn3_prologue_bwd(bp, pa, wp, pb, dp, rates, cos, sin, g(dqr, (B, T, H, M, K)),
                                      g(dkr, (B, T, H, M, K)), g(dbg, (B, T, H, M, K)), g(dwg, (B, T, H, M, V)),
                                      g(ddec, (B, T, H, M)), ctx.decay_clamp)
        dq, dk, dbp, dpa, dwp, dpb, ddp = grads
        out = [t.to(d) for t, d in zip((dq, dk, dbp, dpa, dwp, dpb, ddp), ctx.in_dtypes)]
        return (*out, None, None)


class _Epilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, router_logits, norm):
        y = y.contiguous()
        lg = router_logits.to(y.dtype).contiguous()
        nm = norm.float().contiguous()
        out = ops.gdn3_epilogue_fwd(y, lg, nm)
        ctx.save_for_backward(y, lg, nm)
        ctx.in_dtypes = (router_logits.dtype, norm.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        y, lg, nm = ctx.saved_tensors
        dy, dlg, dnm = ops.gdn3_epilogue_bwd(y, lg, nm, dout)
        return dy, dlg.to(ctx.in_dtypes[0]), dnm.to(ctx.in_dtypes[1])


def gdn3_prologue(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, base_decay_rates,
                  decay_clamp=DEFAULT_DECAY_CLAMP):
    """Recurrence inputs of GDN3LinearAttn.forward (gdn3/gdn3_upgrade.py:796-828).

    q, k [B,T,H,K] lane-shared (after the convolution), bf16 or float32 (the
    compute dtype; the other IO inputs are cast to it); b_proj [B,T,H,M,K],
    w_proj [B,T,H,M,V], proj_a, proj_b [B,T,H], decay_proj [B,T,H,M,4],
    base_decay_rates [4].  Returns (q_rope, k_rope [B,T,H,M,K] in q's dtype,
    b_gates [B,T,H,M,K], w_gates [B,T,H,M,V], decay [B,T,H,M] float32)."""
    if q.numel() == 0:
        B, T, H, K = q.shape
        M, V = b_proj.shape[3], w_proj.shape[-1]
        srcs = (q, k, b_proj, proj_a, w_proj, proj_b, decay_proj)
        dt = q.dtype
        return (ops.empty_result((B, T, H, M, K), dt, q.device, *srcs),
                ops.empty_result((B, T, H, M, K), dt, q.device, *srcs),
                ops.empty_result((B, T, H, M, K), torch.float32, q.device, *srcs),
                ops.empty_result((B, T, H, M, V), torch.float32, q.device, *srcs),
                ops.empty_result((B, T, H, M), torch.float32, q.device, *srcs))
    return _Prologue.apply(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, base_decay_rates, float(decay_clamp))


def gdn3_epilogue(y, router_logits, norm):
    """Lane routing and head norm of GDN3LinearAttn.forward
    (gdn3/gdn3_upgrade.py:842-851): y [B,T,H,M,V] (the recurrence output),
    router_logits [B,T,H,M], norm [V] -> [B,T,H,V] in y's dtype."""
    if y.numel() == 0:
        B, T, H, M, V = y.shape
        return ops.empty_result((B, T, H, V), y.dtype, y.device, y, router_logits, norm)
    return _Epilogue.apply(y, router_logits, norm)


def gdn3_layer_core(q, k, v, b_proj, proj_a, w_proj, proj_b, decay_proj, base_decay_rates, router_logits, norm,
                    *, decay_clamp=DEFAULT_DECAY_CLAMP, R=4, P=16, factors=(16, 16, 8, 8), slow_decay=0.97,
                    compact_every=None, sketch=None, return_state=False):
    """Lines 785-851 of GDN3LinearAttn.forward: prologue, the Kronecker-
    residual recurrence on the lane-expanded v, epilogue.  q, k, v [B,T,H,K]
    (lane-shared, after the convolution); the other arguments as
    gdn3_prologue / gdn3_epilogue; recurrence options as
    gdn3.gdn3_recurrent_state.  Returns the routed, normalised heads
    [B,T,H,V] (``aggregated`` before its view to [B,T,H*V]), plus
    (state, comp_err) when return_state."""
    qr, kr, bg, wg, dec = gdn3_prologue(q, k, b_proj, proj_a, w_proj, proj_b, decay_proj, base_decay_rates,
                                        decay_clamp)
    B, T, H, M, _ = qr.shape
    ve = v.to(qr.dtype).unsqueeze(3).expand(B, T, H, M, v.shape[-1])
    res = gdn3.gdn3_recurrent_state(qr, kr, ve, bg, wg, dec, R=R, P=P, factors=factors, slow_decay=slow_decay,
                                    compact_every=compact_every, sketch=sketch, return_state=return_state)
    y = res[0] if return_state else res
    out = gdn3_epilogue(y, router_logits, norm)
    return (out, res[1], res[2]) if return_state else out

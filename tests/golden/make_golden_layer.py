"""Write golden vectors of the GDN3 layer's boundary pre-ops and post-ops from
the reference's own layer forward (run once, CPU, in the build container
where /root/reference exists; never on the GPU box).

GDN3LinearAttn.forward (gdn3/gdn3_upgrade.py:721-884) computes the
recurrence inputs in line; the lane RoPE (:342-401) carries quirks no closed
form pins (the per-lane denominators, the identity lane, and the in-place
update that makes the second half read the rotated first half).  The script
runs the layer on random hidden states and records, through wrappers around
_apply_partial_rope and _gdn3_recurrent_state and hooks on router_proj and
_agg_proj, the tensors that enter and leave the pre-ops and post-ops:
  pro_q, pro_k            q, k before RoPE (lane-shared, [B,T,H,K])
  pro_b_proj, pro_proj_a, pro_w_proj, pro_proj_b, pro_decay_proj, pro_rates
  pro_q_rope, pro_k_rope, pro_b_gates, pro_w_gates, pro_decay   (outputs)
  epi_y, epi_router_logits, epi_norm, epi_out                    (post-ops)
as float32 arrays in gdn3_layer_golden.npz (allow_pickle=False).

Usage:  python tests/golden/make_golden_layer.py [/root/reference]
"""
import os
import sys
from types import SimpleNamespace

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)

from gdn3.gdn3_upgrade import GDN3LinearAttn  # noqa: E402


def main():
    torch.manual_seed(0)
    cfg = SimpleNamespace(hidden_size=64, linear_num_key_heads=2, linear_key_head_dim=128,
                          linear_value_head_dim=128, linear_conv_kernel_dim=4)
    layer = GDN3LinearAttn(cfg, layer_idx=0).eval()
    gen = torch.Generator().manual_seed(2024)
    with torch.no_grad():
        for name in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"):
            p = getattr(layer, name)
            p.copy_(torch.randn(p.shape, generator=gen) * 0.2)
        layer.norm.copy_(0.5 + torch.rand(layer.norm.shape, generator=gen))
        layer.W_decay.mul_(40.0)   # spread softplus over its clamp at 5
    B, T, D = 1, 24, 64
    H, M, K = layer.H, layer.M, layer.K
    x = torch.randn(B, T, D, generator=gen)

    rec = {}
    rope_calls = []
    orig_rope = layer._apply_partial_rope

    def rope(t, t_max):
        out = orig_rope(t, t_max)
        rope_calls.append((t.detach().clone(), out.detach().clone()))
        return out
    layer._apply_partial_rope = rope
    orig_rec = layer._gdn3_recurrent_state

    def recurrence(q, k, v, b, w, dec):
        y = orig_rec(q, k, v, b, w, dec)
        rec.update(b_gates=b.detach().clone(), w_gates=w.detach().clone(), decay=dec.detach().clone(),
                   y=y.detach().clone())
        return y
    layer._gdn3_recurrent_state = recurrence
    layer.router_proj.register_forward_hook(lambda m, i, o: rec.update(router_logits=o.detach().clone()))
    layer._agg_proj.register_forward_pre_hook(lambda m, i: rec.update(aggregated=i[0].detach().clone()))
    with torch.no_grad():
        layer(x)
        b_proj = F.linear(x, layer.W_b.reshape(-1, D)).view(B, T, H, M, K)
        w_proj = F.linear(x, layer.W_w.reshape(-1, D)).view(B, T, H, M, layer.V)
        proj_a = F.linear(x, layer.in_proj_a)
        proj_b = F.linear(x, layer.in_proj_b)
        decay_proj = F.linear(x, layer.W_decay.reshape(-1, D)).view(B, T, H, M, 4)
    (q_in, q_rope), (k_in, k_rope) = rope_calls
    out = dict(pro_q=q_in[:, :, :, 0], pro_k=k_in[:, :, :, 0], pro_b_proj=b_proj, pro_proj_a=proj_a,
               pro_w_proj=w_proj, pro_proj_b=proj_b, pro_decay_proj=decay_proj,
               pro_rates=layer.base_decay_rates.clone(), pro_q_rope=q_rope, pro_k_rope=k_rope,
               pro_b_gates=rec["b_gates"], pro_w_gates=rec["w_gates"], pro_decay=rec["decay"],
               epi_y=rec["y"], epi_router_logits=rec["router_logits"].view(B, T, H, M),
               epi_norm=layer.norm.detach().clone(), epi_out=rec["aggregated"].view(B, T, H, layer.V))
    np.savez(os.path.join(HERE, "gdn3_layer_golden.npz"),
             **{k: v.detach().float().numpy() for k, v in out.items()},
             decay_clamp=np.array([layer.decay_clamp], dtype=np.float32))
    print("wrote", sorted(out))


if __name__ == "__main__":
    main()

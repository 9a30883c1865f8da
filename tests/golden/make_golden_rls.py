"""Write golden vectors of the rank-r RLS T-factor scan from the reference's
own code (run once, CPU, in the build container where /root/reference
exists; never on the GPU box).

Two sources:
  * KMD2LinearAttn._scan (gdn3/kmd2.py:166-214), called unbound on a plain
    namespace carrying the attributes it reads (r, dk, dv, r_out, rls_eps,
    out_mix) -- cases r = 1 (its fast path) and r = 2 with r_out = 2;
  * the testbed mixer KMD2Mixer.forward (research/testbed_mqar.py:172-262)
    with its projections replaced by fixed tensors (q / K / V from _qkv, the
    gate and decay logits from bgate / wgate / decay) and o_proj by the
    identity, with SVD compaction every P tokens, plain and straight-through.
For each case the inputs, y and the gradients of y . dy with respect to every
input are stored as float32 arrays in rls_golden.npz (allow_pickle=False),
keys "<case>/<name>".

Usage:  python tests/golden/make_golden_rls.py [/root/reference]
"""
import os
import sys
from types import SimpleNamespace

import numpy as np
import torch
import torch.nn as nn

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)
sys.path.insert(0, os.path.join(REF, "research"))

from gdn3.kmd2 import KMD2LinearAttn  # noqa: E402
from testbed_mqar import KMD2Mixer  # noqa: E402


def inputs(gen, B, T, H, r, r_out, dk, dv):
    q = torch.nn.functional.normalize(torch.randn(B, T, H, r_out, dk, generator=gen), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, T, H, r, dk, generator=gen), dim=-1)
    V = torch.randn(B, T, H, r, dv, generator=gen)
    Bg = torch.sigmoid(torch.randn(B, T, H, r, dk, generator=gen))
    Wg = torch.sigmoid(torch.randn(B, T, H, r, dv, generator=gen))
    a = torch.sigmoid(torch.randn(B, T, H, dk, generator=gen) + 4.0).clamp(max=0.999)
    return dict(q=q, K=K, V=V, Bg=Bg, Wg=Wg, a=a)


def scan_case(gen, B, T, H, r, r_out, dk, dv, eps):
    x = inputs(gen, B, T, H, r, r_out, dk, dv)
    mix = torch.rand(H, r_out, generator=gen) + 0.2
    leaves = {k: v.clone().requires_grad_(True) for k, v in x.items()}
    mixl = mix.clone().requires_grad_(True)
    fake = SimpleNamespace(r=r, dk=dk, dv=dv, r_out=r_out, rls_eps=eps, out_mix=mixl)
    y = KMD2LinearAttn._scan(fake, leaves["q"], leaves["K"], leaves["V"], leaves["Bg"], leaves["Wg"],
                             leaves["a"])
    dy = torch.randn(y.shape, generator=gen)
    names = list(leaves) + (["out_mix"] if r_out > 1 else [])
    params = list(leaves.values()) + ([mixl] if r_out > 1 else [])
    grads = torch.autograd.grad(y, params, dy)
    out = {k: v for k, v in x.items()}
    out.update(out_mix=mix, y=y.detach(), dy=dy, eps=torch.tensor([eps]))
    out.update({"d" + n: g for n, g in zip(names, grads)})
    return out


class Fixed(nn.Module):
    def __init__(self, t):
        super().__init__()
        self.t = t

    def forward(self, x):
        return self.t


def testbed_case(gen, B, T, H, r, r_out, dk, dv, eps, P, R, ste):
    torch.manual_seed(0)
    mixer = KMD2Mixer(16, H=H, dk=dk, dv=dv, r=r, eps=eps, compact_P=P, compact_R=R, slow_decay=0.97,
                      use_conv=False, compact_ste=ste, r_out=r_out)
    x = inputs(gen, B, T, H, r, r_out, dk, dv)
    logit = {"bg": torch.randn(B, T, H * r * dk, generator=gen), "wg": torch.randn(B, T, H * r * dv, generator=gen),
             "dec": torch.randn(B, T, H * dk, generator=gen) + 5.0}
    leaves = {k: x[k].clone().requires_grad_(True) for k in ("q", "K", "V")}
    ll = {k: v.clone().requires_grad_(True) for k, v in logit.items()}
    mixer._qkv = lambda xx, BB, TT: (leaves["q"], leaves["K"], leaves["V"])
    mixer.bgate, mixer.wgate, mixer.decay = Fixed(ll["bg"]), Fixed(ll["wg"]), Fixed(ll["dec"])
    mixer.o_proj = nn.Identity()
    y = mixer(torch.zeros(B, T, 16)).view(B, T, H, dv)
    dy = torch.randn(y.shape, generator=gen)
    params = list(leaves.values()) + list(ll.values())
    grads = torch.autograd.grad(y, params, dy)
    out = {k: x[k] for k in ("q", "K", "V")}
    out.update(bg_logit=logit["bg"].view(B, T, H, r, dk), wg_logit=logit["wg"].view(B, T, H, r, dv),
               dec_logit=logit["dec"].view(B, T, H, dk), y=y.detach(), dy=dy,
               eps=torch.tensor([eps]), P=torch.tensor([P]), R=torch.tensor([R]))
    out.update({"d" + n: g for n, g in zip(("q", "K", "V", "bg_logit", "wg_logit", "dec_logit"), grads)})
    out["dbg_logit"] = out["dbg_logit"].view(B, T, H, r, dk)
    out["dwg_logit"] = out["dwg_logit"].view(B, T, H, r, dv)
    out["ddec_logit"] = out["ddec_logit"].view(B, T, H, dk)
    return out


def main():
    gen = torch.Generator().manual_seed(77)
    cases = {
        "r1": scan_case(gen, 2, 20, 2, 1, 1, 16, 8, 0.5),
        "r2o2": scan_case(gen, 1, 18, 2, 2, 2, 16, 12, 0.5),
        "tb_plain": testbed_case(gen, 1, 24, 2, 2, 1, 16, 16, 0.5, 8, 3, False),
        "tb_ste": testbed_case(gen, 1, 24, 2, 2, 1, 16, 16, 0.5, 8, 3, True),
    }
    flat = {f"{c}/{k}": v.detach().float().numpy() for c, d in cases.items() for k, v in d.items()}
    np.savez(os.path.join(HERE, "rls_golden.npz"), **flat)
    print("wrote", len(flat), "arrays:", sorted(cases))


if __name__ == "__main__":
    main()

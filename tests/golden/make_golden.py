"""Write golden vectors from the reference's own GDN3 code (run once, CPU, in
the build container where /root/reference exists; never on the GPU box).

Only functions that no closed form, known-answer test or brute force pins are
recorded here (the compaction's LAPACK sign choices and sketch stream, and the
end-to-end sequential recurrence across several compactions); the dense delta
rule is pinned without importing the reference.

Records, as float32 arrays in gdn3_golden.npz (allow_pickle=False):
  compact_*   inputs/outputs of GDN3LinearAttn._compact_vec and _compact_fast
              (gdn3/gdn3_upgrade.py:650-719, :565-624) on a random state
  seqA_*      reference_recurrent_state (gdn3/_reference_recurrence.py:33-94)
              with the layer defaults (R=4, P=16, 16x16 (x) 8x8, s=0.97),
              B=1, T=48, H=1, M=2 (three compactions), channel-wise gates,
              plus gradients of y.pow(2).mean() and the reference's chunked
              _gdn3_recurrent_state output (gdn3/gdn3_upgrade.py:403-531)
  seqB_*      the config-0 shape in GDN3 mode: d=64 with 8x8 (x) 8x8 factors,
              P=64, scalar gates b = w = beta, four compactions, plus the
              chunked path's output

Usage:  python tests/golden/make_golden.py [/root/reference]
"""
import os
import sys
from types import SimpleNamespace

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from gdn3.gdn3_upgrade import GDN3LinearAttn  # noqa: E402
from gdn3._reference_recurrence import reference_recurrent_state  # noqa: E402

from oracle import inputs  # noqa: E402


def make_layer(factors=(16, 16, 8, 8), P=16):
    cfg = SimpleNamespace(hidden_size=64, linear_num_key_heads=2, linear_key_head_dim=128,
                          linear_value_head_dim=128, linear_conv_kernel_dim=4)
    layer = GDN3LinearAttn(cfg, layer_idx=0).eval()
    layer.a_v, layer.a_k, layer.b_v, layer.b_k = factors
    layer.P = P
    return layer


def main():
    out = {}
    torch.manual_seed(0)
    # ---- compaction on a random state ----------------------------------------
    layer = make_layer()
    gen = torch.Generator().manual_seed(4242)
    N, R = 3, 4
    A = torch.randn(N, R, 16, 16, generator=gen) * 0.3
    Bk = torch.randn(N, R, 8, 8, generator=gen) * 0.3
    U = torch.randn(N, 128, 16, generator=gen)
    Vb = torch.randn(N, 128, 16, generator=gen) * 0.1
    with torch.no_grad():
        A1, B1, _, _, err1 = layer._compact_vec(A, Bk, U, Vb, 0.97)
        A2, B2, _, _, err2 = layer._compact_fast(A, Bk, U, Vb)
    out.update(compact_A=A, compact_Bk=Bk, compact_U=U, compact_Vb=Vb,
               compact_vec_A=A1, compact_vec_B=B1, compact_vec_err=err1.reshape(1),
               compact_fast_A=A2, compact_fast_B=B2, compact_fast_err=err2.reshape(1))

    # ---- case A: layer defaults, channel-wise gates, 3 compactions -----------
    gen = torch.Generator().manual_seed(777)
    Bn, T, H, M, K = 1, 48, 1, 2, 128
    q = torch.randn(Bn, T, H, M, K, generator=gen) * 0.5
    k = torch.nn.functional.normalize(torch.randn(Bn, T, H, M, K, generator=gen), dim=-1)
    v = torch.randn(Bn, T, H, M, K, generator=gen)
    bg = torch.sigmoid(torch.randn(Bn, T, H, M, K, generator=gen))
    wg = torch.sigmoid(torch.randn(Bn, T, H, M, K, generator=gen))
    dec = 0.9 + 0.09 * torch.rand(Bn, T, H, M, generator=gen)
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, bg, wg, dec)]
    y = reference_recurrent_state(layer, *ins)
    grads = torch.autograd.grad(y.pow(2).mean(), ins, allow_unused=True)
    with torch.no_grad():
        yc = layer._gdn3_recurrent_state(q, k, v, bg, wg, dec)
    out.update(seqA_q=q, seqA_k=k, seqA_v=v, seqA_bg=bg, seqA_wg=wg, seqA_dec=dec,
               seqA_y=y.detach(), seqA_ychunk=yc)
    for name, g in zip(["q", "k", "v", "bg", "wg", "dec"], grads):
        out["seqA_grad_" + name] = g

    # ---- case B: config-0 shape in GDN3 mode ---------------------------------
    layer8 = make_layer(factors=(8, 8, 8, 8), P=64)
    x = inputs.config0()
    beta = x["beta"]                                   # [1,256,2,1]
    q5 = x["q"].unsqueeze(3)
    k5 = x["k"].unsqueeze(3)
    v5 = x["v"].unsqueeze(3)
    bgB = beta.unsqueeze(-1).expand(*beta.shape, 64).contiguous()
    decB = x["g"].exp()
    with torch.no_grad():
        yB = reference_recurrent_state(layer8, q5, k5, v5, bgB, bgB, decB)
        yBc = layer8._gdn3_recurrent_state(q5, k5, v5, bgB, bgB, decB)
    out.update(seqB_y=yB, seqB_ychunk=yBc)

    arrays = {k_: np.ascontiguousarray(v_.detach().float().numpy()) for k_, v_ in out.items()}
    path = os.path.join(HERE, "gdn3_golden.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, sum(a.nbytes for a in arrays.values()) // 1024, "KiB raw")
    print("case A chunked-vs-sequential max |diff|:", (yc - y.detach()).abs().max().item())
    print("case B chunked-vs-sequential max |diff|:", (yBc - yB).abs().max().item(),
          "rel-L2:", ((yBc - yB).norm() / yB.norm()).item())


if __name__ == "__main__":
    main()

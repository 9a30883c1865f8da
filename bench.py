#!/usr/bin/env python3
"""Headline benchmark: GDN3 scan tokens/s, forward + backward, on one MI355X.

Workload: one GDN3 layer recurrence at B=4, T=4096,
H=16, d_k=d_v=128, 4 MIMO lanes sharing q/k/v (bf16 IO, fp32 state), lane
decays tau in {0.05, 0.02, 0.005, 0.001} plus N(0, 0.01^2) gate noise,
partial RoPE on q/k dims 0..31; synthetic seeded inputs
(gdnx_amd.workloads, seed 1002) already resident in HBM.  One step =
gdnx_amd.gdn3.gdn3_scan forward + backward against a fixed bf16 upstream
gradient dO, producing dq, dk, dv, dbeta, dlog_g.

Prints ONE JSON line.  Besides the step throughput it reports:
  roofline      the dominant kernel's algorithmic FLOP per launch divided by
                its mean duration (HIP events on the launch stream), against
                the 2.5 PFLOP/s dense bf16 MFMA peak;
  roofline_intra_chunk  the intra-chunk phase (delta_prep_kernel) and the
                fused single-kernel forward at C = 64, with MFMA-busy counters;
  config1_fwd_ms, config1_fwd_fused_c64_ms  the inference forward (no
                stash) at the config-1 shape: the default path, and the fused
                single-kernel scan at C = 64;
  decode_ms_per_step, decode_hbm_frac  the config-4 decode step;
  decode_gdn3_ms_per_step, decode_gdn3_hbm_frac  the GDN3 Kronecker-residual
                decode step at the same width (a step that closes no
                compaction interval);
  gdn3_layer_fwd_bwd_ms  the GDN3 layer default regime (compaction every
                16 tokens) forward + backward at B=4, T=4096;
  cpu_baseline  the repository's CPU oracle (a port of the reference's
                sequential recurrence, fp32, torch autograd) on a bounded
                sample of the same workload (4 of the 16 heads), as measured.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_BF16_PEAK = 2.5e15   # dense bf16 FLOP/s
HBM_PEAK = 8.0e12         # B/s


def flops_fwd(B, T, H, M, D, C):
    """Algorithmic FLOP of one forward launch: per (b, h, chunk) the lane-
    shared grams 4C^2 D plus, per lane, 6 C D^2 (E S0, Q S0 and the carry),
    4 C^2 D (triangular solve on D right-hand sides and the masked output
    product) and C^3/3 (inverse)."""
    nchunks = B * H * ((T + C - 1) // C)
    return nchunks * (4 * C * C * D + M * (6 * C * D * D + 4 * C * C * D + C ** 3 / 3))


def flops_prep(B, T, H, M, D, C):
    """The intra-chunk phase (delta_prep_kernel): per (b, h, chunk) the
    lane-shared grams K K^T and Q K^T (2 C^2 D each) and, per lane, the
    unit-lower inverse (C^3 / 3)."""
    nchunks = B * H * ((T + C - 1) // C)
    return nchunks * (4 * C * C * D + M * C ** 3 / 3)


def flops_bwd_state(B, T, H, M, D, C):
    """Reverse state scan: per lane and chunk K dS (2 C D^2), Aq^T dY and
    T^T dR (2 C^2 D each), the dS update (4 C D^2) and P3 = R dS^T
    (2 C D^2)."""
    nchunks = B * H * ((T + C - 1) // C)
    return nchunks * M * (8 * C * D * D + 4 * C * C * D)


def flops_bwd_grads(B, T, H, M, D, C):
    """Gradient kernel (delta_grad_seg_kernel, 32-token sub-chunks): per lane
    and sub-chunk P1 = dY S^T, P2 = dB S^T and the state update (2 C D^2
    each), dAq = dY R^T and dL = -dB R^T (2 C^2 D each); per head and
    sub-chunk the raw grams Q K^T, K K^T (2 C^2 D each) and the gram-gradient
    products into dq and dk (three of 2 C^2 D)."""
    nchunks = B * H * ((T + C - 1) // C)
    return nchunks * (10 * C * C * D + M * (6 * C * D * D + 4 * C * C * D))


def median_time(fn, runs=3):
    """CPU baseline timing: one warm-up run of ``fn``
    at the sample size, then the median wall time of ``runs`` runs."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(T=2048, H=4):
    """Time the CPU oracle (fp32 sequential recurrence + autograd) on
    B=1, H heads x 4 lanes, T tokens (one warm-up, median of 3); tokens/s of
    that sample as measured (tokens of the H-head sample per second)."""
    import torch
    from oracle import delta, inputs
    torch.set_num_threads(os.cpu_count() or 1)
    x = inputs.dense_inputs(1, T, H, 128, M=4, seed=1002, decay="tau", rope=True, with_grad_out=True)

    def run():
        ins = [x[n].float().requires_grad_(True) for n in ("q", "k", "v", "beta", "g")]
        a = delta.gdn3_dense_coeffs(ins[1], ins[3])
        y, _ = delta.lane_delta(ins[0], ins[1], ins[2], a, a, ins[4], dtype=torch.float32)
        (y * x["dO"].float()).sum().backward()
    secs = median_time(run)
    return {
        "value": T / secs,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle.delta.lane_delta fp32 sequential fwd+bwd, B=1 T={T} H={H}x4 lanes "
                  f"d=128 (the headline layer has 16 heads), one warm-up then median of 3 ({secs:.1f} s); "
                  f"value = tokens of this sample per second, not scaled",
    }


def measured_traffic(kernel):
    """HBM bytes per launch of ``kernel`` from the committed counter table
    (FETCH_SIZE + WRITE_SIZE runs, each scaled by the counter's reading for a
    1 GiB device copy), or None when the table has no entry."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("kernels", {}).get(kernel)
    return None if entry is None else entry["traffic"]


def intra_chunk_entry(t_prep, flop, t_fused, flop_fused):
    """Roofline of the intra-chunk phase as the default paths run it
    (delta_prep_kernel at the training chunk, timed alone with HIP events):
    algorithmic FLOP against the dense bf16 MFMA peak, its measured HBM
    traffic against 8 TB/s, and the MFMA-busy fraction read by the
    SQ_VALU_MFMA_BUSY_CYCLES counter in the committed profile.  "fused": the
    same phase on-chip inside the single-kernel forward at C = 64
    (delta_fwd_kernel, which also runs the inter-chunk scan), with its
    counter."""
    busy = {}
    path = os.path.join(ROOT, "profiles", "mfma_busy.json")
    if os.path.exists(path):
        with open(path) as f:
            busy = json.load(f).get("kernels", {})
    name = "delta_prep_kernel"
    achieved = flop / t_prep / 1e12
    traffic = measured_traffic(name)
    entry = {"kernel": name, "bound": "hbm", "achieved_tflops": achieved,
             "peak_tflops": MFMA_BF16_PEAK / 1e12, "frac_mfma": achieved * 1e12 / MFMA_BF16_PEAK,
             "mean_us": t_prep * 1e6, "algorithmic_flop": flop, "traffic": traffic,
             "hbm_gbs": None if traffic is None else traffic / t_prep / 1e9,
             "frac_hbm": None if traffic is None else traffic / t_prep / HBM_PEAK,
             "mfma_busy_counter": busy.get(name)}
    entry["fused"] = {"kernel": "delta_fwd_kernel", "chunk": 64, "mean_us": t_fused * 1e6,
                      "algorithmic_flop": flop_fused, "achieved_tflops": flop_fused / t_fused / 1e12,
                      "frac_mfma": flop_fused / t_fused / MFMA_BF16_PEAK,
                      "mfma_busy_counter": busy.get("delta_fwd_kernel")}
    return entry


def decode_bytes(NS, H, NC, D, io_bytes=2):
    """HBM bytes of one decode step: the fp32 state read and written once,
    q, k, v read once per head, the per-chain scalars (a_e, a_w, log_g) and
    y written once per chain."""
    state = NS * H * NC * D * D * 4
    return 2 * state + 3 * NS * H * D * io_bytes + 3 * NS * H * NC * 4 + NS * H * NC * D * io_bytes


def cpu_baseline_decode(NS_sample=64, H=16, NC=16, D=128, steps=8):
    """Time the CPU oracle's sequential step (fp32) on NS_sample sequences of
    the decode workload; tokens/s scaled to the 256 sequences."""
    import torch
    from oracle import delta
    torch.set_num_threads(os.cpu_count() or 1)
    gen = torch.Generator().manual_seed(1004)
    S = torch.randn(NS_sample, H, NC, D, D, generator=gen) * 0.02
    q, k, v = (torch.randn(NS_sample, 1, H, D, generator=gen) for _ in range(3))
    a = torch.rand(NS_sample, 1, H, NC, generator=gen)
    lg = torch.full((NS_sample, 1, H, NC), -0.01)
    st = {"S": S}

    def run():
        for _ in range(steps):
            _, st["S"] = delta.lane_delta(q, k, v, a, a, lg, state0=st["S"], dtype=torch.float32)
    secs = median_time(run) / steps
    return {
        "value": NS_sample / secs,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle.delta.lane_delta fp32 one-token step, {NS_sample} of the 256 sequences "
                  f"x {H} heads x {NC} chains d={D}, {steps} steps per run, one warm-up run then median of 3 "
                  f"({secs * 1e3:.1f} ms/step); "
                  f"tokens/s = sequences per step time",
    }


def gdn3_decode_bytes(N, NS, H, D, P=16, R=4, io_bytes=2):
    """HBM bytes of one GDN3 decode step without a compaction: per chain the
    Kronecker-residual state read whole (A: R 16x16, B: R 8x8, U and Vb:
    D x P, fp32: 21.5 KB at D = 128, P = 16) and written back except U's
    other slots (A, B, gamma Vb and one U column: 13.5 KB), its three gates
    and its bf16 output; q, k, v once per head."""
    read = (R * 256 + R * 64 + 2 * D * P) * 4
    write = (R * 256 + R * 64 + D * P + D) * 4
    return N * (read + write + 3 * 4 + D * io_bytes) + 3 * NS * H * D * io_bytes


def decode_bytes_chan(NS, H, NC, D, io_bytes=2):
    """The per-key-channel decode step: the dense step's bytes with a
    log-decay per key channel (D floats per chain) in place of one."""
    return decode_bytes(NS, H, NC, D, io_bytes) + NS * H * NC * (D - 1) * 4


def decode_suite_extras(out, steps, q, k, v, a, lg, state, y, timed, gen, nbytes):
    """decode_suite's slot-indexed and per-key-channel steps on its dense states."""
    import torch
    from gdnx_amd import ops
    dev = state.device
    NS, H, NC, D = state.shape[:4]
    n_in = q.shape[0]
    # the state pool addressed through shuffled slots
    perm = torch.randperm(NS, generator=torch.Generator().manual_seed(5)).to(torch.int32).to(dev)

    def step_slots(i):
        j = i % n_in
        ops.delta_decode_step_slots(q[j], k[j], v[j], a[j], a[j], lg[j], state, perm, out=y)

    sec = timed(step_slots, steps, 1)
    out["slots"] = {"kernel": "delta_decode_kernel (slot-indexed)", "ms_per_step": sec * 1e3,
                    "tokens_per_s": NS / sec, "hbm_frac": nbytes / sec / HBM_PEAK,
                    "note": "rows name shuffled slots of a 256-slot state pool"}
    # a log-decay per key channel (KMD-2's decay) on the same states
    lgc = (lg[..., None] + 0.001 * torch.randn(n_in, NS, H, NC, D, device=dev, generator=gen)).contiguous()

    def step_chan(i):
        j = i % n_in
        ops.delta_decode_step_chan(q[j], k[j], v[j], a[j], a[j], lgc[j], state, out=y)

    sec = timed(step_chan, steps, 1)
    nb = decode_bytes_chan(NS, H, NC, D)
    out["chan"] = {"kernel": "delta_decode_chan_kernel", "ms_per_step": sec * 1e3, "tokens_per_s": NS / sec,
                   "algorithmic_bytes": nb, "hbm_frac": nb / sec / HBM_PEAK}
    del lgc


def decode_suite(steps, warmup, extras=True, gdn3_step=None):
    """Config-4 decode measurements (HIP events on the launch stream): the
    dense step (gdnx_delta_decode_step) and, with extras, the same through
    shuffled state slots and the per-key-channel step; with gdn3_step (by
    default as extras) the GDN3 Kronecker-residual step at the same width
    (256 sequences x 16 heads x 16 chains).  Returns a dict of ms per step
    and HBM fractions of the algorithmic bytes."""
    if gdn3_step is None:
        gdn3_step = extras
    import torch
    import torch.nn.functional as F
    from gdnx_amd import gdn3, ops
    from gdnx_amd import workloads as inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    NS, H, M, NT, D = 256, 16, 4, 4, 128
    NC = M * NT
    gen = torch.Generator(device=dev).manual_seed(1004)
    state = torch.randn(NS, H, NC, D, D, device=dev, generator=gen) * 0.02
    n_in = 8  # distinct per-step inputs cycled through the timed steps
    q = F.normalize(torch.randn(n_in, NS, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(n_in, NS, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    v = torch.randn(n_in, NS, H, D, device=dev, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(n_in, NS, H, M, 1, device=dev, generator=gen))
    alpha_c = beta * (k.float() ** 2).sum(-1)[..., None, None]
    a = ((-torch.expm1(-alpha_c)) / alpha_c).mul(beta).expand(n_in, NS, H, M, NT).reshape(n_in, NS, H, NC).contiguous()
    base = torch.log1p(-torch.tensor(inputs.TAUS, device=dev)).repeat(M)
    lg = (base + 0.01 * torch.randn(n_in, NS, H, NC, device=dev, generator=gen)).contiguous()
    y = torch.empty(NS, H, NC, D, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream()

    def timed(fn, n, w):
        for i in range(w):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / n

    def step(i):
        j = i % n_in
        ops.delta_decode_step(q[j], k[j], v[j], a[j], a[j], lg[j], state, out=y)

    sec = timed(step, steps, warmup)
    nbytes = decode_bytes(NS, H, NC, D)
    out = {"dense": {"kernel": "delta_decode_kernel", "ms_per_step": sec * 1e3, "tokens_per_s": NS / sec,
                     "algorithmic_bytes": nbytes, "hbm_gbs": nbytes / sec / 1e9, "hbm_frac": nbytes / sec / HBM_PEAK,
                     "traffic": measured_traffic("delta_decode_kernel")}}
    if extras:
        decode_suite_extras(out, steps, q, k, v, a, lg, state, y, timed, gen, nbytes)
    if not gdn3_step:
        return out
    # the GDN3 Kronecker-residual step: 4 x (16x16 (x) 8x8) + a 16-slot window per chain
    del state
    torch.cuda.empty_cache()
    P = 16
    N = NS * H * NC
    g2 = torch.Generator(device=dev).manual_seed(1005)
    A = torch.randn(NS, H, NC, 4, 16, 16, device=dev, generator=g2) * \
        torch.tensor([0.4, 0.2, 0.1, 0.05], device=dev).view(4, 1, 1)
    Bk = torch.randn(NS, H, NC, 4, 8, 8, device=dev, generator=g2) * 0.5
    U = torch.randn(NS, H, NC, D, P, device=dev, generator=g2) * 0.02
    Vb = F.normalize(torch.randn(NS, H, NC, D, P, device=dev, generator=g2), dim=-2)
    g3 = (A, Bk, U, Vb)
    sk = torch.randn(N, 64, 8, device=dev, generator=g2) / 8.0
    bg = torch.sigmoid(torch.randn(n_in, NS, H, NC, device=dev, generator=g2))
    wg = torch.sigmoid(torch.randn(n_in, NS, H, NC, device=dev, generator=g2))
    dec = torch.exp(lg).clamp(max=1.0)

    def step_g3(pos):
        def run(i):
            j = i % n_in
            gdn3.gdn3_decode_step(q[j], k[j], v[j], bg[j], wg[j], dec[j], g3, pos(i), R=4, P=P,
                                  factors=(16, 16, 8, 8), compact_every=P, sketch=sk)
        return run

    # positions that close no interval, then whole intervals (15 plain steps and
    # the step after which every row compacts); int32 device tensors, built once
    n_int = 16 * max(1, steps // 16)
    pos_t = [torch.full((NS,), i, dtype=torch.int32, device=dev) for i in range(max(n_int, 16 * steps + 2))]
    with torch.no_grad():
        sec_plain = timed(step_g3(lambda i: pos_t[16 * i + 1]), steps, 1)
        sec_int = timed(step_g3(lambda i: pos_t[i]), n_int, 0)
    nb = gdn3_decode_bytes(N, NS, H, D, P)
    out["gdn3"] = {"kernel": "gdn3_decode_kernel", "ms_per_step": sec_plain * 1e3, "tokens_per_s": NS / sec_plain,
                   "algorithmic_bytes": nb, "hbm_frac": nb / sec_plain / HBM_PEAK,
                   "ms_per_step_with_compactions": sec_int * 1e3,
                   "note": "ms_per_step: steps that close no compaction interval; "
                           "ms_per_step_with_compactions: 16 consecutive positions, the last followed "
                           "by every row's compaction (gdn3_compact_kernel)"}
    return out


def bench_decode(args):
    """Config 4: batched one-token decode, 256 sequences x 16 heads x (4 lanes
    x 4 decays) chains of 128x128 fp32 state, bf16 q/k/v per step.  A step is
    one gdnx_delta_decode_step over all chains; value = sequences decoded per
    second (one token each).  The same line reports the slot-indexed step,
    the per-key-channel step and the GDN3 Kronecker-residual step at the
    same width."""
    NS, H, NC, D = 256, 16, 16, 128
    r = decode_suite(args.steps, args.warmup)
    d = r["dense"]
    line = {
        "metric": "GDN3 batched decode tokens/s @256 seq x 16 heads x 4 lanes x 4 decays, d=128",
        "value": d["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": d["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 4: batched one-token decode, 65,536 fp32 128x128 "
                               "states (4.29 GB), bf16 q/k/v per step",
                   "sequences": NS, "heads": H, "chains_per_head": NC, "head_dim": D,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": d["kernel"], "achieved": d["hbm_gbs"],
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": d["hbm_frac"],
                     "traffic": d["traffic"], "mean_us": d["ms_per_step"] * 1e3,
                     "algorithmic_bytes": d["algorithmic_bytes"]},
        "decode_cache": r["slots"],
        "decode_chan": r["chan"],
        "decode_gdn3": r["gdn3"],
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_decode()
    print(json.dumps(line), flush=True)


def cpu_baseline_gdn3(T=2048, B=1, H=16, M=4, compact_every=2048, train=False):
    """Time the CPU oracle's sequential GDN3 recurrence (fp32, all chains of
    the layer batched per token) on the first T tokens of the workload, with
    train its torch-autograd backward too."""
    import torch
    from oracle import gdn3 as og, inputs
    torch.set_num_threads(os.cpu_count() or 1)
    x = inputs.config3(T=T, B=B, H=H, M=M, span=min(4096, T), n_pairs=16)
    D = x["q"].shape[-1]

    def run():
        leaves = [x[n].float().requires_grad_(train) for n in ("q", "k", "v", "b", "w", "dec")]
        args = [t.unsqueeze(3).expand(B, T, H, M, D) for t in leaves[:3]]
        gates = [t.unsqueeze(-1).expand(B, T, H, M, D) for t in leaves[3:5]]
        y = og.gdn3_recurrence(*args, *gates, leaves[5], compact_every=compact_every, dtype=torch.float32,
                               sign_mode="canonical")
        if train:
            torch.autograd.grad(y, leaves, torch.ones_like(y))
    secs = median_time(run)
    return {
        "value": B * T / secs,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle.gdn3.gdn3_recurrence fp32{' fwd+bwd' if train else ''}, B={B} T={T} H={H}x{M} "
                  f"lanes d={D}, compaction every {compact_every}, one warm-up then median of 3 ({secs:.1f} s)",
    }


def bench_gdn3(args, layer_default, train=False):
    """GDN3 Kronecker-residual regime.  longctx: config 3 (B=1, T=32768,
    H=16, 4 lanes, compaction every 2048 tokens).  gdn3-layer: the reference
    layer's default regime (compaction every P=16 tokens) at config 1 width
    (B=4, T=4096, H=16, 4 lanes).  One step = one gdn3_recurrent_state call
    (forward), or with train forward + gradients of q, k, v, both gates and
    the decay against a fixed upstream gradient (gdn3-layer-train)."""
    import torch
    from gdnx_amd import gdn3
    from gdnx_amd import workloads as inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if layer_default:
        B, T, Kc = 4, 4096, 16
        x = inputs.config3(T=T, B=B, n_pairs=64, span=T)
    else:
        B, T, Kc = 1, 32768, 2048
        x = inputs.config3()
    _, _, H, D = x["q"].shape
    M = x["b"].shape[-1]
    q, k, v, bg, wg, dec = (x[n].to(dev).contiguous() for n in ("q", "k", "v", "b", "w", "dec"))
    stream = torch.cuda.current_stream()
    leaves = (q, k, v, bg, wg, dec)
    if train:
        for t in leaves:
            t.requires_grad_(True)
        dy = torch.randn(B, T, H, M, D, generator=torch.Generator().manual_seed(7)).to(q.dtype).to(dev)

    def step():
        if train:
            out = gdn3.gdn3_recurrent_state(q, k, v, bg, wg, dec, compact_every=Kc)
            return torch.autograd.grad(out, leaves, dy)[0]
        return gdn3.gdn3_recurrent_state(q, k, v, bg, wg, dec, compact_every=Kc)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        y = step()
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / args.steps
    # algorithmic bytes: q, k, v (bf16, shared by lanes), b, w, decay (fp32 per lane), y (bf16);
    # the backward reads them and dy again and writes the same-sized gradients
    nbytes = 3 * B * T * H * D * 2 + 3 * B * T * H * M * 4 + B * T * H * M * D * 2
    if train:
        nbytes *= 3
    achieved = nbytes / sec / 1e9
    # the layer default runs one persistent workgroup per chain for the window steps and
    # their compactions; config 3 a pipelined window launch and a compaction launch per interval
    name = ("gdn3_fused_kernel" if layer_default else "gdn3_window_pipe_kernel+gdn3_compact_kernel") + \
        ("+gdn3_bwd_kernel" if train else "")
    if train:
        metric = "GDN3 Kronecker-residual layer tokens/s fwd+bwd @B=4,T=4096, compaction every 16"
    elif layer_default:
        metric = "GDN3 Kronecker-residual layer tokens/s fwd @B=4,T=4096, compaction every 16"
    else:
        metric = "GDN3 long-context tokens/s fwd @B=1,T=32768, compaction every 2048"
    line = {
        "metric": metric,
        "value": B * T / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": ("GDN3 layer default regime (K_c = P = 16) at config 1 width"
                                + (", forward + backward" if train else "")
                                if layer_default else "BASELINE config 3: long context with compaction"),
                   "batch": B, "seq_len": T, "heads": H, "lanes": M, "head_dim": D, "kron": "4 x (16x16 (x) 8x8)",
                   "window": 16, "compact_every": Kc, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": name, "achieved": achieved, "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": achieved * 1e9 / HBM_PEAK, "traffic": measured_traffic(name),
                     "mean_us": sec * 1e6, "algorithmic_bytes": nbytes,
                     "note": "one workgroup per chain walks the windows in order: latency-bound"},
        "finite": bool(torch.isfinite(y.float()).all()),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_gdn3(T=256 if train else (512 if layer_default else 2048), B=B,
                                                 compact_every=Kc, train=train)
    print(json.dumps(line), flush=True)


def gdn3_layer_train_ms(steps=3, warmup=1):
    """The GDN3 layer's default regime (compaction every P = 16 tokens) at
    config-1 width (B=4, T=4096, H=16, 4 lanes, d=128): ms of one
    gdn3_recurrent_state forward + backward (gradients of q, k, v, both gates
    and the decay against a fixed upstream gradient)."""
    import torch
    from gdnx_amd import gdn3
    from gdnx_amd import workloads as inputs
    dev = torch.device("cuda:0")
    x = inputs.config3(T=4096, B=4, n_pairs=64, span=4096)
    leaves = tuple(x[n].to(dev).contiguous().requires_grad_(True) for n in ("q", "k", "v", "b", "w", "dec"))
    B, T, H, D = x["q"].shape
    M = x["b"].shape[-1]
    dy = torch.randn(B, T, H, M, D, generator=torch.Generator().manual_seed(7)).to(leaves[0].dtype).to(dev)
    stream = torch.cuda.current_stream()

    def step():
        out = gdn3.gdn3_recurrent_state(*leaves, compact_every=16)
        return torch.autograd.grad(out, leaves, dy)[0]
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


MFMA_FP32_PEAK = 157.3e12   # dense fp32 FLOP/s


def kmd2_inputs(B, T, H, r_out, d, seed=7):
    """The reference's scan-benchmark distribution (research/kernel_ab/
    bench_scan.py:39-55): q ~ N(0, 1/d), unit keys, per-channel decay
    exp(-softplus(1.2 z - 0.6)) spanning (0, 1), sigmoid gates, out_mix ~ N(0, 1)."""
    import torch
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, r_out, d, generator=g) * d ** -0.5
    k = F.normalize(torch.randn(B, T, H, d, generator=g), dim=-1)
    v = torch.randn(B, T, H, d, generator=g)
    dec = torch.exp(-F.softplus(torch.randn(B, T, H, d, generator=g) * 1.2 - 0.6))
    be = torch.sigmoid(torch.randn(B, T, H, generator=g))
    bw = torch.sigmoid(torch.randn(B, T, H, generator=g))
    mix = torch.randn(H, r_out, generator=g)
    dy = torch.randn(B, T, H, d, generator=g)
    return (q, k, v, dec, be, bw, mix), dy


def flops_chan(B, T, H, D, C=16):
    """Algorithmic FLOP of the per-channel forward per (b, h, chunk): the two
    exact decay-weighted grams 4 C^2 D, Wm and U 4 C^2 D, Wm S0 / Q S0 / the
    carry 6 C D^2, the masked output product 2 C^2 D and the inverse C^3/3;
    forward + backward = 3x."""
    nchunks = B * H * ((T + C - 1) // C)
    return nchunks * (10 * C * C * D + 6 * C * D * D + C ** 3 / 3)


def cpu_baseline_kmd2(T=512, B=1, H=16, H_full=16, r_out=4, d=128):
    """The CPU oracle (fp32 token loop + autograd) on B x T tokens of H heads;
    tokens/s scaled to the benchmark's 16 heads."""
    import torch
    from oracle import delta
    torch.set_num_threads(os.cpu_count() or 1)
    xs, dy = kmd2_inputs(B, T, H, r_out, d)

    def run():
        leaves = [x.detach().requires_grad_(True) for x in xs]
        y = delta.kmd2_scan(*leaves, dtype=torch.float32)
        torch.autograd.grad(y, leaves, dy)
    secs = median_time(run)
    return {"value": B * T / secs * H / H_full, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"oracle.delta.kmd2_scan fp32 fwd+bwd, B={B} T={T} H={H} r_out={r_out} d={d} "
                      f"(one warm-up then median of 3: {secs:.1f} s), scaled to H={H_full}"}


def bench_kmd2(args):
    """KMD-2 native scan with per-channel decay, the reference's kernel-search
    benchmark (research/kernel_ab/bench_scan.py:26-29): primary metric
    forward+backward tokens/s at the train shape B=2, T=512, H=16, r_out=4,
    dk=dv=128, float32; also the eval shape's forward (B=1, T=2048).  One step
    = kmd2.scan forward + gradients of all seven inputs."""
    import torch
    from gdnx_amd import kmd2, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, T, H, R, D = 2, 512, 16, 4, 128
    xs, dy = kmd2_inputs(B, T, H, R, D)
    leaves = [x.to(dev).requires_grad_(True) for x in xs]
    dy = dy.to(dev)
    stream = torch.cuda.current_stream()

    def step():
        y = kmd2.scan(*leaves)
        return torch.autograd.grad(y, leaves, dy)

    def timed(fn, n):
        for _ in range(max(1, args.warmup)):
            fn()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(n):
            out = fn()
        s1.record(stream)
        torch.cuda.synchronize()
        return s0.elapsed_time(s1) * 1e-3 / n, out

    sec, grads = timed(step, args.steps)
    finite = all(bool(torch.isfinite(t).all()) for t in grads)
    # eval shape, forward only
    xe, _ = kmd2_inputs(1, 2048, H, R, D, seed=8)
    xe = [x.to(dev) for x in xe]
    with torch.no_grad():
        sec_eval, _ = timed(lambda: kmd2.scan(*xe), args.steps)

    # per-kernel means at the train shape
    with torch.no_grad():
        q = kmd2._mixed_query(leaves[0].detach(), leaves[6].detach()).contiguous()
        k, v = leaves[1].detach(), leaves[2].detach()
        lg = torch.log(leaves[3].detach().clamp(min=1e-30))
        be, bw = leaves[4].detach(), leaves[5].detach()
        st = {}

        def fwd():
            st["y"], _, st["cs"] = ops.delta_chan_fwd(q, k, v, be, bw, lg, save_states=True)
        t_fwd, _ = timed(fwd, args.kernel_iters)
        t_bwd, _ = timed(lambda: ops.delta_chan_bwd(q, k, v, be, bw, lg, dy, st["cs"]), args.kernel_iters)
    f_fwd = flops_chan(B, T, H, D)
    kernels = {"chan_prep_kernel+chan_scan_fwd_kernel": (t_fwd, f_fwd),
               "chan_scan_bwd_kernel+chan_grads_kernel": (t_bwd, 2 * f_fwd)}
    dom = max(kernels, key=lambda n: kernels[n][0])
    t_dom, f_dom = kernels[dom]
    achieved = f_dom / t_dom / 1e12
    line = {
        "metric": "KMD-2 scan tokens/s fwd+bwd @B=2,T=512 (per-channel decay)",
        "value": B * T / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "reference scan benchmark, train shape: B=2 T=512 H=16 r_out=4 dk=dv=128, "
                               "per-channel decay exp(-softplus(1.2 z - 0.6))",
                   "batch": B, "seq_len": T, "heads": H, "r_out": R, "head_dim": D, "chunk": 16,
                   "parallelism": "single GPU"},
        "eval_fwd_tokens_per_s": 2048 / sec_eval,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": MFMA_FP32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": achieved * 1e12 / MFMA_FP32_PEAK,
                     "traffic": measured_traffic(dom), "mean_us": t_dom * 1e6, "algorithmic_flop": f_dom,
                     "note": "32 chains of 32 chunks: the sequential scans are latency-bound"},
        "kernels_us": {n: round(t * 1e6, 2) for n, (t, _) in kernels.items()},
        "grads_finite": finite,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_kmd2()
    print(json.dumps(line), flush=True)


def boundary_bytes(B, T, H, M, K, V, io=2):
    """Algorithmic HBM bytes per launch of the four boundary kernels: every
    input read once and every output written once (per (b, t, h) row), plus
    the RoPE tables (read once per launch: 2 M T K/2 float32) and norm."""
    rows = B * T * H
    f = 4
    tables = 2 * M * T * (K // 2) * f
    pro_f = rows * ((2 * K + M * K + M * V + 2 + 4 * M) * io + 2 * M * K * io + (M * K + M * V + M) * f) + tables
    pro_b = rows * ((M * K + M * V + 2 + 4 * M) * io + (2 * M * K + M * K + M * V + M) * f
                    + (2 * K + M * K + M * V + 2 + 4 * M) * f) + tables
    epi_f = rows * ((M * V + M) * io + V * io) + V * f
    epi_b = rows * ((M * V + M + V) * io + M * V * io + M * f) + V * f
    return {"g3_prologue_fwd_kernel": pro_f, "g3_prologue_bwd_kernel": pro_b,
            "g3_epilogue_fwd_kernel": epi_f, "g3_epilogue_bwd_kernel": epi_b}


def boundary_inputs(B, T, H, M, K, V, seed=31):
    import torch
    g = torch.Generator().manual_seed(seed)
    xs = {"q": torch.randn(B, T, H, K, generator=g), "k": torch.randn(B, T, H, K, generator=g),
          "b_proj": torch.randn(B, T, H, M, K, generator=g), "proj_a": torch.randn(B, T, H, generator=g),
          "w_proj": torch.randn(B, T, H, M, V, generator=g), "proj_b": torch.randn(B, T, H, generator=g),
          "decay_proj": torch.randn(B, T, H, M, 4, generator=g) * 3,
          "y": torch.randn(B, T, H, M, V, generator=g), "router_logits": torch.randn(B, T, H, M, generator=g),
          "norm": 0.5 + torch.rand(V, generator=g), "d_out": torch.randn(B, T, H, V, generator=g)}
    return xs


def cpu_baseline_boundary(T=4096, B=2, H=16, M=4, K=128, V=128):
    """The float64 oracle (oracle/gdn3_layer.py, torch autograd, float64 as
    it is written) on B=2, T=4096, H=16 -- half of the 262144 rows -- forward
    and backward of prologue and epilogue, scaled to tokens/s."""
    import torch
    from oracle import gdn3_layer as gl
    torch.set_num_threads(os.cpu_count() or 1)
    xs = boundary_inputs(B, T, H, M, K, V, seed=32)
    rates = torch.tensor([0.05, 0.02, 0.005, 0.001])
    names = ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj")

    def run():
        leaves = [xs[n].double().requires_grad_(True) for n in names]
        outs = gl.prologue(*leaves, rates, 0.999)
        torch.autograd.grad(outs, leaves, [torch.ones_like(o) for o in outs])
        el = [xs[n].double().requires_grad_(True) for n in ("y", "router_logits", "norm")]
        out = gl.epilogue(*el)
        torch.autograd.grad(out, el, xs["d_out"].double())
    sec = median_time(run)
    return {"value": B * T / sec, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle prologue+epilogue fwd+bwd, float64 autograd, B={B} T={T} H={H} M={M} K=V={K} "
                      f"({B * T * H} rows), one warm-up then median of 3: {sec:.2f} s"}


def torch_eager_boundary(xs, rates, clamp, K, V):
    """A torch-eager restatement (this repository's code) of the reference's
    element-wise boundary ops (gdn3/gdn3_upgrade.py:796-851, with
    _apply_partial_rope's clone and in-place slices) on the GPU, forward +
    backward: the op sequence the fused kernels replace, timed as a comparator."""
    import math
    import torch
    import torch.nn.functional as F
    from gdnx_amd import layer
    q, k, bp, pa, wp, pb, dp = (xs[n] for n in ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj"))
    B, T, H, M, _ = bp.shape
    cos, sin = layer.lane_rope_tables(M, T, K, q.device)
    pairs = layer.ops.gdn3_lane_rope_pairs(M, K)

    def rope(x):
        res = x.unsqueeze(3).expand(B, T, H, M, K).clone()
        for m, d in enumerate(pairs):
            if d == 0:
                continue
            lane = res[:, :, :, m, :]
            c = cos[m, :, :d].view(1, T, 1, d)
            s = sin[m, :, :d].view(1, T, 1, d)
            x1, x2 = lane[..., :d], lane[..., d:2 * d]
            lane[..., :d] = x1 * c - x2 * s
            lane[..., d:2 * d] = x1 * s + x2 * c
            res[:, :, :, m, :] = lane
        return res
    bg = torch.sigmoid(bp + pa.unsqueeze(3).unsqueeze(4) * 0.1)
    wg = torch.sigmoid(wp + pb.unsqueeze(3).unsqueeze(4) * 0.1)
    dec = torch.exp(-F.softplus(dp).clamp(max=5.0) * rates).mean(-1).clamp(max=clamp)
    outs = (rope(q), rope(k), bg, wg, dec)
    y, lg, nm = xs["y"], xs["router_logits"], xs["norm"]
    w = F.softmax(lg, dim=-1)
    routed = (w.unsqueeze(-1) * y).sum(dim=3)
    out = F.normalize(routed, p=2, dim=-1, eps=1e-6) * math.sqrt(V) * nm
    leaves = [xs[n] for n in ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj", "y",
                              "router_logits", "norm")]
    return torch.autograd.grad(list(outs) + [out], leaves, [torch.ones_like(o) for o in outs] + [xs["d_out"]])


def bench_boundary(args):
    """Fused GDN3 layer boundary (gdnx_gdn3_prologue_* / _epilogue_*) at the
    layer shape of config 1: B=4, T=4096, H=16, M=4, K=V=128, bf16 IO.  One
    step = prologue forward + epilogue forward + epilogue backward + prologue
    backward on resident inputs; all four kernels are HBM-bound."""
    import torch
    from gdnx_amd import layer, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, T, H, M, K, V = 4, 4096, 16, 4, 128, 128
    io = torch.bfloat16
    xs = {n: t.to(dev) for n, t in boundary_inputs(B, T, H, M, K, V).items()}
    for n in ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj", "y", "router_logits", "d_out"):
        xs[n] = xs[n].to(io).contiguous()
    rates = torch.tensor([0.05, 0.02, 0.005, 0.001], device=dev)
    cos, sin = layer.lane_rope_tables(M, T, K, dev)
    pro_in = [xs[n] for n in ("q", "k", "b_proj", "proj_a", "w_proj", "proj_b", "decay_proj")]
    go = [torch.randn(B, T, H, M, K, device=dev), torch.randn(B, T, H, M, K, device=dev),
          torch.randn(B, T, H, M, K, device=dev), torch.randn(B, T, H, M, V, device=dev),
          torch.randn(B, T, H, M, device=dev)]
    stream = torch.cuda.current_stream()
    calls = {
        "g3_prologue_fwd_kernel": lambda: ops.gdn3_prologue_fwd(*pro_in, rates, cos, sin, 0.999),
        "g3_epilogue_fwd_kernel": lambda: ops.gdn3_epilogue_fwd(xs["y"], xs["router_logits"], xs["norm"]),
        "g3_epilogue_bwd_kernel": lambda: ops.gdn3_epilogue_bwd(xs["y"], xs["router_logits"], xs["norm"],
                                                                xs["d_out"]),
        "g3_prologue_bwd_kernel": lambda: ops.gdn3_prologue_bwd(*pro_in[2:], rates, cos, sin, *go, 0.999),
    }

    def timed(fn, n):
        for _ in range(max(1, args.warmup)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / n

    def step():
        for fn in calls.values():
            fn()
    sec = timed(step, args.steps)
    per = {n: timed(fn, args.kernel_iters) for n, fn in calls.items()}
    nbytes = boundary_bytes(B, T, H, M, K, V)
    dom = max(per, key=per.get)
    achieved = nbytes[dom] / per[dom] / 1e9
    # the same work as torch eager ops (the reference's path), for context
    ex = {n: (t.detach().requires_grad_(True) if n != "d_out" else t) for n, t in xs.items()}
    eager = timed(lambda: torch_eager_boundary(ex, rates, 0.999, K, V), max(2, args.steps // 4))
    line = {
        "metric": "GDN3 layer boundary pre/post-ops tokens/s fwd+bwd @B=4,T=4096,H=16,M=4",
        "value": B * T / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "GDN3LinearAttn.forward lines 796-851 around the recurrence: gates, braided "
                               "decay, lane RoPE, routing + head norm; forward and backward",
                   "batch": B, "seq_len": T, "heads": H, "lanes": M, "key_dim": K, "value_dim": V,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved * 1e9 / HBM_PEAK, "traffic": measured_traffic(dom),
                     "mean_us": per[dom] * 1e6, "algorithmic_bytes": nbytes[dom]},
        "kernels": {n: {"us": round(per[n] * 1e6, 2), "GB/s": round(nbytes[n] / per[n] / 1e9, 1)} for n in per},
        "torch_eager_ms_per_step": eager * 1e3,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_boundary()
    print(json.dumps(line), flush=True)


def rls_inputs(B, T, H, r, r_out, dk, dv, seed=41):
    import torch
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, r_out, dk, generator=g), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, T, H, r, dk, generator=g), dim=-1)
    V = torch.randn(B, T, H, r, dv, generator=g)
    Bg = torch.sigmoid(torch.randn(B, T, H, r, dk, generator=g))
    Wg = torch.sigmoid(torch.randn(B, T, H, r, dv, generator=g))
    a = torch.sigmoid(torch.randn(B, T, H, dk, generator=g) * 0.5 + 6.0).clamp(max=0.999)
    dy = torch.randn(B, T, H, dv, generator=g)
    return [q, K, V, Bg, Wg, a], dy


def flops_rls(B, T, H, r, r_out, dk, dv):
    """Algorithmic FLOP of one forward: per token and chain, decay dv dk,
    S Kt^T 2 r dv dk, erase + write 4 r dv dk, reads 2 r_out dv dk, plus the
    T-factor (2 r^2 dk + r^3)."""
    per = dv * dk * (1 + 2 * r + 4 * r + 2 * r_out) + 2 * r * r * dk + r ** 3
    return B * T * H * per


def cpu_baseline_rls(T=1024, B=1, H=16, r=1, r_out=1, dk=64, dv=64):
    """The float64 oracle (oracle/rls.py, per-token torch loop with autograd)
    on B=1, T=1024, H=16 -- 1/8 of the workload's tokens -- forward and
    backward, scaled to tokens/s."""
    import torch
    from oracle import rls as orls
    torch.set_num_threads(os.cpu_count() or 1)
    xs, dy = rls_inputs(B, T, H, r, r_out, dk, dv, seed=42)

    def run():
        leaves = [x.double().requires_grad_(True) for x in xs]
        y = orls.rls_scan(*leaves)
        torch.autograd.grad(y, leaves, dy.double())
    sec = median_time(run)
    return {"value": B * T / sec, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle rls_scan fwd+bwd, float64 autograd, B={B} T={T} H={H} r={r} dk=dv={dk}, one warm-up then median of 3: {sec:.2f} s"}


def torch_eager_rls(xs, eps):
    """A torch-eager restatement (this repository's code) of the reference's
    per-token loop (KMD2LinearAttn._scan's r = 1 path, gdn3/kmd2.py:193-200)
    on the GPU, forward + backward, timed as a comparator."""
    import torch
    q, K, V, Bg, Wg, a = xs
    B, T, H, _, dk = q.shape
    dv = V.shape[-1]
    N = B * H

    def flat(x, *tail):
        return x.permute(1, 0, 2, *range(3, x.dim())).reshape(T, N, *tail)
    q_, K_, V_, Bg_, Wg_, a_ = flat(q, dk), flat(K, dk), flat(V, dv), flat(Bg, dk), flat(Wg, dv), flat(a, dk)
    S = torch.zeros(N, dv, dk, device=q.device)
    outs = []
    for t in range(T):
        S = S * a_[t].unsqueeze(1)
        ktil = Bg_[t] * K_[t]
        Sk = torch.bmm(S, ktil.unsqueeze(2)).squeeze(2)
        denom = eps + ktil.square().sum(-1, keepdim=True)
        S = S - torch.bmm((Sk / denom).unsqueeze(2), ktil.unsqueeze(1))
        S = S + torch.bmm((Wg_[t] * V_[t]).unsqueeze(2), K_[t].unsqueeze(1))
        outs.append(torch.bmm(S, q_[t].unsqueeze(2)).squeeze(2))
    Y = torch.stack(outs, 0)
    return torch.autograd.grad(Y.sum(), xs)


def bench_rls(args):
    """Rank-r RLS T-factor scan (KMD2LinearAttn._scan, gdn3/kmd2.py:166-214) at
    the reference layer's defaults (H=16, dk=dv=64, r=1, r_out=1, eps 0.5) on
    B=8 sequences of T=1024: one step = rls_scan forward + gradients of all
    six inputs, float32."""
    import torch
    from gdnx_amd import rls

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, T, H, r, ro, dk, dv = 8, 1024, 16, 1, 1, 64, 64
    xs, dy = rls_inputs(B, T, H, r, ro, dk, dv)
    leaves = [x.to(dev).requires_grad_(True) for x in xs]
    dy = dy.to(dev)
    stream = torch.cuda.current_stream()

    def timed(fn, n):
        for _ in range(max(1, args.warmup)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / n

    def step():
        y = rls.rls_scan(*leaves)
        return torch.autograd.grad(y, leaves, dy)
    sec = timed(step, args.steps)
    flat = [x.detach().contiguous() for x in xs]
    flat = [t.to(dev) for t in flat]
    with torch.no_grad():
        t_fwd = timed(lambda: rls.rls_fwd(*flat, checkpoint=True), args.kernel_iters)
    f = flops_rls(B, T, H, r, ro, dk, dv)
    t_bwd = max(sec - t_fwd, 1e-9)
    kernels = {"rls_fwd_rb_kernel": (t_fwd, f), "rls_bwd_rb_kernel+rls_bwd_reduce_kernel": (t_bwd, 3 * f)}
    dom = max(kernels, key=lambda n: kernels[n][0])
    achieved = kernels[dom][1] / kernels[dom][0] / 1e12
    # the testbed mixer's shape with its SVD compaction (research/testbed_mqar.py:75-78 defaults
    # H=4, dk=dv=32, r=4; compaction every 32 tokens to rank 8)
    xt, dyt = rls_inputs(16, 512, 4, 4, 1, 32, 32, seed=43)
    lt = [x.to(dev).requires_grad_(True) for x in xt]
    dyt = dyt.to(dev)

    def step_tb():
        y = rls.rls_scan(*lt, compact_P=32, compact_R=8)
        return torch.autograd.grad(y, lt, dyt)
    sec_tb = timed(step_tb, args.steps)
    ex = [x.to(dev).requires_grad_(True) for x in xs]
    Te = 256   # the eager loop is launch-bound: time a prefix and scale
    exs = [x[:, :Te].detach().clone().requires_grad_(True) for x in ex]
    eager = timed(lambda: torch_eager_rls(exs, 0.5), 2) * T / Te
    line = {
        "metric": "RLS T-factor scan tokens/s fwd+bwd @B=8,T=1024,H=16,dk=dv=64,r=1",
        "value": B * T / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "KMD2LinearAttn._scan (rank-r block-Householder delta, RLS T-factor), reference "
                               "layer defaults", "batch": B, "seq_len": T, "heads": H, "slots": r, "r_out": ro,
                   "key_dim": dk, "value_dim": dv, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": MFMA_FP32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": achieved * 1e12 / MFMA_FP32_PEAK, "traffic": measured_traffic(dom),
                     "mean_us": kernels[dom][0] * 1e6, "algorithmic_flop": kernels[dom][1],
                     "note": "sequential per-token recurrence: latency-bound (16 value rows per workgroup, "
                             "dv/16 workgroups per chain, 128 chains); the backward's time is the step minus "
                             "the forward"},
        "kernels_us": {n: round(t * 1e6, 2) for n, (t, _) in kernels.items()},
        "torch_eager_ms_per_step": eager * 1e3,
        "testbed_compaction": {"shape": "B=16 T=512 H=4 r=4 dk=dv=32, SVD compaction every 32 tokens to rank 8",
                               "tokens_per_s": 16 * 512 / sec_tb, "ms_per_step": sec_tb * 1e3},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_rls()
    print(json.dumps(line), flush=True)


def bench_copy(args):
    """Calibration for the HBM traffic counters: a plain device copy of a
    known size (1 GiB read + 1 GiB written per launch).  Prints its own JSON
    line; the FETCH_SIZE / WRITE_SIZE counters of this launch divided by
    2^30 bytes give the factor that converts the counters' units to bytes."""
    import torch
    dev = torch.device("cuda:0")
    n = 1 << 28
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / args.steps
    print(json.dumps({"metric": "device copy GB/s (traffic-counter calibration)",
                      "value": 2 * n * 4 / sec / 1e9, "unit": "GB/s", "bytes_read": n * 4,
                      "bytes_written": n * 4, "steps": args.steps}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=10)
    ap.add_argument("--workload", choices=("train", "decode", "longctx", "gdn3-layer", "gdn3-layer-train", "kmd2",
                                               "gdn3-boundary", "rls", "copy"),
                    default="train",
                    help="train: config 2 scan fwd+bwd (headline); decode: config 4 decode step; "
                         "longctx: config 3 GDN3 with compaction; gdn3-layer: GDN3 compaction every "
                         "16 tokens; gdn3-layer-train: the same forward + backward; kmd2: KMD-2 scan with per-channel decay fwd+bwd (reference scan "
                         "benchmark, train shape); gdn3-boundary: the layer's fused pre-/post-ops fwd+bwd; rls: the rank-r RLS T-factor scan fwd+bwd; copy: 1 GiB device copy used to calibrate the HBM traffic counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the recurrence shards by chains with no "
              "communication (see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.workload == "decode":
        return bench_decode(args)
    if args.workload == "copy":
        return bench_copy(args)
    if args.workload == "kmd2":
        return bench_kmd2(args)
    if args.workload == "gdn3-boundary":
        return bench_boundary(args)
    if args.workload == "rls":
        return bench_rls(args)
    if args.workload in ("longctx", "gdn3-layer", "gdn3-layer-train"):
        return bench_gdn3(args, layer_default=args.workload != "longctx", train=args.workload == "gdn3-layer-train")

    import torch
    from gdnx_amd import gdn3, ops
    from gdnx_amd import workloads as inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, T, H, D, M = 4, 4096, 16, 128, 4
    x = inputs.config2()
    q, k, v = (x[n].to(dev).contiguous() for n in ("q", "k", "v"))
    beta = x["beta"].to(dev).requires_grad_(True)
    g = x["g"].to(dev).requires_grad_(True)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    dO = x["dO"].to(dev)
    params = [q, k, v, beta, g]

    def step():
        y = gdn3.gdn3_scan(q, k, v, beta, g)
        return torch.autograd.grad(y, params, grad_outputs=dO)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        grads = step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    finite = all(bool(torch.isfinite(t.float()).all()) for t in grads)

    # ---- per-kernel mean durations (events on the launch stream) ----
    C = ops.chunk_size(D, q.dtype, train=True)
    with torch.no_grad():
        a = gdn3.gdn3_coeff(k, beta.detach())
        lg = g.detach().contiguous()
        qd, kd, vd = q.detach(), k.detach(), v.detach()
        stream = torch.cuda.current_stream()

        def timed(fn, n):
            fn()
            s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s0.record(stream)
            for _ in range(n):
                fn()
            s1.record(stream)
            torch.cuda.synchronize()
            return s0.elapsed_time(s1) / n * 1e-3

        state = {}

        def run_fwd():
            _, _, state["cs"] = ops.delta_chunk_fwd(qd, kd, vd, a, a, lg, save_states=True, chunk=C)
        t_fwd = timed(run_fwd, args.kernel_iters)
        ws, out = ops.delta_chunk_bwd_stages(qd, kd, vd, a, a, lg, dO, state["cs"], C)
        t_bst = timed(lambda: ops.delta_chunk_bwd_stages(qd, kd, vd, a, a, lg, dO, state["cs"], C,
                                                         ws=ws, out=out), args.kernel_iters)
        t_bgr = timed(lambda: ops.delta_chunk_bwd_grads(qd, kd, vd, a, a, lg, dO, state["cs"], ws, C, out),
                      args.kernel_iters)
        pws = ops.delta_chunk_prep(qd, kd, a, a, lg, chunk=C)
        t_prep = timed(lambda: ops.delta_chunk_prep(qd, kd, a, a, lg, chunk=C, ws=pws), args.kernel_iters)
        # the config-1 forward (inference, no stash) on the same inputs: the default path
        # (two-pass at the training chunk for bf16) and the fused single-kernel scan at 64
        bd = beta.detach()
        t_c1 = timed(lambda: gdn3.gdn3_scan(qd, kd, vd, bd, lg), args.kernel_iters)
        t_c1_fused = timed(lambda: ops.delta_chunk_fwd(qd, kd, vd, a, a, lg, chunk=64, two_pass=False),
                           args.kernel_iters)
    kernels = {
        "delta_prep_kernel+delta_scan_fwd_kernel": (t_fwd, flops_fwd(B, T, H, M, D, C)),
        "delta_scan_bwd_kernel": (t_bst, flops_bwd_state(B, T, H, M, D, C)),
        "delta_grad_seg_kernel": (t_bgr, flops_bwd_grads(B, T, H, M, D, C)),
    }
    dom = max(kernels, key=lambda n: kernels[n][0])
    t_dom, f_dom = kernels[dom]
    achieved = f_dom / t_dom / 1e12
    traffic = measured_traffic(dom)

    line = {
        "metric": "GDN3 scan tokens/s fwd+bwd @B=4,T=4096 bf16",
        "value": B * T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: GDN3 layer recurrence fwd+bwd, B=4 T=4096 H=16 "
                               "d=128, 4 lanes, bf16 IO, fp32 state",
                   "global_batch": B, "seq_len": T, "heads": H, "head_dim": D, "lanes": M,
                   "chunk": C, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved,
                     "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": achieved * 1e12 / MFMA_BF16_PEAK, "traffic": traffic,
                     "mean_us": t_dom * 1e6, "algorithmic_flop": f_dom},
        "roofline_intra_chunk": intra_chunk_entry(t_prep, flops_prep(B, T, H, M, D, C), t_c1_fused,
                                                  flops_fwd(B, T, H, M, D, 64)),
        "kernels_us": {n: round(t * 1e6, 2) for n, (t, _) in kernels.items()},
        "grads_finite": finite,
        "config1_fwd_ms": t_c1 * 1e3,
        "config1_fwd_fused_c64_ms": t_c1_fused * 1e3,
    }
    # config 4 decode (the dense step) and the layer-default GDN3 regime, timed here so
    # the headline run carries them
    decs = decode_suite(steps=20, warmup=3, extras=False, gdn3_step=True)
    line["decode_ms_per_step"] = decs["dense"]["ms_per_step"]
    line["decode_hbm_frac"] = decs["dense"]["hbm_frac"]
    line["decode_gdn3_ms_per_step"] = decs["gdn3"]["ms_per_step"]
    line["decode_gdn3_hbm_frac"] = decs["gdn3"]["hbm_frac"]
    line["gdn3_layer_fwd_bwd_ms"] = gdn3_layer_train_ms()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

// Lean sequential scans of the chunked delta rule (gfx950), fed by the
// parallel per-chunk operands of delta_prep.hip.
//
// Per chain (b, h, m) and chunk of C tokens (T, Aq, gam, dec, aeg, a_w from
// the prep record; see delta_prep.hip):
//   forward   U  = T diag(a_w) V,  Wm = T diag(aeg) K
//             R  = U - Wm S0                                 (net writes)
//             Y  = diag(gam) Q S0 + Aq R
//             S  = gam_last S0 + K^T diag(dec) R
//   backward  dR = diag(dec) K dS + Aq^T dY,   dB = T^T dR
//             dS0 = gam_last dS + Q^T diag(gam) dY - K^T diag(aeg) dB
// (gdn3/_reference_recurrence.py:60-84 in the dense regime and
// research/kernel_ab/ref_scan.py:40-45, restated per chunk).  Every product
// above is independent across value columns given the prep operands, so a
// chain's value columns are split over NVB workgroups of NWV waves, each wave
// owning 16 columns of the fp32 state in registers.  With 256 chains this
// puts several independent workgroups on every CU, which hide each other's
// MFMA, LDS and memory latency; the only per-chunk critical path left is
// the two dependent products R -> S (dR -> dS backward).
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C, int NWV>
struct ScanDims {
  typedef typename FragT<CT>::type Frag;
  static constexpr int KS = FragT<CT>::KSTEP;
  static constexpr int TPS = FragT<CT>::TPS;
  static constexpr int NT = 64 * NWV;       // threads per workgroup
  static constexpr int BV = 16 * NWV;       // value columns per workgroup
  static constexpr int NVB = D / BV;        // workgroups per chain
  static constexpr int NDT = D / 16;
  static constexpr int NCT = C / 16;
  static constexpr int LDD = D + 4;
  static constexpr int LDC = C + 4;
  static constexpr int DTW = NDT / NWV;     // key tiles of -Wm formed per wave
  static_assert(NDT % NWV == 0 && D % BV == 0, "value split must tile the head dim");
  static_assert(C % KS == 0, "chunk must be a multiple of the MFMA k-step");
};

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Staging is double-buffered by chunk parity: chunk c + 1's tiles are
// committed into the other buffer while chunk c computes, so a chunk step
// needs one workgroup barrier.  The net writes are formed per wave as
//   R = T (diag(a_w) V - diag(aeg) (K S0))
// on the wave's own value columns (K S0 contracts over the keys, which the
// wave's state columns hold whole), so no product is shared between waves.
template <typename CT, int D, int C, int NWV>
struct alignas(16) ScanFwdBuf {
  typedef ScanDims<CT, D, C, NWV> Sd;
  CT q[C * Sd::LDD];        // Q rows
  CT k[C * Sd::LDD];        // K rows
  CT kt[D * Sd::LDC];       // K^T
  CT vt[Sd::BV * Sd::LDC];  // V^T of this workgroup's value columns
  CT t[C * Sd::LDC];        // T rows
  CT aq[C * Sd::LDC];       // Aq rows
  float sc[kNumSc * C];     // gam, dec, aeg, a_w
};
// two staging buffers where they fit in LDS (one at 64-token chunks, with a
// second barrier before each commit)
template <typename CT, int D, int C, int NWV>
struct alignas(16) ScanFwdSmem {
  static constexpr int NBUF = 2 * sizeof(ScanFwdBuf<CT, D, C, NWV>) <= 160 * 1024 ? 2 : 1;
  ScanFwdBuf<CT, D, C, NWV> buf[NBUF];
};

template <typename CT, int D, int C, int NWV, bool STASH>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2))) delta_scan_fwd_kernel(DeltaArgs p) {
  typedef ScanDims<CT, D, C, NWV> Sd;
  typedef typename Sd::Frag Frag;
  typedef typename Vec4T<CT>::type V4;
  constexpr int KS = Sd::KS, TPS = Sd::TPS, NDT = Sd::NDT, NCT = Sd::NCT, NT = Sd::NT;
  constexpr int LDD = Sd::LDD, LDC = Sd::LDC, BV = Sd::BV;
  __shared__ ScanFwdSmem<CT, D, C, NWV> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H * p.M;
  const int work = xcd_remap(blockIdx.x, nchains * Sd::NVB);
  const int chain = work / Sd::NVB, vb = work % Sd::NVB;
  const int m = chain % p.M, h = (chain / p.M) % p.H, b = chain / (p.M * p.H);
  const int V = vb * NWV + wave;          // this wave's 16-column value tile
  const int NC = (p.T + C - 1) / C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t NR = (size_t)nchains * NC;
  const StashGeom sg = stash_geom(nchains, p.T, D, C, p.cps);
  // record of chunk c: rec_index(chain, c, nchains)
  const PrepPtrs<CT> pp = prep_ptrs<CT>(p.prep, NR, C);
  const CT* qg = (const CT*)p.q + qoff;
  const CT* kg = (const CT*)p.k + qoff;
  const CT* vg = (const CT*)p.v + qoff + vb * BV;

  f32x4 S[NDT];   // S[dt][i] = S0[16 dt + 4 g + i][16 V + n]
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    S[dt] = zero4();
    if (p.s0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) S[dt][i] = p.s0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // initial state in registers before the loop's own loads

  // Chunk tiles are fetched into registers two chunks ahead of their use:
  // q by every thread, and K, V, T, Aq (with the scalars) each by one group
  // of NWV/4 waves, so every 16-byte unit is loaded once.  Memory operations
  // are unconditional within a group (tail tokens go through buffer
  // resources), so the compiler's wait for the prefetched loads never covers
  // the stores issued after them.
  constexpr int GW = NWV / 4, GT = 64 * GW;
  static_assert(NWV % 4 == 0, "four load groups");
  const int grp = wave / GW, gt = tid - grp * GT;
  Stage<CT, C, D, 1, NT> pq;
  Stage<CT, C, D, 4, GT> pk;
  Stage<CT, C, BV, 4, GT> pv;
  Stage<CT, C, C, 1, GT> pt, pa;
  ScalStage<kNumSc * C, GT> ps;
  const unsigned rsb = (unsigned)(rs * sizeof(CT));
  const unsigned ysb = (unsigned)((size_t)p.H * p.M * D * sizeof(CT));
  auto fetch = [&](int c) {
    const int t0 = c * C;
    const unsigned nb = (unsigned)min(C, p.T - t0) * rsb;
    pq.fetch(buf_rsrc(qg + (size_t)t0 * rs, nb), rsb, tid);
    if (grp == 0) {
      pk.fetch(buf_rsrc(kg + (size_t)t0 * rs, nb), rsb, gt);
    } else if (grp == 1) {
      pv.fetch(buf_rsrc(vg + (size_t)t0 * rs, nb), rsb, gt);
    } else if (grp == 2) {
      pt.fetch_dense(pp.t + rec_index(chain, c, nchains) * C * C, gt);
      ps.fetch(pp.sc + rec_index(chain, c, nchains) * kNumSc * C, gt);
    } else {
      pa.fetch_dense(pp.aq + rec_index(chain, c, nchains) * C * C, gt);
    }
  };
  constexpr int NBUF = ScanFwdSmem<CT, D, C, NWV>::NBUF;
  auto commit = [&](ScanFwdBuf<CT, D, C, NWV>& B) {
    pq.template commit_nat<LDD>(B.q, tid);
    if (grp == 0) {
      pk.template commit_nat<LDD>(B.k, gt);
      pk.template commit_tr<LDC>(B.kt, gt);
    } else if (grp == 1) {
      pv.template commit_tr<LDC>(B.vt, gt);
    } else if (grp == 2) {
      pt.template commit_nat<LDC>(B.t, gt);
      ps.commit(B.sc, gt);
    } else {
      pa.template commit_nat<LDC>(B.aq, gt);
    }
  };
  fetch(0);
  __builtin_amdgcn_s_waitcnt(0);
  commit(sm.buf[0]);
  fetch(min(1, NC - 1));
  __builtin_amdgcn_s_waitcnt(0);   // the loop's waits then only track its own loads and stores
  __syncthreads();

  for (int c = 0; c < NC; ++c) {
    const int t0 = c * C;
    const size_t rec = rec_index(chain, c, nchains);
    const auto& B = sm.buf[c % NBUF];
    const float* gam = &B.sc[kScGam * C];
    const float* dec = &B.sc[kScDec * C];
    const float* aeg = &B.sc[kScAeg * C];
    const float* aw = &B.sc[kScAw * C];

    // ---- S0 as fragments over k = d; stash for the backward ----
    Frag Sf[NDT / TPS];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb) Sf[kb] = acc_frag((CT*)nullptr, S[kb * TPS], S[kb * TPS + TPS - 1]);
    if (STASH && c % p.cps == 0) {
      // the state entering every cps-th chunk (record c / cps), behind a
      // branch: stores to an empty buffer range at the other chunks would
      // still cost their issue (measured 11 us of the scan at config 2)
      const size_t srec = (size_t)(c / p.cps) * nchains + chain;
      const __amdgpu_buffer_rsrc_t sr =
          buf_rsrc((CT*)p.chunk_states + srec * (D * D), (unsigned)(D * D * sizeof(CT)));
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        buf_store4(sr, (unsigned)(stash_tile_offset<CT, D>(dt, V, lane) * sizeof(CT)), (const CT*)nullptr, S[dt][0],
                   S[dt][1], S[dt][2], S[dt][3]);
    }

    // ---- X = diag(a_w) V - diag(aeg) (K S0) on this wave's columns ----
    f32x4 X[NCT];
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) mma(acc, ld_frag(&B.k[(it * 16 + n16) * LDD + kb * KS], g4), Sf[kb]);
      const f32x4 vv = load4(&B.vt[(wave * 16 + n16) * LDC + it * 16 + 4 * g4]);
      const f32x4 a4 = *(const f32x4*)&aw[it * 16 + 4 * g4];
      const f32x4 e4 = *(const f32x4*)&aeg[it * 16 + 4 * g4];
      X[it] = a4 * vv - e4 * acc;
    }
    // ---- R = T X ----
    f32x4 Racc[NCT];
    {
      Frag Xf[NCT / TPS];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) Xf[kb] = acc_frag((CT*)nullptr, X[kb * TPS], X[kb * TPS + TPS - 1]);
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        Racc[it] = zero4();
#pragma unroll
        for (int kb = 0; kb < C / KS; ++kb) mma(Racc[it], ld_frag(&B.t[(it * 16 + n16) * LDC + kb * KS], g4), Xf[kb]);
      }
    }
    // ---- S = gam_last S0 + K^T diag(dec) R (the recurrence first; Y after) ----
    Frag Rf[NCT / TPS];
#pragma unroll
    for (int kb = 0; kb < NCT / TPS; ++kb) Rf[kb] = acc_frag((CT*)nullptr, Racc[kb * TPS], Racc[kb * TPS + TPS - 1]);
    {
      const float gl = gam[C - 1];
      Frag RDf[NCT / TPS];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) {
        const f32x4 d0 = *(const f32x4*)&dec[kb * KS + 4 * g4];
        const f32x4 d1 = *(const f32x4*)&dec[kb * KS + (TPS - 1) * 16 + 4 * g4];
        RDf[kb] = acc_frag((CT*)nullptr, Racc[kb * TPS], Racc[kb * TPS + TPS - 1], d0, d1);
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        S[dt] *= gl;
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) mma(S[dt], ld_frag(&B.kt[(dt * 16 + n16) * LDC + kb * KS], g4), RDf[kb]);
      }
    }
    if constexpr (STASH) {
      CT* rst = (CT*)p.chunk_states + sg.states + rec * (C * D);
#pragma unroll
      for (int it = 0; it < NCT; ++it)
        st4(rst + stash_tile_offset<CT, D>(it, V, lane), Racc[it][0], Racc[it][1], Racc[it][2], Racc[it][3]);
    }
    // ---- Y = diag(gam) Q S0 + Aq R ----
    {
      // this chain's rows of y in this chunk; rows past T fall outside the resource
      const __amdgpu_buffer_rsrc_t yr =
          buf_rsrc((CT*)p.y + (((size_t)(b * p.T + t0) * p.H + h) * p.M + m) * D, (unsigned)min(C, p.T - t0) * ysb);
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        f32x4 Y = zero4();
#pragma unroll
        for (int kb = 0; kb < NDT / TPS; ++kb) mma(Y, ld_frag(&B.q[(it * 16 + n16) * LDD + kb * KS], g4), Sf[kb]);
        Y *= *(const f32x4*)&gam[it * 16 + 4 * g4];
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) mma(Y, ld_frag(&B.aq[(it * 16 + n16) * LDC + kb * KS], g4), Rf[kb]);
        // transposed tile: lane (g, n) holds row 16 it + n, columns 4 g .. 4 g + 3
        const f32x4 yt = tile_transpose((CT*)nullptr, Y, lane);
        buf_store4(yr, (unsigned)(it * 16 + n16) * ysb + (16 * V + 4 * g4) * sizeof(CT), (const CT*)nullptr, yt[0],
                   yt[1], yt[2], yt[3]);
      }
    }
    // ---- chunk c + 1's tiles into the other buffer, chunk c + 2's loads ----
    if constexpr (NBUF == 1) __syncthreads();   // (one buffer: every wave done with chunk c's tiles)
    if (c + 1 < NC) commit(sm.buf[(c + 1) % NBUF]);
    fetch(min(c + 2, NC - 1));   // (the last chunks refetch, unused)
    __syncthreads();
  }

  if (p.s_out) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) p.s_out[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16] = S[dt][i];
  }
}

// ---------------------------------------------------------------------------
// backward: reverse scan of the state gradient
// ---------------------------------------------------------------------------
// With P3S (the checkpointed form: bf16, one workgroup per chain) the scan
// also forms, per chunk, P3 = R dS^T (the net writes against the gradient of
// the state leaving the chunk, [C][key]) and stashes it as bf16 accumulator
// tiles after dB: the gradient kernel then needs no state gradient but the
// segment ends'.  dS is written to LDS as bf16 [key][value] rows so that
// wave w contracts key tile w over every value column.
template <typename CT, int D, int C, int NWV, bool P3S>
struct alignas(16) ScanBwdBuf {
  typedef ScanDims<CT, D, C, NWV> Sd;
  CT k[C * Sd::LDD];        // K rows
  CT kt[D * Sd::LDC];       // K^T
  CT qt[D * Sd::LDC];       // Q^T
  CT dyt[Sd::BV * Sd::LDC]; // dY^T of this workgroup's value columns
  CT tt[C * Sd::LDC];       // T^T
  CT aqt[C * Sd::LDC];      // Aq^T
  float sc[kNumSc * C];
  CT r[(P3S ? C : 1) * Sd::LDD];   // R rows (the forward's net writes; P3S)
};
// staging double-buffered by chunk parity where it fits in LDS (see the forward)
template <typename CT, int D, int C, int NWV, bool P3S>
struct alignas(16) ScanBwdSmem {
  typedef ScanDims<CT, D, C, NWV> Sd;
  static constexpr size_t DSL = P3S ? (size_t)D * Sd::LDD : 8;
  static constexpr int NBUF = 2 * sizeof(ScanBwdBuf<CT, D, C, NWV, P3S>) + DSL * sizeof(CT) <= 160 * 1024 ? 2 : 1;
  ScanBwdBuf<CT, D, C, NWV, P3S> buf[NBUF];
  CT dsl[DSL];              // dS rows [key][value] (P3S)
  float kpr[2][P3S ? C : 1][NWV];   // per-wave parts of k.P3 per token, by chunk parity (P3S)
};

template <typename CT, int D, int C, int NWV, bool P3S>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2))) delta_scan_bwd_kernel(DeltaBwdArgs p) {
  typedef ScanDims<CT, D, C, NWV> Sd;
  typedef typename Sd::Frag Frag;
  constexpr int KS = Sd::KS, TPS = Sd::TPS, NDT = Sd::NDT, NCT = Sd::NCT, NT = Sd::NT;
  constexpr int LDD = Sd::LDD, LDC = Sd::LDC, BV = Sd::BV;
  static_assert(!P3S || (sizeof(CT) == 2 && Sd::NVB == 1), "P3 needs bf16 and one workgroup per chain");
  __shared__ ScanBwdSmem<CT, D, C, NWV, P3S> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H * p.M;
  const int work = xcd_remap(blockIdx.x, nchains * Sd::NVB);
  const int chain = work / Sd::NVB, vb = work % Sd::NVB;
  const int m = chain % p.M, h = (chain / p.M) % p.H, b = chain / (p.M * p.H);
  const int V = vb * NWV + wave;
  const int NC = (p.T + C - 1) / C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t rsy = (size_t)p.H * p.M * D;
  const size_t yoff = (((size_t)b * p.T * p.H + h) * p.M + m) * D + vb * BV;
  const size_t NR = (size_t)nchains * NC;
  const StashGeom sg = stash_geom(nchains, p.T, D, C, p.cps);
  // record of chunk c: rec_index(chain, c, nchains)
  // the forward's prep records sit after its state and net-write stashes
  const PrepPtrs<CT> pp = prep_ptrs<CT>((CT*)p.s_stash + sg.states + sg.tiles, NR, C);
  const CT* qg = (const CT*)p.q + qoff;
  const CT* kg = (const CT*)p.k + qoff;
  const CT* yg = (const CT*)p.dy + yoff;

  f32x4 dS[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dS[dt] = zero4();
    if (p.ds_final) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dS[dt][i] = p.ds_final[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16];
    }
  }

  __builtin_amdgcn_s_waitcnt(0);   // initial gradient in registers before the loop's own loads
  // chunk tiles fetched a chunk ahead, one group of NWV/4 waves per tile
  // (see the forward)
  constexpr int GW = NWV / 4, GT = 64 * GW;
  static_assert(NWV % 4 == 0, "four load groups");
  const int grp = wave / GW, gt = tid - grp * GT;
  Stage<CT, C, D, 4, GT> pq, pk;
  Stage<CT, C, BV, 4, GT> py;
  Stage<CT, C, C, 4, GT> pt, pa;
  ScalStage<3 * C, GT> ps;   // gam, dec, aeg
  // P3S: the chunk's net-write record, one 16-byte unit (C = 32) or two per thread
  constexpr int UPR = P3S ? C * D / (8 * NT) : 1;
  static_assert(!P3S || UPR * 8 * NT == C * D, "R record: whole units per thread");
  uint4 rx[UPR];
  const CT* rst = (const CT*)p.s_stash + sg.states;   // the forward's net writes
  CT* p3st = (CT*)p.ds_stash + sg.states + sg.tiles;   // P3 tiles, after dB
  float* k3st = (float*)(p3st + sg.tiles);             // k.P3 per token, after P3
  // k.P3 of chunk cc's tokens from the waves' parts (wave 0, once they are complete)
  auto k3_out = [&](int cc) {
    if constexpr (P3S) {
      if (wave == 0 && lane < C) {
        float x = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) x += sm.kpr[cc & 1][lane][w];
        k3st[rec_index(chain, cc, nchains) * C + lane] = x;
      }
    }
  };
  const unsigned rsb = (unsigned)(rs * sizeof(CT));
  const unsigned ysb = (unsigned)(rsy * sizeof(CT));
  auto fetch = [&](int c) {
    if constexpr (P3S) {
      const CT* src = rst + rec_index(chain, c, nchains) * C * D;
#pragma unroll
      for (int u = 0; u < UPR; ++u) rx[u] = *(const uint4*)(src + 8 * (tid + u * NT));
    }
    const int t0 = c * C;
    const int nv = min(C, p.T - t0);
    if (grp == 0) {
      pq.fetch(buf_rsrc(qg + (size_t)t0 * rs, (unsigned)nv * rsb), rsb, gt);
    } else if (grp == 1) {
      pk.fetch(buf_rsrc(kg + (size_t)t0 * rs, (unsigned)nv * rsb), rsb, gt);
    } else if (grp == 2) {
      py.fetch(buf_rsrc(yg + (size_t)t0 * rsy, (unsigned)nv * ysb), ysb, gt);
    } else {
      pt.fetch_dense(pp.t + rec_index(chain, c, nchains) * C * C, gt);
      pa.fetch_dense(pp.aq + rec_index(chain, c, nchains) * C * C, gt);
      ps.fetch(pp.sc + rec_index(chain, c, nchains) * kNumSc * C, gt);
    }
  };
  constexpr int NBUF = ScanBwdSmem<CT, D, C, NWV, P3S>::NBUF;
  auto commit = [&](ScanBwdBuf<CT, D, C, NWV, P3S>& B) {
    if constexpr (P3S) {
#pragma unroll
      for (int u = 0; u < UPR; ++u) unit_commit_rows<LDD>(B.r, rx[u], tile_unit_of<D>(tid + u * NT));
    }
    if (grp == 0) {
      pq.template commit_tr<LDC>(B.qt, gt);
    } else if (grp == 1) {
      pk.template commit_nat<LDD>(B.k, gt);
      pk.template commit_tr<LDC>(B.kt, gt);
    } else if (grp == 2) {
      py.template commit_tr<LDC>(B.dyt, gt);
    } else {
      pt.template commit_tr<LDC>(B.tt, gt);
      pa.template commit_tr<LDC>(B.aqt, gt);
      ps.commit(B.sc, gt);
    }
  };
  fetch(NC - 1);
  __builtin_amdgcn_s_waitcnt(0);
  commit(sm.buf[(NC - 1) % NBUF]);
  fetch(max(NC - 2, 0));
  __builtin_amdgcn_s_waitcnt(0);   // the loop's waits then only track its own loads and stores
  __syncthreads();

  for (int c = NC - 1; c >= 0; --c) {
    const size_t rec = rec_index(chain, c, nchains);
    const auto& sb = sm.buf[c % NBUF];
    const float* gam = &sb.sc[kScGam * C];
    const float* dec = &sb.sc[kScDec * C];
    const float* aeg = &sb.sc[kScAeg * C];

    // ---- dS at the chunk end as fragments over k = d; stash ----
    Frag dSf[NDT / TPS];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb) dSf[kb] = acc_frag((CT*)nullptr, dS[kb * TPS], dS[kb * TPS + TPS - 1]);
    if constexpr (P3S) {
      // dS as bf16 rows [key][value]: this wave's value columns of every key.
      // Each tile is transposed first (lane (g, n): key 16 dt + n, values
      // 16 V + 4 g ..), so a lane writes four values of one row at once.
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 y = tile_transpose((CT*)nullptr, dS[dt], lane);
        *(bf16x4*)&sm.dsl[(dt * 16 + n16) * LDD + 16 * V + 4 * g4] = (bf16x4){(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
      }
      lds_barrier();   // every wave's columns written (loads in flight stay in flight)
      if (c + 1 < NC) k3_out(c + 1);   // (its parts were completed before the last step's barrier)
    }
    {
      // the state gradient leaving every cps-th chunk and the last one
      // (record c / cps); other chunks' stores are dropped (empty range),
      // so the loop carries no branch around a store (here a branch
      // measured slower)
      const size_t srec = (size_t)(c / p.cps) * nchains + chain;
      const bool keep = c % p.cps == p.cps - 1 || c == NC - 1;
      const __amdgpu_buffer_rsrc_t sr =
          buf_rsrc((CT*)p.ds_stash + srec * (D * D), keep ? (unsigned)(D * D * sizeof(CT)) : 0u);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        buf_store4(sr, (unsigned)(stash_tile_offset<CT, D>(dt, V, lane) * sizeof(CT)), (const CT*)nullptr, dS[dt][0],
                   dS[dt][1], dS[dt][2], dS[dt][3]);
    }
    // ---- P3^T = dS R^T on key tile `wave` (lane (g, n): keys 16 wave + 4 g + e
    // of token 16 it + n), stored as the gradient kernel's dk tile, and the
    // per-wave parts of k.P3 ----
    auto p3_block = [&]() {
      if constexpr (P3S) {
        f32x4 P3[NCT];
#pragma unroll
        for (int it = 0; it < NCT; ++it) P3[it] = zero4();
#pragma unroll
        for (int kb = 0; kb < D / KS; ++kb) {
          const Frag a = ld_frag(&sm.dsl[(wave * 16 + n16) * LDD + kb * KS], g4);
#pragma unroll
          for (int it = 0; it < NCT; ++it) mma(P3[it], a, ld_frag(&sb.r[(it * 16 + n16) * LDD + kb * KS], g4));
        }
        CT* pst = p3st + rec * (C * D);
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          st4(pst + stash_tile_offset<CT, D>(it, wave, lane), P3[it][0], P3[it][1], P3[it][2], P3[it][3]);
          // the token's k.P3 over this wave's keys, in float32
          const bf16x4 k4 = *(const bf16x4*)&sb.k[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
          float x = (P3[it][0] * (float)k4[0] + P3[it][1] * (float)k4[1]) + (P3[it][2] * (float)k4[2] + P3[it][3] * (float)k4[3]);
          x = sum_rows4(x);
          if (g4 == 0) sm.kpr[c & 1][it * 16 + n16][wave] = x;
        }
      }
    };
    // ---- dR = diag(dec) K dS + Aq^T dY ----
    Frag dYf[C / KS];
#pragma unroll
    for (int kb = 0; kb < C / KS; ++kb) dYf[kb] = ld_frag(&sb.dyt[(wave * 16 + n16) * LDC + kb * KS], g4);
    f32x4 dR[NCT];
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) mma(acc, ld_frag(&sb.k[(it * 16 + n16) * LDD + kb * KS], g4), dSf[kb]);
      acc *= *(const f32x4*)&dec[it * 16 + 4 * g4];
#pragma unroll
      for (int kb = 0; kb < C / KS; ++kb) mma(acc, ld_frag(&sb.aqt[(it * 16 + n16) * LDC + kb * KS], g4), dYf[kb]);
      dR[it] = acc;
    }
    // ---- dB = T^T dR; stash ----
    Frag dBf[NCT / TPS];
    {
      Frag dRf[NCT / TPS];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) dRf[kb] = acc_frag((CT*)nullptr, dR[kb * TPS], dR[kb * TPS + TPS - 1]);
      f32x4 dB[NCT];
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        dB[it] = zero4();
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) mma(dB[it], ld_frag(&sb.tt[(it * 16 + n16) * LDC + kb * KS], g4), dRf[kb]);
      }
      CT* bst = (CT*)p.ds_stash + sg.states + rec * (C * D);
#pragma unroll
      for (int it = 0; it < NCT; ++it)
        st4(bst + stash_tile_offset<CT, D>(it, V, lane), dB[it][0], dB[it][1], dB[it][2], dB[it][3]);
      // fragments of -diag(aeg) dB over k = token
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) {
        const f32x4 s0 = -*(const f32x4*)&aeg[kb * KS + 4 * g4];
        const f32x4 s1 = -*(const f32x4*)&aeg[kb * KS + (TPS - 1) * 16 + 4 * g4];
        dBf[kb] = acc_frag((CT*)nullptr, dB[kb * TPS], dB[kb * TPS + TPS - 1], s0, s1);
      }
    }
    // ---- dS <- gam_last dS + Q^T diag(gam) dY - K^T diag(aeg) dB ----
    {
      const float gl = gam[C - 1];
      Frag gYf[C / KS];
#pragma unroll
      for (int kb = 0; kb < C / KS; ++kb) gYf[kb] = frag_scale(dYf[kb], gam + kb * KS, g4);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        dS[dt] *= gl;
#pragma unroll
        for (int kb = 0; kb < C / KS; ++kb) {
          mma(dS[dt], ld_frag(&sb.qt[(dt * 16 + n16) * LDC + kb * KS], g4), gYf[kb]);
          mma(dS[dt], ld_frag(&sb.kt[(dt * 16 + n16) * LDC + kb * KS], g4), dBf[kb]);
        }
      }
    }
    p3_block();   // (off the dR -> dB -> dS path: measured fastest here)
    // ---- chunk c - 1's tiles into the other buffer, chunk c - 2's loads ----
    if constexpr (NBUF == 1) __syncthreads();   // (one buffer: every wave done with chunk c's tiles)
    if (c > 0) commit(sm.buf[(c - 1) % NBUF]);
    fetch(max(c - 2, 0));   // (the first chunks refetch, unused)
    __syncthreads();
  }
  k3_out(0);
  if (p.ds0) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) p.ds0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16] = dS[dt][i];
  }
}

// ---------------------------------------------------------------------------
// dispatch: one workgroup of D/16 waves per chain (each wave 16 value
// columns), so the chunk's tiles are loaded and the -Wm product formed once
// per chain and shared through LDS
// ---------------------------------------------------------------------------
template <typename CT, int D, int C>
struct ScanCfg {
  static constexpr int NWV = D / 16;
  static_assert(sizeof(ScanFwdSmem<CT, D, C, NWV>) <= 160 * 1024 &&
                    sizeof(ScanBwdSmem<CT, D, C, NWV, false>) <= 160 * 1024 &&
                    (sizeof(CT) != 2 || C != 32 || sizeof(ScanBwdSmem<CT, D, C, NWV, true>) <= 160 * 1024),
                "scan LDS budget");
};

template <typename CT, int D, int C>
static int launch_scan_fwd(const DeltaArgs& a, hipStream_t stream) {
  constexpr int NWV = ScanCfg<CT, D, C>::NWV;
  typedef ScanDims<CT, D, C, NWV> Sd;
  if (a.chunk_states)
    hipLaunchKernelGGL((delta_scan_fwd_kernel<CT, D, C, NWV, true>), dim3(a.B * a.H * a.M * Sd::NVB), dim3(Sd::NT),
                       0, stream, a);
  else
    hipLaunchKernelGGL((delta_scan_fwd_kernel<CT, D, C, NWV, false>), dim3(a.B * a.H * a.M * Sd::NVB), dim3(Sd::NT),
                       0, stream, a);
  return check_launch("delta_scan_fwd_kernel");
}

template <typename CT, int D, int C>
static int launch_scan_bwd(const DeltaBwdArgs& a, hipStream_t stream) {
  constexpr int NWV = ScanCfg<CT, D, C>::NWV;
  typedef ScanDims<CT, D, C, NWV> Sd;
  if constexpr (sizeof(CT) == 2 && C == 32) {
    if (a.cps > 1) {   // checkpointed form: P3 tiles for delta_grad_seg_kernel
      hipLaunchKernelGGL((delta_scan_bwd_kernel<CT, D, C, NWV, true>), dim3(a.B * a.H * a.M * Sd::NVB), dim3(Sd::NT),
                         0, stream, a);
      return check_launch("delta_scan_bwd_kernel");
    }
  }
  hipLaunchKernelGGL((delta_scan_bwd_kernel<CT, D, C, NWV, false>), dim3(a.B * a.H * a.M * Sd::NVB), dim3(Sd::NT), 0,
                     stream, a);
  return check_launch("delta_scan_bwd_kernel");
}

int delta_scan_fwd_dispatch(const DeltaArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 64) return launch_scan_fwd<bf16, 128, 64>(a, stream);
    if (a.D == 128 && a.C == 32) return launch_scan_fwd<bf16, 128, 32>(a, stream);
    if (a.D == 64 && a.C == 64) return launch_scan_fwd<bf16, 64, 64>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_scan_fwd<bf16, 64, 32>(a, stream);
  } else {
    if (a.D == 128 && a.C == 32) return launch_scan_fwd<float, 128, 32>(a, stream);
    if (a.D == 128 && a.C == 16) return launch_scan_fwd<float, 128, 16>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_scan_fwd<float, 64, 32>(a, stream);
    if (a.D == 64 && a.C == 16) return launch_scan_fwd<float, 64, 16>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "scan: unsupported head_dim %d / chunk %d", a.D, a.C);
}

int delta_scan_bwd_dispatch(const DeltaBwdArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 64) return launch_scan_bwd<bf16, 128, 64>(a, stream);
    if (a.D == 128 && a.C == 32) return launch_scan_bwd<bf16, 128, 32>(a, stream);
    if (a.D == 64 && a.C == 64) return launch_scan_bwd<bf16, 64, 64>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_scan_bwd<bf16, 64, 32>(a, stream);
  } else {
    if (a.D == 128 && a.C == 32) return launch_scan_bwd<float, 128, 32>(a, stream);
    if (a.D == 128 && a.C == 16) return launch_scan_bwd<float, 128, 16>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_scan_bwd<float, 64, 32>(a, stream);
    if (a.D == 64 && a.C == 16) return launch_scan_bwd<float, 64, 16>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "backward scan: unsupported head_dim %d / chunk %d", a.D, a.C);
}

}  // namespace gdnx

// Decoupled-erase delta rule with a decay per key channel (gfx950), the
// general KMD-2 scan: per chain (b, h) and token t, with g_t in (0, 1]^dk,
//
//   S <- diag(g_t) S;  r = beta_w v - beta_e S^T k;  S <- S + k r^T;  y = S^T q
//
// (research/kernel_ab/ref_scan.py:37-47, gdn3/kmd2_native.py:109-132, where
// g = exp(g_head + decay_chan) is per key channel).  Chunks of C = 16 tokens,
// float32 throughout.  With the per-channel inclusive prefix G_i = sum_{s<=i}
// log g_s and the chunk's last row G_L:
//
//   M_ij = sum_d x_id k_jd exp(G_id - G_jd)  (j <= i: every exponent <= 0)
//   L = diag(beta_e) M[x=k] (strict),  Aq = M[x=q],  T = (I + L)^-1
//   R = T (diag(beta_w) V - diag(beta_e) (K o e^G) S0)
//   Y = (Q o e^G) S0 + Aq R
//   S = diag(e^{G_L}) S0 + (K o e^{G_L - G})^T R
//
// With a chunk of 16 the decay-weighted grams are formed exactly, channel by
// channel (no sub-chunk factoring whose factors could overflow).  The
// reference's chunked path (gdn3/kmd2_fast_scan.py:198-214) divides keys by
// the cumulative decay product instead, which is valid only at its chunk of
// 16 and moderate decays.  Three kernels, as for the scalar decay: the
// forward state scan, the reverse scan of the state gradient, and the
// per-chunk gradient kernel.  One workgroup of D/16 waves per chain (scans)
// or per chunk (gradients); wave w owns value (and, in the gradient kernel,
// key) columns 16w..16w+15.
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

namespace {

constexpr int CC = 16;        // chunk
constexpr int LDC = CC + 4;   // [*][C] fp32 rows

template <int D>
struct ChD {
  static constexpr int NW = D / 16, NT = 64 * NW, NDT = D / 16, LDD = D + 4;
};

// The chunk's operands in LDS (fp32): q, k, the per-channel prefix G, the
// scalars, the exact grams and T.
template <int D>
struct alignas(16) ChanOps {
  static constexpr int LDD = D + 4;
  float q[CC * LDD];
  float k[CC * LDD];
  float G[CC * LDD];     // raw log-decay on commit, then the clamped prefix
  float L[CC * LDC];     // beta_e,i M_ij (j < i)
  float LT[CC * 20];     // L transposed (the blocked inverse reads it)
  float Td[CC * 20];
  float Aq[CC * LDC];
  float Mk[CC * LDC];    // M_ij[x=k] (j < i), the gram without beta_e
  float T[CC * LDC];     // (I + L)^-1
  float be[CC], bw[CC];
  float eGL[D];          // exp(G_L) per channel
};

// Column prefix of the clamped log-decay (threads t < D, one column each).
template <int D>
__device__ __forceinline__ void chan_prefix(ChanOps<D>& o, int tid) {
  constexpr int LDD = ChD<D>::LDD;
  if (tid < D) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CC; ++i) {
      acc += fmaxf(fminf(o.G[i * LDD + tid], 0.f), kLogFloor);
      o.G[i * LDD + tid] = acc;
    }
    o.eGL[tid] = __expf(acc);
  }
}

// Exact decay-weighted grams: wave w takes rows i = w, w + NW, ...; lane
// (g, n) takes column j = n and the channel quarter [g D/4, (g+1) D/4).
template <int D>
__device__ __forceinline__ void chan_grams(ChanOps<D>& o, int wave, int lane) {
  constexpr int NW = ChD<D>::NW, LDD = ChD<D>::LDD, DQ = D / 4;
  const int g4 = lane >> 4, j = lane & 15;
  for (int i = wave; i < CC; i += NW) {
    float kk = 0.f, qk = 0.f;
    if (j <= i) {
#pragma unroll 4
      for (int d0 = g4 * DQ; d0 < (g4 + 1) * DQ; d0 += 4) {
        const f32x4 ki = *(const f32x4*)&o.k[i * LDD + d0];
        const f32x4 qi = *(const f32x4*)&o.q[i * LDD + d0];
        const f32x4 Gi = *(const f32x4*)&o.G[i * LDD + d0];
        const f32x4 kj = *(const f32x4*)&o.k[j * LDD + d0];
        const f32x4 Gj = *(const f32x4*)&o.G[j * LDD + d0];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ex = __expf(Gi[e] - Gj[e]);
          kk += ki[e] * kj[e] * ex;
          qk += qi[e] * kj[e] * ex;
        }
      }
    }
    kk += __shfl_xor(kk, 16, 64);
    kk += __shfl_xor(kk, 32, 64);
    qk += __shfl_xor(qk, 16, 64);
    qk += __shfl_xor(qk, 32, 64);
    if (g4 == 0) {
      const float mk = (j < i) ? kk : 0.f;
      const float l = o.be[i] * mk;
      o.L[i * LDC + j] = l;
      o.LT[j * 20 + i] = l;
      o.Mk[i * LDC + j] = mk;
      o.Aq[i * LDC + j] = (j <= i) ? qk : 0.f;
    }
  }
}

template <int D>
__device__ __forceinline__ void chan_inverse(ChanOps<D>& o, int wave, int lane) {
  invert_unit_lower<CC>(o.L, o.LT, o.Td, wave, lane, [&](int) { return 0; },
                        [&](int i, int jj, float t, int) { o.T[i * LDC + jj] = t; });
}

// Buffer resource over this chain's rows of a [B, T, H, X] fp32 tensor for
// the chunk at token t0 (rows past T read zero / drop stores).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const float* base, int b, int t0, int T, int H, int h,
                                                             int X) {
  const size_t off = (((size_t)b * T + t0) * H + h) * X;
  return buf_rsrc(base + off, (unsigned)(min(CC, T - t0) * H * X * 4));
}

// per-token scalar (beta) of this chain at t0 + i, zero past T
__device__ __forceinline__ float chunk_scalar(const float* base, int b, int t0, int i, int T, int H, int h) {
  const int t = min(t0 + i, T - 1);
  const float x = base[((size_t)b * T + t) * H + h];
  return (t0 + i < T) ? x : 0.f;
}

}  // namespace

// ---------------------------------------------------------------------------
// per-chunk operand records (state independent, one workgroup per chunk)
//   forward:  U = T diag(beta_w) V, -Wm = -T diag(beta_e) (K o e^G), Q o e^G,
//             (K o e^{G_L - G})^T, Aq, e^{G_L}
//   backward: K o e^{G_L - G}, (Q o e^G)^T, (K o e^G)^T, T^T, Aq^T, beta_e, e^{G_L}
// so that the scans carry only the state-dependent products.
// ---------------------------------------------------------------------------
template <int D>
struct ChRec {
  static constexpr int CD = CC * D;
  static constexpr int F_U = 0, F_NWM = CD, F_QE = 2 * CD, F_KFT = 3 * CD, F_AQ = 4 * CD, F_EGL = 4 * CD + CC * CC;
  static constexpr int FN = 4 * CD + CC * CC + D;
  static constexpr int B_KF = 0, B_QET = CD, B_KET = 2 * CD, B_TT = 3 * CD, B_AQT = 3 * CD + CC * CC,
                       B_BE = 3 * CD + 2 * CC * CC, B_EGL = 3 * CD + 2 * CC * CC + CC;
  static constexpr int BN = 3 * CD + 2 * CC * CC + CC + D;
  static_assert(FN % 4 == 0 && BN % 4 == 0 && F_EGL % 4 == 0 && B_EGL % 4 == 0, "16-byte aligned records");
};

template <int D>
struct alignas(16) ChanPrepSmem {
  ChanOps<D> o;
  float ket[D * LDC];    // (K o e^G)^T
  float kft[D * LDC];    // (K o e^{G_L - G})^T
  float qet[D * LDC];    // (Q o e^G)^T
  float vt[D * LDC];     // V^T
};

template <int D, bool BWD>
__global__ void __launch_bounds__(64 * (D / 16)) chan_prep_kernel(ChanArgs p) {
  typedef ChD<D> Cd;
  typedef ChRec<D> Rc;
  constexpr int NT = Cd::NT, LDD = Cd::LDD;
  __shared__ ChanPrepSmem<D> sm;
  ChanOps<D>& o = sm.o;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int NC = (p.T + CC - 1) / CC;
  const int nchains = p.B * p.H;
  const int blk = xcd_remap(blockIdx.x, nchains * NC);
  const int c = blk % NC, chain = blk / NC;
  const int h = chain % p.H, b = chain / p.H;
  const int t0 = c * CC;
  const size_t rec = rec_index(chain, c, nchains);
  float* fr = p.frec + rec * Rc::FN;
  float* br = BWD ? p.brec + rec * Rc::BN : nullptr;
  const unsigned rsb = (unsigned)((size_t)p.H * D * 4);
  {
    Stage<float, CC, D, 1, NT> sq, sk, sl;
    Stage<float, CC, D, 4, NT> sv;
    sq.fetch(chunk_rsrc(p.q, b, t0, p.T, p.H, h, D), rsb, tid);
    sk.fetch(chunk_rsrc(p.k, b, t0, p.T, p.H, h, D), rsb, tid);
    sl.fetch(chunk_rsrc(p.lg, b, t0, p.T, p.H, h, D), rsb, tid);
    sv.fetch(chunk_rsrc(p.v, b, t0, p.T, p.H, h, D), rsb, tid);
    const float be = chunk_scalar(p.be, b, t0, tid % CC, p.T, p.H, h);
    const float bw = chunk_scalar(p.bw, b, t0, tid % CC, p.T, p.H, h);
    sq.template commit_nat<LDD>(o.q, tid);
    sk.template commit_nat<LDD>(o.k, tid);
    sl.template commit_nat<LDD>(o.G, tid);
    sv.template commit_tr<LDC>(sm.vt, tid);
    if (tid < CC) {
      o.be[tid] = be;
      o.bw[tid] = bw;
    }
  }
  __syncthreads();
  chan_prefix<D>(o, tid);
  __syncthreads();
  chan_grams<D>(o, wave, lane);
  for (int e = tid; e < CC * D; e += NT) {
    const int i = e / D, d = e % D;
    const float G = o.G[i * LDD + d], GL = o.G[(CC - 1) * LDD + d];
    const float E = __expf(G), F = __expf(GL - G), kv = o.k[i * LDD + d], qv = o.q[i * LDD + d] * E;
    fr[Rc::F_QE + e] = qv;
    sm.ket[d * LDC + i] = kv * E;
    sm.kft[d * LDC + i] = kv * F;
    if constexpr (BWD) {
      br[Rc::B_KF + e] = kv * F;
      sm.qet[d * LDC + i] = qv;
    }
  }
  __syncthreads();
  chan_inverse<D>(o, wave, lane);
  __syncthreads();
  {  // -Wm on this wave's key tile: acc[s] = Wm[n][16 wave + 4 g + s]
    const f32x4 bt = frag_scale(ld_frag(&o.T[n16 * LDC], g4), o.be, g4);
    f32x4 acc = zero4();
    mma(acc, ld_frag(&sm.ket[(16 * wave + n16) * LDC], g4), bt);
    *(f32x4*)&fr[Rc::F_NWM + n16 * D + 16 * wave + 4 * g4] = -acc;
  }
  {  // U = T diag(beta_w) V on value tile wave, stored as rows
    f32x4 acc = zero4();
    mma(acc, frag_scale(ld_frag(&o.T[n16 * LDC], g4), o.bw, g4), ld_frag(&sm.vt[(16 * wave + n16) * LDC], g4));
    *(f32x4*)&fr[Rc::F_U + n16 * D + 16 * wave + 4 * g4] = tile_transpose((float*)nullptr, acc, lane);
  }
  for (int e = tid; e < D * CC; e += NT) {
    const int d = e / CC, i = e % CC;
    fr[Rc::F_KFT + e] = sm.kft[d * LDC + i];
    if constexpr (BWD) {
      br[Rc::B_QET + e] = sm.qet[d * LDC + i];
      br[Rc::B_KET + e] = sm.ket[d * LDC + i];
    }
  }
  for (int e = tid; e < CC * CC; e += NT) {
    const int i = e / CC, j = e % CC;
    fr[Rc::F_AQ + e] = o.Aq[i * LDC + j];
    if constexpr (BWD) {
      br[Rc::B_TT + e] = o.T[j * LDC + i];
      br[Rc::B_AQT + e] = o.Aq[j * LDC + i];
    }
  }
  for (int e = tid; e < D; e += NT) {
    fr[Rc::F_EGL + e] = o.eGL[e];
    if constexpr (BWD) br[Rc::B_EGL + e] = o.eGL[e];
  }
  if constexpr (BWD)
    if (tid < CC) br[Rc::B_BE + tid] = o.be[tid];
}

// ---------------------------------------------------------------------------
// forward state scan: one workgroup of NWV waves per (chain, block of 16 NWV
// value columns); per chunk, from the record:
//   R = U - Wm S0,  Y = (Q o e^G) S0 + Aq R,  S = diag(e^{G_L}) S0 + (K o e^{G_L - G})^T R
// With SCORE (|r_t| requested) a chain's value columns stay in one workgroup.
// ---------------------------------------------------------------------------
template <int D, int NWV>
struct alignas(16) ChanScanFSmem {
  static constexpr int LDD = D + 4, BV = 16 * NWV, LDU = BV + 4;
  float nwm[CC * LDD];
  float qe[CC * LDD];
  float kft[D * LDC];
  float aq[CC * LDC];
  float egl[D];
  float u[CC * LDU];
  float rn[NWV][CC];
};

template <int D, int NWV, bool STASH, bool SCORE>
__global__ void __launch_bounds__(64 * NWV) chan_scan_fwd_kernel(ChanArgs p) {
  typedef ChRec<D> Rc;
  typedef ChanScanFSmem<D, NWV> Sm;
  constexpr int NT = 64 * NWV, NDT = D / 16, LDD = Sm::LDD, BV = Sm::BV, LDU = Sm::LDU, NVB = D / BV;
  static_assert(!SCORE || NVB == 1, "the update norm sums over all value columns in one workgroup");
  __shared__ Sm sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H;
  const int work = xcd_remap(blockIdx.x, nchains * NVB);
  const int chain = work / NVB, vb = work % NVB;
  const int h = chain % p.H, b = chain / p.H;
  const int V = vb * NWV + wave;
  const int NC = (p.T + CC - 1) / CC;
  const size_t NR = (size_t)nchains * NC;
  const unsigned rsb = (unsigned)((size_t)p.H * D * 4);

  f32x4 S[NDT];   // S[dt][i] = S0[16 dt + 4 g + i][16 V + n]
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    S[dt] = zero4();
    if (p.s0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) S[dt][i] = p.s0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);

  Stage<float, CC, D, 1, NT> pn, pq;
  Stage<float, D, CC, 1, NT> pk;
  Stage<float, CC, CC, 1, NT> pa;
  Stage<float, 1, D, 1, NT> pe;
  Stage<float, CC, BV, 1, NT> pu;
  auto fetch = [&](int c) {
    const float* fr = p.frec + rec_index(chain, c, nchains) * Rc::FN;
    pn.fetch_dense(fr + Rc::F_NWM, tid);
    pq.fetch_dense(fr + Rc::F_QE, tid);
    pk.fetch_dense(fr + Rc::F_KFT, tid);
    pa.fetch_dense(fr + Rc::F_AQ, tid);
    pe.fetch_dense(fr + Rc::F_EGL, tid);
    pu.fetch(buf_rsrc(fr + Rc::F_U + vb * BV, (unsigned)(Rc::CD * 4)), (unsigned)(D * 4), tid);
  };
  fetch(0);
  __builtin_amdgcn_s_waitcnt(0);

  for (int c = 0; c < NC; ++c) {
    const int t0 = c * CC;
    const size_t rec = rec_index(chain, c, nchains);
    __syncthreads();
    pn.template commit_nat<LDD>(sm.nwm, tid);
    pq.template commit_nat<LDD>(sm.qe, tid);
    pk.template commit_nat<LDC>(sm.kft, tid);
    pa.template commit_nat<LDC>(sm.aq, tid);
    pe.template commit_nat<D>(sm.egl, tid);
    pu.template commit_nat<LDU>(sm.u, tid);
    __syncthreads();
    fetch(min(c + 1, NC - 1));
    if constexpr (STASH) {
      float* cst = (float*)p.chunk_states + rec * (D * D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) *(f32x4*)(cst + stash_tile_offset<float, D>(dt, V, lane)) = S[dt];
    }
    // R = U - Wm S0 (two accumulators)
    f32x4 R0, R1 = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) R0[s] = sm.u[(4 * g4 + s) * LDU + 16 * wave + n16];
#pragma unroll
    for (int kb = 0; kb < NDT; ++kb) mma((kb & 1) ? R1 : R0, ld_frag(&sm.nwm[n16 * LDD + kb * 16], g4), S[kb]);
    const f32x4 R = R0 + R1;
    if constexpr (STASH) {
      float* rst = (float*)p.chunk_states + NR * D * D + rec * (CC * D);
      *(f32x4*)(rst + stash_tile_offset<float, D>(0, V, lane)) = R;
    }
    if constexpr (SCORE) {
      const f32x4 sq = R * R;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = row_prefix16(sq[e]);
        if (n16 == 15) sm.rn[wave][4 * g4 + e] = x;
      }
    }
    // Y = (Q o e^G) S0 + Aq R
    {
      f32x4 Y0 = zero4(), Y1 = zero4();
#pragma unroll
      for (int kb = 0; kb < NDT; ++kb) mma((kb & 1) ? Y1 : Y0, ld_frag(&sm.qe[n16 * LDD + kb * 16], g4), S[kb]);
      mma(Y0, ld_frag(&sm.aq[n16 * LDC], g4), R);
      const f32x4 yt = tile_transpose((float*)nullptr, Y0 + Y1, lane);
      const __amdgpu_buffer_rsrc_t yr = chunk_rsrc((const float*)p.y, b, t0, p.T, p.H, h, D);
      buf_store4(yr, (unsigned)n16 * rsb + (16 * V + 4 * g4) * 4, (const float*)nullptr, yt[0], yt[1], yt[2], yt[3]);
    }
    // S = diag(e^{G_L}) S0 + (K o e^{G_L - G})^T R
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      S[dt] *= *(const f32x4*)&sm.egl[dt * 16 + 4 * g4];
      mma(S[dt], ld_frag(&sm.kft[(dt * 16 + n16) * LDC], g4), R);
    }
    if constexpr (SCORE) {
      __syncthreads();
      if (tid < CC && t0 + tid < p.T) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) s += sm.rn[w][tid];
        p.r_norm[((size_t)b * p.T + t0 + tid) * p.H + h] = sqrtf(s);
      }
    }
  }
  if (p.s_out) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) p.s_out[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16] = S[dt][i];
  }
}

// ---------------------------------------------------------------------------
// reverse scan of the state gradient, value-split like the forward:
//   dR = Aq^T dY + (K o e^{G_L - G}) dS,  dB = T^T dR
//   dS0 = diag(e^{G_L}) dS + (Q o e^G)^T dY - (K o e^G)^T diag(beta_e) dB
// ---------------------------------------------------------------------------
template <int D, int NWV>
struct alignas(16) ChanScanBSmem {
  static constexpr int LDD = D + 4, BV = 16 * NWV;
  float kf[CC * LDD];
  float qet[D * LDC];
  float ket[D * LDC];
  float tt[CC * LDC];
  float aqt[CC * LDC];
  float be[CC];
  float egl[D];
  float dyt[BV * LDC];
};

template <int D, int NWV>
__global__ void __launch_bounds__(64 * NWV) chan_scan_bwd_kernel(ChanBwdArgs p) {
  typedef ChRec<D> Rc;
  typedef ChanScanBSmem<D, NWV> Sm;
  constexpr int NT = 64 * NWV, NDT = D / 16, LDD = Sm::LDD, BV = Sm::BV, NVB = D / BV;
  __shared__ Sm sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H;
  const int work = xcd_remap(blockIdx.x, nchains * NVB);
  const int chain = work / NVB, vb = work % NVB;
  const int h = chain % p.H, b = chain / p.H;
  const int V = vb * NWV + wave;
  const int NC = (p.T + CC - 1) / CC;
  const size_t NR = (size_t)nchains * NC;
  const float* brec = (const float*)p.s_stash + NR * ((size_t)D * D + CC * D + Rc::FN);

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
  __builtin_amdgcn_s_waitcnt(0);

  Stage<float, CC, D, 1, NT> pf;
  Stage<float, D, CC, 1, NT> pqt, pkt;
  Stage<float, CC, CC, 1, NT> ptt, pat;
  Stage<float, 1, CC, 1, NT> pb;
  Stage<float, 1, D, 1, NT> pe;
  Stage<float, CC, BV, 4, NT> py;
  const unsigned rsb = (unsigned)((size_t)p.H * D * 4);
  auto fetch = [&](int c) {
    const float* br = brec + rec_index(chain, c, nchains) * Rc::BN;
    pf.fetch_dense(br + Rc::B_KF, tid);
    pqt.fetch_dense(br + Rc::B_QET, tid);
    pkt.fetch_dense(br + Rc::B_KET, tid);
    ptt.fetch_dense(br + Rc::B_TT, tid);
    pat.fetch_dense(br + Rc::B_AQT, tid);
    pb.fetch_dense(br + Rc::B_BE, tid);
    pe.fetch_dense(br + Rc::B_EGL, tid);
    py.fetch(chunk_rsrc(p.dy + vb * BV, b, c * CC, p.T, p.H, h, D), rsb, tid);
  };
  fetch(NC - 1);
  __builtin_amdgcn_s_waitcnt(0);

  for (int c = NC - 1; c >= 0; --c) {
    const size_t rec = rec_index(chain, c, nchains);
    __syncthreads();
    pf.template commit_nat<LDD>(sm.kf, tid);
    pqt.template commit_nat<LDC>(sm.qet, tid);
    pkt.template commit_nat<LDC>(sm.ket, tid);
    ptt.template commit_nat<LDC>(sm.tt, tid);
    pat.template commit_nat<LDC>(sm.aqt, tid);
    pb.template commit_nat<CC>(sm.be, tid);
    pe.template commit_nat<D>(sm.egl, tid);
    py.template commit_tr<LDC>(sm.dyt, tid);
    __syncthreads();
    fetch(max(c - 1, 0));
    {
      float* cst = (float*)p.ds_stash + rec * (D * D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) *(f32x4*)(cst + stash_tile_offset<float, D>(dt, V, lane)) = dS[dt];
    }
    const f32x4 dYf = ld_frag(&sm.dyt[(16 * wave + n16) * LDC], g4);
    f32x4 dR0 = zero4(), dR1 = zero4();
#pragma unroll
    for (int kb = 0; kb < NDT; ++kb) mma((kb & 1) ? dR1 : dR0, ld_frag(&sm.kf[n16 * LDD + kb * 16], g4), dS[kb]);
    mma(dR0, ld_frag(&sm.aqt[n16 * LDC], g4), dYf);
    const f32x4 dR = dR0 + dR1;
    f32x4 dB = zero4();
    mma(dB, ld_frag(&sm.tt[n16 * LDC], g4), dR);
    {
      float* bst = (float*)p.ds_stash + NR * D * D + rec * (CC * D);
      *(f32x4*)(bst + stash_tile_offset<float, D>(0, V, lane)) = dB;
    }
    const f32x4 dBf = -dB * *(const f32x4*)&sm.be[4 * g4];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      dS[dt] *= *(const f32x4*)&sm.egl[dt * 16 + 4 * g4];
      mma(dS[dt], ld_frag(&sm.qet[(dt * 16 + n16) * LDC], g4), dYf);
      mma(dS[dt], ld_frag(&sm.ket[(dt * 16 + n16) * LDC], g4), dBf);
    }
  }
  if (p.ds0) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) p.ds0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + 16 * V + n16] = dS[dt][i];
  }
}

// ---------------------------------------------------------------------------
// per-chunk gradients (one chain per head: no lane sums)
//   P1 = dY S0^T, P2 = dB S0^T, P3 = R dS^T        (wave w: key tile w)
//   dq  = e^G o P1 + [grams],   dk = -beta_e e^G o P2 + e^{G_L - G} o P3 + [grams]
//   dG  = e^G o (q o P1 - beta_e k o P2) - e^{G_L - G} o k o P3 + [grams]
//   dG_L += sum_i e^{G_L - G} o k o P3 + e^{G_L} o rowsum(dS o S0)
//   dlog_g_t = sum_{i >= t} dG_i (zero where the log-decay was clamped)
//   dv = diag(beta_w) dB,  dbeta_w = rowsum(dB o V),
//   dbeta_e = -rowsum(e^G o k o P2) + rowsum(dL o M[x=k])
// with dAq = dY R^T (j <= i), dL = -dB R^T (j < i) entering the grams
// exactly, channel by channel.
// ---------------------------------------------------------------------------
template <int D>
struct alignas(16) ChanGradSmem {
  static constexpr int LDD = D + 4;
  ChanOps<D> o;
  float v[CC * LDD];
  float dy[CC * LDD];
  float R[CC * LDD];
  float dB[CC * LDD];
  float raw[CC * LDD];   // unclamped log-decay (gradient mask)
  float dAq[CC * LDC];
  float dL[CC * LDC];
  float sdot[D];         // rowsum(dS o S0) per key channel
  float red[2][ChD<D>::NW][CC];   // per-wave partial row sums: dbeta_e, dbeta_w
};

template <int D>
__global__ void __launch_bounds__(64 * (D / 16)) chan_grads_kernel(ChanBwdArgs p) {
  typedef ChD<D> Cd;
  constexpr int NW = Cd::NW, NT = Cd::NT, NDT = Cd::NDT, LDD = Cd::LDD;
  __shared__ ChanGradSmem<D> sm;
  ChanOps<D>& o = sm.o;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int NC = (p.T + CC - 1) / CC;
  const int nchains = p.B * p.H;
  const int blk = xcd_remap(blockIdx.x, nchains * NC);
  const int c = blk % NC, chain = blk / NC;
  const int h = chain % p.H, b = chain / p.H;
  const int t0 = c * CC;
  const size_t NR = (size_t)nchains * NC;
  const size_t rec = rec_index(chain, c, nchains);
  const int d = 16 * wave + n16;   // this lane's key (and value) column
  const unsigned rsb = (unsigned)((size_t)p.H * D * 4);

  // stage the chunk: q, k, v, log-decay, dY (rows), scalars; this wave's R and
  // dB tiles into LDS rows; this wave's key rows of S0 and dS into registers
  f32x4 s0t[NDT], dst[NDT];
  {
    Stage<float, CC, D, 1, NT> sq, sk, sv, sl, sy;
    sq.fetch(chunk_rsrc(p.q, b, t0, p.T, p.H, h, D), rsb, tid);
    sk.fetch(chunk_rsrc(p.k, b, t0, p.T, p.H, h, D), rsb, tid);
    sv.fetch(chunk_rsrc(p.v, b, t0, p.T, p.H, h, D), rsb, tid);
    sl.fetch(chunk_rsrc(p.lg, b, t0, p.T, p.H, h, D), rsb, tid);
    sy.fetch(chunk_rsrc(p.dy, b, t0, p.T, p.H, h, D), rsb, tid);
    const float* srec = (const float*)p.s_stash + rec * (D * D);
    const float* drec = (const float*)p.ds_stash + rec * (D * D);
#pragma unroll
    for (int V = 0; V < NDT; ++V) {
      s0t[V] = *(const f32x4*)(srec + stash_tile_offset<float, D>(wave, V, lane));
      dst[V] = *(const f32x4*)(drec + stash_tile_offset<float, D>(wave, V, lane));
    }
    const f32x4 rt = *(const f32x4*)((const float*)p.s_stash + NR * D * D + rec * (CC * D) +
                                     stash_tile_offset<float, D>(0, wave, lane));
    const f32x4 bt = *(const f32x4*)((const float*)p.ds_stash + NR * D * D + rec * (CC * D) +
                                     stash_tile_offset<float, D>(0, wave, lane));
    const float be = chunk_scalar(p.be, b, t0, tid % CC, p.T, p.H, h);
    const float bw = chunk_scalar(p.bw, b, t0, tid % CC, p.T, p.H, h);
    sq.template commit_nat<LDD>(o.q, tid);
    sk.template commit_nat<LDD>(o.k, tid);
    sv.template commit_nat<LDD>(sm.v, tid);
    sl.template commit_nat<LDD>(o.G, tid);
    sl.template commit_nat<LDD>(sm.raw, tid);
    sy.template commit_nat<LDD>(sm.dy, tid);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sm.R[(4 * g4 + i) * LDD + d] = rt[i];
      sm.dB[(4 * g4 + i) * LDD + d] = bt[i];
    }
    if (tid < CC) {
      o.be[tid] = be;
      o.bw[tid] = bw;
    }
  }
  {   // rowsum(dS o S0) over this wave's key rows 16 wave + 4 g + i
    f32x4 s = zero4();
#pragma unroll
    for (int V = 0; V < NDT; ++V) s += s0t[V] * dst[V];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = s[e];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off, 64);
      if (n16 == 0) sm.sdot[16 * wave + 4 * g4 + e] = x;
    }
  }
  __syncthreads();
  chan_prefix<D>(o, tid);
  __syncthreads();
  chan_grams<D>(o, wave, lane);
  if (wave == 0 || wave == 1) {   // dAq = dY R^T (j <= i), dL = -dB R^T (j < i)
    const float* arow = (wave == 0) ? &sm.dy[n16 * LDD] : &sm.dB[n16 * LDD];
    const f32x4 acc = tile_nt<float, D>(arow, &sm.R[n16 * LDD], g4);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * g4 + ii, j = n16;
      if (wave == 0) sm.dAq[i * LDC + j] = (j <= i) ? acc[ii] : 0.f;
      else sm.dL[i * LDC + j] = (j < i) ? -acc[ii] : 0.f;
    }
  }
  __syncthreads();

  // P products on this wave's key tile (S0 / dS rows as fragments over k = v)
  f32x4 P1 = zero4(), P2 = zero4(), P3 = zero4();
#pragma unroll
  for (int kb = 0; kb < NDT; ++kb) {
    const f32x4 Sf = tile_transpose_raw(s0t[kb], lane);
    const f32x4 dSf = tile_transpose_raw(dst[kb], lane);
    mma(P1, ld_frag(&sm.dy[n16 * LDD + kb * 16], g4), Sf);
    mma(P2, ld_frag(&sm.dB[n16 * LDD + kb * 16], g4), Sf);
    mma(P3, ld_frag(&sm.R[n16 * LDD + kb * 16], g4), dSf);
  }
  // lane (g, n): rows i = 4 g + ii of column d; the column's operands in registers
  float Gc[CC], kc[CC], qc[CC];
#pragma unroll
  for (int j = 0; j < CC; ++j) {
    Gc[j] = o.G[j * LDD + d];
    kc[j] = o.k[j * LDD + d];
    qc[j] = o.q[j * LDD + d];
  }
  const float GL = Gc[CC - 1];
  float dq[4], dk[4], dG[4], dGLp = 0.f, pbe[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int i = 4 * g4 + ii;
    const float E = __expf(Gc[i]), F = __expf(GL - Gc[i]);
    const float bei = o.be[i];
    dq[ii] = E * P1[ii];
    dk[ii] = -bei * E * P2[ii] + F * P3[ii];
    dG[ii] = E * (qc[i] * P1[ii] - bei * kc[i] * P2[ii]) - F * kc[i] * P3[ii];
    dGLp += F * kc[i] * P3[ii];
    pbe[ii] = -E * kc[i] * P2[ii];
    // grams, row i as the query / erase side (j <= i) and as the key side (i <= j')
#pragma unroll
    for (int j = 0; j < CC; ++j) {
      if (j <= i) {
        const float ex = __expf(Gc[i] - Gc[j]);
        const float t1 = sm.dAq[i * LDC + j] * ex, t2 = sm.dL[i * LDC + j] * bei * ex;
        dq[ii] += t1 * kc[j];
        dk[ii] += t2 * kc[j];
        dG[ii] += (t1 * qc[i] + t2 * kc[i]) * kc[j];
      }
      if (j >= i) {
        const float ex = __expf(Gc[j] - Gc[i]);
        const float cc = (sm.dAq[j * LDC + i] * qc[j] + sm.dL[j * LDC + i] * o.be[j] * kc[j]) * ex;
        dk[ii] += cc;
        dG[ii] -= cc * kc[i];
      }
    }
  }
  // chunk-end decay: the column's dG_L, added to every token's suffix sum
  dGLp += __shfl_xor(dGLp, 16, 64);
  dGLp += __shfl_xor(dGLp, 32, 64);
  const float dGL = dGLp + o.eGL[d] * sm.sdot[d];
  // suffix sums over the chunk's rows (within the lane, then across g)
  float tot = (dG[0] + dG[1]) + (dG[2] + dG[3]);
  const float t1 = __shfl_down(tot, 16, 64), t2 = __shfl_down(tot, 32, 64), t3 = __shfl_down(tot, 48, 64);
  float above = dGL + (g4 < 3 ? t1 : 0.f) + (g4 < 2 ? t2 : 0.f) + (g4 < 1 ? t3 : 0.f);
  float dlg[4];
#pragma unroll
  for (int ii = 3; ii >= 0; --ii) {
    above += dG[ii];
    const float raw = sm.raw[(4 * g4 + ii) * LDD + d];
    dlg[ii] = (raw <= 0.f && raw >= kLogFloor) ? above : 0.f;
  }
  // per-token sums: dbeta_e over the key columns, dbeta_w over the value columns
  float dvv[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int i = 4 * g4 + ii;
    const float dbv = sm.dB[i * LDD + d];
    dvv[ii] = o.bw[i] * dbv;
    float xe = pbe[ii], xw = dbv * sm.v[i * LDD + d];
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      xe += __shfl_xor(xe, off, 64);
      xw += __shfl_xor(xw, off, 64);
    }
    if (n16 == 0) {
      sm.red[0][wave][i] = xe;
      sm.red[1][wave][i] = xw;
    }
  }
  // stores: rows past T fall outside the buffer resources
  {
    const __amdgpu_buffer_rsrc_t rq = chunk_rsrc((const float*)p.dq, b, t0, p.T, p.H, h, D);
    const __amdgpu_buffer_rsrc_t rk = chunk_rsrc((const float*)p.dk, b, t0, p.T, p.H, h, D);
    const __amdgpu_buffer_rsrc_t rv = chunk_rsrc((const float*)p.dv, b, t0, p.T, p.H, h, D);
    const __amdgpu_buffer_rsrc_t rg = chunk_rsrc(p.dlg, b, t0, p.T, p.H, h, D);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const unsigned off = (unsigned)(4 * g4 + ii) * rsb + d * 4;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dq[ii]), rq, (int)off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dk[ii]), rk, (int)off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dvv[ii]), rv, (int)off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dlg[ii]), rg, (int)off, 0, 0);
    }
  }
  __syncthreads();
  if (tid < CC && t0 + tid < p.T) {
    float se = 0.f, sw = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      se += sm.red[0][w][tid];
      sw += sm.red[1][w][tid];
    }
    // the erase coefficient also scales L: + sum_j dL_ij M_ij
#pragma unroll
    for (int j = 0; j < CC; ++j) se += sm.dL[tid * LDC + j] * o.Mk[tid * LDC + j];
    const size_t si = ((size_t)b * p.T + t0 + tid) * p.H + h;
    p.dbe[si] = se;
    p.dbw[si] = sw;
  }
}

template <int D>
static int launch_chan_fwd(ChanArgs a, hipStream_t stream) {
  typedef ChRec<D> Rc;
  const int nchains = a.B * a.H, NC = (a.T + CC - 1) / CC;
  const size_t NR = (size_t)nchains * NC;
  const bool train = a.chunk_states != nullptr;
  a.frec = train ? (float*)a.chunk_states + NR * ((size_t)D * D + CC * D) : (float*)a.workspace;
  a.brec = train ? a.frec + NR * Rc::FN : nullptr;
  if (train)
    hipLaunchKernelGGL((chan_prep_kernel<D, true>), dim3(nchains * NC), dim3(64 * (D / 16)), 0, stream, a);
  else
    hipLaunchKernelGGL((chan_prep_kernel<D, false>), dim3(nchains * NC), dim3(64 * (D / 16)), 0, stream, a);
  int rc = check_launch("chan_prep_kernel");
  if (rc) return rc;
  if (a.r_norm) {   // one workgroup per chain: the update norm sums every value column
    constexpr int NW = D / 16;
    if (train)
      hipLaunchKernelGGL((chan_scan_fwd_kernel<D, NW, true, true>), dim3(nchains), dim3(64 * NW), 0, stream, a);
    else
      hipLaunchKernelGGL((chan_scan_fwd_kernel<D, NW, false, true>), dim3(nchains), dim3(64 * NW), 0, stream, a);
  } else {
    constexpr int NW = 4, NVB = D / 64;
    if (train)
      hipLaunchKernelGGL((chan_scan_fwd_kernel<D, NW, true, false>), dim3(nchains * NVB), dim3(64 * NW), 0, stream, a);
    else
      hipLaunchKernelGGL((chan_scan_fwd_kernel<D, NW, false, false>), dim3(nchains * NVB), dim3(64 * NW), 0, stream, a);
  }
  return check_launch("chan_scan_fwd_kernel");
}

template <int D>
static int launch_chan_bwd(const ChanBwdArgs& a, hipStream_t stream) {
  const int NC = (a.T + CC - 1) / CC;
  constexpr int NW = 4, NVB = D / 64;
  hipLaunchKernelGGL((chan_scan_bwd_kernel<D, NW>), dim3(a.B * a.H * NVB), dim3(64 * NW), 0, stream, a);
  int rc = check_launch("chan_scan_bwd_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((chan_grads_kernel<D>), dim3(a.B * a.H * NC), dim3(64 * (D / 16)), 0, stream, a);
  return check_launch("chan_grads_kernel");
}

int chan_fwd_dispatch(const ChanArgs& a, hipStream_t stream) {
  if (a.D == 128) return launch_chan_fwd<128>(a, stream);
  if (a.D == 64) return launch_chan_fwd<64>(a, stream);
  return set_error(GDNX_ERR_SHAPE, "per-channel decay: head_dim %d unsupported (64 or 128)", a.D);
}

int chan_bwd_dispatch(const ChanBwdArgs& a, hipStream_t stream) {
  if (a.D == 128) return launch_chan_bwd<128>(a, stream);
  if (a.D == 64) return launch_chan_bwd<64>(a, stream);
  return set_error(GDNX_ERR_SHAPE, "per-channel decay: head_dim %d unsupported (64 or 128)", a.D);
}

size_t chan_states_bytes(int nchains, int T, int D) {
  const size_t NR = (size_t)nchains * ((T + CC - 1) / CC);
  const size_t rec = D == 128 ? ChRec<128>::FN + ChRec<128>::BN : ChRec<64>::FN + ChRec<64>::BN;
  return NR * ((size_t)D * D + (size_t)CC * D + rec) * 4;
}

size_t chan_fwd_workspace_bytes(int nchains, int T, int D) {
  const size_t NR = (size_t)nchains * ((T + CC - 1) / CC);
  return NR * (size_t)(D == 128 ? ChRec<128>::FN : ChRec<64>::FN) * 4;
}

}  // namespace gdnx

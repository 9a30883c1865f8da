// Chunked decoupled-erase delta rule, backward (gfx950).
//
// Forward per chunk (see delta_fwd.hip): R = T (W - diag(exp G) E S0),
// Y = diag(exp G) Q S0 + Aq R, S_C = gamma_C S0 + K^T diag(dec) R with
// E = diag(a_e) K, W = diag(a_w) V.  Given dY and dS_C:
//
//   dR   = diag(dec) K dS_C + Aq^T dY            dB = T^T dR
//   dS0  = gamma_C dS_C + (diag(exp G) Q)^T dY - (diag(a_e exp G) K)^T dB
//   dV   = diag(a_w) dB                          da_w = rowsum(dB o V)
//   dAq  = dY R^T (j<=i),  dL = -dB R^T (j<i)    (then through D, a_e, grams)
//   dQ   = diag(exp G) dY S0^T + dQK K
//   dK   = diag(dec) R dS_C^T - diag(a_e exp G) dB S0^T + dQK^T Q + (dKK + dKK^T) K
//   dG_i = exp(G_i) q_i.(dY S0^T)_i - a_e,i exp(G_i) k_i.(dB S0^T)_i + mask terms
//          + chunk-end terms; dg = reverse cumulative sum of dG in the chunk.
//
// Two kernels:
//   delta_bwd_state_kernel  one workgroup per chain, chunks in reverse order,
//     carries dS in registers (value columns split over the waves, like the
//     forward's S) and stashes dS_C of every chunk.  Needs no S0.
//   delta_bwd_grads_kernel  one workgroup per (batch, head, chunk), looping
//     over the M lanes that share q/k/v: recomputes T, R, dR, dB from the two
//     state stashes, runs the contractions over value columns with S0 / dS
//     staged in LDS, and sums the lanes' dq/dk/dv in registers (fixed order,
//     no atomics), so the lane expansion of the reference
//     (gdn3/gdn3_upgrade.py:785-787) costs no extra memory traffic.
// The reference differentiates its chunk graph with torch autograd
// (gdn3/gdn3_upgrade.py:467-521) and its KMD-2 TRSM by hand
// (gdn3/kmd2_fast_scan.py:143-160).
#include "delta_common.hpp"

namespace gdnx {

// ---------------------------------------------------------------------------
// reverse state scan
// ---------------------------------------------------------------------------
template <typename CT, int D, int C>
struct alignas(16) BwdStateSmem {
  typedef Dims<CT, D, C> Dm;
  CT q[C * Dm::LDD];
  CT k[C * Dm::LDD];
  CT kt[D * Dm::LDC];
  CT qt[D * Dm::LDC];    // (diag(exp G) Q)^T
  CT dyt[D * Dm::LDC];   // dY^T
  CT aqt[C * Dm::LDC];   // Aq^T [j][i]
  CT tt[C * Dm::LDC];    // T^T  [i][j] = T[j][i]
  float L[C * Dm::LDF];
  float LT[C * Dm::LDT];
  float Td[C * Dm::LDT];
  float G[C], gam[C], dec[C], ae[C];
};

template <typename CT, int D, int C>
__global__ void __launch_bounds__((Dims<CT, D, C>::NT)) delta_bwd_state_kernel(DeltaBwdArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NDT = Dm::NDT, NCT = Dm::NCT, VS = Dm::VS, NVT = Dm::NVT;
  constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF, NT = Dm::NT;
  __shared__ BwdStateSmem<CT, D, C> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H * p.M;
  const int chain = xcd_remap(blockIdx.x, nchains);
  const int m = chain % p.M;
  const int h = (chain / p.M) % p.H;
  const int b = chain / (p.M * p.H);
  const int v0 = wave * VS;
  const int NC = (p.T + C - 1) / C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t rsy = (size_t)p.H * p.M * D;
  const size_t yoff = (((size_t)b * p.T * p.H + h) * p.M + m) * D;
  const size_t st = (size_t)p.H * p.M;
  const size_t soff = ((size_t)b * p.T * p.H + h) * p.M + m;
  const ChunkScalars cs{sm.G, sm.gam, sm.dec, sm.ae, nullptr, nullptr};

  for (int i = tid; i < C * LDC; i += NT) {
    sm.aqt[i] = from_f<CT>(0.f);
    sm.tt[i] = from_f<CT>(0.f);
  }

  f32x4 dS[NDT][NVT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int vt = 0; vt < NVT; ++vt) {
      dS[dt][vt] = zero4();
      if (p.ds_final) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dS[dt][vt][i] = p.ds_final[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + v0 + vt * 16 + n16];
      }
    }

  const CT* qg = (const CT*)p.q + qoff;
  const CT* kg = (const CT*)p.k + qoff;
  const CT* yg = (const CT*)p.dy + yoff;
  TileRegs rq, rk, ry;
  ScalarRegs rsc;
  tile_fetch<CT, D, C>(rq, qg, rs, (NC - 1) * C, p.T, tid);
  tile_fetch<CT, D, C>(rk, kg, rs, (NC - 1) * C, p.T, tid);
  tile_fetch<CT, D, C>(ry, yg, rsy, (NC - 1) * C, p.T, tid);
  if (wave == 0) scal_fetch<C>(rsc, p.ae + soff, nullptr, p.g + soff, st, (NC - 1) * C, p.T, lane);

  for (int c = NC - 1; c >= 0; --c) {
    const int t0 = c * C;
    __syncthreads();
    tile_commit<CT, D, C>(rq, sm.q, sm.qt, tid);
    tile_commit<CT, D, C>(rk, sm.k, sm.kt, tid);
    tile_commit<CT, D, C>(ry, nullptr, sm.dyt, tid);
    if (wave == 0) scal_commit<C>(cs, rsc, lane);
    __syncthreads();
    if (c > 0) {
      tile_fetch<CT, D, C>(rq, qg, rs, t0 - C, p.T, tid);
      tile_fetch<CT, D, C>(rk, kg, rs, t0 - C, p.T, tid);
      tile_fetch<CT, D, C>(ry, yg, rsy, t0 - C, p.T, tid);
      if (wave == 0) scal_fetch<C>(rsc, p.ae + soff, nullptr, p.g + soff, st, t0 - C, p.T, lane);
    }
    for (int idx = tid; idx < D * C; idx += NT) {
      const int d = idx / C, i = idx % C;
      sm.qt[d * LDC + i] = from_f<CT>(to_f(sm.qt[d * LDC + i]) * sm.gam[i]);
    }
    chunk_grams<CT, D, C>(sm.k, sm.q, sm.L, sm.LT, sm.G, sm.ae, wave, lane, [&](int i, int j0, const float* v) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sm.aqt[(j0 + e) * LDC + i] = from_f<CT>(v[e]);
    });
    __syncthreads();
    invert_unit_lower<C>(
        sm.L, sm.LT, sm.Td, wave, lane, [&](int) { return 0; },
        [&](int i, int j, float t, int) { sm.tt[j * LDC + i] = from_f<CT>(t); });
    __syncthreads();

    // stash dS_C of this chunk
    Frag dSf[NDT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        dSf[kb][vt] = acc_frag((CT*)nullptr, dS[kb * TPS][vt], dS[kb * TPS + TPS - 1][vt]);
    {
      Frag* cst = (Frag*)p.ds_stash + ((size_t)chain * NC + c) * (NT * Dm::STASH_FRAGS);
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) cst[(kb * NVT + vt) * NT + tid] = dSf[kb][vt];
    }
    // dR = diag(dec) K dS + Aq^T dY
    f32x4 dR[NCT][NVT];
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      const f32x4 dj = *(const f32x4*)&sm.dec[it * 16 + 4 * g4];
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kb = 0; kb < NDT / TPS; ++kb)
          mma(acc, ld_frag(&sm.k[(it * 16 + n16) * LDD + kb * KS], g4), dSf[kb][vt]);
        acc *= dj;
#pragma unroll
        for (int kb = 0; kb < C; kb += KS)
          mma(acc, ld_frag(&sm.aqt[(it * 16 + n16) * LDC + kb], g4),
              ld_frag(&sm.dyt[(v0 + vt * 16 + n16) * LDC + kb], g4));
        dR[it][vt] = acc;
      }
    }
    // dB = T^T dR
    Frag dRf[NCT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NCT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) dRf[kb][vt] = acc_frag((CT*)nullptr, dR[kb * TPS][vt], dR[kb * TPS + TPS - 1][vt]);
    Frag dBf[NCT / TPS][NVT];
    {
      f32x4 dB[NCT][NVT];
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < NCT / TPS; ++kb)
            mma(acc, ld_frag(&sm.tt[(it * 16 + n16) * LDC + kb * KS], g4), dRf[kb][vt]);
          dB[it][vt] = acc;
        }
      // fragments of -diag(a_e exp G) dB over k = i
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) {
        const int r0 = kb * KS + 4 * g4, r1 = kb * KS + (TPS - 1) * 16 + 4 * g4;
        f32x4 s0, s1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s0[e] = -sm.ae[r0 + e] * sm.gam[r0 + e];
          s1[e] = -sm.ae[r1 + e] * sm.gam[r1 + e];
        }
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
          dBf[kb][vt] = acc_frag((CT*)nullptr, dB[kb * TPS][vt], dB[kb * TPS + TPS - 1][vt], s0, s1);
      }
    }
    // dS <- gamma_C dS + (diag(exp G) Q)^T dY - (diag(a_e exp G) K)^T dB
    {
      const float gl = sm.gam[C - 1];
      Frag dYf[NCT / TPS][NVT];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) dYf[kb][vt] = ld_frag(&sm.dyt[(v0 + vt * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) dS[dt][vt] *= gl;
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) {
          const Frag aq = ld_frag(&sm.qt[(dt * 16 + n16) * LDC + kb * KS], g4);
          const Frag ak = ld_frag(&sm.kt[(dt * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
          for (int vt = 0; vt < NVT; ++vt) {
            mma(dS[dt][vt], aq, dYf[kb][vt]);
            mma(dS[dt][vt], ak, dBf[kb][vt]);
          }
        }
      }
    }
  }
  if (p.ds0) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p.ds0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + v0 + vt * 16 + n16] = dS[dt][vt][i];
  }
}

// ---------------------------------------------------------------------------
// per-chunk gradients, lanes summed in-block
// ---------------------------------------------------------------------------
template <typename CT, int D, int C>
struct alignas(16) BwdGradSmem {
  typedef Dims<CT, D, C> Dm;
  static constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF;
  CT q[C * LDD];
  CT k[C * LDD];
  CT dy[C * LDD];
  CT qt[D * LDC];
  CT kt[D * LDC];
  CT vt[D * LDC];
  float KK[C * LDF];   // k_i . k_j  (lower)
  float QK[C * LDF];   // q_i . k_j  (lower incl. diagonal)
  float dQK[C * LDF];  // sum over lanes of dL/d(q_i.k_j)
  float dKK[C * LDF];  // sum over lanes of dL/d(k_i.k_j), j < i
  float G[C], gam[C], dec[C], ae[C], aw[C], graw[C], tmp[C];
  float red[4][Dm::NW][C];  // [quantity][wave][row] partial sums
  float scal[Dm::NW];
  union alignas(16) U {
    struct alignas(16) {
      CT dyt[D * LDC];
      CT ta[C * LDC], tb[C * LDC], tt[C * LDC], aqt[C * LDC];
      CT wm[C * LDD];
      float L[C * LDF], LT[C * Dm::LDT], Td[C * Dm::LDT];
    } p1;
    struct alignas(16) {
      CT X[D * LDD];   // S0, then dS  ([d][v], value-contiguous)
      CT R[C * LDD];
      CT dB[C * LDD];
      float Xm[C * LDF], AE[C * LDF];
    } p2;
    struct alignas(16) {
      CT A1[C * LDC], A2[C * LDC], A3[C * LDC];
    } p3;
  } u;
};

// sum a per-row value over the 16 lanes that share g (lane bits 0..3)
__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 4, 64);
  x += __shfl_xor(x, 8, 64);
  return x;
}

template <typename CT, int D, int C>
__global__ void __launch_bounds__((Dims<CT, D, C>::NT)) delta_bwd_grads_kernel(DeltaBwdArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NDT = Dm::NDT, NCT = Dm::NCT, VS = Dm::VS, NVT = Dm::NVT;
  constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF, NT = Dm::NT, NW = Dm::NW;
  constexpr int DPW = Dm::DPW;  // d tiles per wave in the d-partitioned phase
  constexpr int FL = FragLen<CT>::value;
  __shared__ BwdGradSmem<CT, D, C> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int NC = (p.T + C - 1) / C;
  const int nblocks = p.B * p.H * NC;
  const int blk = xcd_remap(blockIdx.x, nblocks);
  const int c = blk % NC;
  const int h = (blk / NC) % p.H;
  const int b = blk / (NC * p.H);
  const int t0 = c * C;
  const int v0 = wave * VS;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t rsy = (size_t)p.H * p.M * D;
  const size_t st = (size_t)p.H * p.M;

  stage_tile<CT, D, C>((const CT*)p.q + qoff, rs, t0, p.T, sm.q, sm.qt, tid);
  stage_tile<CT, D, C>((const CT*)p.k + qoff, rs, t0, p.T, sm.k, sm.kt, tid);
  stage_tile<CT, D, C>((const CT*)p.v + qoff, rs, t0, p.T, nullptr, sm.vt, tid);
  for (int i = tid; i < C * LDF; i += NT) {
    sm.dQK[i] = 0.f;
    sm.dKK[i] = 0.f;
  }
  f32x4 dQacc[NCT][DPW], dKacc[NCT][DPW], dVacc[NCT][NVT];
#pragma unroll
  for (int it = 0; it < NCT; ++it) {
#pragma unroll
    for (int dd = 0; dd < DPW; ++dd) dQacc[it][dd] = dKacc[it][dd] = zero4();
#pragma unroll
    for (int vt = 0; vt < NVT; ++vt) dVacc[it][vt] = zero4();
  }
  __syncthreads();
  {  // raw grams (shared by the lanes)
    constexpr int NP = NCT * (NCT + 1) / 2;
    for (int task = wave; task < 2 * NP; task += NW) {
      int it, jt;
      tri_pair(task >> 1, it, jt);
      const CT* arow = ((task & 1) == 0) ? &sm.k[(it * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
      const f32x4 acc = tile_nt<CT, D>(arow, &sm.k[(jt * 16 + n16) * LDD], g4);
      float* dst = ((task & 1) == 0) ? sm.KK : sm.QK;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) dst[(it * 16 + 4 * g4 + ii) * LDF + jt * 16 + n16] = acc[ii];
    }
  }
  __syncthreads();

  for (int m = 0; m < p.M; ++m) {
    const size_t chain = ((size_t)b * p.H + h) * p.M + m;
    const size_t yoff = (((size_t)b * p.T * p.H + h) * p.M + m) * D;
    const size_t soff = ((size_t)b * p.T * p.H + h) * p.M + m;
    const ChunkScalars cs{sm.G, sm.gam, sm.dec, sm.ae, sm.aw, sm.graw};
    stage_tile<CT, D, C>((const CT*)p.dy + yoff, rsy, t0, p.T, sm.dy, sm.u.p1.dyt, tid);
    if (wave == 0) prep_scalars<C>(cs, p.ae + soff, p.aw + soff, p.g + soff, st, t0, p.T, lane);
    __syncthreads();
    for (int idx = tid; idx < C * C; idx += NT) {
      const int i = idx / C, j = idx % C;
      const float Dij = (j <= i) ? __expf(sm.G[i] - sm.G[j]) : 0.f;
      const float Lij = (j < i) ? Dij * sm.ae[i] * sm.KK[i * LDF + j] : 0.f;
      sm.u.p1.L[i * LDF + j] = Lij;
      if ((i >> 4) == (j >> 4)) sm.u.p1.LT[j * Dm::LDT + (i & 15)] = Lij;
      sm.u.p1.aqt[j * LDC + i] = from_f<CT>((j <= i) ? Dij * sm.QK[i * LDF + j] : 0.f);
      sm.u.p1.ta[i * LDC + j] = from_f<CT>(0.f);
      sm.u.p1.tb[i * LDC + j] = from_f<CT>(0.f);
      sm.u.p1.tt[i * LDC + j] = from_f<CT>(0.f);
    }
    __syncthreads();
    invert_unit_lower<C>(
        sm.u.p1.L, sm.u.p1.LT, sm.u.p1.Td, wave, lane,
        [&](int j) { return make_float2(sm.aw[j], sm.ae[j] * sm.gam[j]); },
        [&](int i, int j, float t, float2 f) {
          sm.u.p1.ta[i * LDC + j] = from_f<CT>(t * f.x);
          sm.u.p1.tb[i * LDC + j] = from_f<CT>(t * f.y);
          sm.u.p1.tt[j * LDC + i] = from_f<CT>(t);
        });
    __syncthreads();
#pragma unroll
    for (int dd = 0; dd < DPW; ++dd) {
      const int dt = wave * DPW + dd;
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        const f32x4 acc = tile_nt<CT, C>(&sm.kt[(dt * 16 + n16) * LDC], &sm.u.p1.tb[(it * 16 + n16) * LDC], g4);
        st4(&sm.u.p1.wm[(it * 16 + n16) * LDD + dt * 16 + 4 * g4], -acc[0], -acc[1], -acc[2], -acc[3]);
      }
    }
    f32x4 Racc[NCT][NVT];
#pragma unroll
    for (int it = 0; it < NCT; ++it)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Racc[it][vt] = tile_nt<CT, C>(&sm.u.p1.ta[(it * 16 + n16) * LDC], &sm.vt[(v0 + vt * 16 + n16) * LDC], g4);
    __syncthreads();

    // ---- phase 1 (value columns split over waves) ----
    Frag Sf[NDT / TPS][NVT], dSf[NDT / TPS][NVT];
    {
      const Frag* s = (const Frag*)p.s_stash + (chain * NC + c) * (NT * Dm::STASH_FRAGS);
      const Frag* ds = (const Frag*)p.ds_stash + (chain * NC + c) * (NT * Dm::STASH_FRAGS);
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          Sf[kb][vt] = s[(kb * NVT + vt) * NT + tid];
          dSf[kb][vt] = ds[(kb * NVT + vt) * NT + tid];
        }
    }
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) {
        const Frag a = ld_frag(&sm.u.p1.wm[(it * 16 + n16) * LDD + kb * KS], g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) mma(Racc[it][vt], a, Sf[kb][vt]);
      }
    }
    f32x4 dB[NCT][NVT];
    {
      f32x4 dR[NCT][NVT];
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        const f32x4 dj = *(const f32x4*)&sm.dec[it * 16 + 4 * g4];
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < NDT / TPS; ++kb)
            mma(acc, ld_frag(&sm.k[(it * 16 + n16) * LDD + kb * KS], g4), dSf[kb][vt]);
          acc *= dj;
#pragma unroll
          for (int kb = 0; kb < C; kb += KS)
            mma(acc, ld_frag(&sm.u.p1.aqt[(it * 16 + n16) * LDC + kb], g4),
                ld_frag(&sm.u.p1.dyt[(v0 + vt * 16 + n16) * LDC + kb], g4));
          dR[it][vt] = acc;
        }
      }
      Frag dRf[NCT / TPS][NVT];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) dRf[kb][vt] = acc_frag((CT*)nullptr, dR[kb * TPS][vt], dR[kb * TPS + TPS - 1][vt]);
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < NCT / TPS; ++kb)
            mma(acc, ld_frag(&sm.u.p1.tt[(it * 16 + n16) * LDC + kb * KS], g4), dRf[kb][vt]);
          dB[it][vt] = acc;
        }
    }
    // dV += diag(a_w) dB ; da_w = rowsum(dB o V)
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      const f32x4 awi = *(const f32x4*)&sm.aw[it * 16 + 4 * g4];
      f32x4 part = zero4();
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) {
        dVacc[it][vt] += awi * dB[it][vt];
        const CT* vrow = &sm.vt[(v0 + vt * 16 + n16) * LDC + it * 16 + 4 * g4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) part[ii] += dB[it][vt][ii] * to_f(vrow[ii]);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const float s = sum16(part[ii]);
        if (n16 == 0) sm.red[0][wave][it * 16 + 4 * g4 + ii] = s;
      }
    }
    {  // <dS_C, S0>
      float s = 0.f;
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
          for (int e = 0; e < FL; ++e) s += to_f(Sf[kb][vt][e]) * to_f(dSf[kb][vt][e]);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) s += __shfl_xor(s, off, 64);
      if (lane == 0) sm.scal[wave] = s;
    }
    __syncthreads();  // phase-1 LDS (union p1) is dead from here on

    // ---- stage R, dB, S0 value-contiguous ----
#pragma unroll
    for (int it = 0; it < NCT; ++it)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int r = (it * 16 + 4 * g4 + ii) * LDD + v0 + vt * 16 + n16;
          sm.u.p2.R[r] = from_f<CT>(Racc[it][vt][ii]);
          sm.u.p2.dB[r] = from_f<CT>(dB[it][vt][ii]);
        }
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int e = 0; e < FL; ++e)
          sm.u.p2.X[(kb * KS + frag_row<CT>(e, g4)) * LDD + v0 + vt * 16 + n16] = Sf[kb][vt][e];
    __syncthreads();

    // ---- phase 2 (key columns split over waves): P1 = dY S0^T, P2 = dB S0^T ----
    {
      f32x4 r1[NCT], r2[NCT];
#pragma unroll
      for (int it = 0; it < NCT; ++it) r1[it] = r2[it] = zero4();
#pragma unroll
      for (int dd = 0; dd < DPW; ++dd) {
        const int dt = wave * DPW + dd;
        const int d = dt * 16 + n16;
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          const f32x4 P1 = tile_nt<CT, D>(&sm.dy[(it * 16 + n16) * LDD], &sm.u.p2.X[(dt * 16 + n16) * LDD], g4);
          const f32x4 P2 = tile_nt<CT, D>(&sm.u.p2.dB[(it * 16 + n16) * LDD], &sm.u.p2.X[(dt * 16 + n16) * LDD], g4);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = it * 16 + 4 * g4 + ii;
            dQacc[it][dd][ii] += sm.gam[i] * P1[ii];
            dKacc[it][dd][ii] -= sm.ae[i] * sm.gam[i] * P2[ii];
            r1[it][ii] += P1[ii] * to_f(sm.q[i * LDD + d]);
            r2[it][ii] += P2[ii] * to_f(sm.k[i * LDD + d]);
          }
        }
      }
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const float s1 = sum16(r1[it][ii]), s2 = sum16(r2[it][ii]);
          if (n16 == 0) {
            sm.red[1][wave][it * 16 + 4 * g4 + ii] = s1;
            sm.red[2][wave][it * 16 + 4 * g4 + ii] = s2;
          }
        }
    }
    // dAq = dY R^T (j <= i) and dL = -dB R^T (j < i), lower tiles
    {
      constexpr int NP = NCT * (NCT + 1) / 2;
      for (int pidx = wave; pidx < NP; pidx += NW) {
        int it, jt;
        tri_pair(pidx, it, jt);
        const f32x4 aA = tile_nt<CT, D>(&sm.dy[(it * 16 + n16) * LDD], &sm.u.p2.R[(jt * 16 + n16) * LDD], g4);
        const f32x4 aL = tile_nt<CT, D>(&sm.u.p2.dB[(it * 16 + n16) * LDD], &sm.u.p2.R[(jt * 16 + n16) * LDD], g4);
        const int j = jt * 16 + n16;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = it * 16 + 4 * g4 + ii;
          float xm = 0.f, ae = 0.f;
          if (j <= i) {
            const float Dij = __expf(sm.G[i] - sm.G[j]);
            const float dqk = aA[ii] * Dij;
            sm.dQK[i * LDF + j] += dqk;
            xm = dqk * sm.QK[i * LDF + j];
            if (j < i) {
              const float dl = -aL[ii];
              const float dkk = dl * Dij * sm.ae[i];
              sm.dKK[i * LDF + j] += dkk;
              xm += dkk * sm.KK[i * LDF + j];
              ae = dl * Dij * sm.KK[i * LDF + j];
            }
          }
          sm.u.p2.Xm[i * LDF + j] = xm;
          sm.u.p2.AE[i * LDF + j] = ae;
        }
      }
    }
    __syncthreads();
    // ---- P3 = R dS^T ----
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int e = 0; e < FL; ++e)
          sm.u.p2.X[(kb * KS + frag_row<CT>(e, g4)) * LDD + v0 + vt * 16 + n16] = dSf[kb][vt][e];
    __syncthreads();
    {
      f32x4 r3[NCT];
#pragma unroll
      for (int it = 0; it < NCT; ++it) r3[it] = zero4();
#pragma unroll
      for (int dd = 0; dd < DPW; ++dd) {
        const int dt = wave * DPW + dd;
        const int d = dt * 16 + n16;
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          const f32x4 P3 = tile_nt<CT, D>(&sm.u.p2.R[(it * 16 + n16) * LDD], &sm.u.p2.X[(dt * 16 + n16) * LDD], g4);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int j = it * 16 + 4 * g4 + ii;
            dKacc[it][dd][ii] += sm.dec[j] * P3[ii];
            r3[it][ii] += P3[ii] * to_f(sm.k[j * LDD + d]);
          }
        }
      }
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const float s3 = sum16(r3[it][ii]);
          if (n16 == 0) sm.red[3][wave][it * 16 + 4 * g4 + ii] = s3;
        }
    }
    __syncthreads();
    // ---- per-token scalar gradients of this lane ----
    float dGi = 0.f, daei = 0.f, dawi = 0.f;
    if (tid < C) {
      const int i = tid;
      float r1 = 0.f, r2 = 0.f, r3 = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        dawi += sm.red[0][w][i];
        r1 += sm.red[1][w][i];
        r2 += sm.red[2][w][i];
        r3 += sm.red[3][w][i];
      }
      dGi = sm.gam[i] * r1 - sm.gam[i] * sm.ae[i] * r2 - sm.dec[i] * r3;
      daei = -sm.gam[i] * r2;
      for (int j = 0; j <= i; ++j) dGi += sm.u.p2.Xm[i * LDF + j];
      for (int j = i; j < C; ++j) dGi -= sm.u.p2.Xm[j * LDF + i];
      for (int j = 0; j < i; ++j) daei += sm.u.p2.AE[i * LDF + j];
      sm.tmp[i] = sm.dec[i] * r3;
    }
    __syncthreads();
    if (wave == 0) {
      if (lane == C - 1) {
        float s = 0.f;
        for (int w = 0; w < NW; ++w) s += sm.scal[w];
        s *= sm.gam[C - 1];
        for (int j = 0; j < C; ++j) s += sm.tmp[j];
        dGi += s;
      }
      // dg_s = sum_{i >= s} dG_i (suffix sum within the chunk)
      float sfx = (lane < C) ? dGi : 0.f;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_down(sfx, off, 64);
        if (lane + off < 64) sfx += o;
      }
      const int t = t0 + lane;
      if (lane < C && t < p.T) {
        const size_t si = ((size_t)(b * p.T + t) * p.H + h) * p.M + m;
        const float raw = sm.graw[lane];
        p.dae[si] = daei;
        p.daw[si] = dawi;
        p.dg[si] = (raw <= 0.f && raw >= kLogFloor) ? sfx : 0.f;
      }
    }
    __syncthreads();
  }

  // ---- gram gradient products, shared over lanes ----
  for (int idx = tid; idx < C * C; idx += NT) {
    const int i = idx / C, j = idx % C;
    sm.u.p3.A1[i * LDC + j] = from_f<CT>((j <= i) ? sm.dQK[i * LDF + j] : 0.f);
    sm.u.p3.A2[i * LDC + j] = from_f<CT>((i <= j) ? sm.dQK[j * LDF + i] : 0.f);
    const float s = (j < i) ? sm.dKK[i * LDF + j] : ((i < j) ? sm.dKK[j * LDF + i] : 0.f);
    sm.u.p3.A3[i * LDC + j] = from_f<CT>(s);
  }
  __syncthreads();
#pragma unroll
  for (int dd = 0; dd < DPW; ++dd) {
    const int dt = wave * DPW + dd;
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      dQacc[it][dd] += tile_nt<CT, C>(&sm.u.p3.A1[(it * 16 + n16) * LDC], &sm.kt[(dt * 16 + n16) * LDC], g4);
      dKacc[it][dd] += tile_nt<CT, C>(&sm.u.p3.A2[(it * 16 + n16) * LDC], &sm.qt[(dt * 16 + n16) * LDC], g4);
      dKacc[it][dd] += tile_nt<CT, C>(&sm.u.p3.A3[(it * 16 + n16) * LDC], &sm.kt[(dt * 16 + n16) * LDC], g4);
    }
  }
  CT* dq = (CT*)p.dq;
  CT* dk = (CT*)p.dk;
  CT* dv = (CT*)p.dv;
#pragma unroll
  for (int it = 0; it < NCT; ++it)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int t = t0 + it * 16 + 4 * g4 + ii;
      if (t < p.T) {
        const size_t row = ((size_t)(b * p.T + t) * p.H + h) * D;
#pragma unroll
        for (int dd = 0; dd < DPW; ++dd) {
          const int d = (wave * DPW + dd) * 16 + n16;
          dq[row + d] = from_f<CT>(dQacc[it][dd][ii]);
          dk[row + d] = from_f<CT>(dKacc[it][dd][ii]);
        }
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) dv[row + v0 + vt * 16 + n16] = from_f<CT>(dVacc[it][vt][ii]);
      }
    }
}

// stages: bit 0 = reverse state scan, bit 1 = gradient kernel
template <typename CT, int D, int C>
static int launch_bwd(const DeltaBwdArgs& a, int stages, hipStream_t stream) {
  const int NC = (a.T + C - 1) / C;
  if (stages & 1) {
    hipLaunchKernelGGL((delta_bwd_state_kernel<CT, D, C>), dim3(a.B * a.H * a.M), dim3(Dims<CT, D, C>::NT), 0, stream, a);
    const int rc = check_launch("delta_bwd_state_kernel");
    if (rc) return rc;
  }
  if (stages & 2) {
    hipLaunchKernelGGL((delta_bwd_grads_kernel<CT, D, C>), dim3(a.B * a.H * NC), dim3(Dims<CT, D, C>::NT), 0, stream, a);
    return check_launch("delta_bwd_grads_kernel");
  }
  return GDNX_OK;
}

int delta_bwd_dispatch(const DeltaBwdArgs& a, int stages, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 32) return launch_bwd<bf16, 128, 32>(a, stages, stream);
    if (a.D == 64 && a.C == 32) return launch_bwd<bf16, 64, 32>(a, stages, stream);
  } else {
    if (a.D == 128 && a.C == 16) return launch_bwd<float, 128, 16>(a, stages, stream);
    if (a.D == 64 && a.C == 16) return launch_bwd<float, 64, 16>(a, stages, stream);
    if (a.D == 64 && a.C == 32) return launch_bwd<float, 64, 32>(a, stages, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "backward: unsupported head dim %d / chunk %d for this dtype (use "
                   "gdnx_delta_train_chunk_size)", a.D, a.C);
}

}  // namespace gdnx

// Chunked decoupled-erase delta rule, forward (gfx950).
//
// One workgroup (4 waves) per chain = (batch, head, lane).  The lanes of a
// head share q/k/v (the reference expands them, gdn3/gdn3_upgrade.py:785-787)
// and differ in the per-token erase/write coefficients a_e, a_w and the
// log-decay g.  Per chunk of C tokens with carried state S0 [Dk, Dv] (fp32,
// in registers, wave w owning value columns [w*D/4, (w+1)*D/4)):
//
//   G_i  = sum_{s<=i} g_s,  D_ij = exp(G_i - G_j) [j<=i]
//   L_ij = D_ij a_e,i (k_i.k_j) [j<i],  T = (I + L)^-1       (fp32, blocked)
//   U    = T diag(a_w) V,   Wm = T diag(a_e exp G) K           (WY form)
//   R    = U - Wm S0                                           (net writes)
//   Y    = diag(exp G) Q S0 + (D o Q K^T) R
//   S    = exp(G_last) S0 + K^T diag(D_last,:) R
//
// which is gdn3/_reference_recurrence.py:60-84 (dense regime) and
// research/kernel_ab/ref_scan.py:40-45 restated per chunk.  All products run
// on MFMA (bf16 with fp32 accumulation, or fp32 MFMA for the fp32 path); K,
// Q, V, T-derived tiles are staged in LDS; S0 and R stay in registers.
#include "delta_common.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct alignas(16) FwdSmem {
  typedef Dims<CT, D, C> Dm;
  CT q[C * Dm::LDD];
  CT k[C * Dm::LDD];
  CT wm[C * Dm::LDD];   // -Wm
  CT kt[D * Dm::LDC];   // K^T
  CT vt[D * Dm::LDC];   // V^T
  CT ta[C * Dm::LDC];   // T diag(a_w)
  CT tb[C * Dm::LDC];   // T diag(a_e exp G)
  CT aq[C * Dm::LDC];   // D o Q K^T
  float L[C * Dm::LDF];
  float T[C * Dm::LDF];
  float G[C], gam[C], dec[C], ae[C], aw[C];
};

template <typename CT, int D, int C>
__global__ void __launch_bounds__(256) delta_fwd_kernel(DeltaArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NDT = Dm::NDT, NCT = Dm::NCT, VS = Dm::VS, NVT = Dm::NVT;
  constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF;

  __shared__ FwdSmem<CT, D, C> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int nchains = p.B * p.H * p.M;
  const int chain = xcd_remap(blockIdx.x, nchains);
  const int m = chain % p.M;
  const int h = (chain / p.M) % p.H;
  const int b = chain / (p.M * p.H);
  const int v0 = wave * VS;
  const int NC = (p.T + C - 1) / C;
  const size_t rs = (size_t)p.H * D;                                  // q/k/v token stride
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t st = (size_t)p.H * p.M;                                // scalar token stride
  const size_t soff = ((size_t)b * p.T * p.H + h) * p.M + m;
  const ChunkScalars cs{sm.G, sm.gam, sm.dec, sm.ae, sm.aw, nullptr};

  // strictly-upper parts never written below must read as zero
  for (int i = tid; i < C * LDF; i += 256) sm.T[i] = 0.f;
  for (int i = tid; i < C * LDC; i += 256) sm.aq[i] = from_f<CT>(0.f);

  f32x4 S[NDT][NVT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int vt = 0; vt < NVT; ++vt) {
      S[dt][vt] = zero4();
      if (p.s0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          S[dt][vt][i] = p.s0[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + v0 + vt * 16 + n16];
      }
    }

  for (int c = 0; c < NC; ++c) {
    const int t0 = c * C;
    __syncthreads();
    stage_tile<CT, D, C>((const CT*)p.q + qoff, rs, t0, p.T, sm.q, nullptr, tid);
    stage_tile<CT, D, C>((const CT*)p.k + qoff, rs, t0, p.T, sm.k, sm.kt, tid);
    stage_tile<CT, D, C>((const CT*)p.v + qoff, rs, t0, p.T, nullptr, sm.vt, tid);
    if (wave == 0) prep_scalars<C>(cs, p.ae + soff, p.aw + soff, p.g + soff, st, t0, p.T, lane);
    __syncthreads();

    // ---- grams: L (from K K^T, lower) and Aq (from K Q^T, lower) ----
    {
      constexpr int NP = NCT * (NCT + 1) / 2;
      for (int task = wave; task < 2 * NP; task += 4) {
        int it, jt;
        tri_pair(task >> 1, it, jt);
        if ((task & 1) == 0) {
          // acc[ii] = k_i . k_j, i = it*16+4g+ii, j = jt*16+n
          const f32x4 acc = tile_nt<CT, D>(&sm.k[(it * 16 + n16) * LDD], &sm.k[(jt * 16 + n16) * LDD], g4);
          const int j = jt * 16 + n16;
          const float Gj = sm.G[j];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = it * 16 + 4 * g4 + ii;
            sm.L[i * LDF + j] = (j < i) ? __expf(sm.G[i] - Gj) * sm.ae[i] * acc[ii] : 0.f;
          }
        } else {
          // acc[ii] = q_i . k_j, i = it*16+n, j = jt*16+4g+ii
          const f32x4 acc = tile_nt<CT, D>(&sm.k[(jt * 16 + n16) * LDD], &sm.q[(it * 16 + n16) * LDD], g4);
          const int i = it * 16 + n16;
          const float Gi = sm.G[i];
          float vals[4];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int j = jt * 16 + 4 * g4 + ii;
            vals[ii] = (j <= i) ? __expf(Gi - sm.G[j]) * acc[ii] : 0.f;
          }
          st4(&sm.aq[i * LDC + jt * 16 + 4 * g4], vals[0], vals[1], vals[2], vals[3]);
        }
      }
    }
    __syncthreads();
    invert_unit_lower<C>(sm.L, sm.T, wave, lane);

    // ---- TA = T diag(a_w), TB = T diag(a_e exp G) ----
    for (int idx = tid; idx < C * C; idx += 256) {
      const int i = idx / C, j = idx % C;
      const float t = sm.T[i * LDF + j];
      sm.ta[i * LDC + j] = from_f<CT>(t * sm.aw[j]);
      sm.tb[i * LDC + j] = from_f<CT>(t * sm.ae[j] * sm.gam[j]);
    }
    __syncthreads();

    // ---- -Wm (rows i, cols d) via Wm^T = K^T TB^T; this wave's d tiles ----
#pragma unroll
    for (int dd = 0; dd < NDT / 4; ++dd) {
      const int dt = wave * (NDT / 4) + dd;
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        // acc[ii] = Wm[i = it*16+n][d = dt*16+4g+ii]
        const f32x4 acc = tile_nt<CT, C>(&sm.kt[(dt * 16 + n16) * LDC], &sm.tb[(it * 16 + n16) * LDC], g4);
        st4(&sm.wm[(it * 16 + n16) * LDD + dt * 16 + 4 * g4], -acc[0], -acc[1], -acc[2], -acc[3]);
      }
    }
    // ---- U = TA V (this wave's value columns) into the R accumulators ----
    f32x4 Racc[NCT][NVT];
#pragma unroll
    for (int it = 0; it < NCT; ++it)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Racc[it][vt] = tile_nt<CT, C>(&sm.ta[(it * 16 + n16) * LDC], &sm.vt[(v0 + vt * 16 + n16) * LDC], g4);
    __syncthreads();

    // ---- S0 fragments over k = d (stashed for the backward) ----
    Frag Sf[NDT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Sf[kb][vt] = acc_frag((CT*)nullptr, S[kb * TPS][vt], S[kb * TPS + TPS - 1][vt]);
    if (p.chunk_states) {
      Frag* cst = (Frag*)p.chunk_states + ((size_t)chain * NC + c) * (256 * Dm::STASH_FRAGS);
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) cst[(kb * NVT + vt) * 256 + tid] = Sf[kb][vt];
    }

    // ---- R = U - Wm S0 ----
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      const CT* arow = &sm.wm[(it * 16 + n16) * LDD];
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) {
        const Frag a = ld_frag(arow + kb * KS, g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) mma(Racc[it][vt], a, Sf[kb][vt]);
      }
    }
    // ---- Y = diag(exp G) Q S0 + Aq R ----
    f32x4 Yacc[NCT][NVT];
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) Yacc[it][vt] = zero4();
      const CT* arow = &sm.q[(it * 16 + n16) * LDD];
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) {
        const Frag a = ld_frag(arow + kb * KS, g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) mma(Yacc[it][vt], a, Sf[kb][vt]);
      }
      const f32x4 gi = *(const f32x4*)&sm.gam[it * 16 + 4 * g4];
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) Yacc[it][vt] *= gi;
    }
    Frag Rf[NCT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NCT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Rf[kb][vt] = acc_frag((CT*)nullptr, Racc[kb * TPS][vt], Racc[kb * TPS + TPS - 1][vt]);
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      const CT* arow = &sm.aq[(it * 16 + n16) * LDC];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) {
        const Frag a = ld_frag(arow + kb * KS, g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) mma(Yacc[it][vt], a, Rf[kb][vt]);
      }
    }
    {
      CT* yg = (CT*)p.y;
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int t = t0 + it * 16 + 4 * g4 + ii;
          if (t < p.T) {
            const size_t off = (((size_t)(b * p.T + t) * p.H + h) * p.M + m) * D + v0 + n16;
#pragma unroll
            for (int vt = 0; vt < NVT; ++vt) yg[off + vt * 16] = from_f<CT>(Yacc[it][vt][ii]);
          }
        }
    }
    // ---- S = exp(G_last) S0 + K^T diag(dec) R ----
    {
      const float gl = sm.gam[C - 1];
      Frag RDf[NCT / TPS][NVT];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb) {
        const f32x4 d0 = *(const f32x4*)&sm.dec[kb * KS + 4 * g4];
        const f32x4 d1 = *(const f32x4*)&sm.dec[kb * KS + (TPS - 1) * 16 + 4 * g4];
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
          RDf[kb][vt] = acc_frag((CT*)nullptr, Racc[kb * TPS][vt], Racc[kb * TPS + TPS - 1][vt], d0, d1);
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const CT* arow = &sm.kt[(dt * 16 + n16) * LDC];
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) S[dt][vt] *= gl;
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) {
          const Frag a = ld_frag(arow + kb * KS, g4);
#pragma unroll
          for (int vt = 0; vt < NVT; ++vt) mma(S[dt][vt], a, RDf[kb][vt]);
        }
      }
    }
  }

  if (p.s_out) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p.s_out[(size_t)chain * D * D + (dt * 16 + 4 * g4 + i) * D + v0 + vt * 16 + n16] = S[dt][vt][i];
  }
}

template <typename CT, int D, int C>
static int launch_fwd(const DeltaArgs& a, hipStream_t stream) {
  const int nblocks = a.B * a.H * a.M;
  hipLaunchKernelGGL((delta_fwd_kernel<CT, D, C>), dim3(nblocks), dim3(256), 0, stream, a);
  return check_launch("delta_fwd_kernel");
}

int delta_fwd_dispatch(const DeltaArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 64) return launch_fwd<bf16, 128, 64>(a, stream);
    if (a.D == 128 && a.C == 32) return launch_fwd<bf16, 128, 32>(a, stream);
    if (a.D == 64 && a.C == 64) return launch_fwd<bf16, 64, 64>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_fwd<bf16, 64, 32>(a, stream);
  } else {
    if (a.D == 128 && a.C == 32) return launch_fwd<float, 128, 32>(a, stream);
    if (a.D == 128 && a.C == 16) return launch_fwd<float, 128, 16>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_fwd<float, 64, 32>(a, stream);
    if (a.D == 64 && a.C == 16) return launch_fwd<float, 64, 16>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "unsupported head dim %d / chunk %d for this dtype", a.D, a.C);
}

}  // namespace gdnx

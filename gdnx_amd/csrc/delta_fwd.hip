// Chunked decoupled-erase delta rule, forward (gfx950).
//
// One workgroup (NW waves, see Dims) per chain = (batch, head, lane).  The lanes of a
// head share q/k/v (the reference expands them, gdn3/gdn3_upgrade.py:785-787)
// and differ in the per-token erase/write coefficients a_e, a_w and the
// log-decay g.  Per chunk of C tokens with carried state S0 [Dk, Dv] (fp32,
// in registers, wave w owning value columns [w*D/NW, (w+1)*D/NW)):
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
  float LT[C * Dm::LDT];
  float Td[C * Dm::LDT];
  float G[C], gam[C], dec[C], ae[C], aw[C];
  float rn[4][C];       // per-wave partial |r_i|^2 (scored forward)
};

template <typename CT, int D, int C>
__global__ void __launch_bounds__((Dims<CT, D, C>::NT)) delta_fwd_kernel(DeltaArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NDT = Dm::NDT, NCT = Dm::NCT, VS = Dm::VS, NVT = Dm::NVT;
  constexpr int LDD = Dm::LDD, LDC = Dm::LDC, NT = Dm::NT, DPW = Dm::DPW;

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
  const CT* qg = (const CT*)p.q + qoff;
  const CT* kg = (const CT*)p.k + qoff;
  const CT* vg = (const CT*)p.v + qoff;

  // never-written strictly-upper parts of TA, TB, Aq must read as zero
  for (int i = tid; i < C * LDC; i += NT) {
    sm.ta[i] = from_f<CT>(0.f);
    sm.tb[i] = from_f<CT>(0.f);
    sm.aq[i] = from_f<CT>(0.f);
  }

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

  TileRegs rq, rk, rv;
  ScalarRegs rsc;
  tile_fetch<CT, D, C>(rq, qg, rs, 0, p.T, tid);
  tile_fetch<CT, D, C>(rk, kg, rs, 0, p.T, tid);
  tile_fetch<CT, D, C>(rv, vg, rs, 0, p.T, tid);
  if (wave == 0) scal_fetch<C>(rsc, p.ae + soff, p.aw + soff, p.g + soff, st, 0, p.T, lane);

  for (int c = 0; c < NC; ++c) {
    const int t0 = c * C;
    __syncthreads();
    tile_commit<CT, D, C>(rq, sm.q, nullptr, tid);
    tile_commit<CT, D, C>(rk, sm.k, sm.kt, tid);
    tile_commit<CT, D, C>(rv, nullptr, sm.vt, tid);
    if (wave == 0) scal_commit<C>(cs, rsc, lane);
    __syncthreads();
    // prefetch the next chunk while this one computes
    if (c + 1 < NC) {
      tile_fetch<CT, D, C>(rq, qg, rs, t0 + C, p.T, tid);
      tile_fetch<CT, D, C>(rk, kg, rs, t0 + C, p.T, tid);
      tile_fetch<CT, D, C>(rv, vg, rs, t0 + C, p.T, tid);
      if (wave == 0) scal_fetch<C>(rsc, p.ae + soff, p.aw + soff, p.g + soff, st, t0 + C, p.T, lane);
    }

    {
      // ---- grams: L (K K^T) and Aq (Q K^T) ----
      chunk_grams<CT, D, C>(sm.k, sm.q, sm.L, sm.LT, sm.G, sm.ae, wave, lane,
                            [&](int i, int j0, const float* v) { st4(&sm.aq[i * LDC + j0], v[0], v[1], v[2], v[3]); });
      __syncthreads();
      // ---- T = (I + L)^-1, emitted as TA = T diag(a_w), TB = T diag(a_e exp G) ----
      invert_unit_lower<C>(
          sm.L, sm.LT, sm.Td, wave, lane,
          [&](int j) { return make_float2(sm.aw[j], sm.ae[j] * sm.gam[j]); },
          [&](int i, int j, float t, float2 f) {
            sm.ta[i * LDC + j] = from_f<CT>(t * f.x);
            sm.tb[i * LDC + j] = from_f<CT>(t * f.y);
          });
      __syncthreads();
    }

    // ---- -Wm (rows i, cols d) via Wm^T = K^T TB^T; this wave's d tiles ----
#pragma unroll
    for (int dd = 0; dd < DPW; ++dd) {
      const int dt = wave * DPW + dd;
      Frag a[C / KS];
#pragma unroll
      for (int kb = 0; kb < C / KS; ++kb) a[kb] = ld_frag(&sm.kt[(dt * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kb = 0; kb < C / KS; ++kb) mma(acc, a[kb], ld_frag(&sm.tb[(it * 16 + n16) * LDC + kb * KS], g4));
        // acc[ii] = Wm[i = it*16+n][d = dt*16+4g+ii]
        st4(&sm.wm[(it * 16 + n16) * LDD + dt * 16 + 4 * g4], -acc[0], -acc[1], -acc[2], -acc[3]);
      }
    }
    // ---- U = TA V (this wave's value columns) into the R accumulators ----
    f32x4 Racc[NCT][NVT];
    {
      Frag bv[NVT][C / KS];
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
#pragma unroll
        for (int kb = 0; kb < C / KS; ++kb) bv[vt][kb] = ld_frag(&sm.vt[(v0 + vt * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        Frag a[C / KS];
#pragma unroll
        for (int kb = 0; kb < C / KS; ++kb) a[kb] = ld_frag(&sm.ta[(it * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          Racc[it][vt] = zero4();
#pragma unroll
          for (int kb = 0; kb < C / KS; ++kb) mma(Racc[it][vt], a[kb], bv[vt][kb]);
        }
      }
    }

    // ---- S0 fragments over k = d ----
    Frag Sf[NDT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Sf[kb][vt] = acc_frag((CT*)nullptr, S[kb * TPS][vt], S[kb * TPS + TPS - 1][vt]);
    if (p.chunk_states && c % p.cps == 0) {  // stash S0 for the backward (raw tiles), every cps-th chunk
      CT* cst = (CT*)p.chunk_states + ((size_t)(c / p.cps) * nchains + chain) * (D * D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
          st4(cst + stash_tile_offset<CT, D>(dt, wave * NVT + vt, lane), S[dt][vt][0], S[dt][vt][1], S[dt][vt][2],
              S[dt][vt][3]);
    }
    __syncthreads();   // -Wm complete

    // ---- R = U - Wm S0 ----
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb) {
        const Frag a = ld_frag(&sm.wm[(it * 16 + n16) * LDD + kb * KS], g4);
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) mma(Racc[it][vt], a, Sf[kb][vt]);
      }
    }
    if (p.chunk_states) {  // stash R after all states: raw accumulator tiles (stash_tiles layout)
      CT* rst = (CT*)p.chunk_states + stash_geom(nchains, p.T, D, C, p.cps).states +
                rec_index(chain, c, nchains) * (C * D);
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
          st4(rst + ((it * NDT + wave * NVT + vt) * 64 + lane) * 4, Racc[it][vt][0], Racc[it][vt][1],
              Racc[it][vt][2], Racc[it][vt][3]);
    }
    if (p.r_norm) {  // |r_i| per token: squares over this wave's value columns, then across waves
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        f32x4 ss = zero4();
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) ss += Racc[it][vt] * Racc[it][vt];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = ss[e];
#pragma unroll
          for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off, 64);
          if (n16 == 0) sm.rn[wave][it * 16 + 4 * g4 + e] = x;
        }
      }
      __syncthreads();
      if (tid < C && t0 + tid < p.T)
        p.r_norm[((size_t)(b * p.T + t0 + tid) * p.H + h) * p.M + m] =
            sqrtf((sm.rn[0][tid] + sm.rn[1][tid]) + (sm.rn[2][tid] + sm.rn[3][tid]));
    }
    // ---- Y = diag(exp G) Q S0 + Aq R, one 16-row block at a time ----
    {
      Frag Rf[NCT / TPS][NVT];
#pragma unroll
      for (int kb = 0; kb < NCT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt)
          Rf[kb][vt] = acc_frag((CT*)nullptr, Racc[kb * TPS][vt], Racc[kb * TPS + TPS - 1][vt]);
      CT* yg = (CT*)p.y;
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        f32x4 Yacc[NVT];
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) Yacc[vt] = zero4();
#pragma unroll
        for (int kb = 0; kb < NDT / TPS; ++kb) {
          const Frag a = ld_frag(&sm.q[(it * 16 + n16) * LDD + kb * KS], g4);
#pragma unroll
          for (int vt = 0; vt < NVT; ++vt) mma(Yacc[vt], a, Sf[kb][vt]);
        }
        const f32x4 gi = *(const f32x4*)&sm.gam[it * 16 + 4 * g4];
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) Yacc[vt] *= gi;
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) {
          const Frag a = ld_frag(&sm.aq[(it * 16 + n16) * LDC + kb * KS], g4);
#pragma unroll
          for (int vt = 0; vt < NVT; ++vt) mma(Yacc[vt], a, Rf[kb][vt]);
        }
        // transposed tiles: lane (g, n) holds row it*16+n, columns 4g..4g+3
        const int t = t0 + it * 16 + n16;
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) {
          const f32x4 yt = tile_transpose((CT*)nullptr, Yacc[vt], lane);
          if (t < p.T) {
            const size_t off = (((size_t)(b * p.T + t) * p.H + h) * p.M + m) * D + v0 + vt * 16 + 4 * g4;
            st4(yg + off, yt[0], yt[1], yt[2], yt[3]);
          }
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
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) S[dt][vt] *= gl;
#pragma unroll
        for (int kb = 0; kb < NCT / TPS; ++kb) {
          const Frag a = ld_frag(&sm.kt[(dt * 16 + n16) * LDC + kb * KS], g4);
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
  hipLaunchKernelGGL((delta_fwd_kernel<CT, D, C>), dim3(a.B * a.H * a.M), dim3(Dims<CT, D, C>::NT), 0, stream, a);
  return check_launch("delta_fwd_kernel");
}

static int delta_fused_dispatch(const DeltaArgs& a, hipStream_t stream) {
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

// With somewhere to put the per-chunk operands (the prep region of
// chunk_states, else the workspace) the forward is the parallel prep kernel
// plus the value-split lean scan; the scored variant (|r_t| needs every value
// column of a token in one workgroup) and calls without either buffer run
// the fused single-kernel scan.  A stash for the backward always gets its
// prep records, which the reverse scan reads.
int delta_fwd_dispatch(const DeltaArgs& a, hipStream_t stream) {
  DeltaArgs b = a;
  if (a.chunk_states)
    b.prep = (char*)a.chunk_states + delta_stash_bytes(a.B * a.H * a.M, a.T, a.D, a.C, a.dtype, a.cps);
  if (b.prep && !a.r_norm) {
    const int rc = delta_prep_dispatch(b, stream);
    return rc ? rc : delta_scan_fwd_dispatch(b, stream);
  }
  const int rc = delta_fused_dispatch(a, stream);
  if (rc || !a.chunk_states) return rc;
  return delta_prep_dispatch(b, stream);
}

}  // namespace gdnx

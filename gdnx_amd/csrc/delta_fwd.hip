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
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct alignas(16) FwdSmem {
  static constexpr int LDD = D + 4;   // row length for [*, D] tiles
  static constexpr int LDC = C + 4;   // row length for [*, C] tiles
  static constexpr int LDF = C + 1;   // fp32 scratch rows
  CT q[C * LDD];
  CT k[C * LDD];
  CT wm[C * LDD];   // -Wm
  CT kt[D * LDC];   // K^T
  CT vt[D * LDC];   // V^T
  CT ta[C * LDC];   // T diag(a_w)
  CT tb[C * LDC];   // T diag(a_e exp G)
  CT aq[C * LDC];   // D o Q K^T
  float L[C * LDF];
  float T[C * LDF];
  float G[C], gam[C], dec[C], ae[C], aw[C];
};

// Load one chunk's q/k/v rows into LDS (natural layouts for q, k; transposed
// layouts for k, v) plus the per-token scalars and their prefix sums.
template <typename CT, int D, int C>
__device__ __forceinline__ void load_chunk(FwdSmem<CT, D, C>& sm, const DeltaArgs& p, int b, int h,
                                           int m, int t0, int tid) {
  constexpr int VEC = 16 / sizeof(CT);
  constexpr int DG = D / VEC;
  constexpr int LDD = FwdSmem<CT, D, C>::LDD;
  constexpr int LDC = FwdSmem<CT, D, C>::LDC;
  const CT* qg = (const CT*)p.q;
  const CT* kg = (const CT*)p.k;
  const CT* vg = (const CT*)p.v;
  for (int u = tid; u < (C / 4) * DG; u += 256) {
    const int tg = u / DG, dg = u % DG;
    CT xq[4][VEC], xk[4][VEC], xv[4][VEC];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * tg + r;
      if (t < p.T) {
        const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + dg * VEC;
        *(uint4*)xq[r] = *(const uint4*)(qg + off);
        *(uint4*)xk[r] = *(const uint4*)(kg + off);
        *(uint4*)xv[r] = *(const uint4*)(vg + off);
      } else {
        *(uint4*)xq[r] = make_uint4(0, 0, 0, 0);
        *(uint4*)xk[r] = make_uint4(0, 0, 0, 0);
        *(uint4*)xv[r] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      CT* dq = &sm.q[(4 * tg + r) * LDD + dg * VEC];
      CT* dk = &sm.k[(4 * tg + r) * LDD + dg * VEC];
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        *(uint2*)(dq + e) = *(const uint2*)(&xq[r][e]) ;
        *(uint2*)(dk + e) = *(const uint2*)(&xk[r][e]);
        if constexpr (sizeof(CT) == 4) {
          *(uint2*)(dq + e + 2) = *(const uint2*)(&xq[r][e + 2]);
          *(uint2*)(dk + e + 2) = *(const uint2*)(&xk[r][e + 2]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      CT* dkt = &sm.kt[(dg * VEC + e) * LDC + 4 * tg];
      CT* dvt = &sm.vt[(dg * VEC + e) * LDC + 4 * tg];
      st4(dkt, to_f(xk[0][e]), to_f(xk[1][e]), to_f(xk[2][e]), to_f(xk[3][e]));
      st4(dvt, to_f(xv[0][e]), to_f(xv[1][e]), to_f(xv[2][e]), to_f(xv[3][e]));
    }
  }
  if (tid < 64) {
    float ae = 0.f, aw = 0.f, g = 0.f;
    const int t = t0 + tid;
    if (tid < C && t < p.T) {
      const size_t si = ((size_t)(b * p.T + t) * p.H + h) * p.M + m;
      ae = p.ae[si];
      aw = p.aw[si];
      g = fmaxf(fminf(p.g[si], 0.f), kLogFloor);
    }
    // inclusive prefix sum over the wave
    float G = g;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      float o = __shfl_up(G, off, 64);
      if (tid >= off) G += o;
    }
    const float Glast = __shfl(G, C - 1, 64);
    if (tid < C) {
      sm.G[tid] = G;
      sm.gam[tid] = __expf(G);
      sm.dec[tid] = __expf(Glast - G);
      sm.ae[tid] = ae;
      sm.aw[tid] = aw;
    }
  }
}

template <typename CT, int D, int C>
__global__ void __launch_bounds__(256) delta_fwd_kernel(DeltaArgs p) {
  typedef typename FragT<CT>::type Frag;
  constexpr int KS = FragT<CT>::KSTEP;
  constexpr int TPS = FragT<CT>::TPS;
  constexpr int NDT = D / 16;      // d tiles
  constexpr int NCT = C / 16;      // chunk tiles
  constexpr int VS = D / 4;        // value columns per wave
  constexpr int NVT = VS / 16;     // value tiles per wave
  constexpr int LDD = FwdSmem<CT, D, C>::LDD;
  constexpr int LDC = FwdSmem<CT, D, C>::LDC;
  constexpr int LDF = FwdSmem<CT, D, C>::LDF;
  static_assert(NVT >= 1 && NDT % 4 == 0, "D must be 64 or 128");

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

  // zero the strictly-upper parts that are never written (T, and Aq's
  // upper tiles); they must read as zero in the full-width products.
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
    load_chunk<CT, D, C>(sm, p, b, h, m, t0, tid);
    __syncthreads();

    // ---- grams: L (from K K^T) and Aq (from K Q^T), lower tiles only ----
    {
      constexpr int NP = NCT * (NCT + 1) / 2;
      for (int task = wave; task < 2 * NP; task += 4) {
        const int pidx = task >> 1, type = task & 1;
        int it = 0, acc_p = 0;
        while (acc_p + it + 1 <= pidx) { acc_p += it + 1; ++it; }
        const int jt = pidx - acc_p;   // jt <= it
        f32x4 acc = zero4();
        const CT* arow = (type == 0) ? &sm.k[(it * 16 + n16) * LDD] : &sm.k[(jt * 16 + n16) * LDD];
        const CT* brow = (type == 0) ? &sm.k[(jt * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
#pragma unroll
        for (int kb = 0; kb < D; kb += KS) mma(acc, ld_frag(arow + kb, g4), ld_frag(brow + kb, g4));
        if (type == 0) {
          // acc[i] = (k_i . k_j), i = it*16+4g+ii, j = jt*16+n
          const int j = jt * 16 + n16;
          const float Gj = sm.G[j];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = it * 16 + 4 * g4 + ii;
            const float val = (j < i) ? __expf(sm.G[i] - Gj) * sm.ae[i] * acc[ii] : 0.f;
            sm.L[i * LDF + j] = val;
          }
        } else {
          // acc[ii] = (q_i . k_j), i = it*16+n, j = jt*16+4g+ii
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

    // ---- T = (I + L)^-1: 16x16 diagonal blocks by substitution ----
    if (wave == 0) {
      const int bb = lane >> 4, col = lane & 15;
      if (bb < NCT) {
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float s = (i == col) ? 1.f : 0.f;
          const float* Lrow = &sm.L[(16 * bb + i) * LDF + 16 * bb];
#pragma unroll
          for (int j = 0; j < i; ++j) s -= Lrow[j] * x[j];
          x[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sm.T[(16 * bb + i) * LDF + 16 * bb + col] = x[i];
      }
    }
    __syncthreads();
    // off-diagonal blocks: T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj, by distance
#pragma unroll
    for (int dist = 1; dist < NCT; ++dist) {
      if (wave < NCT - dist) {
        const int jb = wave, ib = wave + dist;
        f32x4 X = zero4();
        for (int kb = jb; kb < ib; ++kb) {
          f32x4 a, bq;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            a[s] = sm.L[(16 * ib + n16) * LDF + 16 * kb + 4 * g4 + s];
            bq[s] = sm.T[(16 * kb + 4 * g4 + s) * LDF + 16 * jb + n16];
          }
          mma(X, a, bq);
        }
        f32x4 a;
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = sm.T[(16 * ib + n16) * LDF + 16 * ib + 4 * g4 + s];
        f32x4 Y = zero4();
        mma(Y, a, X);
#pragma unroll
        for (int s = 0; s < 4; ++s) sm.T[(16 * ib + 4 * g4 + s) * LDF + 16 * jb + n16] = -Y[s];
      }
      __syncthreads();
    }

    // ---- TA = T diag(a_w), TB = T diag(a_e exp G) ----
    for (int idx = tid; idx < C * C; idx += 256) {
      const int i = idx / C, j = idx % C;
      const float t = sm.T[i * LDF + j];
      sm.ta[i * LDC + j] = from_f<CT>(t * sm.aw[j]);
      sm.tb[i * LDC + j] = from_f<CT>(t * sm.ae[j] * sm.gam[j]);
    }
    __syncthreads();

    // ---- -Wm (rows i, cols d) via Wm^T = K^T TB^T; this wave's d tiles ----
    {
      constexpr int DPW = NDT / 4;
#pragma unroll
      for (int dd = 0; dd < DPW; ++dd) {
        const int dt = wave * DPW + dd;
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          f32x4 acc = zero4();
          const CT* arow = &sm.kt[(dt * 16 + n16) * LDC];
          const CT* brow = &sm.tb[(it * 16 + n16) * LDC];
#pragma unroll
          for (int kb = 0; kb < C; kb += KS) mma(acc, ld_frag(arow + kb, g4), ld_frag(brow + kb, g4));
          // acc[ii] = Wm[i = it*16+n][d = dt*16+4g+ii]
          st4(&sm.wm[(it * 16 + n16) * LDD + dt * 16 + 4 * g4], -acc[0], -acc[1], -acc[2], -acc[3]);
        }
      }
    }
    // ---- U = TA V (this wave's value columns) into the R accumulators ----
    f32x4 Racc[NCT][NVT];
#pragma unroll
    for (int it = 0; it < NCT; ++it)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt) {
        f32x4 acc = zero4();
        const CT* arow = &sm.ta[(it * 16 + n16) * LDC];
        const CT* brow = &sm.vt[(v0 + vt * 16 + n16) * LDC];
#pragma unroll
        for (int kb = 0; kb < C; kb += KS) mma(acc, ld_frag(arow + kb, g4), ld_frag(brow + kb, g4));
        Racc[it][vt] = acc;
      }
    __syncthreads();

    // ---- S0 fragments over k = d ----
    Frag Sf[NDT / TPS][NVT];
#pragma unroll
    for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
      for (int vt = 0; vt < NVT; ++vt)
        Sf[kb][vt] = acc_frag((CT*)nullptr, S[kb * TPS][vt], S[kb * TPS + TPS - 1][vt]);
    if (p.chunk_states) {
      Frag* cs = (Frag*)p.chunk_states + ((size_t)chain * NC + c) * (256 * (NDT / TPS) * NVT);
#pragma unroll
      for (int kb = 0; kb < NDT / TPS; ++kb)
#pragma unroll
        for (int vt = 0; vt < NVT; ++vt) cs[(kb * NVT + vt) * 256 + tid] = Sf[kb][vt];
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
    if (a.D == 128) return launch_fwd<bf16, 128, 64>(a, stream);
    if (a.D == 64) return launch_fwd<bf16, 64, 64>(a, stream);
  } else {
    if (a.D == 128) return launch_fwd<float, 128, 32>(a, stream);
    if (a.D == 64) return launch_fwd<float, 64, 32>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "unsupported head dim %d (64 or 128)", a.D);
}

}  // namespace gdnx

// Per-chunk operands of the chunked delta rule that do not depend on the
// carried state, computed for every (b, h, chunk) and lane in parallel
// (gfx950).  The sequential scans (delta_scan.hip) then only carry the
// state (forward) or its gradient (backward).
//
// For chain (b, h, m) and chunk c with inclusive log-decay prefix G (clamped
// to [kLogFloor, 0] per token):
//   L  = (exp(G_i - G_j) a_e,i k_i . k_j)_{j<i},   T = (I + L)^-1
//   Aq = (exp(G_i - G_j) q_i . k_j)_{j<=i}
//   gam = exp(G),  dec = exp(G_last - G),  aeg = a_e exp(G),  a_w
// (the reference's chunk structure gdn3/gdn3_upgrade.py:467-521 and the
// KMD-2 chunk derivation gdn3/kmd2_fast_scan.py:1-18, with the decay ratios
// prefix_i / prefix_j replaced by log-space differences, which never
// underflow).  One workgroup per (b, h, chunk): the raw grams K K^T and
// Q K^T are formed once on MFMA and kept in registers, then the M lanes
// (which share q and k), LP at a time, apply their own decay and erase
// scaling, invert their unit-lower L by 16x16 blocks and store T, Aq and
// the scalars.  The LP lanes of a group go through each phase together:
// wave w forms lane w's scalars, the diagonal blocks of every lane are
// inverted at once (a 16-lane group per block), wave w forms lane w's
// blocks below the diagonal, so a group costs one lane's chain of
// dependent steps and barriers.
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct alignas(16) PrepLane {   // one lane's operands
  typedef Dims<CT, D, C> Dm;
  CT t[C * Dm::LDC];    // T (strictly upper tiles stay zero)
  CT aq[C * Dm::LDC];   // Aq (same)
  float L[C * Dm::LDF];
  float LT[C * Dm::LDT];
  float Td[C * Dm::LDT];
  float G[C], gam[C], dec[C], ae[C], aw[C];
};
template <typename CT, int D, int C, int LP>
struct alignas(16) PrepSmem {
  typedef Dims<CT, D, C> Dm;
  CT q[C * Dm::LDD];
  CT k[C * Dm::LDD];
  PrepLane<CT, D, C> ln[LP];
};
// lanes prepared together: as many (of 4, 2, 1) as leave LDS for two
// workgroups per CU
template <typename CT, int D, int C>
struct PrepCfg {
  static constexpr int LP = sizeof(PrepSmem<CT, D, C, 4>) <= 80 * 1024   ? 4
                            : sizeof(PrepSmem<CT, D, C, 2>) <= 80 * 1024 ? 2
                                                                          : 1;
};

// [C][LDC] LDS tile -> row-major [C][C] global, 16-byte stores
template <typename CT, int C, int LDC>
__device__ __forceinline__ void store_cc(CT* __restrict__ dst, const CT* src, int tid, int nt) {
  constexpr int PER = 16 / sizeof(CT), NU = C * C / PER;
  for (int u = tid; u < NU; u += nt) {
    const int i = (u * PER) / C, j = (u * PER) % C;
    const uint2* s = (const uint2*)&src[i * LDC + j];
    *(uint4*)&dst[(size_t)u * PER] = make_uint4(s[0].x, s[0].y, s[1].x, s[1].y);
  }
}

template <typename CT, int D, int C>
__global__ void __launch_bounds__((Dims<CT, D, C>::NT)) __attribute__((amdgpu_waves_per_eu(2))) delta_prep_kernel(DeltaArgs p) {
  typedef Dims<CT, D, C> Dm;
  constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF, NT = Dm::NT, NW = Dm::NW, NCT = Dm::NCT;
  constexpr int NP = NCT * (NCT + 1) / 2;          // lower 16x16 tile pairs of a C x C gram
  constexpr int NTPW = (2 * NP + NW - 1) / NW;      // gram tiles per wave (K K^T and Q K^T)
  constexpr int LP = PrepCfg<CT, D, C>::LP;
  static_assert(LP <= NW && LP * NCT <= 4 * NW, "a wave per lane; a 16-lane group per diagonal block");
  __shared__ PrepSmem<CT, D, C, LP> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int NC = (p.T + C - 1) / C;
  const int nblk = p.B * p.H * NC;
  const int blk = xcd_remap(blockIdx.x, nblk);
  const int c = blk % NC, h = (blk / NC) % p.H, b = blk / (NC * p.H);
  const int t0 = c * C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t st = (size_t)p.H * p.M;
  const size_t NR = (size_t)p.B * p.H * p.M * NC;
  const PrepPtrs<CT> po = prep_ptrs<CT>(p.prep, NR, C);

#pragma unroll
  for (int l = 0; l < LP; ++l)
    for (int i = tid; i < C * LDC; i += NT) {  // strictly upper tiles are never written
      sm.ln[l].t[i] = from_f<CT>(0.f);
      sm.ln[l].aq[i] = from_f<CT>(0.f);
    }
  // the first lane group's token scalars are issued before the q/k tiles:
  // loads retire in order, so issued after the tiles they would wait for them
  const size_t sbase = ((size_t)b * p.T * p.H + h) * p.M + wave;
  ScalarVals sv{0.f, 0.f, 0.f};
  if (wave < min(LP, p.M)) sv = prep_scalars_load<C>(p.ae + sbase, p.aw + sbase, p.g + sbase, st, t0, p.T, lane);
  {
    Stage<CT, C, D, 1, NT> sq, sk;
    const unsigned rsb = (unsigned)(rs * sizeof(CT)), nb = (unsigned)min(C, p.T - t0) * rsb;
    sq.fetch(buf_rsrc((const CT*)p.q + qoff + (size_t)t0 * rs, nb), rsb, tid);
    sk.fetch(buf_rsrc((const CT*)p.k + qoff + (size_t)t0 * rs, nb), rsb, tid);
    sq.template commit_nat<LDD>(sm.q, tid);
    sk.template commit_nat<LDD>(sm.k, tid);
  }
  __syncthreads();

  // raw grams, kept in registers: task s of this wave is tile pair
  // (wave + NW s) >> 1 of K K^T (even) or Q K^T (odd)
  f32x4 gram[NTPW];
#pragma unroll
  for (int s = 0; s < NTPW; ++s) {
    const int task = wave + NW * s;
    gram[s] = zero4();
    if (task < 2 * NP) {
      int it, jt;
      tri_pair(task >> 1, it, jt);
      // K K^T: acc[ii] = k_i . k_j, i = 16 it + 4 g + ii, j = 16 jt + n
      // Q K^T: acc[ii] = q_i . k_j, i = 16 it + n,        j = 16 jt + 4 g + ii
      const CT* arow = &sm.k[(((task & 1) == 0 ? it : jt) * 16 + n16) * LDD];
      const CT* brow = ((task & 1) == 0) ? &sm.k[(jt * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
      gram[s] = tile_nt<CT, D>(arow, brow, g4);
    }
  }

  for (int m0 = 0; m0 < p.M; m0 += LP) {
    const int nl = min(LP, p.M - m0);
    if (m0 > 0) __syncthreads();   // the previous group's stores have read its lanes' operands
    // ---- the lanes' token scalars (wave w: lane m0 + w) ----
    if (wave < nl) {
      PrepLane<CT, D, C>& P = sm.ln[wave];
      const ChunkScalars cs{P.G, P.gam, P.dec, P.ae, P.aw, nullptr};
      if (m0 > 0) sv = prep_scalars_load<C>(p.ae + sbase + m0, p.aw + sbase + m0, p.g + sbase + m0, st, t0, p.T, lane);
      prep_scalars_commit<C>(cs, sv, lane);
    }
    __syncthreads();
    // ---- each lane's L (fp32, plus transposed diagonal blocks) and Aq ----
#pragma unroll
    for (int l = 0; l < LP; ++l) {
      if (l >= nl) break;
      PrepLane<CT, D, C>& P = sm.ln[l];
#pragma unroll
      for (int s = 0; s < NTPW; ++s) {
        const int task = wave + NW * s;
        if (task < 2 * NP) {
          int it, jt;
          tri_pair(task >> 1, it, jt);
          if ((task & 1) == 0) {
            const f32x4 G4 = *(const f32x4*)&P.G[it * 16 + 4 * g4];
            const f32x4 ae4 = *(const f32x4*)&P.ae[it * 16 + 4 * g4];
            const int j = jt * 16 + n16;
            const float Gj = P.G[j];
            f32x4 val;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int i = it * 16 + 4 * g4 + ii;
              val[ii] = (j < i) ? __expf(G4[ii] - Gj) * ae4[ii] * gram[s][ii] : 0.f;
              P.L[i * LDF + j] = val[ii];
            }
            if (jt == it) *(f32x4*)&P.LT[j * 20 + 4 * g4] = val;
          } else {
            const int i = it * 16 + n16;
            const float Gi = P.G[i];
            const f32x4 Gj4 = *(const f32x4*)&P.G[jt * 16 + 4 * g4];
            float v[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int j = jt * 16 + 4 * g4 + ii;
              v[ii] = (j <= i) ? __expf(Gi - Gj4[ii]) * gram[s][ii] : 0.f;
            }
            st4(&P.aq[i * LDC + jt * 16 + 4 * g4], v[0], v[1], v[2], v[3]);
          }
        }
      }
    }
    __syncthreads();
    // ---- T = (I + L)^-1: every lane's diagonal blocks at once (16-lane
    // group g of wave w: block (4 w + g) mod NCT of lane (4 w + g) / NCT) ----
    {
      const int pair = 4 * wave + g4;
      if (pair < nl * NCT) {
        PrepLane<CT, D, C>& P = sm.ln[pair / NCT];
        diag_block_inverse(P.LT, P.Td, pair % NCT, n16, 0,
                           [&](int i, int j, float t, int) { P.t[i * LDC + j] = from_f<CT>(t); });
      }
    }
    if constexpr (NCT > 1) {
      __syncthreads();
      // the blocks below the diagonal: wave w, lane m0 + w
      if (wave < nl) {
        PrepLane<CT, D, C>& P = sm.ln[wave];
#pragma unroll
        for (int jb = 0; jb < NCT - 1; ++jb)
          offdiag_block_column<C>(P.L, P.Td, jb, lane, 0,
                                  [&](int i, int j, float t, int) { P.t[i * LDC + j] = from_f<CT>(t); });
      }
    }
    __syncthreads();
    // ---- records: T, Aq and the scalars of each lane ----
#pragma unroll
    for (int l = 0; l < LP; ++l) {
      if (l >= nl) break;
      const PrepLane<CT, D, C>& P = sm.ln[l];
      const size_t rec = rec_index(((size_t)b * p.H + h) * p.M + m0 + l, c, (size_t)p.B * p.H * p.M);
      store_cc<CT, C, LDC>(po.t + rec * C * C, P.t, tid, NT);
      store_cc<CT, C, LDC>(po.aq + rec * C * C, P.aq, tid, NT);
      if (wave == l && lane < C) {
        float* sc = po.sc + rec * kNumSc * C;
        sc[kScGam * C + lane] = P.gam[lane];
        sc[kScDec * C + lane] = P.dec[lane];
        sc[kScAeg * C + lane] = P.ae[lane] * P.gam[lane];
        sc[kScAw * C + lane] = P.aw[lane];
      }
    }
  }
}

template <typename CT, int D, int C>
static int launch_prep(const DeltaArgs& a, hipStream_t stream) {
  const int NC = (a.T + C - 1) / C;
  hipLaunchKernelGGL((delta_prep_kernel<CT, D, C>), dim3(a.B * a.H * NC), dim3(Dims<CT, D, C>::NT), 0, stream, a);
  return check_launch("delta_prep_kernel");
}

int delta_prep_dispatch(const DeltaArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 64) return launch_prep<bf16, 128, 64>(a, stream);
    if (a.D == 128 && a.C == 32) return launch_prep<bf16, 128, 32>(a, stream);
    if (a.D == 64 && a.C == 64) return launch_prep<bf16, 64, 64>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_prep<bf16, 64, 32>(a, stream);
  } else {
    if (a.D == 128 && a.C == 32) return launch_prep<float, 128, 32>(a, stream);
    if (a.D == 128 && a.C == 16) return launch_prep<float, 128, 16>(a, stream);
    if (a.D == 64 && a.C == 32) return launch_prep<float, 64, 32>(a, stream);
    if (a.D == 64 && a.C == 16) return launch_prep<float, 64, 16>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "prep: unsupported head_dim %d / chunk %d", a.D, a.C);
}

size_t delta_prep_bytes(int nchains, int T, int C, int dtype) {
  const size_t NR = (size_t)nchains * ((T + C - 1) / C);
  return NR * prep_bytes_per_record(C, dtype == GDNX_DTYPE_BF16 ? 2 : 4);
}

}  // namespace gdnx

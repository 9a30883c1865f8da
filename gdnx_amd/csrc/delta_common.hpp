// Device building blocks shared by the chunked delta-rule kernels
// (forward, reverse state scan, gradient kernel).  All assume 256 threads
// (4 waves) per workgroup.
#pragma once
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct Dims {
  typedef typename FragT<CT>::type Frag;
  static constexpr int KS = FragT<CT>::KSTEP;  // k per MFMA step
  static constexpr int TPS = FragT<CT>::TPS;   // accumulator tiles per k-step
  static constexpr int NDT = D / 16;           // 16-row tiles over a feature dim
  static constexpr int NCT = C / 16;           // 16-row tiles over the chunk
  static constexpr int VS = D / 4;             // feature columns owned by a wave
  static constexpr int NVT = VS / 16;          // 16-col tiles owned by a wave
  static constexpr int LDD = D + 4;            // LDS row length, [*, D] tiles
  static constexpr int LDC = C + 4;            // LDS row length, [*, C] tiles
  static constexpr int LDF = C + 1;            // fp32 [C, C] scratch rows
  // fragments of one chunk-state stash per workgroup (tile-native layout)
  static constexpr int STASH_FRAGS = (NDT / TPS) * NVT;
  static_assert(C % KS == 0, "chunk must be a multiple of the MFMA k-step");
  static_assert(NVT >= 1 && NDT % 4 == 0, "head dim must be 64 or 128");
};

// Stage C rows (tokens t0..t0+C-1, zero beyond T) of a [.., T, .., D] tensor
// into LDS: `nat` gets rows [C][D+4] (feature-contiguous), `tr` gets the
// transpose [D][C+4] (token-contiguous), each optional.  `src` points at
// token 0, feature 0 of this (batch, head[, lane]); rows are `rs` apart.
template <typename CT, int D, int C>
__device__ __forceinline__ void stage_tile(const CT* __restrict__ src, size_t rs, int t0, int T,
                                           CT* nat, CT* tr, int tid) {
  constexpr int VEC = 16 / sizeof(CT);
  constexpr int DG = D / VEC;
  constexpr int LDD = D + 4, LDC = C + 4;
  for (int u = tid; u < (C / 4) * DG; u += 256) {
    const int tg = u / DG, dg = u % DG;
    CT x[4][VEC];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * tg + r;
      if (t < T)
        *(uint4*)x[r] = *(const uint4*)(src + (size_t)t * rs + dg * VEC);
      else
        *(uint4*)x[r] = make_uint4(0, 0, 0, 0);
    }
    if (nat) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint2* d = (uint2*)(nat + (4 * tg + r) * LDD + dg * VEC);
        const uint2* s = (const uint2*)x[r];
        d[0] = s[0];
        d[1] = s[1];
      }
    }
    if (tr) {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        st4(&tr[(dg * VEC + e) * LDC + 4 * tg], to_f(x[0][e]), to_f(x[1][e]), to_f(x[2][e]),
            to_f(x[3][e]));
    }
  }
}

// Per-token scalars of one chunk for one chain (wave 0 only): erase/write
// coefficients, clamped log-decay, inclusive prefix G, exp(G) and the decay
// to the chunk end exp(G_last - G).  `base` = &arr[b][0][h][m]; tokens are
// `st` apart.  graw (optional) keeps the unclamped log-decay.
struct ChunkScalars {
  float *G, *gam, *dec, *ae, *aw, *graw;
};

template <int C>
__device__ __forceinline__ void prep_scalars(const ChunkScalars& s, const float* ae, const float* aw,
                                             const float* g, size_t st, int t0, int T, int lane) {
  float vae = 0.f, vaw = 0.f, vg = 0.f, raw = 0.f;
  const int t = t0 + lane;
  if (lane < C && t < T) {
    if (ae) vae = ae[(size_t)t * st];
    if (aw) vaw = aw[(size_t)t * st];
    raw = g[(size_t)t * st];
    vg = fmaxf(fminf(raw, 0.f), kLogFloor);
  }
  float G = vg;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(G, off, 64);
    if (lane >= off) G += o;
  }
  const float Glast = __shfl(G, C - 1, 64);
  if (lane < C) {
    s.G[lane] = G;
    s.gam[lane] = __expf(G);
    s.dec[lane] = __expf(Glast - G);
    if (s.ae) s.ae[lane] = vae;
    if (s.aw) s.aw[lane] = vaw;
    if (s.graw) s.graw[lane] = raw;
  }
}

// T = (I + L)^-1 for a unit-lower C x C matrix (L strictly lower, fp32,
// rows LDF apart; only the lower blocks are read).  T's strictly-upper part
// must already be zero.  16x16 diagonal blocks by substitution (wave 0, one
// lane per column), then T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj by distance
// on fp32 MFMA.  Contains barriers: every thread must call it.
template <int C>
__device__ __forceinline__ void invert_unit_lower(const float* sL, float* sT, int wave, int lane) {
  constexpr int NCT = C / 16, LDF = C + 1;
  const int g4 = lane >> 4, n16 = lane & 15;
  if (wave == 0) {
    const int bb = lane >> 4, col = lane & 15;
    if (bb < NCT) {
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == col) ? 1.f : 0.f;
        const float* Lrow = &sL[(16 * bb + i) * LDF + 16 * bb];
#pragma unroll
        for (int j = 0; j < i; ++j) s -= Lrow[j] * x[j];
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[(16 * bb + i) * LDF + 16 * bb + col] = x[i];
    }
  }
  __syncthreads();
#pragma unroll
  for (int dist = 1; dist < NCT; ++dist) {
    if (wave < NCT - dist) {
      const int jb = wave, ib = wave + dist;
      f32x4 X = zero4();
      for (int kb = jb; kb < ib; ++kb) {
        f32x4 a, bq;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          a[s] = sL[(16 * ib + n16) * LDF + 16 * kb + 4 * g4 + s];
          bq[s] = sT[(16 * kb + 4 * g4 + s) * LDF + 16 * jb + n16];
        }
        mma(X, a, bq);
      }
      f32x4 a;
#pragma unroll
      for (int s = 0; s < 4; ++s) a[s] = sT[(16 * ib + n16) * LDF + 16 * ib + 4 * g4 + s];
      f32x4 Y = zero4();
      mma(Y, a, X);
#pragma unroll
      for (int s = 0; s < 4; ++s) sT[(16 * ib + 4 * g4 + s) * LDF + 16 * jb + n16] = -Y[s];
    }
    __syncthreads();
  }
}

// Lower-triangular 16x16 tile pair index -> (it, jt) with jt <= it.
__device__ __forceinline__ void tri_pair(int pidx, int& it, int& jt) {
  int row = 0, start = 0;
  while (start + row + 1 <= pidx) {
    start += row + 1;
    ++row;
  }
  it = row;
  jt = pidx - start;
}

// 16x16 NT tile product over K (both operands K-contiguous LDS rows).
template <typename CT, int K>
__device__ __forceinline__ f32x4 tile_nt(const CT* arow, const CT* brow, int g4) {
  f32x4 acc = zero4();
#pragma unroll
  for (int kb = 0; kb < K; kb += FragT<CT>::KSTEP) mma(acc, ld_frag(arow + kb, g4), ld_frag(brow + kb, g4));
  return acc;
}

// Frag element e of a tile-native fragment sits at row offset frag_row(e, g4)
// within the k-step (see gdnx_common.hpp).
template <typename CT>
__device__ __forceinline__ int frag_row(int e, int g4) {
  if constexpr (sizeof(CT) == 2) return (e < 4) ? 4 * g4 + e : 16 + 4 * g4 + (e - 4);
  return 4 * g4 + e;
}
template <typename CT> struct FragLen { static constexpr int value = sizeof(CT) == 2 ? 8 : 4; };

}  // namespace gdnx

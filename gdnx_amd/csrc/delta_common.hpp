// Device building blocks shared by the chunked delta-rule kernels
// (forward, reverse state scan, gradient kernel).  Workgroups have NW = 4
// waves (one per SIMD): with the whole 512-entry register file per wave the
// fp32 state, the MFMA accumulators and the next chunk's prefetched tiles all
// stay in registers (8 waves halve the budget and spill).
#pragma once
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct Dims {
  typedef typename FragT<CT>::type Frag;
  static constexpr int KS = FragT<CT>::KSTEP;  // k per MFMA step
  static constexpr int TPS = FragT<CT>::TPS;   // accumulator tiles per k-step
  static constexpr int NW = 4;                 // waves per workgroup
  static constexpr int NT = 64 * NW;           // threads per workgroup
  static constexpr int NDT = D / 16;           // 16-row tiles over a feature dim
  static constexpr int NCT = C / 16;           // 16-row tiles over the chunk
  static constexpr int VS = D / NW;            // feature columns owned by a wave
  static constexpr int DPW = NDT / NW;         // 16-row feature tiles owned by a wave
  static constexpr int NVT = VS / 16;          // 16-col tiles owned by a wave
  static constexpr int LDD = D + 4;            // LDS row length, [*, D] tiles
  static constexpr int LDC = C + 4;            // LDS row length, [*, C] tiles
  static constexpr int LDF = C + 4;            // fp32 [C, C] scratch rows (16-byte aligned)
  static constexpr int LDT = 20;               // fp32 diagonal-block scratch [C][LDT]
  static_assert(C % KS == 0, "chunk must be a multiple of the MFMA k-step");
  static_assert(NVT >= 1 && DPW >= 1 && NDT % NW == 0, "head dim must be 64 or 128");
};

// Per-token scalars of one chunk for one chain (wave 0 only): erase/write
// coefficients, clamped log-decay, inclusive prefix G, exp(G) and the decay
// to the chunk end exp(G_last - G).  `base` = &arr[b][0][h][m]; tokens are
// `st` apart.  graw (optional) keeps the unclamped log-decay.
struct ChunkScalars {
  float *G, *gam, *dec, *ae, *aw, *graw;
};

// Per-chunk records (stashes and prep operands) are chunk-major: record
// (chain, chunk) = chunk * nchains + chain.  The chains of a scan run in
// lockstep, so the records written or read at one time are contiguous and
// spread over the memory channels (chain-major records would sit a whole
// chain's stash apart and pile onto the same channels).
__host__ __device__ __forceinline__ size_t rec_index(size_t chain, int chunk, size_t nchains) {
  return (size_t)chunk * nchains + chain;
}

// Per-chunk operands written by the prep kernel, for NR = chains x chunks
// records (indexed by rec_index): the unit-lower inverse T = (I + L)^-1
// and the decay-masked Q K^T (Aq) as row-major [C][C] compute-dtype
// matrices, then per token [4][C] floats: gam = exp(G), dec = exp(G_last - G),
// aeg = a_e exp(G) and a_w.  Consumers scale T on the fly:
// T diag(a_w) V and T diag(aeg) K are the chunk's U and Wm.
enum { kScGam = 0, kScDec = 1, kScAeg = 2, kScAw = 3, kNumSc = 4 };
template <typename CT>
struct PrepPtrs {
  CT* t;
  CT* aq;
  float* sc;
};
template <typename CT>
__host__ __device__ __forceinline__ PrepPtrs<CT> prep_ptrs(void* base, size_t NR, int C) {
  CT* t = (CT*)base;
  CT* aq = t + NR * C * C;
  return PrepPtrs<CT>{t, aq, (float*)(aq + NR * C * C)};
}
__host__ __device__ __forceinline__ size_t prep_bytes_per_record(int C, size_t es) {
  return 2 * (size_t)C * C * es + (size_t)kNumSc * C * sizeof(float);
}

// Inclusive prefix sum over the 16 lanes of each DPP row (lane bits 0..3);
// lane 15 of a row ends with the row's total.
__device__ __forceinline__ float row_prefix16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, true));
  return x;
}

// Inclusive suffix sum over the 16 lanes of each DPP row (row_shl steps).
__device__ __forceinline__ float row_suffix16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x101, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x102, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x104, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x108, 0xf, 0xf, true));
  return x;
}

__device__ __forceinline__ float lane_value(float x, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

// Wave scans on DPP rows plus scalar reads of the row totals (no LDS
// permutes on the dependent path).  N: the lanes that take part (lanes at
// or past N must hold 0 for the suffix).
template <int N>
__device__ __forceinline__ float lane_prefix(float x, int lane) {
  const float rp = row_prefix16(x);
  float add = 0.f;
  if constexpr (N > 16) {
    const float t0 = lane_value(rp, 15);
    add += lane >= 16 ? t0 : 0.f;
  }
  if constexpr (N > 32) {
    const float t1 = lane_value(rp, 31);
    add += lane >= 32 ? t1 : 0.f;
  }
  if constexpr (N > 48) {
    const float t2 = lane_value(rp, 47);
    add += lane >= 48 ? t2 : 0.f;
  }
  return rp + add;
}
template <int N>
__device__ __forceinline__ float lane_suffix(float x, int lane) {
  const float rs = row_suffix16(x);
  float add = 0.f;
  if constexpr (N > 16) {
    const float t1 = lane_value(rs, 16);
    add += lane < 16 ? t1 : 0.f;
  }
  if constexpr (N > 32) {
    const float t2 = lane_value(rs, 32);
    add += lane < 32 ? t2 : 0.f;
  }
  if constexpr (N > 48) {
    const float t3 = lane_value(rs, 48);
    add += lane < 48 ? t3 : 0.f;
  }
  return rs + add;
}
// the sum over all 64 lanes, in every lane
__device__ __forceinline__ float wave_sum(float x) {
  const float rp = row_prefix16(x);
  return (lane_value(rp, 15) + lane_value(rp, 31)) + (lane_value(rp, 47) + lane_value(rp, 63));
}

// Prefetched per-token scalars of one lane (token t0 + lane).
struct ScalarRegs {
  float ae, aw, g;
};

template <int C>
__device__ __forceinline__ void scal_fetch(ScalarRegs& r, const float* ae, const float* aw, const float* g,
                                           size_t st, int t0, int T, int lane) {
  r.ae = r.aw = r.g = 0.f;
  const int t = t0 + lane;
  if (lane < C && t < T) {
    if (ae) r.ae = ae[(size_t)t * st];
    if (aw) r.aw = aw[(size_t)t * st];
    r.g = g[(size_t)t * st];
  }
}

// scal_fetch without branches: every lane loads (lanes past the chunk or
// past T read a clamped token) and the values of tokens outside [t0, T) are
// zeroed afterwards.
template <int C>
__device__ __forceinline__ void scal_fetch_all(ScalarRegs& r, const float* ae, const float* aw, const float* g,
                                               size_t st, int t0, int T, int lane) {
  const int t = t0 + lane;
  const size_t tc = (size_t)min(t, T - 1) * st;
  const bool ok = lane < C && t < T;
  const float vae = ae[tc], vaw = aw[tc], vg = g[tc];
  r.ae = ok ? vae : 0.f;
  r.aw = ok ? vaw : 0.f;
  r.g = ok ? vg : 0.f;
}

template <int C>
__device__ __forceinline__ void scal_commit(const ChunkScalars& s, const ScalarRegs& r, int lane) {
  const float G = lane_prefix<C>(fmaxf(fminf(r.g, 0.f), kLogFloor), lane);
  const float Glast = lane_value(G, C - 1);
  if (lane < C) {
    s.G[lane] = G;
    s.gam[lane] = __expf(G);
    s.dec[lane] = __expf(Glast - G);
    if (s.ae) s.ae[lane] = r.ae;
    if (s.aw) s.aw[lane] = r.aw;
    if (s.graw) s.graw[lane] = r.g;
  }
}

// The loads of prep_scalars (issued early, consumed later: loads retire in
// order, so what is issued before a larger stream does not wait for it)
struct ScalarVals {
  float ae, aw, raw;
};
template <int C>
__device__ __forceinline__ ScalarVals prep_scalars_load(const float* ae, const float* aw, const float* g, size_t st,
                                                        int t0, int T, int lane) {
  ScalarVals v{0.f, 0.f, 0.f};
  const int t = t0 + lane;
  if (lane < C && t < T) {
    if (ae) v.ae = ae[(size_t)t * st];
    if (aw) v.aw = aw[(size_t)t * st];
    v.raw = g[(size_t)t * st];
  }
  return v;
}
template <int C>
__device__ __forceinline__ void prep_scalars_commit(const ChunkScalars& s, const ScalarVals& v, int lane) {
  const float vae = v.ae, vaw = v.aw, raw = v.raw;
  const float vg = lane < C ? fmaxf(fminf(raw, 0.f), kLogFloor) : 0.f;
  const float G = lane_prefix<C>(vg, lane);
  const float Glast = lane_value(G, C - 1);
  if (lane < C) {
    s.G[lane] = G;
    s.gam[lane] = __expf(G);
    s.dec[lane] = __expf(Glast - G);
    if (s.ae) s.ae[lane] = vae;
    if (s.aw) s.aw[lane] = vaw;
    if (s.graw) s.graw[lane] = raw;
  }
}

template <int C>
__device__ __forceinline__ void prep_scalars(const ChunkScalars& s, const float* ae, const float* aw,
                                             const float* g, size_t st, int t0, int T, int lane) {
  prep_scalars_commit<C>(s, prep_scalars_load<C>(ae, aw, g, st, t0, T, lane), lane);
}

// Registers holding one thread's share of a chunk tile ([C][D] rows, 4
// consecutive tokens x 16 bytes), used to prefetch the next chunk while the
// current one computes.  Every (C, D, dtype) used here maps to at most one
// such unit per thread.
struct TileRegs {
  uint4 x[4];
};

template <typename CT, int D, int C>
__device__ __forceinline__ bool tile_unit(int tid, int& tg, int& dg) {
  constexpr int VEC = 16 / sizeof(CT);
  constexpr int DG = D / VEC;
  static_assert((C / 4) * DG <= Dims<CT, D, C>::NT, "one staging unit per thread");
  tg = tid / DG;
  dg = tid % DG;
  return tid < (C / 4) * DG;
}

template <typename CT, int D, int C>
__device__ __forceinline__ void tile_fetch(TileRegs& r, const CT* __restrict__ src, size_t rs, int t0,
                                           int T, int tid) {
  constexpr int VEC = 16 / sizeof(CT);
  int tg, dg;
  if (!tile_unit<CT, D, C>(tid, tg, dg)) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = t0 + 4 * tg + q;
    r.x[q] = (t < T) ? *(const uint4*)(src + (size_t)t * rs + dg * VEC) : make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ unsigned word_of(const uint4& v, int w) {
  return w == 0 ? v.x : (w == 1 ? v.y : (w == 2 ? v.z : v.w));
}

template <typename CT, int D, int C>
__device__ __forceinline__ void tile_commit(const TileRegs& r, CT* nat, CT* tr, int tid) {
  constexpr int VEC = 16 / sizeof(CT);
  constexpr int LDD = D + 4, LDC = C + 4;
  int tg, dg;
  if (!tile_unit<CT, D, C>(tid, tg, dg)) return;
  if (nat) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint2* d = (uint2*)(nat + (4 * tg + q) * LDD + dg * VEC);
      d[0] = make_uint2(r.x[q].x, r.x[q].y);
      d[1] = make_uint2(r.x[q].z, r.x[q].w);
    }
  }
  if (tr) {
    if constexpr (sizeof(CT) == 2) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {   // (byte permutes as in Stage::commit_tr)
        const unsigned r0 = word_of(r.x[0], w), r1 = word_of(r.x[1], w);
        const unsigned r2 = word_of(r.x[2], w), r3 = word_of(r.x[3], w);
        *(uint2*)&tr[(dg * VEC + 2 * w) * LDC + 4 * tg] =
            make_uint2(__builtin_amdgcn_perm(r1, r0, 0x05040100u), __builtin_amdgcn_perm(r3, r2, 0x05040100u));
        *(uint2*)&tr[(dg * VEC + 2 * w + 1) * LDC + 4 * tg] =
            make_uint2(__builtin_amdgcn_perm(r1, r0, 0x07060302u), __builtin_amdgcn_perm(r3, r2, 0x07060302u));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *(uint4*)&tr[(dg * VEC + e) * LDC + 4 * tg] =
            make_uint4(word_of(r.x[0], e), word_of(r.x[1], e), word_of(r.x[2], e), word_of(r.x[3], e));
    }
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

// Grams of a chunk.  L-type tiles (K K^T, strictly lower, scaled by
// exp(G_i - G_j) a_e,i) go to sL (rows i, fp32) and, for diagonal blocks, to
// sLT transposed (compact: row j holds L[16b+.][j] at [j*20 + i-16b]);
// Aq-type tiles (Q K^T, lower incl. diagonal, scaled by exp(G_i - G_j)) are
// handed to emit_aq(i, j0, v[4]) as 4 consecutive j.  The lower tiles of both
// grams are dealt round-robin to the NW waves; each task loads all its
// operand fragments before its MFMAs.
template <typename CT, int D, int C, typename EmitAq>
__device__ __forceinline__ void chunk_grams(const CT* sk, const CT* sq, float* sL, float* sLT,
                                            const float* sG, const float* sae, int wave, int lane,
                                            EmitAq emit_aq) {
  typedef typename FragT<CT>::type Frag;
  constexpr int KS = FragT<CT>::KSTEP, NCT = C / 16, LDD = D + 4, LDF = C + 4;
  constexpr int NW = Dims<CT, D, C>::NW, NP = NCT * (NCT + 1) / 2;
  const int g4 = lane >> 4, n16 = lane & 15;
  for (int task = wave; task < 2 * NP; task += NW) {
    const int type = task & 1;
    int it, jt;
    tri_pair(task >> 1, it, jt);
    const CT* arow = &sk[((type == 0 ? it : jt) * 16 + n16) * LDD];
    const CT* brow = (type == 0) ? &sk[(jt * 16 + n16) * LDD] : &sq[(it * 16 + n16) * LDD];
    Frag a[D / KS], b[D / KS];
#pragma unroll
    for (int kb = 0; kb < D / KS; ++kb) {
      a[kb] = ld_frag(arow + kb * KS, g4);
      b[kb] = ld_frag(brow + kb * KS, g4);
    }
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < D / KS; ++kb) mma(acc, a[kb], b[kb]);
    if (type == 0) {
      // acc[ii] = k_i . k_j, i = it*16+4g+ii, j = jt*16+n
      const f32x4 G4 = *(const f32x4*)&sG[it * 16 + 4 * g4];
      const f32x4 ae4 = *(const f32x4*)&sae[it * 16 + 4 * g4];
      const int j = jt * 16 + n16;
      const float Gj = sG[j];
      f32x4 val;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = it * 16 + 4 * g4 + ii;
        val[ii] = (j < i) ? __expf(G4[ii] - Gj) * ae4[ii] * acc[ii] : 0.f;
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) sL[(it * 16 + 4 * g4 + ii) * LDF + j] = val[ii];
      if (jt == it) *(f32x4*)&sLT[j * 20 + 4 * g4] = val;
    } else {
      // acc[ii] = q_i . k_j, i = it*16+n, j = jt*16+4g+ii
      const int i = it * 16 + n16;
      const float Gi = sG[i];
      const f32x4 Gj4 = *(const f32x4*)&sG[jt * 16 + 4 * g4];
      float v[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int j = jt * 16 + 4 * g4 + ii;
        v[ii] = (j <= i) ? __expf(Gi - Gj4[ii]) * acc[ii] : 0.f;
      }
      emit_aq(i, jt * 16 + 4 * g4, v);
    }
  }
}

// Diagonal block b of T = (I + L)^-1, one column per thread: forward
// substitution of column `col` of the unit-lower 16x16 block whose
// transpose sits in sLT (rows 16 b .. 16 b + 15, row length 20).
// Right-looking: after step j, x_j is final; row j of the transposed block
// holds L[16b+i][16b+j] for all i.  Rows are loaded PF steps ahead so each
// step's LDS latency overlaps earlier steps' FMAs.  Writes the column to
// sTd and emits it (x[i] == 0 for i < col).
template <typename Emit, typename F>
__device__ __forceinline__ void diag_block_inverse(const float* sLT, float* sTd, int b, int col, F f, Emit emit) {
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = (i == col) ? 1.f : 0.f;
  constexpr int PF = 4;
  f32x4 win[PF][4];
#pragma unroll
  for (int r = 0; r < PF; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) win[r][q] = *(const f32x4*)&sLT[(16 * b + r) * 20 + 4 * q];
#pragma unroll
  for (int j = 0; j < 15; ++j) {
    f32x4 c4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) c4[q] = win[j % PF][q];
    if (j + PF < 15) {
#pragma unroll
      for (int q = 0; q < 4; ++q) win[j % PF][q] = *(const f32x4*)&sLT[(16 * b + j + PF) * 20 + 4 * q];
    }
#pragma unroll
    for (int i = j + 1; i < 16; ++i) x[i] -= c4[i >> 2][i & 3] * x[j];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    sTd[(16 * b + i) * 20 + col] = x[i];
    emit(16 * b + i, 16 * b + col, x[i], f);
  }
}

// Block column jb of T below the diagonal, by one wave, from L (row length
// C + 4) and the diagonal blocks of T (sTd): T_ib,jb = -T_ib,ib sum_kb
// L_ib,kb T_kb,jb on fp32 MFMA.
template <int C, typename Emit, typename F>
__device__ __forceinline__ void offdiag_block_column(const float* sL, const float* sTd, int jb, int lane, F f,
                                                     Emit emit) {
  constexpr int NCT = C / 16, LDF = C + 4;
  const int g4 = lane >> 4, n16 = lane & 15;
  f32x4 Tk[NCT];
  // T_jj as a B fragment: lane (g, n) holds T_jj[4g+s][n]
#pragma unroll
  for (int s = 0; s < 4; ++s) Tk[jb][s] = sTd[(16 * jb + 4 * g4 + s) * 20 + n16];
#pragma unroll
  for (int ib = jb + 1; ib < NCT; ++ib) {
    f32x4 X = zero4();
#pragma unroll
    for (int kb = jb; kb < ib; ++kb) {
      const f32x4 a = *(const f32x4*)&sL[(16 * ib + n16) * LDF + 16 * kb + 4 * g4];
      mma(X, a, Tk[kb]);
    }
    const f32x4 a = *(const f32x4*)&sTd[(16 * ib + n16) * 20 + 4 * g4];
    f32x4 Y = zero4();
    mma(Y, a, X);
    Tk[ib] = -Y;
#pragma unroll
    for (int s = 0; s < 4; ++s) emit(16 * ib + 4 * g4 + s, 16 * jb + n16, Tk[ib][s], f);
  }
}

// T = (I + L)^-1 of one unit-lower C x C matrix by the whole workgroup:
// the diagonal blocks by waves 0 .. NCT - 1 (16 lanes each), then block
// column jb by wave jb.
template <int C, typename ColPrep, typename Emit>
__device__ __forceinline__ void invert_unit_lower(const float* sL, const float* sLT, float* sTd, int wave,
                                                  int lane, ColPrep colprep, Emit emit) {
  constexpr int NCT = C / 16;
  const int n16 = lane & 15;
  if (wave < NCT && lane < 16) {
    const auto f = colprep(16 * wave + lane);
    diag_block_inverse(sLT, sTd, wave, lane, f, emit);
  }
  __syncthreads();
#pragma unroll
  for (int jb = 0; jb < NCT - 1; ++jb) {
    if (wave != jb) continue;   // block column jb (compile-time, so Tk stays in registers)
    const auto f = colprep(16 * jb + n16);
    offdiag_block_column<C>(sL, sTd, jb, lane, f, emit);
  }
}

// Four consecutive compute-dtype values (8 bytes for bf16, 16 for fp32).
template <typename CT> struct Vec4T;
template <> struct Vec4T<bf16> { typedef bf16x4 type; };
template <> struct Vec4T<float> { typedef f32x4 type; };

// Transpose of a 16x16 tile held as raw values (lane (g, n) holds rows 4g..4g+3
// of column n): returns lane (g, n) holding row n, columns 4g..4g+3.  Exact.
__device__ __forceinline__ f32x4 tile_transpose_raw(const bf16x4& x, int lane) {
  const int g4 = lane >> 4, n16 = lane & 15;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = x[e];
    a[e + 4] = (bf16)0.f;
    b[e] = (bf16)((4 * g4 + e == n16) ? 1.f : 0.f);
    b[e + 4] = (bf16)0.f;
  }
  f32x4 y = zero4();
  mma(y, a, b);
  return y;
}
__device__ __forceinline__ f32x4 tile_transpose_raw(const f32x4& x, int lane) {
  const int g4 = lane >> 4, n16 = lane & 15;
  f32x4 b;
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = (4 * g4 + e == n16) ? 1.f : 0.f;
  f32x4 y = zero4();
  mma(y, x, b);
  return y;
}

// Transpose of a 16x16 fp32 accumulator tile via MFMA with an identity
// operand: returns Y with lane (g, n) holding X[n][4g+s] in element s.
// The bf16 variant rounds the values to bf16 (used for bf16 outputs).
__device__ __forceinline__ f32x4 tile_transpose(bf16*, const f32x4& X, int lane) {
  const int g4 = lane >> 4, n16 = lane & 15;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = (bf16)X[e];
    a[e + 4] = (bf16)0.f;
    b[e] = (bf16)((4 * g4 + e == n16) ? 1.f : 0.f);
    b[e + 4] = (bf16)0.f;
  }
  f32x4 y = zero4();
  mma(y, a, b);
  return y;
}
__device__ __forceinline__ f32x4 tile_transpose(float*, const f32x4& X, int lane) {
  const int g4 = lane >> 4, n16 = lane & 15;
  f32x4 b;
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = (4 * g4 + e == n16) ? 1.f : 0.f;
  f32x4 y = zero4();
  mma(y, X, b);
  return y;
}


// 16x16 NT tile product over K (both operands K-contiguous LDS rows).
template <typename CT, int K>
__device__ __forceinline__ f32x4 tile_nt(const CT* arow, const CT* brow, int g4) {
  f32x4 acc = zero4();
#pragma unroll
  for (int kb = 0; kb < K; kb += FragT<CT>::KSTEP) mma(acc, ld_frag(arow + kb, g4), ld_frag(brow + kb, g4));
  return acc;
}

template <typename CT> struct FragLen { static constexpr int value = sizeof(CT) == 2 ? 8 : 4; };

// ---- stash layouts (written by the scans, read by the gradient kernel) ----
// Both stashes hold raw 16x16 accumulator tiles: a record's block X (the
// d x d state entering or leaving a chunk, or the chunk's C x d net writes
// / dB) as tile (it, V) = rows 16 it.., columns 16 V.., lane l = 16 g + n
// holding rows 16 it + 4 g + i (i = 0..3) of column 16 V + n at
// ((it (D/16) + V) 64 + l) 4 + i.  A wave reads or writes a tile as 64
// consecutive 4-value groups, and any split of the value columns over waves
// or workgroups writes whole tiles.
template <typename CT, int D>
__device__ __forceinline__ size_t stash_tile_offset(int it, int V, int lane) {
  return (((size_t)it * (D / 16) + V) * 64 + lane) * 4;
}
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  const bf16x4 x = *(const bf16x4*)p;
  return (f32x4){(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}
__device__ __forceinline__ f32x4 load4(const float* p) { return *(const f32x4*)p; }

// X[16 dt + 4 g + i][16 V + n], i = 0..3, for lane (g, n) of a state record
template <typename CT, int D, int C>
__device__ __forceinline__ const CT* stash_state_ptr(const CT* rec, int dt, int V, int lane) {
  return rec + stash_tile_offset<CT, D>(dt, V, lane);
}

// One 16-byte unit of a [C][D] tile record in the scans' raw
// accumulator-tile layout (unit u: tile u / 32 = (token tile, value tile),
// lanes 2 (u % 32) and 2 (u % 32) + 1): 4 consecutive tokens of two
// adjacent value columns.
struct TileUnit {
  int tok, col;   // first token (within the sub-chunk), first column
};
template <int D>
__device__ __forceinline__ TileUnit tile_unit_of(int u) {
  constexpr int NDT = D / 16;
  const int tl = u >> 5, lp = u & 31;
  const int it = tl / NDT, V = tl % NDT, g = lp >> 3, n0 = 2 * (lp & 7);
  return TileUnit{16 * it + 4 * g, 16 * V + n0};
}
// rows [tok + i][col], [tok + i][col + 1], i = 0..3 (two bf16 per store)
template <int LD>
__device__ __forceinline__ void unit_commit_rows(bf16* dst, const uint4& x, TileUnit t) {
  const unsigned w[4] = {x.x, x.y, x.z, x.w};   // x.x, x.y: column col, tokens 0..3; x.z, x.w: column col + 1
#pragma unroll
  for (int i = 0; i < 4; ++i)   // token i: the low (even i) or high half of each column's word, one byte permute
    *(unsigned*)&dst[(t.tok + i) * LD + t.col] =
        __builtin_amdgcn_perm(w[2 + (i >> 1)], w[i >> 1], (i & 1) ? 0x07060302u : 0x05040100u);
}
// Sum of x over the four 16-lane rows of the wave, in every lane (gfx950
// permlane swaps: lane l is added to l ^ 16, then to l ^ 32).
__device__ __forceinline__ float sum_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Frag element e of a tile-native fragment sits at row offset frag_row(e, g4)
// within the k-step (see gdnx_common.hpp).
template <typename CT>
__device__ __forceinline__ int frag_row(int e, int g4) {
  if constexpr (sizeof(CT) == 2) return (e < 4) ? 4 * g4 + e : 16 + 4 * g4 + (e - 4);
  return 4 * g4 + e;
}

// Raw buffer resource over nbytes at base: buffer loads beyond nbytes
// return zero and buffer stores beyond it are dropped, so a chunk's tail
// tokens need no branch (a branch around a memory op makes the compiler wait
// for every outstanding load and store at the next loop iteration).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, unsigned nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// 4 consecutive values of the compute dtype from floats (8 or 16 bytes)
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, unsigned off, const bf16*, float a, float b,
                                           float c, float d) {
  const bf16x4 x = (bf16x4){(bf16)a, (bf16)b, (bf16)c, (bf16)d};
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, x), r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, unsigned off, const float*, float a, float b,
                                           float c, float d) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128((u32x4){__float_as_uint(a), __float_as_uint(b), __float_as_uint(c),
                                                 __float_as_uint(d)},
                                         r, (int)off, 0, 0);
}

// Register staging of a [ROWS][COLS] compute-dtype tile for NTH threads:
// unit u = (RU consecutive rows, 16 bytes of columns); thread tid owns units
// tid, tid + NTH, ...  Fetched a chunk ahead into registers, then committed
// to LDS either as rows (commit_nat, row stride LD) or transposed
// (commit_tr, [col][row] with row stride LD; needs RU = 4: 4 consecutive
// rows per store).  Every thread issues the same loads (a thread past the
// last unit repeats it), so the loads are unconditional.
template <typename CT, int ROWS, int COLS, int RU, int NTH>
struct Stage {
  static constexpr int VEC = 16 / sizeof(CT);
  static constexpr int CG = COLS / VEC;
  static constexpr int NU = (ROWS / RU) * CG;
  static constexpr int UPT = (NU + NTH - 1) / NTH;
  static_assert(COLS % VEC == 0 && ROWS % RU == 0, "tile not a whole number of units");
  uint4 x[UPT][RU];

  __device__ __forceinline__ static int unit(int tid, int u) {
    const int e = tid + u * NTH;
    return (NU % NTH == 0 || e < NU) ? e : NU - 1;
  }
  __device__ __forceinline__ static bool owns(int tid, int u) { return NU % NTH == 0 || tid + u * NTH < NU; }
  // rows rsb bytes apart in a buffer resource (rows past its end read zero)
  __device__ __forceinline__ void fetch(__amdgpu_buffer_rsrc_t r, unsigned rsb, int tid) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int e = unit(tid, u), rg = e / CG, cg = e % CG;
#pragma unroll
      for (int q = 0; q < RU; ++q) x[u][q] = buf_load16(r, (unsigned)(rg * RU + q) * rsb + cg * 16);
    }
  }
  // a dense row-major [ROWS][COLS] tile
  __device__ __forceinline__ void fetch_dense(const CT* __restrict__ src, int tid) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int e = unit(tid, u), rg = e / CG, cg = e % CG;
#pragma unroll
      for (int q = 0; q < RU; ++q) x[u][q] = *(const uint4*)(src + (rg * RU + q) * COLS + cg * VEC);
    }
  }
  template <int LD>
  __device__ __forceinline__ void commit_nat(CT* dst, int tid) const {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      if (!owns(tid, u)) continue;
      const int e = tid + u * NTH, rg = e / CG, cg = e % CG;
#pragma unroll
      for (int q = 0; q < RU; ++q) {
        uint2* d = (uint2*)(dst + (rg * RU + q) * LD + cg * VEC);
        d[0] = make_uint2(x[u][q].x, x[u][q].y);
        d[1] = make_uint2(x[u][q].z, x[u][q].w);
      }
    }
  }
  template <int LD>
  __device__ __forceinline__ void commit_tr(CT* dst, int tid) const {
    static_assert(RU == 4, "transposed commit stores 4 consecutive rows");
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      if (!owns(tid, u)) continue;
      const int e = tid + u * NTH, rg = e / CG, cg = e % CG;
      if constexpr (sizeof(CT) == 2) {
        // word w of a row holds columns 2 w (low half) and 2 w + 1 (high
        // half); one byte permute pairs the halves of two rows
        // (v_perm_b32: selector bytes 0-3 pick the second operand's bytes,
        // 4-7 the first's)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const unsigned r0 = word_of(x[u][0], w), r1 = word_of(x[u][1], w);
          const unsigned r2 = word_of(x[u][2], w), r3 = word_of(x[u][3], w);
          *(uint2*)&dst[(cg * VEC + 2 * w) * LD + 4 * rg] =
              make_uint2(__builtin_amdgcn_perm(r1, r0, 0x05040100u), __builtin_amdgcn_perm(r3, r2, 0x05040100u));
          *(uint2*)&dst[(cg * VEC + 2 * w + 1) * LD + 4 * rg] =
              make_uint2(__builtin_amdgcn_perm(r1, r0, 0x07060302u), __builtin_amdgcn_perm(r3, r2, 0x07060302u));
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *(uint4*)&dst[(cg * VEC + c) * LD + 4 * rg] =
              make_uint4(word_of(x[u][0], c), word_of(x[u][1], c), word_of(x[u][2], c), word_of(x[u][3], c));
      }
    }
  }
};

// N floats staged by NTH threads (one dword each, a chunk ahead).
template <int N, int NTH>
struct ScalStage {
  static constexpr int PT = (N + NTH - 1) / NTH;
  float x[PT];
  __device__ __forceinline__ void fetch(const float* __restrict__ src, int t) {
#pragma unroll
    for (int i = 0; i < PT; ++i) x[i] = src[min(t + i * NTH, N - 1)];
  }
  __device__ __forceinline__ void commit(float* dst, int t) const {
#pragma unroll
    for (int i = 0; i < PT; ++i)
      if (N % NTH == 0 || t + i * NTH < N) dst[t + i * NTH] = x[i];
  }
};

// A fragment over k with element e (k index kb + frag_row(e, g)) scaled by
// s[frag_row(e, g)]; s points at the k-step's first scale factor (LDS,
// 16-byte aligned).
__device__ __forceinline__ bf16x8 frag_scale(const bf16x8& f, const float* s, int g4) {
  const f32x4 s0 = *(const f32x4*)&s[4 * g4], s1 = *(const f32x4*)&s[16 + 4 * g4];
  return (bf16x8){(bf16)((float)f[0] * s0[0]), (bf16)((float)f[1] * s0[1]), (bf16)((float)f[2] * s0[2]),
                  (bf16)((float)f[3] * s0[3]), (bf16)((float)f[4] * s1[0]), (bf16)((float)f[5] * s1[1]),
                  (bf16)((float)f[6] * s1[2]), (bf16)((float)f[7] * s1[3])};
}
__device__ __forceinline__ f32x4 frag_scale(const f32x4& f, const float* s, int g4) {
  return f * *(const f32x4*)&s[4 * g4];
}

}  // namespace gdnx

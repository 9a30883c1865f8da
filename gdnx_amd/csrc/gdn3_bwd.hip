// GDN3 Kronecker-residual recurrence, backward (gfx950).
//
// Gradient semantics of the frozen oracle (gdn3/_reference_recurrence.py:
// 60-90): the compaction runs under no_grad, so the factors A, B it leaves
// are constants, while the residual slots (U, Vb) keep their graph across
// compactions.  With chunks aligned to the P-slot window (see gdn3.hip), a
// chunk's outputs depend on
//   its own tokens, the previous chunk's net writes U_old and keys decayed to
//   that chunk's end Vbd_old, the Kronecker matrix S_kron of the last
//   compaction (a constant) and the log decay Gacc accumulated since it.
// Per chunk, with G_i the inclusive log-decay prefix, gamma_i = e^{G_i},
// e2_i = e^{2(Gacc + G_i)}, H = b o k, u = w o v, alpha_i = alpha(k_i . h_i):
//   Lm_ij = alpha_i e^{G_i-G_j} (h_i.k_j) (j<i),  T = (I + Lm)^-1
//   Ho_ip = alpha_i gamma_i (h_i.Vbd_old_p) (p>=i), Qo_ip = gamma_i (q_i.Vbd_old_p) (p>=i)
//   Aq_ij = e^{G_i-G_j} (q_i.k_j) (j<=i)
//   U = T (diag(alpha) u - diag(alpha e2) H S_kron^T - Ho U_old)
//   Y = diag(e2) Q S_kron^T + Qo U_old + Aq U
//   Vbd_j = k_j e^{G_last - G_j} (what the next chunk sees), Gacc' = Gacc + G_last
// The backward walks the chunks in reverse, one workgroup per chain, carrying
// dU (for the previous chunk's U), dVbd (for its decayed keys) and dGacc
// (reset at every compaction boundary), and recomputes each chunk's grams,
// inverse and coefficients from its inputs and the forward's stash (U per
// chunk, Gacc per chunk, the factors after every compaction).  Every
// product is fp32 MFMA.  The reference differentiates its chunk graph with
// torch autograd (gdn3/gdn3_upgrade.py:467-521).
#include "gdn3_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int BP = 16;  // tokens per sub-chunk (the forward's): the P-slot window is P / 16 blocks

// S_kron^T stays in LDS when it fits beside the window blocks (SKL), else
// each wave keeps the fragments of its key tiles in registers
template <typename CT, int D, int P, bool SKL>
struct alignas(16) G3BwdSmem {
  static constexpr int NB = P / BP;
  static constexpr int LR = D + 4;                              // fp32 rows
  static constexpr int LK = D + (sizeof(CT) == 2 ? 8 : 4);      // compute-dtype rows
  static constexpr int LP = BP + 4;                             // 16 x 16 matrices
  float h[BP][LR], q[BP][LR], k[BP][LR];  // H = b o k, Q, K of the sub-chunk
  float dy[BP][LR], u[BP][LR];
  float dr[BP][LR];                       // dRhs (and the factors while S_kron^T is rebuilt)
  CT kb[P][LK];                           // raw keys of the window blocks (block b: slots 16 b ..)
  float uo[P][LR];                        // the blocks' net writes
  CT skt[SKL ? D : 1][LK];                // S_kron^T: skt[k][v] = sum_r A_r (x) B_r at (v, k)
  float m0[BP][LP], lm[BP][LP];           // raw H K^T, Lm
  float aqt[BP][LP], tt[BP][LP];          // Aq^T, T^T
  float w[BP][LP], z[BP][LP], wt[BP][LP], zt[BP][LP];   // dLm, dAq gradient factors and transposes
  float m2[NB][BP][LP];                   // per block: raw H Vbd_b^T (keys decayed)
  float hot[NB][BP][LP], qot[NB][BP][LP]; // Ho_b^T, Qo_b^T
  float vv[NB][BP][LP], wq[NB][BP][LP];   // dHo_b, dQo_b gradient factors
  float kd[P];                            // block slot: its key's decay to the start of the sub-chunk
  float lg[BP], lgp[P], dec[BP], alpha[BP], cdot[BP], bsc[BP];   // bsc: scalar erase gates
  float G[BP], e2[BP], kco[BP], qco[BP], vsc[BP], dc[BP], su[BP];
  float red[8][4][BP];                    // per-wave partial per-token sums, slots kR*
  float carry[4];
};
constexpr int kRdA = 0, kRgRow = 1, kRgCol = 2, kRhG = 3, kRqG = 4, kRsvb = 5, kRdb = 6, kRdd = 7;

template <typename CT>
__device__ __forceinline__ void load8(const CT* p, float* f);
template <>
__device__ __forceinline__ void load8<bf16>(const bf16* p, float* f) {
  const bf16x8 x = *(const bf16x8*)p;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)x[e];
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* f) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
}
__device__ __forceinline__ void store8f(float* p, const float* f) {
  *(f32x4*)p = (f32x4){f[0], f[1], f[2], f[3]};
  *(f32x4*)(p + 4) = (f32x4){f[4], f[5], f[6], f[7]};
}
// Sum over the 16 lanes of each DPP row, the same bits in all 16 (a
// butterfly of row rotations by 8, 4, 2, 1)
__device__ __forceinline__ float row_sum16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
  return x;
}

// 8 consecutive elements held raw (one 16-byte vector per 8 bf16, two per 8
// floats), converted to float where they are used
template <typename CT> struct Row8 { uint4 w[sizeof(CT) / 2]; };
template <typename CT>
__device__ __forceinline__ void raw8(const CT* p, Row8<CT>& r) {
#pragma unroll
  for (int i = 0; i < (int)(sizeof(CT) / 2); ++i) r.w[i] = ((const uint4*)p)[i];
}
template <typename CT>
__device__ __forceinline__ void zero8(Row8<CT>& r) {
#pragma unroll
  for (int i = 0; i < (int)(sizeof(CT) / 2); ++i) r.w[i] = make_uint4(0u, 0u, 0u, 0u);
}
__device__ __forceinline__ void cvt8(const Row8<bf16>& r, float* f) {
  const bf16x8 x = *(const bf16x8*)&r.w[0];
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)x[e];
}
__device__ __forceinline__ void cvt8(const Row8<float>& r, float* f) {
  const f32x4 a = *(const f32x4*)&r.w[0], b = *(const f32x4*)&r.w[1];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
}


// A bf16 k-step fragment (k = 4 g + i and 16 + 4 g + i, i < 4) of an fp32 LDS
// row as hi + lo bf16 parts: x - hi - lo is ~2^-17 of x
__device__ __forceinline__ void split_frag(const float* p, int g, bf16x8& hi, bf16x8& lo) {
  const f32x4 x0 = *(const f32x4*)(p + 4 * g), x1 = *(const f32x4*)(p + 16 + 4 * g);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16 h0 = (bf16)x0[i], h1 = (bf16)x1[i];
    hi[i] = h0;
    hi[4 + i] = h1;
    lo[i] = (bf16)(x0[i] - (float)h0);
    lo[4 + i] = (bf16)(x1[i] - (float)h1);
  }
}

// 16x16 NT tile product over K of fp32 LDS rows on bf16 MFMA: each operand
// enters as hi + lo parts (an operand that holds bf16 values exactly needs no
// lo part); lo x lo is dropped, so the product is within ~2^-16 of fp32
// (every step's operands are read before the first split and MFMA, behind a
// scheduling barrier: the compiler, short of registers, waited for each
// step's LDS reads)
__device__ __forceinline__ void split8(const f32x4& x0, const f32x4& x1, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16 h0 = (bf16)x0[i], h1 = (bf16)x1[i];
    hi[i] = h0;
    hi[4 + i] = h1;
    lo[i] = (bf16)(x0[i] - (float)h0);
    lo[4 + i] = (bf16)(x1[i] - (float)h1);
  }
}
template <int K>
__device__ __forceinline__ f32x4 tile_nt_split(const float* arow, const float* brow, int g4, bool a_exact,
                                               bool b_exact) {
  constexpr int NS = K / 32;
  f32x4 ra[NS][2], rb[NS][2];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    ra[u][0] = *(const f32x4*)(arow + 32 * u + 4 * g4);
    ra[u][1] = *(const f32x4*)(arow + 32 * u + 16 + 4 * g4);
    rb[u][0] = *(const f32x4*)(brow + 32 * u + 4 * g4);
    rb[u][1] = *(const f32x4*)(brow + 32 * u + 16 + 4 * g4);
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = zero4();
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    bf16x8 ah, al, bh, bl;
    split8(ra[u][0], ra[u][1], ah, al);
    split8(rb[u][0], rb[u][1], bh, bl);
    mma(acc, ah, bh);
    if (!b_exact) mma(acc, ah, bl);
    if (!a_exact) mma(acc, al, bh);
  }
  return acc;
}

// The same with B a raw compute-dtype row: bf16 values are exact (no lo part)
template <int K>
__device__ __forceinline__ f32x4 tile_nt_fb(const float* arow, const bf16* brow, int g4, bool a_exact) {
  constexpr int NS = K / 32;
  f32x4 ra[NS][2];
  bf16x8 bh[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    ra[u][0] = *(const f32x4*)(arow + 32 * u + 4 * g4);
    ra[u][1] = *(const f32x4*)(arow + 32 * u + 16 + 4 * g4);
    bh[u] = ld_frag(brow + 32 * u, g4);
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = zero4();
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    bf16x8 ah, al;
    split8(ra[u][0], ra[u][1], ah, al);
    mma(acc, ah, bh[u]);
    if (!a_exact) mma(acc, al, bh[u]);
  }
  return acc;
}
template <int K>
__device__ __forceinline__ f32x4 tile_nt_fb(const float* arow, const float* brow, int g4, bool) {
  return tile_nt<float, K>(arow, brow, g4);
}

// 8 values to 8 consecutive entries of the compute dtype (16-byte aligned)
__device__ __forceinline__ void store8c(float* p, const float* f) { store8f(p, f); }
__device__ __forceinline__ void store8c(bf16* p, const float* f) {
  *(bf16x8*)p = (bf16x8){(bf16)f[0], (bf16)f[1], (bf16)f[2], (bf16)f[3],
                         (bf16)f[4], (bf16)f[5], (bf16)f[6], (bf16)f[7]};
}

// lane (g, n): X[4 g + s][col], s = 0..3 -- a fragment over k = rows of a
// row-major P x D LDS matrix
template <int LR>
__device__ __forceinline__ f32x4 col_frag(const float (*X)[LR], int col, int g4) {
  return (f32x4){X[4 * g4][col], X[4 * g4 + 1][col], X[4 * g4 + 2][col], X[4 * g4 + 3][col]};
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <typename CT, int D, int P>
__global__ void __launch_bounds__(kNT) gdn3_bwd_kernel(G3BwdArgs p) {
  typedef G3D<D> Ge;
  constexpr bool SKL = sizeof(G3BwdSmem<CT, D, P, true>) <= 160 * 1024;
  typedef G3BwdSmem<CT, D, P, SKL> Sm;
  __shared__ Sm sm;
  static_assert(sizeof(Sm) <= 160 * 1024, "LDS budget");
  constexpr int NB = Sm::NB, DG = D / 8, UNITS = BP * DG, NDT = D / 16, VPW = NDT / 4, LR = Sm::LR;
  static_assert(UNITS <= kNT && VPW >= 1, "one load unit per thread, a tile per wave");
  static_assert(P % BP == 0 && NB >= 1 && NB <= 4, "whole blocks of 16 slots, at most 4");
  constexpr int NT = 2 + 2 * NB;      // gram / gradient tiles: H K^T, Q K^T, then H, Q against block b
  constexpr int TPW = (NT + 3) / 4;   // tile ti on wave ti mod 4
  constexpr int KS = FragT<CT>::KSTEP;
  typedef typename FragT<CT>::type Frag;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), g4 = lane >> 4, n16 = lane & 15;
  const int H = p.H, M = p.M, T = p.T;
  const int N = p.B * H * M;
  const int chain = xcd_remap(blockIdx.x, N);
  const int b = chain / (H * M), hm = chain % (H * M), h = hm / M, m = hm % M;
  const bool has_unit = tid < UNITS;
  const int ui = tid / DG, ud = 8 * (tid % DG);
  const int L = p.qkv_lanes, gc = p.gate_ch;
  const size_t qkv_tok = (size_t)H * L * D;
  const size_t qkv_base = ((size_t)b * T * H + h) * L * D + (L > 1 ? (size_t)m * D : 0);
  const size_t gate_tok = (size_t)H * M * gc;
  const size_t gate_base = (((size_t)b * T * H + h) * M + m) * gc;
  const size_t dec_tok = (size_t)H * M;
  const size_t dec_base = ((size_t)b * T * H + h) * M + m;
  const size_t y_tok = (size_t)H * M * D;
  const size_t y_base = (((size_t)b * T * H + h) * M + m) * D;
  const int nch = (T + BP - 1) / BP, per = p.Kc / BP, ncomp = T / p.Kc;
  const G3Stash ts = g3_stash(const_cast<void*>(p.train_states), N, nch, ncomp, D, BP, Ge::RMN);

  // carried per window block b (this wave's value / key tiles): dUa, d/dU of
  // the sub-chunk the block holds (complete once every later reader is
  // processed), and dVa, d/dVbd of its keys as seen at the start of the
  // sub-chunk after the one being processed
  f32x4 dUa[NB][VPW], dVa[NB][VPW];
#pragma unroll
  for (int bl = 0; bl < NB; ++bl)
#pragma unroll
    for (int a = 0; a < VPW; ++a) dUa[bl][a] = dVa[bl][a] = zero4();
  float dgacc = 0.f;          // d/dGacc of the sub-chunk after the current one
  Frag skf[SKL ? 1 : VPW][SKL ? 1 : D / KS];   // S_kron^T fragments of this wave's key tiles (!SKL)

  // the factors of the interval a sub-chunk rebuilds S_kron^T from, fetched
  // into registers a sub-chunk ahead (their loads land while the one before
  // computes)
  constexpr int NAB = (Ge::RMN + kNT - 1) / kNT;
  float abr[NAB];
  auto rebuilds = [&](int cc) { return cc / per > 0 && (cc == nch - 1 || (cc + 1) % per == 0); };
  auto fetch_ab = [&](int cc) {
    const float* ab = ts.ab + ((size_t)(cc / per - 1) * N + chain) * Ge::RMN;
    // (a clamped index, no branch: a load under a branch drew a wait for every
    // load issued before it)
#pragma unroll
    for (int u = 0; u < NAB; ++u) abr[u] = ab[min(tid + u * kNT, Ge::RMN - 1)];
  };
  if (nch > 0 && rebuilds(nch - 1)) fetch_ab(nch - 1);

  // a window block: sub-chunk mb's raw keys and net writes (zero before the
  // sequence) into block mb mod NB
  auto load_block = [&](int mb, Row8<CT>& rk, Row8<float>& ru) {
    zero8(rk), zero8(ru);
    if (has_unit && mb >= 0) {
      raw8<CT>((const CT*)p.k + qkv_base + (size_t)(mb * BP + ui) * qkv_tok + ud, rk);
      raw8<float>(ts.u + ((size_t)chain * nch + mb) * BP * D + (size_t)ui * D + ud, ru);
    }
  };
  auto store_block = [&](int mb, const Row8<CT>& rk, const Row8<float>& ru) {
    if (!has_unit) return;
    const int sl = BP * (((mb % NB) + NB) % NB) + ui;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(CT) / 2); ++i) *(uint4*)&sm.kb[sl][ud + i * (16 / sizeof(CT))] = rk.w[i];
    *(uint4*)&sm.uo[sl][ud] = ru.w[0];
    *(uint4*)&sm.uo[sl][ud + 4] = ru.w[1];
  };
  // the blocks the last sub-chunk sees whole (sub-chunks nch - NB .. nch - 2)
  for (int mb = nch - NB; mb <= nch - 2; ++mb) {
    Row8<CT> rk;
    Row8<float> ru;
    load_block(mb, rk, ru);
    store_block(mb, rk, ru);
  }

  for (int c = nch - 1; c >= 0; --c) {
    const int iv = c / per;
    const bool live = iv > 0;
    const int beta = c % NB;
    if ((c + 1) % per == 0 && (long long)(c + 1) * BP <= T) dgacc = 0.f;  // compaction after this sub-chunk
    const float gacc = ts.gacc[(size_t)chain * nch + c];
    f32x4 dUc[VPW], dVc[VPW];   // this sub-chunk's complete d/dU and d/d(keys decayed to its end)
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
      if (bl == beta)
#pragma unroll
        for (int a = 0; a < VPW; ++a) {
          dUc[a] = dUa[bl][a];
          dVc[a] = dVa[bl][a];
        }
    // the previous sub-chunk is done with LDS (an LDS-only barrier: its gradient
    // stores to global memory stay in flight, nothing reads them back)
    lds_barrier();
    // the factors S_kron^T is rebuilt from (fetched a sub-chunk ahead) go to
    // LDS before this sub-chunk's input loads are issued, so that waiting for
    // them does not wait for those
    const bool rebuild = live && rebuilds(c);
    float* st = &sm.dr[0][0];
    if (rebuild) {
#pragma unroll
      for (int u = 0; u < NAB; ++u) {
        const int e = tid + u * kNT;
        if (e < Ge::RMN) st[e] = abr[u];
      }
    }
    // the next rebuild's factors, issued ahead of this sub-chunk's input loads
    if (c > 0 && rebuilds(c - 1)) fetch_ab(c - 1);
    // the decay of token c BP - P + tid (tid < P), loaded unconditionally at an
    // in-bounds token and used raw in A: a load in a branch drew its clamp in
    // after it, whose wait then held every input load issued above; issued
    // before the inputs (its address arithmetic after them reused a register
    // of a pending input load and so waited for all of them)
    const int tpv = c * BP - P + (tid < P ? tid : 0);
    const float dvp = p.dec[dec_base + (size_t)(tpv > 0 ? tpv : 0) * dec_tok];

    // the sub-chunk's inputs, the block entering the window (sub-chunk c -
    // NB) and the decays of the P tokens before the sub-chunk, loaded raw
    // before the S_kron^T rebuild so that their latency hides behind it
    const int t = c * BP + ui;
    const bool tv = has_unit && t < T;
    Row8<CT> rk, rq, rv, rdy, rkp;
    Row8<float> rb, rw, ru, ruo;
    float bs = 0.f, ws = 0.f, dv = 1.f;
    zero8(rk), zero8(rq), zero8(rv), zero8(rdy), zero8(rb), zero8(rw), zero8(ru);
    if (tv) {
      raw8<CT>((const CT*)p.k + qkv_base + (size_t)t * qkv_tok + ud, rk);
      raw8<CT>((const CT*)p.q + qkv_base + (size_t)t * qkv_tok + ud, rq);
      raw8<CT>((const CT*)p.v + qkv_base + (size_t)t * qkv_tok + ud, rv);
      raw8<CT>((const CT*)p.dy + y_base + (size_t)t * y_tok + ud, rdy);
      // the scalar gates (channel 0 of per-channel gates, unused then) load
      // unconditionally: a value set in one branch and loaded in the other made
      // the merge wait for every load issued before
      bs = p.bg[gate_base + (size_t)t * gate_tok];
      ws = p.wg[gate_base + (size_t)t * gate_tok];
      if (gc > 1) {
        raw8<float>(p.bg + gate_base + (size_t)t * gate_tok + ud, rb);
        raw8<float>(p.wg + gate_base + (size_t)t * gate_tok + ud, rw);
      }
      dv = p.dec[dec_base + (size_t)t * dec_tok];
      raw8<float>(ts.u + ((size_t)chain * nch + c) * BP * D + (size_t)ui * D + ud, ru);
    }
    // per-channel erase gates at this wave's key tiles (used in G), loaded with
    // the rest (in G they would sit between stores the compiler cannot reorder
    // them past); scalar gates go through LDS from A
    float bgc[VPW][4];
#pragma unroll
    for (int a = 0; a < VPW; ++a)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) bgc[a][s4] = 0.f;
    if (gc > 1) {
#pragma unroll
      for (int a = 0; a < VPW; ++a)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const int tt_ = c * BP + 4 * g4 + s4, d = 16 * (wave * VPW + a) + n16;
          if (tt_ < T) bgc[a][s4] = p.bg[gate_base + (size_t)tt_ * gate_tok + d];
        }
    }
    load_block(c - NB, rkp, ruo);

    // ---- S_kron^T of this interval (the factors of compaction iv - 1), rebuilt on entry ----
    if (rebuild) {
      lds_barrier();   // the inputs loaded above stay in flight across it
      const float* Bf = st + Ge::R * Ge::m;
      if constexpr (SKL) {
        // skt[k][v] (k = ik b_k + jk, v = iv b_v + jv) = sum_r B_r[jv][jk] A_r[iv][ik]:
        // for a tile of 16 (jk, jv) rows (16 / b_v values of jk) and 16
        // (ik, iv) columns (16 / a_v values of ik) a product with K = R = 4,
        // one fp32 MFMA.  Lane (g, l) holds rows 4 g .. 4 g + 3, i.e. 4
        // consecutive jv of one jk, and column l: 4 consecutive v of row k, one
        // 4-element store.  The tiles go round the 4 waves.
        static_assert(Ge::R == 4 && 16 % Ge::bv == 0 && 16 % Ge::av == 0 && Ge::bv % 4 == 0, "K = R = 4 MFMA tiles");
        constexpr int JKT = 16 / Ge::bv, IKT = 16 / Ge::av;   // jk and ik per tile
        constexpr int NJ = Ge::bk / JKT, NT = NJ * (Ge::ak / IKT);
        static_assert(NT % 4 == 0, "whole tiles per wave");
        // Every operand is read before the first MFMA and every MFMA issued
        // before the first store: in a read / MFMA / store chain per tile the
        // stores (which might alias the factors, as far as the compiler can
        // tell) would hold each next read, one LDS round trip per tile.
        const int g = lane >> 4, l16 = lane & 15;
        constexpr int TW = NT / 4;   // tiles per wave
        float av[TW], bv[TW];
#pragma unroll
        for (int u = 0; u < TW; ++u) {
          const int t = wave + 4 * u, jk0 = (t % NJ) * JKT, ik0 = (t / NJ) * IKT;
          av[u] = Bf[g * Ge::n + (l16 % Ge::bv) * Ge::bk + jk0 + l16 / Ge::bv];
          bv[u] = st[g * Ge::m + (l16 % Ge::av) * Ge::ak + ik0 + l16 / Ge::av];
        }
        f32x4 acc[TW];
#pragma unroll
        for (int u = 0; u < TW; ++u)
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], zero4(), 0, 0, 0);
#pragma unroll
        for (int u = 0; u < TW; ++u) {
          const int t = wave + 4 * u, jk0 = (t % NJ) * JKT, ik0 = (t / NJ) * IKT;
          const int i0 = 4 * g, jk = jk0 + i0 / Ge::bv, jv = i0 % Ge::bv;
          const int ik = ik0 + l16 / Ge::av, iv = l16 % Ge::av;
          st4(&sm.skt[ik * Ge::bk + jk][iv * Ge::bv + jv], acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
        }
      } else {
        // the fragments this lane feeds the Kronecker products: row k = d of
        // its key tiles, values v = kb KS + (the fragment's k set)
#pragma unroll
        for (int a = 0; a < VPW; ++a) {
          const int d = 16 * (wave * VPW + a) + n16, ik = d >> Ge::lbk, jk = d & (Ge::bk - 1);
#pragma unroll
          for (int kb = 0; kb < D / KS; ++kb) {
            float sv[sizeof(CT) == 2 ? 8 : 4];
#pragma unroll
            for (int e = 0; e < (int)(sizeof(CT) == 2 ? 8 : 4); ++e) {
              const int v = kb * KS + (e < 4 ? 4 * g4 + e : 16 + 4 * g4 + e - 4);
              const int ivv = v >> Ge::lbv, jv = v & (Ge::bv - 1);
              float x = 0.f;
#pragma unroll
              for (int r = 0; r < Ge::R; ++r) x += st[r * Ge::m + ivv * Ge::ak + ik] * Bf[r * Ge::n + jv * Ge::bk + jk];
              sv[e] = x;
            }
            if constexpr (sizeof(CT) == 2)
              skf[a][kb] = (bf16x8){(bf16)sv[0], (bf16)sv[1], (bf16)sv[2], (bf16)sv[3],
                                    (bf16)sv[4], (bf16)sv[5], (bf16)sv[6], (bf16)sv[7]};
            else
              skf[a][kb] = (f32x4){sv[0], sv[1], sv[2], sv[3]};
          }
        }
      }
    }

    // ---- A: the sub-chunk's inputs to LDS (h = b o k, alpha, log decays), the entering block ----
    float vf[8], wf[8];
    {
      float kf[8], qf[8], bf[8], dyf[8], us[8];
      cvt8(rk, kf);
      cvt8(rq, qf);
      cvt8(rv, vf);
      cvt8(rdy, dyf);
      cvt8(ru, us);
      if (gc > 1) {
        cvt8(rb, bf);
        cvt8(rw, wf);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          bf[e] = bs;
          wf[e] = ws;
        }
      }
      float hf[8], part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hf[e] = bf[e] * kf[e];
        part += kf[e] * hf[e];
      }
      if (has_unit) {
        store8f(&sm.h[ui][ud], hf);
        store8f(&sm.q[ui][ud], qf);
        store8f(&sm.k[ui][ud], kf);
        store8f(&sm.dy[ui][ud], dyf);
        store8f(&sm.u[ui][ud], us);
      }
      store_block(c - NB, rkp, ruo);
      if constexpr (DG == 16) {   // a token row is one DPP row
        part = row_sum16(part);
      } else {
#pragma unroll
        for (int off = 1; off < DG; off <<= 1) part += __shfl_xor(part, off, 64);
      }
      if (has_unit && tid % DG == 0) {
        sm.cdot[ui] = part;
        sm.alpha[ui] = stable_alpha_f(part);
        sm.lg[ui] = tv ? log_decay(dv) : 0.f;
        sm.dec[ui] = dv;
        sm.bsc[ui] = bs;
      }
      if (tid < P) sm.lgp[tid] = c * BP - P + tid >= 0 ? log_decay(dvp) : 0.f;
    }
    __syncthreads();

    // ---- B: per-token scalars and key decays (every wave scans for itself), the grams ----
    float gl = lane < BP ? sm.lg[lane] : 0.f;
#pragma unroll
    for (int off = 1; off < BP; off <<= 1) {
      const float o = __shfl_up(gl, off, 64);
      if (lane >= off) gl += o;
    }
    // lane j < P: token 16 c - P + j (block (c + j / 16) mod NB, slot j mod 16),
    // its key decayed to the start of this sub-chunk by exp(sum of the later log decays)
    float lp = lane < P ? sm.lgp[lane] : 0.f;
#pragma unroll
    for (int off = 1; off < P; off <<= 1) {
      const float o = __shfl_up(lp, off, 64);
      if (lane >= off) lp += o;
    }
    const float kdv = expf(__shfl(lp, P - 1, 64) - lp);
    const float gl_last = __shfl(gl, BP - 1, 64);
    if (wave == 0) {
      if (lane < BP) {
        const float e2 = expf(2.f * (gacc + gl));
        sm.G[lane] = gl;
        sm.e2[lane] = e2;
        sm.kco[lane] = sm.alpha[lane] * e2;
        sm.qco[lane] = e2;
        sm.vsc[lane] = expf(gl_last - gl);
      }
      if (lane < P) sm.kd[BP * ((c + lane / BP) % NB) + lane % BP] = kdv;
    }
    {
      const int j = n16;
      const float Gj = __shfl(gl, j, 64);
      // the rows' alpha read once, before the tile stores (a read after a store
      // to LDS the compiler cannot tell apart waits for that store)
      float Gi[4], ali[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        Gi[s] = __shfl(gl, 4 * g4 + s, 64);
        ali[s] = sm.alpha[4 * g4 + s];
      }
#pragma unroll
      for (int r = 0; r < TPW; ++r) {
        const int ti = wave + 4 * r;
        if (ti < NT) {
          const bool isq = ti & 1;
          const float* ar = isq ? &sm.q[0][0] : &sm.h[0][0];
          const int bl = (ti - 2) >> 1;
          f32x4 acc;
          if (ti < 2) {
            if constexpr (sizeof(CT) == 2)   // bf16 IO: q and k are bf16 values exactly
              acc = tile_nt_split<D>(ar + n16 * LR, &sm.k[n16][0], g4, isq, true);
            else
              acc = tile_nt<float, D>(ar + n16 * LR, &sm.k[n16][0], g4);
          } else {
            acc = tile_nt_fb<D>(ar + n16 * LR, &sm.kb[BP * bl + n16][0], g4, isq);
          }
          if (ti == 0) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const int i = 4 * g4 + s;
              sm.m0[i][j] = acc[s];
              sm.lm[i][j] = (j < i) ? ali[s] * expf(Gi[s] - Gj) * acc[s] : 0.f;
            }
          } else if (ti == 1) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const int i = 4 * g4 + s;
              sm.aqt[j][i] = (j <= i) ? expf(Gi[s] - Gj) * acc[s] : 0.f;
            }
          } else {
            // block bl holds window tokens jb 16 .. jb 16 + 15 (jb = (bl - c) mod NB)
            const int jb = ((bl - c) % NB + NB) % NB;
            const float kdj = __shfl(kdv, jb * BP + j, 64);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const int i = 4 * g4 + s;
              const bool vis = bl != beta || j >= i;
              const float ga = expf(Gi[s]), m2 = kdj * acc[s];
              if (!isq) {
                sm.m2[bl][i][j] = m2;
                sm.hot[bl][j][i] = vis ? ali[s] * ga * m2 : 0.f;
              } else {
                sm.qot[bl][j][i] = vis ? ga * m2 : 0.f;
              }
            }
          }
        }
      }
    }
    __syncthreads();

    // ---- C: T = (I + Lm)^-1 (wave 0) ----
    if (wave == 0) {
      // Lm is strictly lower: (I + Lm)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8)
      f32x4 xa, ta;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        xa[s] = sm.lm[i][n16];
        ta[s] = (i == n16 ? 1.f : 0.f) - xa[s];
      }
      const float* src = &sm.lm[0][0];
#pragma unroll
      for (int step = 0; step < 3; ++step) {
        float* dst = (step & 1) ? &sm.w[0][0] : &sm.z[0][0];
        f32x4 sq = zero4();
        mma(sq, *(const f32x4*)&src[n16 * Sm::LP + 4 * g4], xa);
        xa = sq;
#pragma unroll
        for (int s = 0; s < 4; ++s) dst[(4 * g4 + s) * Sm::LP + n16] = sq[s];
        wave_lds_sync();
        mma(ta, *(const f32x4*)&dst[n16 * Sm::LP + 4 * g4], ta);
        src = dst;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) sm.tt[n16][4 * g4 + s] = ta[s];   // T^T
    }
    __syncthreads();

    // ---- D: dU_tot = dU + Aq^T dY, dRhs = T^T dU_tot, the blocks' dU ----
    {
      // every operand read before the first dRhs store (reads after a store the
      // compiler cannot tell apart would wait for it)
      const f32x4 aqf = ld_frag(&sm.aqt[n16][0], g4), ttf = ld_frag(&sm.tt[n16][0], g4);
      f32x4 qof[NB], hof[NB], dYf[VPW];
#pragma unroll
      for (int bl = 0; bl < NB; ++bl) {
        qof[bl] = ld_frag(&sm.qot[bl][n16][0], g4);
        hof[bl] = ld_frag(&sm.hot[bl][n16][0], g4);
      }
#pragma unroll
      for (int a = 0; a < VPW; ++a) dYf[a] = col_frag<LR>(sm.dy, 16 * (wave * VPW + a) + n16, g4);
#pragma unroll
      for (int a = 0; a < VPW; ++a) {
        const int col = 16 * (wave * VPW + a) + n16;
        f32x4 dut = dUc[a];
        mma(dut, aqf, dYf[a]);
        f32x4 drh = zero4();
        mma(drh, ttf, dut);
#pragma unroll
        for (int s = 0; s < 4; ++s) sm.dr[4 * g4 + s][col] = drh[s];
#pragma unroll
        for (int bl = 0; bl < NB; ++bl) {
          f32x4 nd = zero4();
          mma(nd, qof[bl], dYf[a]);
          mma(nd, hof[bl], -drh);
          dUa[bl][a] = (bl == beta) ? nd : dUa[bl][a] + nd;
        }
      }
    }
    __syncthreads();

    // ---- E: gradients of the 16 x 16 coefficient tiles, the Kronecker
    // products, the value / write-gate gradients ----
    {
      const int j = n16;
      const float Gj = sm.G[j];
      float cg = 0.f, rda[4] = {0.f, 0.f, 0.f, 0.f}, rg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < TPW; ++r) {
        const int ti = wave + 4 * r;
        if (ti < NT) {
          const bool isq = ti & 1;   // dY rows (else -dRhs)
          const float* ar = isq ? &sm.dy[0][0] : &sm.dr[0][0];
          const int bl = (ti - 2) >> 1;
          const float* br = ti < 2 ? &sm.u[0][0] : &sm.uo[BP * bl][0];
          f32x4 acc;
          if constexpr (sizeof(CT) == 2)   // bf16 IO: dY holds bf16 values exactly
            acc = tile_nt_split<D>(ar + n16 * LR, br + n16 * LR, g4, isq, false);
          else
            acc = tile_nt<float, D>(ar + n16 * LR, br + n16 * LR, g4);
          if (!isq) acc = -acc;
          // the element loop's operands, read before its first store (a read
          // after a store the compiler cannot tell apart waits for it)
          float Gv[4], alv[4], o1[4], o2[4];
          const int blc = bl < 0 ? 0 : bl;   // (tiles 0 and 1 read no block)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int i = 4 * g4 + s;
            Gv[s] = sm.G[i];
            alv[s] = sm.alpha[i];
            o1[s] = ti == 0 ? sm.m0[i][j] : ti == 1 ? sm.aqt[j][i] : isq ? 0.f : sm.m2[blc][i][j];
            o2[s] = ti < 2 ? 0.f : isq ? sm.qot[blc][j][i] : sm.hot[blc][j][i];
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int i = 4 * g4 + s;
            const float Gi = Gv[s], al = alv[s], ga = expf(Gi);
            if (ti == 0) {          // dLm (j < i)
              const float x = (j < i) ? acc[s] : 0.f, e = expf(Gi - Gj), m0 = o1[s];
              const float wv = x * al * e;
              sm.w[i][j] = wv;
              sm.wt[j][i] = wv;
              rda[s] += x * e * m0;
              const float g = x * al * e * m0;
              rg[s] += g;
              cg += g;
            } else if (ti == 1) {   // dAq (j <= i)
              const float x = (j <= i) ? acc[s] : 0.f, e = expf(Gi - Gj);
              const float zv = x * e;
              sm.z[i][j] = zv;
              sm.zt[j][i] = zv;
              const float g = x * o1[s];
              rg[s] += g;
              cg += g;
            } else {
              const bool vis = bl != beta || j >= i;
              const float x = vis ? acc[s] : 0.f;
              if (!isq) {           // dHo_b
                sm.vv[bl][i][j] = x * al * ga;
                rda[s] += x * ga * o1[s];
                rg[s] += x * o2[s];
              } else {              // dQo_b
                sm.wq[bl][i][j] = x * ga;
                rg[s] += x * o2[s];
              }
            }
          }
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        const float a_ = row_prefix16(rda[s]), g_ = row_prefix16(rg[s]);
        if (n16 == 15) {
          sm.red[kRdA][wave][i] = a_;
          sm.red[kRgRow][wave][i] = g_;
        }
      }
      cg += __shfl_xor(cg, 16, 64);
      cg += __shfl_xor(cg, 32, 64);
      if (g4 == 0) sm.red[kRgCol][wave][j] = cg;   // zero on waves without tile 0 or 1
    }
    // Kronecker products G_h = dRhs S_kron, G_q = dY S_kron on this wave's key tiles,
    // and per-token partials h . G_h, q . G_q, dVbd . Vbd
    f32x4 Gh[VPW], Gq[VPW];
    // bf16 MFMA: S_kron^T is bf16, dY holds bf16 values exactly, dRhs enters as
    // hi + lo parts; the dRhs and dY fragments are read and split once for
    // both key tiles, every read ahead of its MFMAs behind a scheduling barrier
    constexpr int NKB = D / 32;
    bf16x8 rfh[sizeof(CT) == 2 ? NKB : 1], rfl[sizeof(CT) == 2 ? NKB : 1], yfh[sizeof(CT) == 2 ? NKB : 1];
    if constexpr (sizeof(CT) == 2) {
      if (live) {
        f32x4 xr[NKB][2], xy[NKB][2];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          xr[kb][0] = *(const f32x4*)&sm.dr[n16][kb * 32 + 4 * g4];
          xr[kb][1] = *(const f32x4*)&sm.dr[n16][kb * 32 + 16 + 4 * g4];
          xy[kb][0] = *(const f32x4*)&sm.dy[n16][kb * 32 + 4 * g4];
          xy[kb][1] = *(const f32x4*)&sm.dy[n16][kb * 32 + 16 + 4 * g4];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          bf16x8 yl;
          split8(xr[kb][0], xr[kb][1], rfh[kb], rfl[kb]);
          split8(xy[kb][0], xy[kb][1], yfh[kb], yl);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < VPW; ++a) {
      const int kt = wave * VPW + a, d = 16 * kt + n16;
      Gh[a] = Gq[a] = zero4();
      if (live) {
        if constexpr (sizeof(CT) == 2) {
          bf16x8 sf[NKB];
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            if constexpr (SKL) sf[kb] = ld_frag(&sm.skt[d][kb * 32], g4);
            else sf[kb] = skf[a][kb];
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            mma(Gh[a], rfh[kb], sf[kb]);
            mma(Gh[a], rfl[kb], sf[kb]);
            mma(Gq[a], yfh[kb], sf[kb]);
          }
        } else {
#pragma unroll 4
          for (int kb = 0; kb < D / 16; ++kb) {
            f32x4 sf;
            if constexpr (SKL) sf = load4(&sm.skt[d][kb * 16 + 4 * g4]);
            else sf = skf[a][kb];
            mma(Gh[a], ld_frag(&sm.dr[n16][kb * 16], g4), sf);
            mma(Gq[a], ld_frag(&sm.dy[n16][kb * 16], g4), sf);
          }
        }
      }
    }
    {
      // all rows' partials before the first store to red (reads after it
      // would wait for it)
      float xh[4], xq[4], xv[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        xh[s] = xq[s] = xv[s] = 0.f;
#pragma unroll
        for (int a = 0; a < VPW; ++a) {
          const int d = 16 * (wave * VPW + a) + n16;
          xh[s] += sm.h[i][d] * Gh[a][s];
          xq[s] += sm.q[i][d] * Gq[a][s];
          xv[s] += dVc[a][s] * sm.k[i][d];
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        const float ph = row_prefix16(xh[s]), pq = row_prefix16(xq[s]), pv = row_prefix16(xv[s]);
        if (n16 == 15) {
          sm.red[kRhG][wave][i] = ph;
          sm.red[kRqG][wave][i] = pq;
          sm.red[kRsvb][wave][i] = pv;   // times vsc_i below
        }
      }
    }
    // the blocks this sub-chunk leaves in the window decay by e^{G_last}:
    // sum over them of dVa . (keys decayed to the start of this sub-chunk)
    if constexpr (NB > 1) {
      float xd = 0.f;
#pragma unroll
      for (int bl = 0; bl < NB; ++bl)
        if (bl != beta)
#pragma unroll
          for (int a = 0; a < VPW; ++a) {
            const int d = 16 * (wave * VPW + a) + n16;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const int sl = BP * bl + 4 * g4 + s;
              xd += dVa[bl][a][s] * (float)sm.kb[sl][d] * sm.kd[sl];
            }
          }
      xd = row_sum16(xd);
      xd += __shfl_xor(xd, 16, 64);
      xd += __shfl_xor(xd, 32, 64);
      if (lane == 0) sm.red[kRdd][wave][0] = xd;
    }
    // u = w o v: dv = w alpha dRhs, dw = v alpha dRhs, and sum_v w v dRhs per token
    {
      float dr8[8], dvo[8], dwo[8], ut = 0.f, dws = 0.f;
      const float al = has_unit ? sm.alpha[ui] : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dr8[e] = has_unit ? sm.dr[ui][ud + e] : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float du = al * dr8[e];
        dvo[e] = wf[e] * du;
        dwo[e] = vf[e] * du;
        dws += dwo[e];
        ut += wf[e] * vf[e] * dr8[e];
      }
      if constexpr (DG == 16) {
        ut = row_sum16(ut);
        dws = row_sum16(dws);
      } else {
#pragma unroll
        for (int off = 1; off < DG; off <<= 1) {
          ut += __shfl_xor(ut, off, 64);
          dws += __shfl_xor(dws, off, 64);
        }
      }
      if (tv) {
        store8f(p.dv + y_base + (size_t)t * y_tok + ud, dvo);
        if (gc > 1) store8f(p.dwg + gate_base + (size_t)t * gate_tok + ud, dwo);
        else if (tid % DG == 0) p.dwg[gate_base + (size_t)t * gate_tok] = dws;
      }
      if (has_unit && tid % DG == 0) sm.su[ui] = ut;
    }
    __syncthreads();

    // ---- F: per-token scalar gradients (wave 0, lane = token) ----
    const float egl = expf(sm.G[BP - 1]);   // the sub-chunk's total decay
    if (wave == 0) {
      float dG = 0.f, dE = 0.f, svb = 0.f;
      if (lane < BP) {
        const int i = lane;
        float da = sm.su[i], dkco = 0.f, dqco = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          da += sm.red[kRdA][w][i];
          dG += sm.red[kRgRow][w][i] - sm.red[kRgCol][w][i];
          svb += sm.red[kRsvb][w][i];
          if (live) {
            dkco -= sm.red[kRhG][w][i];
            dqco += sm.red[kRqG][w][i];
          }
        }
        svb *= sm.vsc[i];
        const float e2 = sm.e2[i], al = sm.alpha[i];
        da += dkco * e2;
        dE = 2.f * e2 * (dkco * al + dqco);
        dG += dE - svb;
        sm.dc[i] = da * stable_dalpha_f(sm.cdot[i]);
      }
      float svt = row_sum16(svb), det = row_sum16(dE);   // then across the four DPP rows
      svt += __shfl_xor(svt, 16, 64);
      det += __shfl_xor(det, 16, 64);
      svt += __shfl_xor(svt, 32, 64);
      det += __shfl_xor(det, 32, 64);
      float gdd = 0.f;   // G_last through the older blocks' decay
      if constexpr (NB > 1)
        gdd = egl * ((sm.red[kRdd][0][0] + sm.red[kRdd][1][0]) + (sm.red[kRdd][2][0] + sm.red[kRdd][3][0]));
      // G_last: the decayed keys, the next sub-chunk's Gacc and the older blocks
      if (lane == BP - 1) dG += svt + dgacc + gdd;
      // d log-decay_s = sum_{i >= s} dG_i: the 16 tokens are DPP row 0
      const float sfx = row_suffix16(lane < BP ? dG : 0.f);
      const int tt_ = c * BP + lane;
      if (lane < BP && tt_ < T) p.ddec[dec_base + (size_t)tt_ * dec_tok] = sfx * dlog_decay(sm.dec[lane]);
      if (lane == 0) sm.carry[0] = det + dgacc;
    }
    __syncthreads();
    dgacc = sm.carry[0];

    // ---- G: dH, dQ, dK on this wave's key tiles; the blocks' dVbd ----
    float dbs[4] = {0.f, 0.f, 0.f, 0.f};   // per-token partial k . dh (scalar erase gates)
    // every LDS operand read ahead of the MFMAs, behind a scheduling barrier
    // (the compiler, short of registers, waited for each MFMA's reads); the
    // coefficient fragments and per-token scalars serve both key tiles
    const f32x4 fw = ld_frag(&sm.w[n16][0], g4), fz = ld_frag(&sm.z[n16][0], g4);
    const f32x4 fwt = ld_frag(&sm.wt[n16][0], g4), fzt = ld_frag(&sm.zt[n16][0], g4);
    f32x4 fvv[NB], fwq[NB], vvt[NB], wqt[NB];
#pragma unroll
    for (int bl = 0; bl < NB; ++bl) {
      fvv[bl] = ld_frag(&sm.vv[bl][n16][0], g4);
      fwq[bl] = ld_frag(&sm.wq[bl][n16][0], g4);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        vvt[bl][s] = sm.vv[bl][4 * g4 + s][n16];
        wqt[bl][s] = sm.wq[bl][4 * g4 + s][n16];
      }
    }
    float dcv[4], kcv[4], qcv[4], vsv[4], bsv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g4 + s;
      dcv[s] = sm.dc[i];
      kcv[s] = sm.kco[i];
      qcv[s] = sm.qco[i];
      vsv[s] = sm.vsc[i];
      bsv[s] = sm.bsc[i];
    }
    f32x4 Kcv[VPW], Hcv[VPW], Qcv[VPW], Vcv[VPW][NB];
#pragma unroll
    for (int a = 0; a < VPW; ++a) {
      const int d = 16 * (wave * VPW + a) + n16;
      Kcv[a] = col_frag<LR>(sm.k, d, g4);
      Hcv[a] = col_frag<LR>(sm.h, d, g4);
      Qcv[a] = col_frag<LR>(sm.q, d, g4);
#pragma unroll
      for (int bl = 0; bl < NB; ++bl)
#pragma unroll
        for (int s = 0; s < 4; ++s) {   // the block's keys decayed to the start of this sub-chunk (k = slot)
          const int sl = BP * bl + 4 * g4 + s;
          Vcv[a][bl][s] = (float)sm.kb[sl][d] * sm.kd[sl];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int a = 0; a < VPW; ++a) {
      const int d = 16 * (wave * VPW + a) + n16;
      const f32x4 Kc = Kcv[a], Hc = Hcv[a], Qc = Qcv[a];
      f32x4 dH = zero4(), dQ = zero4(), dK = zero4();
      mma(dH, fw, Kc);
      mma(dQ, fz, Kc);
      mma(dK, fwt, Hc);
      mma(dK, fzt, Qc);
#pragma unroll
      for (int bl = 0; bl < NB; ++bl) {
        mma(dH, fvv[bl], Vcv[a][bl]);
        mma(dQ, fwq[bl], Vcv[a][bl]);
        // d/dVbd_b = dHo_b^T H + dQo_b^T Q (A operand: the transposes, read by column)
        f32x4 dVo = zero4();
        mma(dVo, vvt[bl], Hc);
        mma(dVo, wqt[bl], Qc);
        dVa[bl][a] = (bl == beta) ? dVo : egl * dVa[bl][a] + dVo;
      }
      float dbp[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s, tt_ = c * BP + i;
        const bool ok = tt_ < T;
        const float dci = dcv[s];
        float dh = dH[s] + dci * Kc[s];
        if (live) dh -= kcv[s] * Gh[a][s];
        const float dq = dQ[s] + (live ? qcv[s] * Gq[a][s] : 0.f);
        const float bgv = gc > 1 ? bgc[a][s] : bsv[s];
        const float dk = dK[s] + dci * Hc[s] + dVc[a][s] * vsv[s] + bgv * dh;
        dbp[s] = Kc[s] * dh;
        dbs[s] += dbp[s];
        if (ok) {
          const size_t o = y_base + (size_t)tt_ * y_tok + d;
          p.dq[o] = dq;
          p.dk[o] = dk;
          if (gc > 1) p.dbg[gate_base + (size_t)tt_ * gate_tok + d] = dbp[s];
        }
      }
    }
    if (gc == 1) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float x = row_prefix16(dbs[s]);
        if (n16 == 15) sm.red[kRdb][wave][4 * g4 + s] = x;
      }
      __syncthreads();
      if (tid < BP && c * BP + tid < T) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) s += sm.red[kRdb][w][tid];
        p.dbg[gate_base + (size_t)(c * BP + tid) * gate_tok] = s;
      }
    }
  }
}

template <typename CT, int D, int P>
int launch_bwd(const G3BwdArgs& a, hipStream_t stream) {
  const int N = a.B * a.H * a.M;
  hipLaunchKernelGGL((gdn3_bwd_kernel<CT, D, P>), dim3(N), dim3(kNT), 0, stream, a);
  return check_launch("gdn3_bwd_kernel");
}

template <typename CT, int D>
int launch_bwd_p(const G3BwdArgs& a, hipStream_t stream) {
  if (a.P == 16) return launch_bwd<CT, D, 16>(a, stream);
  if (a.P == 32) return launch_bwd<CT, D, 32>(a, stream);
  if (a.P == 64) return launch_bwd<CT, D, 64>(a, stream);
  return set_error(GDNX_ERR_SHAPE, "gdn3 backward: window P=%d unsupported (16, 32 or 64)", a.P);
}

}  // namespace

int gdn3_bwd_dispatch(const G3BwdArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128) return launch_bwd_p<bf16, 128>(a, stream);
    if (a.D == 64) return launch_bwd_p<bf16, 64>(a, stream);
  } else {
    if (a.D == 128) return launch_bwd_p<float, 128>(a, stream);
    if (a.D == 64) return launch_bwd_p<float, 64>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "gdn3 backward: unsupported head_dim %d", a.D);
}

}  // namespace gdnx

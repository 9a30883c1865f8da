// GDN3 Kronecker-residual recurrence on gfx950: the fused per-chain forward
// (banded residual window + Kronecker read + periodic compaction), and the
// standalone compaction and Kronecker-read kernels.
//
// Reference semantics (frozen oracle gdn3/_reference_recurrence.py:33-94):
// per chain, state S = sum_r A_r (x) B_r + U Vb^T with a P-slot circular
// residual buffer.  Per token t: gamma = clamp(dec, 0, 1); A, B, Vb *= gamma;
// h = b.k; u = w.v; r = u - S h; alpha = alpha(k.h) (gdn3_upgrade.py:641-648);
// y = S q + alpha (k.q) r; slot t mod P <- (alpha r, k); after token t with
// (t+1) mod K_c == 0 the compaction (_compact_vec, gdn3_upgrade.py:650-719)
// refits A, B from R_mat = sum_r vec(A_r) vec(B_r)^T + rearrange(U Vb^T) by a
// randomized SVD and blends them (A <- s A + (1-s) A_svd, U, Vb unchanged).
//
// Chunked form (one chunk = the P-token window, aligned with the slots).
// With G_i the inclusive log-decay prefix inside the chunk, Gacc the log
// decay since the last compaction, U_old / Vbd the previous chunk's net
// writes and keys (keys decayed to the chunk start):
//   U_i = alpha_i (u_i - e^{2(Gacc+G_i)} Kr(h_i) - e^{G_i} sum_{p>=i} (h_i.Vbd_p) U_old_p)
//         - alpha_i sum_{j<i} e^{G_i-G_j} (h_i.k_j) U_j
//   y_i = e^{2(Gacc+G_i)} Kr(q_i) + e^{G_i} sum_{p>=i} (q_i.Vbd_p) U_old_p
//         + sum_{j<=i} e^{G_i-G_j} (q_i.k_j) U_j
// (slot p of the previous chunk is still visible to token i while p >= i;
// the Kronecker part decays by gamma^2 since A and B each decay by gamma).
// Kr(x) = (sum_r A_r (x) B_r) x is read on MFMA against the materialised
// d x d Kronecker matrix, rebuilt after every compaction.
//
// One workgroup per chain carries the whole state in LDS; the chunk loop
// is sequential because every compaction depends on the window it closes.
#include <mutex>

#include "gdn3_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

// Sum over the 64 lanes of a wave, the same bits in every lane: DPP row
// rotations by 8, 4, 2, 1 (a butterfly inside each 16-lane row, so all lanes
// of a row form the same sum), then across the four rows.
template <int CTL>
__device__ __forceinline__ double dpp_f64(double x) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(b & 0xffffffffll), CTL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTL, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}
// lane l's x, wave-uniform (l uniform)
__device__ __forceinline__ double readlane_f64(double x, int l) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}
// (the four row sums are read out of lanes 0, 16, 32, 48 and added as
// (r0 + r1) + (r2 + r3): a uniform value, no LDS round trip)
__device__ __forceinline__ double wave_sum_f64(double x) {
  x += dpp_f64<0x128>(x);
  x += dpp_f64<0x124>(x);
  x += dpp_f64<0x122>(x);
  x += dpp_f64<0x121>(x);
  return (readlane_f64(x, 0) + readlane_f64(x, 16)) + (readlane_f64(x, 32) + readlane_f64(x, 48));
}

// Sum of NV doubles over the 256 threads of the block, in a fixed order;
// every thread receives the totals.  red: 4 * NV doubles of LDS.
template <int NV>
__device__ __forceinline__ void block_sum(double (&v)[NV], double* red, int tid) {
#pragma unroll
  for (int e = 0; e < NV; ++e) v[e] = wave_sum_f64(v[e]);
  if ((tid & 63) == 0)
#pragma unroll
    for (int e = 0; e < NV; ++e) red[(tid >> 6) * NV + e] = v[e];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < NV; ++e) v[e] = (red[e] + red[NV + e]) + (red[2 * NV + e] + red[3 * NV + e]);
  __syncthreads();
}

// LDS of one compaction.  STG: the window's writes and keys are staged
// through ut / vt a block of 16 slots at a time (they come from global
// memory); without, they are read where they lie (LDS of the fused kernel).
// Row stride (doubles) of the compaction's row-major [rows][kQ] double arrays:
// where a thread reads or writes a whole row, 9 doubles put the 64 lanes' rows
// on distinct bank pairs (a stride of 8 put 16 lanes on each).
constexpr int kLQ = kQ + 1;

template <int D, int P, bool STG = true>
struct G3Compact {
  static constexpr int m = G3D<D>::m, n = G3D<D>::n;
  static constexpr int ldr = n + 4;                 // R_mat row stride: 16-byte rows, 4 banks apart
  static constexpr int lym = m + 16, lzn = n + 16;  // strides of the column-major fp32 copies
  alignas(16) float rm[m * ldr];          // R_mat
  alignas(16) double y[m * kLQ];          // range basis, rows of kQ (stride kLQ)
  alignas(16) double z[n * kLQ];          // R_mat^T Y, then Bm^T = R_mat^T Q (rows of kQ, stride kLQ)
  alignas(16) float yt[kQ * lym];         // y in fp32, column-major: the B operand of R_mat^T Y
  alignas(16) float zt[kQ * lzn];         // the sketch (zero padded), then z, in fp32 column-major
  alignas(16) float ut[STG ? 16 : 1][D + 4];   // a block of 16 window slots: net writes U_p
  alignas(16) float vt[STG ? 16 : 1][D + 4];   // and keys Vb_p
  double red[4 * 64];
  double rinv[kQ * kQ];                   // the summed Gram Y^T Y of a Cholesky-QR pass (row-major)
  double ev[kQ * kQ];                     // eigenvectors of Bm Bm^T (rows, in rank order)
  double lam[kQ];
  double sig[kRMax];
  double isig[kRMax];                     // 1 / sig (0 where sig is)
  double sgn[kRMax];
};

// Partial Gram X^T X (kQ x kQ) of NR rows of X (rows of kQ doubles, stride
// kLQ) on v_mfma_f64_4x4x4_4b_f64, four rows per step: block b = 2 P + Q is
// the 4 x 4 block (P, Q) of the Gram, so all 64 outputs are live (a 16 x 16
// tile left three quarters of its outputs dead at four times the cycles).
// Lane l = 16 k + 4 b + i supplies X[k][4 P + i] as A[b][i][k] and X[k][4 Q + i]
// as B[b][k][i]; it returns G[4 P + l / 16][4 Q + l % 4], the row-major entry
// gram_entry(l).  Two accumulation chains (even and odd steps) hide the
// MFMA's dependent latency.
__device__ __forceinline__ int gram_entry(int lane) {
  const int b = (lane >> 2) & 3;
  return (4 * (b >> 1) + (lane >> 4)) * kQ + 4 * (b & 1) + (lane & 3);
}
template <int NR>
__device__ __forceinline__ double gram_mfma(const double* x, int lane) {
  static_assert(NR % 8 == 0, "two chains of 4-row steps");
  const int k = lane >> 4, b = (lane >> 2) & 3, i = lane & 3;
  const int ca = 4 * (b >> 1) + i, cb = 4 * (b & 1) + i;
  double acc0 = 0.0, acc1 = 0.0;
#pragma unroll
  for (int r = 0; r < NR; r += 8) {
    acc0 = __builtin_amdgcn_mfma_f64_4x4x4f64(x[(r + k) * kLQ + ca], x[(r + k) * kLQ + cb], acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f64_4x4x4f64(x[(r + 4 + k) * kLQ + ca], x[(r + 4 + k) * kLQ + cb], acc1, 0, 0, 0);
  }
  return acc0 + acc1;
}

// C[M x kQ] = A[M x K] B[K x kQ] on fp32 MFMA: A is R_mat (fp32, row stride
// ldr, a multiple of 4) read as is (TRANS = false, M = m, K = n) or transposed
// (TRANS = true, M = n, K = m); B is fp32 and column-major (column j at bt +
// j ldb, zero where it has no column), so every product is exact and the sums
// are fp32.  v_mfma_f32_4x4x1_16b_f32 (16 blocks of 4 x 4 x 1, a quarter of the
// 16 x 16 x 4 instruction's cycles) takes the kQ = 8 columns as two blocks of
// 4, so no MFMA column is dead (16 x 16 tiles left half of theirs unused).
// Lane l = 4 b + q supplies row q of block b's A operand and column q of its B
// operand and holds D[b][r][q] in element r.  A wave owns RW = M / 4 rows of C; its 16 blocks are RG = RW / 4
// row groups times KP = 64 / RW partitions of k (k = 4 (KP t + p) + s for
// partition p, which puts the lanes of every LDS read on distinct banks),
// summed across the partitions (lane bits 4 and 5) at the end.  C goes to c
// (rows of kQ at stride kLQ, fp64) and, when ct is given, column-major in fp32
// to ct (stride ldc); GR: also this wave's partial Gram C^T C over its rows,
// in the layout of gram_mfma, formed from its rows of c.
template <bool TRANS, int M, int K, int ldr, int ldb, int ldc = 0, bool GR = false>
__device__ __forceinline__ void rm_mfma(const float* rm, const float* bt, double* c, float* ct, int tid,
                                         double* gp = nullptr) {
  constexpr int RW = M / 4, KP = 64 / RW, RG = RW / 4, NG = K / (4 * KP), BATCH = 4;
  static_assert(RW == 16 || RW == 64, "a wave's rows: one or four partitions of k");
  static_assert(NG % BATCH == 0 && ldr % 4 == 0 && ldb % 4 == 0 && ldc % 4 == 0, "whole batches, 16-byte rows");
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = lane >> 2, q = lane & 3, kp = b / RG, rg = b % RG;
  const int row = wave * RW + 4 * rg + q;   // the A row this lane supplies
  auto lda = [&](int t) {
    const int k0 = 4 * (KP * t + kp);
    f32x4 x;
    if constexpr (TRANS) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) x[s4] = rm[(k0 + s4) * ldr + row];
    } else {
      x = *(const f32x4*)&rm[row * ldr + k0];
    }
    return x;
  };
  f32x4 c1 = {0.f, 0.f, 0.f, 0.f}, c2 = {0.f, 0.f, 0.f, 0.f};   // columns q and 4 + q
#pragma unroll
  for (int t0 = 0; t0 < NG; t0 += BATCH) {
    f32x4 av[BATCH], b1[BATCH], b2[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int k0 = 4 * (KP * (t0 + u) + kp);
      av[u] = lda(t0 + u);
      b1[u] = *(const f32x4*)&bt[q * ldb + k0];
      b2[u] = *(const f32x4*)&bt[(4 + q) * ldb + k0];
    }
    __builtin_amdgcn_sched_barrier(0);   // (the scheduler would interleave them again)
#pragma unroll
    for (int u = 0; u < BATCH; ++u)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(av[u][s4], b1[u][s4], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_4x4x1f32(av[u][s4], b2[u][s4], c2, 0, 0, 0);
      }
  }
  if constexpr (KP > 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      c1[r] = sum_rows4(c1[r]);
      c2[r] = sum_rows4(c2[r]);
    }
  }
  // rows r0 + r of C; with KP = 4 the four partitions' lanes share the stores
  const int r0 = wave * RW + 4 * rg;
  if (KP == 1 || kp == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r) c[(r0 + r) * kLQ + q] = (double)c1[r];
  if (KP == 1 || kp == 1)
#pragma unroll
    for (int r = 0; r < 4; ++r) c[(r0 + r) * kLQ + 4 + q] = (double)c2[r];
  if constexpr (ldc > 0) {
    if (KP == 1 || kp == 2) *(f32x4*)&ct[q * ldc + r0] = c1;
    if (KP == 1 || kp == 3) *(f32x4*)&ct[(4 + q) * ldc + r0] = c2;
  }
  if constexpr (GR) {
    wave_lds_sync();   // the wave's rows of c, written by its lanes above
    *gp = gram_mfma<RW>(c + wave * RW * kLQ, lane);
  }
}

// 1 / sqrt(x) for x > 0 to fp64 rounding: the hardware estimate r0 and the
// Halley-order correction r0 (1 + t/2 + 3 t^2/8), t = 1 - x r0^2 (error
// O(t^3)).  x = 0 gives a NaN (callers select it away).
__device__ __forceinline__ double rsqrt_f64(double x) {
  const double r0 = __builtin_amdgcn_rsq(x);
  const double t = fma(-x * r0, r0, 1.0);
  return fma(r0 * t, fma(t, 0.375, 0.5), r0);
}

// Jacobi rotation zeroing a_pq (Numerical Recipes convention):
// J[p][p] = J[q][q] = c, J[p][q] = s, J[q][p] = -s, with the smaller angle
// t = sgn(th) / (|th| + sqrt(th^2 + 1)), th = (a_qq - a_pp) / (2 a_pq).
// Multiplying through by |2 a_pq| gives it without divisions: with
// d = a_qq - a_pp, e = 2 a_pq, h = sqrt(d^2 + e^2) and w = |d| + h,
// t = sgn(d) e / w, so c = w / sqrt(w^2 + e^2), s = sgn(d) e / sqrt(w^2 + e^2)
// (c^2 + s^2 = 1 by construction; d = +0 counts as positive, and at d = 0
// either sign of the 45-degree rotation zeroes a_pq).
__device__ __forceinline__ void jacobi_rot(double app, double aqq, double apq, double& c, double& s) {
  // the round is bound by its instruction count (one wave issues it), so no
  // selects: h only sets the angle (x times the hardware reciprocal square
  // root, about 2^-23 relative, 0 at x = 0; a rotation that leaves 1e-7 of
  // a_pq behind still converges within the same sweeps), w carries 2^-500,
  // which vanishes against any |d| or h above 2^-447 and makes d = e = 0 give
  // c = 1, s = 0, and sgn(d) e is a sign-bit copy.  c and s are normalised by
  // the refined reciprocal square root, so c^2 + s^2 = 1 to rounding.
  const double d = aqq - app, e = 2.0 * apq;
  const double e2 = e * e;
  const double x = fma(d, d, e2);
  const double h = x * __builtin_amdgcn_rsq(fmax(x, 2.2250738585072014e-308));
  const double w = (fabs(d) + 3.0549363634996047e-151) + h;
  const double r = rsqrt_f64(fma(w, w, e2));
  const long long sb = __double_as_longlong(d) & (long long)0x8000000000000000ull;
  c = w * r;
  s = __longlong_as_double(__double_as_longlong(e) ^ sb) * r;
}

// x as held by lane src of the wave (ds_bpermute, one per 32-bit half)
__device__ __forceinline__ double lane_f64(int src, double x) {
  const long long v = __double_as_longlong(x);
  const unsigned lo = (unsigned)__builtin_amdgcn_ds_bpermute(4 * src, (int)(unsigned)v);
  const unsigned hi = (unsigned)__builtin_amdgcn_ds_bpermute(4 * src, (int)(unsigned)(v >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Round-robin (circle method) partner of index x in round st of 7 for 8 indices.
__device__ __forceinline__ int rr_partner(int x, int st) {
  if (x == 7) return st;
  if (x == st) return 7;
  return (2 * st - x + 14) % 7;
}

// One Cholesky-QR pass leaves Q^T Q - I at about cond(Y)^2 * 1.1e-16 in fp64;
// the pivots' spread (largest / smallest, about cond(Y)^2) below this bound
// makes a second pass unnecessary (Q orthonormal to ~1e-10).
constexpr double kOrthCut = 1e6;
// Pivot spread (about cond(Y)^2) below which an intermediate basis enters the
// next product unnormalised: cond(Y) < 10 costs the fp32 products at most a
// decimal digit in its weakest direction, against their 1e-7
constexpr double kKeepCut = 1e2;

// Y <- Y R^{-1} with Y^T Y = R^T R (Cholesky QR, up to `passes` times: one
// pass keeps the intermediate power-iteration bases well conditioned; the
// final basis takes a second where the first pass's pivots spread by more
// than kOrthCut or a column was dropped); the result also goes column-major in fp32 to yt.  Columns whose pivot falls below 1e-24 of the largest
// diagonal are set to zero.  The Gram runs on fp64 MFMA over 4 row segments;
// each row of Y is then solved against R by forward substitution.
template <int D, int P, int M, bool STG>
__device__ __forceinline__ void orth_rows(G3Compact<D, P, STG>& cs, int tid, int passes, const double* pre = nullptr,
                                          double keep = 0.0) {
  static_assert(M % 16 == 0 && M <= kNT, "rows: 4 segments of whole MFMA steps, one row per thread");
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int seg = M / 4;
  for (int pass = 0; pass < passes; ++pass) {
    {   // this wave's partial Gram (the first pass's may come from the product that formed Y)
      const double g = (pass == 0 && pre) ? *pre : gram_mfma<seg>(cs.y + wave * seg * kLQ, lane);
      cs.red[wave * 64 + gram_entry(lane)] = g;
    }
    __syncthreads();
    if (wave == 0)   // the Gram, summed over the segments (rinv holds it row-major)
      cs.rinv[lane] = (cs.red[lane] + cs.red[64 + lane]) + (cs.red[128 + lane] + cs.red[192 + lane]);
    __syncthreads();
    // every thread factors the 8 x 8 Gram itself, in registers (right-looking
    // Cholesky, lower triangle; a dropped column gets rd = 0), and solves its
    // row of Y against R = L^T: no second exchange through LDS
    double L[kQ][kQ], rdv[kQ];
#pragma unroll
    for (int i = 0; i < kQ; ++i)
#pragma unroll
      for (int j = 0; j <= i; ++j) L[i][j] = cs.rinv[i * kQ + j];
    double dmax = 0.0;
#pragma unroll
    for (int k = 0; k < kQ; ++k) dmax = fmax(dmax, L[k][k]);
    const double tol = dmax * 1e-24;
    double pmin = dmax, pmax = 0.0;   // the spread of the pivots
#pragma unroll
    for (int k = 0; k < kQ; ++k) {
      const double akk = L[k][k];
      pmin = fmin(pmin, akk);
      pmax = fmax(pmax, akk);
      const double rq = rsqrt_f64(fmax(akk, 2.2250738585072014e-308));  // unconditional: a select, no branch
      const double rd = (akk > tol && akk > 0.0) ? rq : 0.0;
      rdv[k] = rd;   // 1 / R[k][k] (R[k][k] = akk rd = sqrt(akk))
#pragma unroll
      for (int i = k + 1; i < kQ; ++i) L[i][k] *= rd;
#pragma unroll
      for (int i = k + 1; i < kQ; ++i)
#pragma unroll
        for (int j = k + 1; j <= i; ++j) L[i][j] -= L[i][k] * L[j][k];
    }
    // keep > 0 (an intermediate basis, whose fp32 copy the product wrote):
    // where the pivots spread by less than keep, Y is conditioned well enough
    // to enter the next product as it is (the basis only has to stay well
    // conditioned; its span is what the power iteration carries)
    if (keep > 0.0 && __builtin_amdgcn_readfirstlane(pmin * keep > pmax ? 1 : 0)) return;
    if (tid < M) {
      double x[kQ];
#pragma unroll
      for (int j = 0; j < kQ; ++j) x[j] = cs.y[tid * kLQ + j];
      // x R = y, column by column: x_j = (y_j - sum_{i<j} x_i R[i][j]) / R[j][j], R[i][j] = L[j][i]
#pragma unroll
      for (int j = 0; j < kQ; ++j) {
        double sacc = x[j];
#pragma unroll
        for (int i = 0; i < j; ++i) sacc -= x[i] * L[j][i];
        x[j] = sacc * rdv[j];
      }
#pragma unroll
      for (int j = 0; j < kQ; ++j) {
        cs.y[tid * kLQ + j] = x[j];
        cs.yt[j * cs.lym + tid] = (float)x[j];
      }
    }
    __syncthreads();
    // a later pass only where this one can have lost orthogonality: every
    // thread factored the same Gram, so the test is uniform
    if (pass + 1 < passes && __builtin_amdgcn_readfirstlane(pmin * kOrthCut > pmax ? 1 : 0)) break;
  }
}

// Sums of squares of the first kRMax columns of a row-major [M][kQ] double
// array, into out[0..kRMax) (every thread waits for them).
template <int M>
__device__ __forceinline__ void col_sumsq(const double* y, double* red, double* out, int tid) {
  const int r = tid & (kRMax - 1), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  double part = 0.0;
  for (int row = tid / kRMax; row < M; row += kNT / kRMax) {
    const double x = y[row * kLQ + r];
    part += x * x;
  }
#pragma unroll
  for (int off = kRMax; off < 64; off <<= 1) part += __shfl_xor(part, off, 64);
  if (lane < kRMax) red[wave * kRMax + lane] = part;
  __syncthreads();
  if (tid < kRMax) out[tid] = (red[tid] + red[kRMax + tid]) + (red[2 * kRMax + tid] + red[3 * kRMax + tid]);
  __syncthreads();
}

struct G3NoOp {
  __device__ void operator()() const {}
};

// Compaction of one chain (gdn3/gdn3_upgrade.py:650-719): ab = [A (R x m) |
// B (R x n)] in LDS as stored (the Kronecker part is decayed by e^{gacc} per
// factor); the window's P net writes U and keys Vb (decayed to now) are read
// from global memory, slot p column d at p u_sp + d u_sd.  Writes the blended A, B back into ab and, from
// thread 0, stats = (|R_mat|^2, sum of the R kept sigma^2).  Sign
// convention: each (u_r, v_r) pair is flipped so that the largest-magnitude
// entry of v_r is positive (first index on ties).
// mode 1 is the reference's 'sketch' / 'sketch_noqr' (both run the same
// branch, gdn3/gdn3_upgrade.py:579-592): no range finder and no SVD, with a
// sketch of qs = R columns, Q = the column-normalised R_mat G,
// Bm = Q^T R_mat, A_svd_r = |Bm_r| Q_r, B_svd_r = Bm_r / |Bm_r| (norms
// clamped at 1e-12); it reports no error (stats = (|R_mat|^2, |R_mat|^2)).
// issue / commit: work of the caller's that uses no compaction state and
// runs in the eigen-solve's shadow (every thread calls issue before it; waves
// 1-3 call commit while wave 0 solves, wave 0 after); 'svd' mode only.
// pre: the sketch entries this thread stages, loaded by the caller (a chain's
// sketch is the same at every compaction), else they are loaded here.
template <int D>
struct G3Sketch {
  static constexpr int N = (G3D<D>::n * kQ + kNT - 1) / kNT;
  float v[N];   // entry e = tid + u kNT: sketch row e / kQ, column e % kQ (zero past its qs columns)
};
template <int D>
__device__ __forceinline__ void g3_sketch_load(G3Sketch<D>& g, const float* __restrict__ sketch, int qs, int tid) {
#pragma unroll
  for (int u = 0; u < G3Sketch<D>::N; ++u) {
    const int e = tid + u * kNT, c = e / kQ, j = e % kQ;
    g.v[u] = (e < G3D<D>::n * kQ && j < qs) ? sketch[c * qs + j] : 0.f;
  }
}
template <int D, int P, bool STG, typename Issue = G3NoOp, typename Commit = G3NoOp>
__device__ __forceinline__ void g3_compact(G3Compact<D, P, STG>& cs, float* ab, const float* __restrict__ U,
                                           const float* __restrict__ Vb, size_t u_sp, size_t u_sd, float gacc,
                                           float sdec, const float* __restrict__ sketch, double* stats, int tid,
                                           int mode = 0, Issue issue = Issue(), Commit commit = Commit(),
                                           const G3Sketch<D>* pre = nullptr) {
  typedef G3D<D> Ge;
  constexpr int R = Ge::R, m = Ge::m, n = Ge::n, q = Ge::q, ak = Ge::ak, bk = Ge::bk;
  constexpr int lbv = Ge::lbv, lbk = Ge::lbk, ln = Ge::ln;
  constexpr int ldr = G3Compact<D, P, STG>::ldr, lym = G3Compact<D, P, STG>::lym, lzn = G3Compact<D, P, STG>::lzn;
  float* A = ab;
  float* Bv = ab + R * m;
  tid = opaque(tid);
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // the sketch's global loads (unless the caller holds it) are issued first
  // and land in LDS after the residual part (which does not read them)
  constexpr int NGS = G3Sketch<D>::N;
  G3Sketch<D> gs;
  if (pre) gs = *pre;
  else g3_sketch_load<D>(gs, sketch, mode ? R : q, tid);
  double en[1] = {0.0};
  // residual part rearrange(U Vb^T) on fp32 MFMA: out[v][k] = sum_p U_p[v] Vb_p[k]
  // (A[v][p] = U_p[v], B[p][k] = Vb_p[k]), accumulated over the window's
  // blocks of 16 slots staged through LDS; wave w owns the value-row tiles
  // w VTW .. w VTW + VTW - 1 against every key-column tile, and scatters each
  // entry to its rearranged place (iv a_k + ik, jv b_k + jk)
  {
    constexpr int NT16 = D / 16, VTW = NT16 / 4;
    static_assert(NT16 % 4 == 0 && P % 16 == 0, "whole 16x16 tiles on 4 waves, blocks of 16 window slots");
    const int g4 = lane >> 4, n16 = lane & 15;
    f32x4 racc[VTW][NT16];
#pragma unroll
    for (int vi = 0; vi < VTW; ++vi)
#pragma unroll
      for (int kt = 0; kt < NT16; ++kt) racc[vi][kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int pb = 0; pb < P / 16; ++pb) {
      if constexpr (STG) {
        if (pb > 0) __syncthreads();   // the previous block is consumed
        for (int e = tid; e < 16 * D; e += kNT) {
          const int i = e / D, d = e % D;
          const size_t o = (size_t)(16 * pb + i) * u_sp + (size_t)d * u_sd;
          cs.ut[i][d] = U[o];
          cs.vt[i][d] = Vb[o];
        }
        __syncthreads();
      }
      // slot 16 pb + i, column d
      auto uval = [&](int i, int d) {
        if constexpr (STG) return cs.ut[i][d];
        else return U[(size_t)(16 * pb + i) * u_sp + (size_t)d * u_sd];
      };
      auto vval = [&](int i, int d) {
        if constexpr (STG) return cs.vt[i][d];
        else return Vb[(size_t)(16 * pb + i) * u_sp + (size_t)d * u_sd];
      };
      // every operand read before the MFMAs, behind a scheduling barrier (the
      // compiler, short of registers, waited for each tile's reads); the
      // key fragments serve every value tile
      f32x4 ua[VTW], kb4[NT16];
#pragma unroll
      for (int vi = 0; vi < VTW; ++vi)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) ua[vi][s4] = uval(4 * g4 + s4, (wave * VTW + vi) * 16 + n16);
#pragma unroll
      for (int kt = 0; kt < NT16; ++kt)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) kb4[kt][s4] = vval(4 * g4 + s4, kt * 16 + n16);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int vi = 0; vi < VTW; ++vi)
#pragma unroll
        for (int kt = 0; kt < NT16; ++kt) mma(racc[vi][kt], ua[vi], kb4[kt]);
    }
    // plus the Kronecker part sum_r A_r[iv][ik] B_r[jv][jk] (each factor decayed
    // by e^{gacc}), and the energy |R_mat|^2.  With b_v = b_k = 8 a lane's
    // jk = n16 mod 8 and jv = (4 g4 + i) mod 8 are fixed (its B entries load
    // once), iv = 2 vt + g4 / 2 follows the value tile and ik = 2 kt + n16 / 8
    // the key tile (R A entries per tile pair, 4 addresses per wave)
    static_assert(Ge::bv == 8 && Ge::bk == 8, "lane-fixed Kronecker columns");
    const float sc2 = expf(2.f * gacc);
    float bl[4][kRMax];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < kRMax; ++r)
        bl[i][r] = r < R ? sc2 * Bv[r * n + ((4 * g4 + i) & 7) * bk + (n16 & 7)] : 0.f;
    double e4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int vi = 0; vi < VTW; ++vi) {
      const int vt = wave * VTW + vi, iv = 2 * vt + (g4 >> 1);
      float alv[NT16][kRMax];   // (read before use, as above)
#pragma unroll
      for (int kt = 0; kt < NT16; ++kt)
#pragma unroll
        for (int r = 0; r < kRMax; ++r) alv[kt][r] = r < R ? A[r * m + iv * ak + 2 * kt + (n16 >> 3)] : 0.f;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kt = 0; kt < NT16; ++kt) {
        const int ik = 2 * kt + (n16 >> 3), jk = n16 & 7, row = iv * ak + ik;
        const float* al = alv[kt];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int jv = (4 * g4 + i) & 7;
          float sv = racc[vi][kt][i];
#pragma unroll
          for (int r = 0; r < kRMax; ++r)
            if (r < R) sv += al[r] * bl[i][r];
          cs.rm[row * ldr + jv * bk + jk] = sv;
          e4[i] += (double)sv * (double)sv;
        }
      }
    }
    en[0] = (e4[0] + e4[1]) + (e4[2] + e4[3]);
  }
#pragma unroll
  for (int u = 0; u < NGS; ++u) {
    const int e = tid + u * kNT;
    if (e < n * kQ) cs.zt[(e % kQ) * lzn + e / kQ] = gs.v[u];
  }
  block_sum<1>(en, cs.red, tid);

  if (mode) {   // 'sketch': one product, column and row normalisation
    rm_mfma<false, m, n, ldr, lzn>(cs.rm, cs.zt, cs.y, nullptr, tid);   // Y = R_mat G (columns >= R are zero)
    __syncthreads();
    col_sumsq<m>(cs.y, cs.red, cs.lam, tid);
    for (int e = tid; e < m * kQ; e += kNT) {
      const int j = e % kQ;
      const double qv = j < R ? cs.y[(e / kQ) * kLQ + j] / fmax(sqrt(cs.lam[j]), 1e-12) : 0.0;   // Q
      cs.y[(e / kQ) * kLQ + j] = qv;
      cs.yt[j * lym + e / kQ] = (float)qv;
    }
    __syncthreads();
    rm_mfma<true, n, m, ldr, lym>(cs.rm, cs.yt, cs.z, nullptr, tid);      // Bm^T = R_mat^T Q
    __syncthreads();
    col_sumsq<n>(cs.z, cs.red, cs.sig, tid);
    const float dk = expf(gacc);
    const float s1 = sdec, s2 = 1.f - sdec;
    for (int e = tid; e < R * m; e += kNT) {
      const int r = e / m, row = e % m;
      const double sv = cs.y[row * kLQ + r] * fmax(sqrt(cs.sig[r]), 1e-12);
      A[e] = s1 * (A[e] * dk) + s2 * (float)sv;
    }
    for (int e = tid; e < R * n; e += kNT) {
      const int r = e / n, col = e % n;
      const double sv = cs.z[col * kLQ + r] / fmax(sqrt(cs.sig[r]), 1e-12);
      Bv[e] = s1 * (Bv[e] * dk) + s2 * (float)sv;
    }
    if (tid == 0 && stats) {
      stats[0] = en[0];
      stats[1] = en[0];
    }
    __syncthreads();
    return;
  }

  // range finder with two power iterations; orthonormalising between the
  // products leaves the final basis unchanged (up to column signs)
  // (each Y = R_mat Z product hands its partial Grams straight to the first
  // Cholesky-QR pass, whose barrier then also publishes Y)
  double gp;
  rm_mfma<false, m, n, ldr, lzn, lym, true>(cs.rm, cs.zt, cs.y, cs.yt, tid, &gp);
  orth_rows<D, P, m, STG>(cs, tid, 1, &gp, kKeepCut);
  for (int it = 0; it < 2; ++it) {
    rm_mfma<true, n, m, ldr, lym, lzn>(cs.rm, cs.yt, cs.z, cs.zt, tid);
    __syncthreads();
    rm_mfma<false, m, n, ldr, lzn, lym, true>(cs.rm, cs.zt, cs.y, cs.yt, tid, &gp);
    orth_rows<D, P, m, STG>(cs, tid, it == 1 ? 2 : 1, &gp, it == 1 ? 0.0 : kKeepCut);
  }
  // Bm^T = R_mat^T Q  [n][kQ]
  rm_mfma<true, n, m, ldr, lym>(cs.rm, cs.yt, cs.z, nullptr, tid);
  __syncthreads();
  {  // W = Bm Bm^T: each wave's partial Gram over a quarter of the rows of Bm^T
    static_assert(n % 32 == 0, "quarters of whole MFMA steps");
    cs.red[wave * 64 + gram_entry(lane)] = gram_mfma<n / 4>(cs.z + wave * (n / 4) * kLQ, lane);
  }
  __syncthreads();
  issue();
  // eigen-decomposition of W = Bm Bm^T by cyclic Jacobi in wave 0: lane
  // (i, j) holds W[i][j] and V[i][j].  Each round rotates 4 disjoint pairs;
  // a lane gathers every operand of its round in one exchange and forms the
  // rotation of its column's pair (that of j); the rotation of i it takes
  // from lane (i, i), whose column pair that is.  The exchange goes through
  // LDS (xa, xv), ordered by wave_lds_sync (the next round's writes depend
  // on this round's reads, so they cannot move above them).
  if (wave == 0) {
    const int i = lane >> 3, j = lane & 7;
    double* xa = cs.rinv;   // 64 doubles each, free after the last Cholesky-QR pass
    double* xv = cs.ev;
    double a;
    {  // the partials summed, upper entry for both (i, j) and (j, i)
      const int e = min(i, j) * kQ + max(i, j);
      a = (cs.red[e] + cs.red[64 + e]) + (cs.red[128 + e] + cs.red[192 + e]);
    }
    double vv = (i == j) ? 1.0 : 0.0;
    // |W|_F^2, which the rotations keep: the diagonal's mass is fro - off
    const double fro = wave_sum_f64(a * a);
    for (int sweep = 0; sweep < 12; ++sweep) {
      if (sweep >= 4) {   // (fewer than four sweeps rarely suffice; extra sweeps over a diagonal W rotate by identities)
        const double off = wave_sum_f64(i != j ? a * a : 0.0);
        // stop at off-diagonal entries ~1e-8 of the diagonal's (in norm): the
        // eigenvectors then sit within ~1e-8 / (relative gap) of W's, an order
        // below what the fp32 products that formed Bm already left in W
        if (!(off > 1e-16 * (fro - off))) break;  // uniform across the wave
      }
#pragma unroll
      for (int st = 0; st < 7; ++st) {
        const int pi = rr_partner(i, st), pj = rr_partner(j, st);
        const int j0 = min(j, pj), j1 = max(j, pj);
        xa[lane] = a;
        xv[lane] = vv;
        wave_lds_sync();
        const double aj0 = xa[9 * j0], aj1 = xa[9 * j1], ajo = xa[8 * j0 + j1];
        const double a_ipj = xa[8 * i + pj], a_pij = xa[8 * pi + j];
        const double a_pipj = xa[8 * pi + pj], v_ipj = xv[8 * i + pj];
        double cj, sj;
        jacobi_rot(aj0, aj1, ajo, cj, sj);
        // J[x][x] = c; J[partner][x] = -s if x < partner else +s
        const double xj = (j < pj) ? -sj : sj;
        // the rotation of i: lane (i, i) formed it as the rotation of its column
        const double ci = lane_f64(9 * i, cj), xi = lane_f64(9 * i, xj);
        a = cj * fma(ci, a, xi * a_pij) + xj * fma(ci, a_ipj, xi * a_pipj);
        vv = vv * cj + v_ipj * xj;
      }
    }
    // (still wave 0 alone, ordered by wave_lds_sync) the rank of eigenvalue j,
    // descending, ties by index; the eigenvectors in rank order,
    // ev[r][i] = component i of the r-th; the kept singular values
    if (i == j) cs.lam[i] = a;
    wave_lds_sync();
    const double lj = cs.lam[j];
    int rk = 0;
#pragma unroll
    for (int k = 0; k < kQ; ++k) rk += (cs.lam[k] > lj || (cs.lam[k] == lj && k < j)) ? 1 : 0;
    cs.ev[rk * kQ + i] = vv;
    if (i == 0 && rk < R) {   // sigma = l / sqrt(l) and 1 / sigma from one refined reciprocal square root
      const double rs = rsqrt_f64(fmax(lj, 2.2250738585072014e-308));
      cs.sig[rk] = lj > 0.0 ? lj * rs : 0.0;
      cs.isig[rk] = lj > 0.0 ? rs : 0.0;
    }
    commit();
  } else {
    commit();
  }
  __syncthreads();
  // leading singular vectors: u_r = Q ev_r (a row per thread, kept in
  // registers for the blend), v_r = Bm^T ev_r / sigma_r
  static_assert(m <= kNT && n <= 64, "left vectors: a row per thread; right vectors: a column per lane of a wave");
  const float dk = expf(gacc);
  const float s1 = sdec, s2 = 1.f - sdec;
  double ur[kRMax];
  if (tid < m) {
    double yv[kQ];
#pragma unroll
    for (int j = 0; j < kQ; ++j) yv[j] = cs.y[tid * kLQ + j];
#pragma unroll
    for (int r = 0; r < kRMax; ++r) {
      double s = 0.0;
#pragma unroll
      for (int j = 0; j < kQ; ++j) s += yv[j] * cs.ev[r * kQ + j];
      ur[r] = s;
    }
  }
  // wave r: v_r (one column per lane) and the pair's canonical sign,
  // argmax_c |v_r[c]| with the first index on ties (an all-reduce by row
  // rotations inside each 16-lane row, then across the rows), then the
  // blend of B's row r, which needs nothing from the other waves
  static_assert(R <= 4, "one factor per wave");
  if (wave < R) {
    const int r = wave, c = lane;
    const bool on = c < n;
    double vr = 0.0;
    if (on) {
      double sv = 0.0;
#pragma unroll
      for (int j = 0; j < kQ; ++j) sv += cs.z[c * kLQ + j] * cs.ev[r * kQ + j];
      vr = cs.sig[r] > 0.0 ? sv * cs.isig[r] : (c == r ? 1.0 : 0.0);
    }
    double bv_ = on ? fabs(vr) : -1.0;
    int bi = on ? c : 0x7fffffff;
    auto take = [&](double ov, int oi) {
      const bool t = (ov > bv_) | ((ov == bv_) & (oi < bi));  // selects, no branches
      bv_ = t ? ov : bv_;
      bi = t ? oi : bi;
    };
    take(dpp_f64<0x128>(bv_), __builtin_amdgcn_update_dpp(0, bi, 0x128, 0xf, 0xf, false));
    take(dpp_f64<0x124>(bv_), __builtin_amdgcn_update_dpp(0, bi, 0x124, 0xf, 0xf, false));
    take(dpp_f64<0x122>(bv_), __builtin_amdgcn_update_dpp(0, bi, 0x122, 0xf, 0xf, false));
    take(dpp_f64<0x121>(bv_), __builtin_amdgcn_update_dpp(0, bi, 0x121, 0xf, 0xf, false));
    // the four rows' results out of lanes 0, 16, 32, 48 (the order does not
    // matter: max value, then least index, is a total order): wave-uniform
    double mv = readlane_f64(bv_, 0);
    int mi = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int rr = 1; rr < 4; ++rr) {
      const double ov = readlane_f64(bv_, 16 * rr);
      const int oi = __builtin_amdgcn_readlane(bi, 16 * rr);
      const bool t = (ov > mv) | ((ov == mv) & (oi < mi));
      mv = t ? ov : mv;
      mi = t ? oi : mi;
    }
    const double vb = readlane_f64(vr, mi & 63);
    const double sg = (mi != 0x7fffffff && vb < 0.0) ? -1.0 : 1.0;
    if (lane == 0) cs.sgn[r] = sg;
    if (on) Bv[r * n + c] = s1 * (Bv[r * n + c] * dk) + s2 * (float)(sg * vr);
  }
  __syncthreads();
  // two-timescale blend of the decayed factors with the SVD factors (B above)
  if (tid < m)
#pragma unroll
    for (int r = 0; r < kRMax; ++r)
      if (r < R) {
        const double sv = cs.sgn[r] * cs.sig[r] * ur[r];
        A[r * m + tid] = s1 * (A[r * m + tid] * dk) + s2 * (float)sv;
      }
  if (tid == 0 && stats) {
    double kept = 0.0;
    for (int r = 0; r < R; ++r) kept += cs.sig[r] * cs.sig[r];
    stats[0] = en[0];
    stats[1] = kept;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// fused forward
// ---------------------------------------------------------------------------
// The window runs in sub-chunks of kSC = 16 tokens aligned with the slots:
// the P slots are NB = P / 16 blocks, block b holding slots 16 b .. 16 b + 15.
// Sub-chunk c (global tokens 16 c .. 16 c + 15) writes block c mod NB.  Token
// i of it sees the other NB - 1 blocks whole (the writes of sub-chunks c - 1
// .. c - NB + 1) and, of block c mod NB, the slots p >= i the writes of
// sub-chunk c - NB still hold; at P = 16 that is the banded previous chunk.
constexpr int kSC = 16;

template <typename CT, int D, int P, int NVB>
struct G3WinSmem {
  static constexpr int NB = P / kSC;
  static constexpr bool KF = sizeof(CT) == 4;  // fp32 IO: the grams read the fp32 window keys
  alignas(16) CT x[3 * kSC][D + 8];      // rows: H (0..15), Q (16..31), K (32..47)
  alignas(16) float u[kSC][D + 4];       // w (.) v
  alignas(16) float kr[2 * kSC][D + 4];  // Kronecker reads of H and Q
  alignas(16) float pp[4][kSC][kSC + 4]; // H K^T (then inverse scratch), Aq, T, inverse scratch
  alignas(16) float po[2][kSC][P + 4];   // Ho, Qo over the P slots
  alignas(16) CT skron[D / NVB][D + 8];  // sum_r A_r (x) B_r, this workgroup's rows v
  alignas(16) float vbd[P][D + 4];       // window keys: block b decayed to e^{-boff_b} of now
  alignas(16) CT vbx[KF ? 1 : P][D + 8]; // the same in the compute dtype (bf16 IO)
  float G[kSC], alpha[kSC], lg[kSC], kco[kSC], qco[kSC], gam[kSC], vsc[kSC];
  float boff[NB];                        // log decay of block b's keys since they were last rebased
};
template <typename CT, int D, int P, int NVB>
constexpr bool win_fits() { return sizeof(G3WinSmem<CT, D, P, NVB>) <= 160 * 1024; }

template <typename CT> struct W16Of { static constexpr int value = 8 * sizeof(CT) / 16; };

__device__ __forceinline__ void unpack8(const uint4* w, float* f, const bf16*) {
  const unsigned ws[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(ws[e] << 16);
    f[2 * e + 1] = __uint_as_float(ws[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack8(const uint4* w, float* f, const float*) {
  const unsigned ws[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = __uint_as_float(ws[e]);
}
__device__ __forceinline__ void store8(bf16* dst, const float* f) {
  *(bf16x8*)dst = (bf16x8){(bf16)f[0], (bf16)f[1], (bf16)f[2], (bf16)f[3],
                           (bf16)f[4], (bf16)f[5], (bf16)f[6], (bf16)f[7]};
}
__device__ __forceinline__ void store8(float* dst, const float* f) {
  *(f32x4*)dst = (f32x4){f[0], f[1], f[2], f[3]};
  *(f32x4*)(dst + 4) = (f32x4){f[4], f[5], f[6], f[7]};
}

// A thread's share of a sub-chunk's token rows as loaded: 8 consecutive
// channels of one token (raw q, k, v; gates and decay as float).  The loads
// always go to an in-bounds token and the validity is applied when the rows
// are committed: loaded registers that branches merge would make the
// prefetch wait for its own loads.
template <typename CT> struct G3Raw {
  uint4 k[W16Of<CT>::value], q[W16Of<CT>::value], v[W16Of<CT>::value];
  f32x4 b0, b1, w0, w1;   // per-channel gates
  float bs, ws, dec;      // scalar gates, decay
  bool ok;                // a token of this call (else zeros and decay 1)
};

// Per-chain offsets of the token-major inputs and outputs
struct G3Tok {
  size_t qkv_tok, qkv_base, gate_tok, gate_base, dec_tok, dec_base, y_tok, y_base;
  int gc;
  __device__ __forceinline__ G3Tok(const G3FwdArgs& p, int chain, int D) {
    const int H = p.H, M = p.M, T = p.T, L = p.qkv_lanes;
    const int b = chain / (H * M), hm = chain % (H * M), h = hm / M, m = hm % M;
    gc = p.gate_ch;
    qkv_tok = (size_t)H * L * D;
    qkv_base = ((size_t)b * T * H + h) * L * D + (L > 1 ? (size_t)m * D : 0);
    gate_tok = (size_t)H * M * gc;
    gate_base = (((size_t)b * T * H + h) * M + m) * gc;
    dec_tok = (size_t)H * M;
    dec_base = ((size_t)b * T * H + h) * M + m;
    y_tok = (size_t)H * M * D;
    y_base = (((size_t)b * T * H + h) * M + m) * D;
  }
};

// local token t (marked invalid outside [0, T) or for a thread without a
// unit; the loads then read token min(max(t, 0), T - 1)).  GL: the gate
// layout, 1 a scalar per lane, 2 per channel, 0 read from o.gc (a runtime
// branch, whose merge costs the prefetch a wait)
template <typename CT, int GL = 0>
__device__ __forceinline__ void g3_fetch(const G3FwdArgs& p, const G3Tok& o, G3Raw<CT>& r, int t, bool on,
                                         int ud) {
  constexpr int W16 = W16Of<CT>::value;
  r.ok = on && t >= 0 && t < p.T;
  const size_t tc = (size_t)min(max(t, 0), p.T - 1);
  const uint4* kp = (const uint4*)((const CT*)p.k + o.qkv_base + tc * o.qkv_tok + ud);
  const uint4* qp = (const uint4*)((const CT*)p.q + o.qkv_base + tc * o.qkv_tok + ud);
  const uint4* vp = (const uint4*)((const CT*)p.v + o.qkv_base + tc * o.qkv_tok + ud);
#pragma unroll
  for (int w = 0; w < W16; ++w) {
    r.k[w] = kp[w];
    r.q[w] = qp[w];
    r.v[w] = vp[w];
  }
  // both branches define every gate field, so no loaded register is merged
  if (GL == 2 || (GL == 0 && o.gc > 1)) {
    const float* bp = p.bg + o.gate_base + tc * o.gate_tok + ud;
    const float* wp = p.wg + o.gate_base + tc * o.gate_tok + ud;
    r.b0 = *(const f32x4*)bp;
    r.b1 = *(const f32x4*)(bp + 4);
    r.w0 = *(const f32x4*)wp;
    r.w1 = *(const f32x4*)(wp + 4);
    if constexpr (GL == 0) r.bs = r.ws = 0.f;
  } else {
    r.bs = p.bg[o.gate_base + tc * o.gate_tok];
    r.ws = p.wg[o.gate_base + tc * o.gate_tok];
    if constexpr (GL == 0) r.b0 = r.b1 = r.w0 = r.w1 = zero4();
  }
  r.dec = p.dec[o.dec_base + tc * o.dec_tok];
}

// the raw q / k vector w of a thread's row, zero for an invalid token
template <typename CT>
__device__ __forceinline__ uint4 g3_raw(const G3Raw<CT>& r, const uint4& x) {
  return r.ok ? x : make_uint4(0u, 0u, 0u, 0u);
}

// h = b o k and u = w o v of the thread's 8 channels (gc: gate channels);
// returns the row sum of k . h over the token's DG threads (consecutive lanes)
template <typename CT, int DG, int GL = 0>
__device__ __forceinline__ float g3_unpack(const G3Raw<CT>& r, int gc, float* hf, float* uu) {
  float kf[8], vf[8], bb[8], ww[8];
  unpack8(r.k, kf, (const CT*)nullptr);
  unpack8(r.v, vf, (const CT*)nullptr);
  if (GL == 2 || (GL == 0 && gc > 1)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bb[e] = r.b0[e];
      bb[4 + e] = r.b1[e];
      ww[e] = r.w0[e];
      ww[4 + e] = r.w1[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bb[e] = r.bs;
      ww[e] = r.ws;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {   // an invalid token commits zeros
    kf[e] = r.ok ? kf[e] : 0.f;
    vf[e] = r.ok ? vf[e] : 0.f;
  }
  float part = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    hf[e] = bb[e] * kf[e];
    uu[e] = ww[e] * vf[e];
    part += kf[e] * hf[e];
  }
  if constexpr (DG == 16) {
    // the 16 lanes of a token row are one DPP row: rotations by 8, 4, 2, 1
    part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0x128, 0xf, 0xf, false));
    part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0x124, 0xf, 0xf, false));
    part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0x122, 0xf, 0xf, false));
    part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0x121, 0xf, 0xf, false));
  } else {
#pragma unroll
    for (int off = 1; off < DG; off <<= 1) part += __shfl_xor(part, off, 64);
  }
  return part;
}

// The window LDS a sub-chunk step works on (pointers into one workgroup's
// shared memory)
template <typename CT, int D, int P>
struct G3WinView {
  CT (*x)[D + 8];               // rows: H (0..15), Q (16..31), K (32..47)
  float (*u)[D + 4];            // w (.) v
  float (*kr)[D + 4];           // Kronecker reads of H and Q
  float (*pp)[kSC][kSC + 4];    // [4]: H K^T (then inverse scratch), Aq, T, inverse scratch
  float (*po)[kSC][P + 4];      // [2]: Ho, Qo over the P slots
  CT (*skron)[D + 8];           // this workgroup's rows of sum_r A_r (x) B_r
  float (*vbd)[D + 4];          // window keys: block b decayed to e^{-boff_b} of now
  CT (*vbx)[D + 8];             // the same in the compute dtype (bf16 IO)
  float *G, *alpha, *lg, *kco, *qco, *gam, *vsc;
  float* boff;                  // log decay of block b's keys since they were rebased
};

// The log-decay prefix sums of a sub-chunk (lane i < 16 holds G_i).
template <typename CT, int D, int P>
__device__ __forceinline__ float g3_scan_g(const G3WinView<CT, D, P>& w, int lane) {
  float gl = lane < kSC ? w.lg[lane] : 0.f;
#pragma unroll
  for (int off = 1; off < kSC; off <<= 1) {
    const float o = __shfl_up(gl, off, 64);
    if (lane >= off) gl += o;
  }
  return gl;
}

// The per-token coefficients of a sub-chunk (one wave): G, e^G, kco = alpha
// e^{2 (gacc + G)}, qco = e^{2 (gacc + G)} and the key scale e^{G_last - G}.
template <typename CT, int D, int P>
__device__ __forceinline__ void g3_scalars(const G3WinView<CT, D, P>& w, float gl, float gacc, int lane) {
  const float gl_last = __shfl(gl, kSC - 1, 64);
  if (lane < kSC) {
    const float e2 = expf(2.f * (gacc + gl));
    w.G[lane] = gl;
    w.gam[lane] = expf(gl);
    w.kco[lane] = w.alpha[lane] * e2;
    w.qco[lane] = e2;
    w.vsc[lane] = expf(gl_last - gl);
  }
}

// Gram tile ti of a sub-chunk (one wave; 2 + 2 NB tiles):
//   0: H K^T (raw; the inverse turns it into T),  1: Aq = [j <= i] e^{G_i - G_j} q_i.k_j,
//   2 + 2 b: Ho_b = vis alpha_i e^{G_i + boff_b} h_i.Vb_b[j],  3 + 2 b: Qo_b = vis e^{G_i + boff_b} q_i.Vb_b[j]
// with vis = [b != beta or j >= i or j < lo]
template <typename CT, int D, int P>
__device__ __forceinline__ void g3_gram_tile(const G3WinView<CT, D, P>& w, int ti, float gl, int beta, int lo,
                                             int lane) {
  constexpr bool KF = sizeof(CT) == 4;
  const int g4 = lane >> 4, n16 = lane & 15;
  const float gj = __shfl(gl, n16, 64);
  float gi[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) gi[s] = __shfl(gl, 4 * g4 + s, 64);
  const bool isq = ti & 1;
  const CT* arow = &w.x[(isq ? kSC : 0) + n16][0];
  const int bl = (ti - 2) >> 1;
  const CT* brow;
  if (ti < 2) brow = &w.x[2 * kSC + n16][0];
  else if constexpr (KF) brow = (const CT*)&w.vbd[kSC * bl + n16][0];
  else brow = &w.vbx[kSC * bl + n16][0];
  const f32x4 acc = tile_nt<CT, D>(arow, brow, g4);
  const int j = n16;
  if (ti == 0) {
#pragma unroll
    for (int s = 0; s < 4; ++s) w.pp[0][4 * g4 + s][j] = acc[s];
  } else if (ti == 1) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g4 + s;
      w.pp[1][i][j] = (j <= i) ? expf(gi[s] - gj) * acc[s] : 0.f;
    }
  } else {
    const float bo = w.boff[bl];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g4 + s;
      const bool vis = bl != beta || j >= i || j < lo;
      const float sc = expf(gi[s] + bo) * (isq ? 1.f : w.alpha[i]);
      w.po[isq ? 1 : 0][i][kSC * bl + j] = vis ? sc * acc[s] : 0.f;
    }
  }
}

// T = (I + Lm)^-1 into pp[2] (one wave, the one that formed tile 0 and the
// coefficients: it reads what its own lanes wrote, ordered by the fences).
// Lm[i][j] = alpha_i e^{G_i - G_j} (h_i . k_j), j < i, is strictly lower
// (nilpotent): (I + Lm)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8), factors that
// commute; squarings and products on fp32 MFMA.  An accumulator tile is a
// k-fragment (B operand); the A operand of each square goes through LDS.
template <typename CT, int D, int P>
__device__ __forceinline__ void g3_inverse(const G3WinView<CT, D, P>& w, int lane) {
  const int g4 = lane >> 4, n16 = lane & 15;
  wave_lds_sync();
  f32x4 xa, ta;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int i = 4 * g4 + s;
    xa[s] = (n16 < i) ? w.alpha[i] * expf(w.G[i] - w.G[n16]) * w.pp[0][i][n16] : 0.f;
    w.pp[3][i][n16] = xa[s];
    ta[s] = (i == n16 ? 1.f : 0.f) - xa[s];
  }
  wave_lds_sync();
  int src = 3;
#pragma unroll
  for (int step = 0; step < 3; ++step) {
    const int dst = step & 1 ? 3 : 0;
    f32x4 sq = zero4();
    mma(sq, *(const f32x4*)&w.pp[src][n16][4 * g4], xa);  // X^2
    xa = sq;
#pragma unroll
    for (int s = 0; s < 4; ++s) w.pp[dst][4 * g4 + s][n16] = sq[s];
    wave_lds_sync();
    mma(ta, *(const f32x4*)&w.pp[dst][n16][4 * g4], ta);  // T += X^2 T
    src = dst;
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) w.pp[2][4 * g4 + s][n16] = ta[s];
}

// The commit of a sub-chunk's prefetched token rows into the window LDS: H =
// b (.) k, the Q and K rows, u = w (.) v, and per token alpha and the log
// decay (thread tid holds load unit (tid / (D / 8), 8 (tid mod (D / 8)))).
template <typename CT, int D, int P>
__device__ __forceinline__ void g3_commit(const G3WinView<CT, D, P>& w, const G3Tok& tk, const G3Raw<CT>& r, int tid) {
  constexpr int DG = D / 8, W16 = W16Of<CT>::value;
  if (tid >= kSC * DG) return;
  const int ui = tid / DG, ud = 8 * (tid % DG);
  float hf[8], uu[8];
  const float part = g3_unpack<CT, DG>(r, tk.gc, hf, uu);
  store8(&w.x[ui][ud], hf);
#pragma unroll
  for (int q16 = 0; q16 < W16; ++q16) {
    *(uint4*)&w.x[kSC + ui][ud + q16 * (16 / sizeof(CT))] = g3_raw(r, r.q[q16]);
    *(uint4*)&w.x[2 * kSC + ui][ud + q16 * (16 / sizeof(CT))] = g3_raw(r, r.k[q16]);
  }
  *(f32x4*)&w.u[ui][ud] = (f32x4){uu[0], uu[1], uu[2], uu[3]};
  *(f32x4*)&w.u[ui][ud + 4] = (f32x4){uu[4], uu[5], uu[6], uu[7]};
  if (tid % DG == 0) {
    w.alpha[ui] = stable_alpha_f(part);
    w.lg[ui] = log_decay(r.ok ? r.dec : 1.f);
  }
}

// The state-independent half of sub-chunk c's step, formed on waves 1..3
// while wave 0 runs a compaction's eigen-solve (no workgroup barrier can be
// used then): every one of the three waves loads and commits all 16 token
// rows itself (identical values, so the concurrent writes agree), two load
// passes in flight at a time, and reads only what it wrote; then wave 1 forms
// the coefficients, H K^T and the inverse, wave 2 Aq and wave 3 the window
// grams.  The commit's x, u and scalars and the tiles' pp, po must lie in LDS
// the compaction no longer uses.
template <typename CT, int D, int P>
__device__ __forceinline__ void g3_stage_a_shadow(const G3WinView<CT, D, P>& w, const G3FwdArgs& p,
                                                  const G3Tok& tk, G3Raw<CT>& ra, G3Raw<CT>& rb, int c,
                                                  int wave, int lane) {
  constexpr int NB = P / kSC, DG = D / 8, PASSES = kSC * DG / 64;
  static_assert(PASSES % 2 == 0, "load passes in pairs");
  auto fetch = [&](G3Raw<CT>& r, int pass) {
    const int u = pass * 64 + lane;
    g3_fetch<CT>(p, tk, r, c * kSC + u / DG - p.t0, true, 8 * (u % DG));
  };
#pragma unroll
  for (int pass = 0; pass < PASSES; pass += 2) {
    fetch(ra, pass);
    fetch(rb, pass + 1);
    g3_commit<CT, D, P>(w, tk, ra, pass * 64 + lane);
    g3_commit<CT, D, P>(w, tk, rb, (pass + 1) * 64 + lane);
  }
  wave_lds_sync();
  const int lo = max(0, p.t0 - c * kSC), beta = c % NB;
  const float gl = g3_scan_g(w, lane);
  if (wave == 1) {
    g3_scalars(w, gl, 0.f, lane);
    g3_gram_tile<CT, D, P>(w, 0, gl, beta, lo, lane);
    g3_inverse(w, lane);
  } else if (wave == 2) {
    g3_gram_tile<CT, D, P>(w, 1, gl, beta, lo, lane);
  } else {
#pragma unroll
    for (int ti = 2; ti < 2 + 2 * NB; ++ti) g3_gram_tile<CT, D, P>(w, ti, gl, beta, lo, lane);
  }
}

// One sub-chunk c of the single-stage window recurrence for one workgroup
// (value tiles vb NVTW .. of chain): commit of its prefetched token rows (and
// the loads of sub-chunk next, if >= 0), the grams, the inverse, the
// Kronecker reads, the window algebra on the U tiles uo, y and the training
// stash, then the window keys.  first: no sub-chunk before it in this launch;
// committed: its token rows are in LDS already (g3_commit ran earlier).
template <typename CT, int D, int P, int NVB>
__device__ __forceinline__ void g3_window_step(const G3WinView<CT, D, P>& w, const G3FwdArgs& p, const G3Tok& tk,
                                               int chain, int vb, int c, bool first, int next, bool live,
                                               float& gacc, f32x4 (&uo)[P / kSC][(D / 16 / NVB + 3) / 4],
                                               G3Raw<CT>& raw, bool committed = false) {
  constexpr int NB = P / kSC;
  constexpr bool KF = sizeof(CT) == 4;
  constexpr int DG = D / 8;  // 8-element load units per token row
  constexpr int UNITS = kSC * DG;
  constexpr int W16 = W16Of<CT>::value;
  constexpr int KS = FragT<CT>::KSTEP;
  typedef typename FragT<CT>::type Frag;
  constexpr int NVTW = D / 16 / NVB;   // value tiles of this workgroup: vb NVTW + [0, NVTW)
  constexpr int VPW = (NVTW + 3) / 4;
  const int tid = opaque(threadIdx.x), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, n16 = lane & 15;
  const int T = p.T;
  const bool has_unit = tid < UNITS;
  const int ui = tid / DG, ud = 8 * (tid % DG);
  auto fetch = [&](G3Raw<CT>& r, int cc) { g3_fetch<CT>(p, tk, r, cc * kSC + ui - p.t0, has_unit, ud); };
  auto commit = [&](const G3Raw<CT>& r) { g3_commit<CT, D, P>(w, tk, r, tid); };
  // after sub-chunk cc: its block is rebased (boff 0), the others decayed by its G_last
  auto advance_boff = [&](int cc, float glast) {
    if (tid < NB) w.boff[tid] = (tid == cc % NB) ? 0.f : w.boff[tid] + glast;
  };
  auto vown = [&](int a) { return wave + 4 * a < NVTW; };
  auto vtile = [&](int a) { return vb * NVTW + wave + 4 * a; };

    // slots [lo, hi) of block beta receive this call's tokens; the others (the
    // head a previous call wrote, the tail after the last token) keep the
    // writes they hold and stay visible to every token of the sub-chunk
    const int lo = max(0, p.t0 - c * kSC), hi = min(kSC, p.t0 + T - c * kSC);
    const int beta = c % NB;
    __syncthreads();
    if (!first) advance_boff(c - 1, w.G[kSC - 1]);
    if (!committed) commit(raw);
    if (next >= 0) fetch(raw, next);
    __syncthreads();
    // per-token scalars | grams and Kronecker reads (MFMA).  Every wave forms
    // the log-decay prefix sums G (lane i holds G_i); wave 0 publishes the
    // per-token coefficients, the gram tiles go round the waves, and wave 0
    // forms the inverse while waves 1..3 do the Kronecker reads.  A committed
    // sub-chunk had all of this formed in the previous compaction's shadow.
    if (!committed) {
      const float gl = g3_scan_g(w, lane);
      if (wave == 0) g3_scalars(w, gl, gacc, lane);
#pragma unroll
      for (int r = 0; r < (2 + 2 * NB + 3) / 4; ++r)
        if (wave + 4 * r < 2 + 2 * NB) g3_gram_tile<CT, D, P>(w, wave + 4 * r, gl, beta, lo, lane);
      if (wave == 0) g3_inverse(w, lane);
    }
    if (live && (committed || wave > 0)) {
      // this workgroup's value tiles over waves 1..3 (wave 0 forms the inverse), or all four
      const int w0 = committed ? wave : wave - 1, ws = committed ? 4 : 3;
      // the H and Q fragments serve every value tile; each tile's Kronecker
      // fragments are read ahead of its MFMAs behind a scheduling barrier (the
      // compiler, short of registers, waited for each MFMA's reads)
      Frag xf[2][D / KS];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kb = 0; kb < D / KS; ++kb) xf[rt][kb] = ld_frag(&w.x[rt * 16 + n16][kb * KS], g4);
      for (int l = w0; l < NVTW; l += ws) {
        const int vt = vb * NVTW + l;
        Frag bf[D / KS];
#pragma unroll
        for (int kb = 0; kb < D / KS; ++kb) bf[kb] = ld_frag(&w.skron[l * 16 + n16][kb * KS], g4);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < D / KS; ++kb) mma(acc, xf[rt][kb], bf[kb]);
#pragma unroll
          for (int s = 0; s < 4; ++s) w.kr[rt * 16 + 4 * g4 + s][vt * 16 + n16] = acc[s];
        }
      }
    }
    __syncthreads();
    // window algebra on fp32 MFMA, per wave its VPW value tiles:
    //   Rhs = alpha u - kco KRh - sum_b Ho_b U_b;  U = T Rhs
    //   Y   = qco KRq + sum_b Qo_b U_b + Aq U
    // (an accumulator tile over rows = tokens is directly a k-fragment)
    // (every LDS operand read ahead, behind a scheduling barrier; the
    // coefficient tiles and per-token scalars serve every value tile)
    f32x4 po0[NB], po1[NB];
#pragma unroll
    for (int bl = 0; bl < NB; ++bl) {
      po0[bl] = *(const f32x4*)&w.po[0][n16][kSC * bl + 4 * g4];
      po1[bl] = *(const f32x4*)&w.po[1][n16][kSC * bl + 4 * g4];
    }
    const f32x4 ptf = *(const f32x4*)&w.pp[2][n16][4 * g4], paf = *(const f32x4*)&w.pp[1][n16][4 * g4];
    float alv[4], kcv[4], qcv[4], uv[VPW][4], khv[VPW][4], kqv[VPW][4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g4 + s;
      alv[s] = w.alpha[i];
      kcv[s] = w.kco[i];
      qcv[s] = w.qco[i];
    }
#pragma unroll
    for (int a = 0; a < VPW; ++a)
      if (vown(a)) {
        const int v = vtile(a) * 16 + n16;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int i = 4 * g4 + s;
          uv[a][s] = w.u[i][v];
          khv[a][s] = w.kr[i][v];
          kqv[a][s] = w.kr[kSC + i][v];
        }
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int a = 0; a < VPW; ++a) {
      if (!vown(a)) continue;
      const int v = vtile(a) * 16 + n16;
      f32x4 acc = zero4();
#pragma unroll
      for (int bl = 0; bl < NB; ++bl) mma(acc, po0[bl], uo[bl][a]);
      f32x4 rhs;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float r = alv[s] * uv[a][s] - acc[s];
        if (live) r -= kcv[s] * khv[a][s];
        rhs[s] = r;
      }
      f32x4 un = zero4();
      mma(un, ptf, rhs);
      f32x4 yv = zero4();
#pragma unroll
      for (int bl = 0; bl < NB; ++bl) mma(yv, po1[bl], uo[bl][a]);
      mma(yv, paf, un);
      CT* yp = (CT*)p.y + tk.y_base + v;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        float out = yv[s];
        if (live) out += qcv[s] * kqv[a][s];
        const int t = c * kSC + i - p.t0;
        if (t >= 0 && t < T) yp[(size_t)t * tk.y_tok] = from_f<CT>(out);
      }
#pragma unroll
      for (int bl = 0; bl < NB; ++bl)
        if (bl == beta)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int i = 4 * g4 + s;
            if (i >= lo && i < hi) uo[bl][a][s] = un[s];
          }
      if (p.ts_u) {   // training stash: this sub-chunk's net writes
        float* us = p.ts_u + ((size_t)chain * p.nch + c) * kSC * D + v;
#pragma unroll
        for (int s = 0; s < 4; ++s) us[(size_t)(4 * g4 + s) * D] = un[s];
      }
    }
    if (p.ts_g && tid == 0 && vb == 0) p.ts_g[(size_t)chain * p.nch + c] = gacc;
    // block beta's keys for the next sub-chunks: the slots this sub-chunk
    // wrote take k_j decayed to its end, the others their old keys decayed
    // over it (8 consecutive keys per thread); the block's offset restarts
    {
      const float olds = expf(w.boff[beta] + w.G[kSC - 1]);
      for (int u8 = tid; u8 < kSC * D / 8; u8 += kNT) {
        const int j = u8 / DG, d = 8 * (u8 % DG), sl = kSC * beta + j;
        uint4 kw[W16];
#pragma unroll
        for (int q16 = 0; q16 < W16; ++q16) kw[q16] = *(const uint4*)&w.x[2 * kSC + j][d + q16 * (16 / sizeof(CT))];
        float kf[8];
        unpack8(kw, kf, (const CT*)nullptr);
        float sc = w.vsc[j];
        if (j < lo || j >= hi) {
          sc = olds;
          const f32x4 o0 = *(const f32x4*)&w.vbd[sl][d], o1 = *(const f32x4*)&w.vbd[sl][d + 4];
          kf[0] = o0[0], kf[1] = o0[1], kf[2] = o0[2], kf[3] = o0[3];
          kf[4] = o1[0], kf[5] = o1[1], kf[6] = o1[2], kf[7] = o1[3];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] *= sc;
        *(f32x4*)&w.vbd[sl][d] = (f32x4){kf[0], kf[1], kf[2], kf[3]};
        *(f32x4*)&w.vbd[sl][d + 4] = (f32x4){kf[4], kf[5], kf[6], kf[7]};
        if constexpr (!KF) store8(&w.vbx[sl][d], kf);
      }
    }
    gacc += w.G[kSC - 1];
}

// Sub-chunks [c0, c1) of one compaction interval (or the tail) for every
// chain; the window state enters and leaves through the workspace.  A
// chain's value columns are split over NVB workgroups (D / 16 / NVB value
// tiles each): the grams, the triangular inverse and the window keys depend
// on no value column and are formed by each of them; the Kronecker reads, the
// window algebra, the net writes U and y are split.
template <typename CT, int D, int P, int NVB>
__global__ void __launch_bounds__(kNT) gdn3_window_kernel(G3FwdArgs p) {
  typedef G3WinSmem<CT, D, P, NVB> Sm;
  __shared__ Sm sm;
  constexpr int NB = Sm::NB;
  constexpr int DG = D / 8;  // 8-element load units per token row
  constexpr int UNITS = kSC * DG;
  constexpr int W16 = W16Of<CT>::value;
  constexpr int KS = FragT<CT>::KSTEP;
  typedef typename FragT<CT>::type Frag;
  static_assert(UNITS <= kNT && UNITS % 64 == 0, "one load unit per thread");
  static_assert(P % kSC == 0 && NB >= 1 && NB <= 4, "whole 16-slot blocks, at most 4");
  static_assert(sizeof(Sm) <= 160 * 1024, "LDS budget");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, n16 = lane & 15;
  const int H = p.H, M = p.M, T = p.T;
  const int N = p.B * H * M;
  const int work = xcd_remap(blockIdx.x, N * NVB);   // a chain's NVB workgroups land on one XCD
  const int chain = work / NVB, vb = work % NVB;
  typedef G3D<D> Ge;
  constexpr int NVTW = D / 16 / NVB;   // value tiles of this workgroup: vb NVTW + [0, NVTW)
  static_assert(NVTW >= 1 && (D / 16) % NVB == 0, "value split");

  const bool has_unit = tid < UNITS;
  const int ui = tid / DG, ud = 8 * (tid % DG);
  typedef G3Raw<CT> Raw;
  const G3Tok tk(p, chain, D);
  // sub-chunk c covers global tokens [16 c, 16 c + 16): local token 16 c + i - t0
  auto fetch = [&](Raw& r, int c) { g3_fetch<CT>(p, tk, r, c * kSC + ui - p.t0, has_unit, ud); };

  // window state: zero for the first interval, else from the workspace.
  // Wave w holds value tiles vtile(a) = vb NVTW + w + 4 a of the workgroup's
  // (a < VPW, where w + 4 a < NVTW), of every block
  constexpr int VPW = (NVTW + 3) / 4;
  auto vown = [&](int a) { return wave + 4 * a < NVTW; };
  auto vtile = [&](int a) { return vb * NVTW + wave + 4 * a; };
  f32x4 uo[NB][VPW];
  float* uw = p.uw + (size_t)chain * P * D;
  float* vw = p.vw + (size_t)chain * P * D;
  if (p.first) {
    for (int e = tid; e < P * (D + 4); e += kNT) (&sm.vbd[0][0])[e] = 0.f;
    if constexpr (!Sm::KF)
      for (int e = tid; e < P * (D + 8); e += kNT) (&sm.vbx[0][0])[e] = (CT)0.f;
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int a = 0; a < VPW; ++a) uo[bl][a] = zero4();
  } else {
    for (int e = tid; e < P * D; e += kNT) {
      const int j = e / D, d = e % D;
      const float kv = vw[e];
      sm.vbd[j][d] = kv;
      if constexpr (!Sm::KF) sm.vbx[j][d] = from_f<CT>(kv);
    }
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int a = 0; a < VPW; ++a)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          uo[bl][a][s] = vown(a) ? uw[(bl * kSC + 4 * g4 + s) * D + vtile(a) * 16 + n16] : 0.f;
  }
  if (tid < NB) sm.boff[tid] = 0.f;
  const bool live = p.live;
  if (live) {   // this workgroup's value rows of the Kronecker matrix
    constexpr int PER = 16 / sizeof(CT);  // elements per 16-byte load
    const uint4* src = (const uint4*)((const CT*)p.skron + ((size_t)chain * D + vb * NVTW * 16) * D);
    for (int e = tid; e < NVTW * 16 * D / PER; e += kNT) {
      const int v = (e * PER) / D, k = (e * PER) % D;   // (local row)
      *(uint4*)&sm.skron[v][k] = src[e];
    }
  }
  float gacc = 0.f;

  Raw raw;
  fetch(raw, p.c0);
  const G3WinView<CT, D, P> w{sm.x, sm.u, sm.kr, sm.pp, sm.po, sm.skron, sm.vbd, sm.vbx, sm.G,
                              sm.alpha, sm.lg, sm.kco, sm.qco, sm.gam, sm.vsc, sm.boff};
  for (int c = p.c0; c < p.c1; ++c)
    g3_window_step<CT, D, P, NVB>(w, p, tk, chain, vb, c, c == p.c0, c + 1 < p.c1 ? c + 1 : -1, live, gacc, uo,
                                  raw);
  __syncthreads();
  if (p.c1 > p.c0 && tid < NB)   // the last sub-chunk's block rebased, the others decayed
    sm.boff[tid] = (tid == (p.c1 - 1) % NB) ? 0.f : sm.boff[tid] + sm.G[kSC - 1];
  __syncthreads();
  // window state out (and the final state after the last sub-chunk): the
  // value columns from their workgroup, the keys and decays from the first
#pragma unroll
  for (int a = 0; a < VPW; ++a) {
    if (!vown(a)) continue;
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = bl * kSC + 4 * g4 + s, v = vtile(a) * 16 + n16;
        uw[i * D + v] = uo[bl][a][s];
        if (p.last && p.U_out) p.U_out[((size_t)chain * D + v) * P + i] = uo[bl][a][s];
      }
  }
  if (vb != 0) return;
  for (int e = tid; e < P * D; e += kNT) {
    const int j = e / D, d = e % D;
    const float kv = sm.vbd[j][d] * expf(sm.boff[j / kSC]);
    vw[e] = kv;
    if (p.last && p.Vb_out) p.Vb_out[((size_t)chain * D + d) * P + j] = kv;
  }
  if (tid == 0) p.gsum[chain] = gacc;
  if (p.last && !p.complete) {  // no compaction follows: A, B decayed since the last one
    // the workspace holds every chain's A [N][R m], then every chain's B [N][R n]
    const float dk = expf(gacc);
    const float* af = p.ab + (size_t)chain * Ge::R * Ge::m;
    const float* bf = p.ab + (size_t)N * Ge::R * Ge::m + (size_t)chain * Ge::R * Ge::n;
    if (p.A_out)
      for (int e = tid; e < Ge::R * Ge::m; e += kNT) p.A_out[(size_t)chain * Ge::R * Ge::m + e] = af[e] * dk;
    if (p.B_out)
      for (int e = tid; e < Ge::R * Ge::n; e += kNT) p.B_out[(size_t)chain * Ge::R * Ge::n + e] = bf[e] * dk;
  }
}

// Long intervals: the same sub-chunk recurrence as a two-stage software
// pipeline over the sub-chunks with one barrier per step.  In step c:
//   wave 0: the G scan and per-token coefficients of sub-chunk c, H K^T and
//           the inverse T (the longest chain of a step);
//   wave 1: Ho_b, Qo_b against the window keys of sub-chunk c, then sub-chunk
//           c's keys into block c mod NB (the window keys are read and
//           written by wave 1 alone);
//   waves 2, 3: the window algebra of sub-chunk c - 1 on their value tiles (U
//           resident in their registers; wave 2 takes the first), then
//           sub-chunk c's Kronecker reads; wave 3 also forms Aq = Q K^T;
//   waves 0, 2, 3: the token rows of sub-chunk c + 1 into LDS (loaded a step
//           ahead), wave 3 also wave 1's.
// What a step writes for the next alternates by sub-chunk parity; the
// per-token inputs sub-chunk c + 1 commits while sub-chunk c - 1's algebra
// still reads its own rotate over three.
template <typename CT, int D, int P, int NVB>
struct G3PipeSmem {
  static constexpr int NB = P / kSC;
  static constexpr int NVTW = D / 16 / NVB;
  static constexpr int VW = NVTW * 16;        // this workgroup's value columns
  static constexpr bool KF = sizeof(CT) == 4; // fp32 IO: the grams read the fp32 window keys
  alignas(16) CT x[2][3 * kSC][D + 8];        // H, Q, K rows (parity)
  alignas(16) float uu[3][kSC][VW + 4];       // w (.) v at this workgroup's value columns (c mod 3)
  alignas(16) float kr[2][2 * kSC][VW + 4];   // Kronecker reads of H and Q at those columns (parity)
  alignas(16) float ws[2][kSC][kSC + 4];      // wave 0's inverse scratch
  alignas(16) float tt[2][kSC][kSC + 4];      // T (parity)
  alignas(16) float aq[2][kSC][kSC + 4];      // Aq (parity)
  alignas(16) float po[2][2][kSC][P + 4];     // Ho, Qo over the P slots (parity)
  alignas(16) CT skron[VW][D + 8];            // sum_r A_r (x) B_r, this workgroup's rows v
  alignas(16) float vbd[P][D + 4];            // window keys: block b decayed to e^{-boff_b} of now
  alignas(16) CT vbx[KF ? 1 : P][D + 8];      // the same in the compute dtype (bf16 IO)
  float cr[2][kSC], dr[2][kSC];               // k . h and the decay as committed (parity)
  float al[2][kSC];                           // alpha (parity)
  float kco[2][kSC], qco[2][kSC];             // alpha e^{2(Gacc + G)}, e^{2(Gacc + G)} (parity)
  float boff[NB];                             // log decay of block b's keys since they were rebased
  float gfin;                                 // Gacc after the last sub-chunk
};
template <typename CT, int D, int P, int NVB>
constexpr size_t pipe_lds() { return sizeof(G3PipeSmem<CT, D, P, NVB>); }

template <typename CT, int D, int P, int NVB, int GL>
__global__ void __launch_bounds__(kNT) gdn3_window_pipe_kernel(G3FwdArgs p) {
  typedef G3PipeSmem<CT, D, P, NVB> Sm;
  __shared__ Sm sm;
  constexpr int NB = Sm::NB, NVTW = Sm::NVTW, VW = Sm::VW;
  constexpr int DG = D / 8, UNITS = kSC * DG, W16 = W16Of<CT>::value, KS = FragT<CT>::KSTEP;
  typedef typename FragT<CT>::type Frag;
  static_assert(UNITS <= kNT && UNITS % 64 == 0, "one load unit per thread");
  static_assert(P % kSC == 0 && NB >= 1 && NB <= 4, "whole 16-slot blocks, at most 4");
  static_assert(NVTW >= 1 && (D / 16) % NVB == 0, "value split");
  static_assert(sizeof(Sm) <= 160 * 1024, "LDS budget");
  typedef G3D<D> Ge;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, n16 = lane & 15;
  const int T = p.T;
  const int N = p.B * p.H * p.M;
  const int work = xcd_remap(blockIdx.x, N * NVB);   // a chain's NVB workgroups land on one XCD
  const int chain = work / NVB, vb = work % NVB;
  typedef G3Raw<CT> Raw;
  const G3Tok tk(p, chain, D);
  const bool live = p.live;

  // load unit un (< UNITS: token row un / DG, channels 8 (un mod DG) ..);
  // sub-chunk c covers global tokens [16 c, 16 c + 16): local token 16 c + i - t0
  auto fetch = [&](Raw& r, int c, int un) {
    g3_fetch<CT, GL>(p, tk, r, c * kSC + un / DG - p.t0, un < UNITS, 8 * (un % DG));
  };
  auto commit = [&](const Raw& r, int c, int un) {
    if (un >= UNITS) return;
    const int ui = un / DG, ud = 8 * (un % DG);
    float hf[8], uu[8];
    const float part = g3_unpack<CT, DG, GL>(r, tk.gc, hf, uu);
    const int s2 = c & 1, s3 = c % 3;
    store8(&sm.x[s2][ui][ud], hf);
#pragma unroll
    for (int w = 0; w < W16; ++w) {
      *(uint4*)&sm.x[s2][kSC + ui][ud + w * (16 / sizeof(CT))] = g3_raw(r, r.q[w]);
      *(uint4*)&sm.x[s2][2 * kSC + ui][ud + w * (16 / sizeof(CT))] = g3_raw(r, r.k[w]);
    }
    const int uc = ud - vb * VW;   // this workgroup's value columns only
    if (uc >= 0 && uc < VW) {
      *(f32x4*)&sm.uu[s3][ui][uc] = (f32x4){uu[0], uu[1], uu[2], uu[3]};
      *(f32x4*)&sm.uu[s3][ui][uc + 4] = (f32x4){uu[4], uu[5], uu[6], uu[7]};
    }
    if (un % DG == 0) {   // alpha and the log decay are formed lane-parallel in stage A
      sm.cr[s2][ui] = part;
      sm.dr[s2][ui] = r.ok ? r.dec : 1.f;
    }
  };
  // the units a wave commits: its own (waves 0, 2, 3) and, for wave 3, wave 1's
  const int u_own = tid, u_w1 = 64 + lane;
  // stage A's per-token scalars of sub-chunk c: lane i < 16 gets G_i (the
  // log-decay prefix) and alpha_i
  auto scan_g = [&](int c) {
    float gl = lane < kSC ? log_decay(sm.dr[c & 1][lane]) : 0.f;
#pragma unroll
    for (int off = 1; off < kSC; off <<= 1) {
      const float o = __shfl_up(gl, off, 64);
      if (lane >= off) gl += o;
    }
    return gl;
  };
  auto token_scalars = [&](int c, float& alpha_l, float& gl) {
    alpha_l = lane < kSC ? stable_alpha_f(sm.cr[c & 1][lane]) : 0.f;
    gl = scan_g(c);
  };

  // window state: zero for the first interval, else from the workspace.
  // Algebra wave 2 + w2 holds the workgroup's local value tiles w2 + 2 a
  // (a < VPW, where w2 + 2 a < NVTW), of every block
  constexpr int VPW = (NVTW + 1) / 2;
  const int w2 = wave - 2;
  auto vown = [&](int a) { return w2 >= 0 && w2 + 2 * a < NVTW; };
  f32x4 uo[NB][VPW];
  float* uw = p.uw + (size_t)chain * P * D;
  float* vw = p.vw + (size_t)chain * P * D;
  if (p.first) {
    for (int e = tid; e < P * (D + 4); e += kNT) (&sm.vbd[0][0])[e] = 0.f;
    if constexpr (!Sm::KF)
      for (int e = tid; e < P * (D + 8); e += kNT) (&sm.vbx[0][0])[e] = (CT)0.f;
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int a = 0; a < VPW; ++a) uo[bl][a] = zero4();
  } else {
    for (int e = tid; e < P * D; e += kNT) {
      const int j = e / D, d = e % D;
      const float kv = vw[e];
      sm.vbd[j][d] = kv;
      if constexpr (!Sm::KF) sm.vbx[j][d] = from_f<CT>(kv);
    }
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int a = 0; a < VPW; ++a)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          uo[bl][a][s] = vown(a) ? uw[(bl * kSC + 4 * g4 + s) * D + vb * VW + (w2 + 2 * a) * 16 + n16] : 0.f;
  }
  if (tid < NB) sm.boff[tid] = 0.f;
  if (live) {   // this workgroup's value rows of the Kronecker matrix
    constexpr int PER = 16 / sizeof(CT);  // elements per 16-byte load
    const uint4* src = (const uint4*)((const CT*)p.skron + ((size_t)chain * D + vb * VW) * D);
    for (int e = tid; e < VW * D / PER; e += kNT) {
      const int v = (e * PER) / D, k = (e * PER) % D;   // (local row)
      *(uint4*)&sm.skron[v][k] = src[e];
    }
  }
  float gacc = 0.f;   // (wave 0) log decay since the last compaction, at the current sub-chunk

  Raw raw, raw1;   // raw1: wave 3's copy of wave 1's units
  fetch(raw, p.c0, u_own);
  commit(raw, p.c0, u_own);
  if (p.c0 + 1 < p.c1) fetch(raw, p.c0 + 1, u_own);
  if (wave == 3 && p.c0 + 1 < p.c1) fetch(raw1, p.c0 + 1, u_w1);
  __syncthreads();
  for (int c = p.c0; c <= p.c1; ++c) {
    const bool sa = c < p.c1, sb = c > p.c0;   // stage A of c, stage B of c - 1
    const int s2 = c & 1;
    if (wave == 0 && sa) {
      // per-token coefficients and T = (I + Lm)^-1 of sub-chunk c
      float alpha_l, gl;
      token_scalars(c, alpha_l, gl);
      const float gl_last = __shfl(gl, kSC - 1, 64);
      if (lane < kSC) {
        const float e2 = expf(2.f * (gacc + gl));
        sm.al[s2][lane] = alpha_l;
        sm.kco[s2][lane] = alpha_l * e2;
        sm.qco[s2][lane] = e2;
      }
      if (p.ts_g && lane == 0 && vb == 0) p.ts_g[(size_t)chain * p.nch + c] = gacc;
      gacc += gl_last;
      const f32x4 acc = tile_nt<CT, D>(&sm.x[s2][n16][0], &sm.x[s2][2 * kSC + n16][0], g4);
      // Lm[i][j] = alpha_i e^{G_i - G_j} (h_i . k_j), j < i, is strictly lower
      // (nilpotent): (I + Lm)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8), factors
      // that commute; squarings and products on fp32 MFMA.  An accumulator
      // tile is a k-fragment (B operand); the A operand of each square goes
      // through LDS.
      const float gj = __shfl(gl, n16, 64);
      f32x4 xa, ta;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = 4 * g4 + s;
        const float gi = __shfl(gl, i, 64), ai = __shfl(alpha_l, i, 64);
        xa[s] = (n16 < i) ? ai * expf(gi - gj) * acc[s] : 0.f;
        sm.ws[0][i][n16] = xa[s];
        ta[s] = (i == n16 ? 1.f : 0.f) - xa[s];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
      for (int step = 0; step < 3; ++step) {
        const int src = step & 1, dst = src ^ 1;
        f32x4 sq = zero4();
        mma(sq, *(const f32x4*)&sm.ws[src][n16][4 * g4], xa);  // X^2
        xa = sq;
#pragma unroll
        for (int s = 0; s < 4; ++s) sm.ws[dst][4 * g4 + s][n16] = sq[s];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        mma(ta, *(const f32x4*)&sm.ws[dst][n16][4 * g4], ta);  // T += X^2 T
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) sm.tt[s2][4 * g4 + s][n16] = ta[s];
    } else if (wave == 1 && sa) {
      // Ho_b, Qo_b of sub-chunk c, then its keys into block c mod NB:
      //   Ho_b = vis alpha_i e^{G_i + boff_b} h_i.Vb_b[j],  Qo_b = vis e^{G_i + boff_b} q_i.Vb_b[j]
      // with vis = [b != beta or j >= i or j < lo]
      const int beta = c % NB, lo = max(0, p.t0 - c * kSC), hi = min(kSC, p.t0 + T - c * kSC);
      float alpha_l, gl;
      token_scalars(c, alpha_l, gl);
      float gi[4], ai[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        gi[s] = __shfl(gl, 4 * g4 + s, 64);
        ai[s] = __shfl(alpha_l, 4 * g4 + s, 64);
      }
#pragma unroll
      for (int t2 = 0; t2 < 2 * NB; ++t2) {
        const int bl = t2 >> 1;
        const bool isq = t2 & 1;
        const CT* brow;
        if constexpr (Sm::KF) brow = (const CT*)&sm.vbd[kSC * bl + n16][0];
        else brow = &sm.vbx[kSC * bl + n16][0];
        const f32x4 acc = tile_nt<CT, D>(&sm.x[s2][(isq ? kSC : 0) + n16][0], brow, g4);
        const float bo = sm.boff[bl];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int i = 4 * g4 + s;
          const bool vis = bl != beta || n16 >= i || n16 < lo;
          const float sc = expf(gi[s] + bo) * (isq ? 1.f : ai[s]);
          sm.po[s2][isq ? 1 : 0][i][kSC * bl + n16] = vis ? sc * acc[s] : 0.f;
        }
      }
      // block beta's keys for the next sub-chunks: the slots sub-chunk c wrote
      // take k_j decayed to its end, the others their old keys decayed over
      // it; then the block's offset restarts and the others' grow by G_last
      const float gl_last = __shfl(gl, kSC - 1, 64);
      const float vsc = expf(gl_last - gl);   // lane j < 16
      const float olds = expf(sm.boff[beta] + gl_last);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      for (int u8 = lane; u8 < kSC * D / 8; u8 += 64) {
        const int j = u8 / DG, d = 8 * (u8 % DG), sl = kSC * beta + j;
        uint4 w[W16];
#pragma unroll
        for (int q16 = 0; q16 < W16; ++q16)
          w[q16] = *(const uint4*)&sm.x[s2][2 * kSC + j][d + q16 * (16 / sizeof(CT))];
        float kf[8];
        unpack8(w, kf, (const CT*)nullptr);
        float sc = __shfl(vsc, j, 64);
        if (j < lo || j >= hi) {
          sc = olds;
          const f32x4 o0 = *(const f32x4*)&sm.vbd[sl][d], o1 = *(const f32x4*)&sm.vbd[sl][d + 4];
          kf[0] = o0[0], kf[1] = o0[1], kf[2] = o0[2], kf[3] = o0[3];
          kf[4] = o1[0], kf[5] = o1[1], kf[6] = o1[2], kf[7] = o1[3];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] *= sc;
        *(f32x4*)&sm.vbd[sl][d] = (f32x4){kf[0], kf[1], kf[2], kf[3]};
        *(f32x4*)&sm.vbd[sl][d + 4] = (f32x4){kf[4], kf[5], kf[6], kf[7]};
        if constexpr (!Sm::KF) store8(&sm.vbx[sl][d], kf);
      }
      if (lane < NB) sm.boff[lane] = (lane == beta) ? 0.f : sm.boff[lane] + gl_last;
    } else if (wave >= 2) {
      if (wave == 3 && sa) {   // Aq = [j <= i] e^{G_i - G_j} q_i.k_j of sub-chunk c
        const float gl = scan_g(c);
        const float gj = __shfl(gl, n16, 64);
        const f32x4 acc = tile_nt<CT, D>(&sm.x[s2][kSC + n16][0], &sm.x[s2][2 * kSC + n16][0], g4);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int i = 4 * g4 + s;
          const float gi = __shfl(gl, i, 64);
          sm.aq[s2][i][n16] = (n16 <= i) ? expf(gi - gj) * acc[s] : 0.f;
        }
      }
      if (sb) {
        // window algebra of sub-chunk cb = c - 1 on fp32 MFMA, per value tile:
        //   Rhs = alpha u - kco KRh - sum_b Ho_b U_b;  U = T Rhs
        //   Y   = qco KRq + sum_b Qo_b U_b + Aq U
        const int cb = c - 1, t2 = cb & 1, t3 = cb % 3, beta = cb % NB;   // uu by c mod 3, the rest by parity
        const int lo = max(0, p.t0 - cb * kSC), hi = min(kSC, p.t0 + T - cb * kSC);
#pragma unroll
        for (int a = 0; a < VPW; ++a) {
          if (!vown(a)) continue;
          const int vl = (w2 + 2 * a) * 16 + n16, v = vb * VW + vl;
          f32x4 acc = zero4();
#pragma unroll
          for (int bl = 0; bl < NB; ++bl) mma(acc, *(const f32x4*)&sm.po[t2][0][n16][kSC * bl + 4 * g4], uo[bl][a]);
          f32x4 rhs;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int i = 4 * g4 + s;
            float r = sm.al[t2][i] * sm.uu[t3][i][vl] - acc[s];
            if (live) r -= sm.kco[t2][i] * sm.kr[t2][i][vl];
            rhs[s] = r;
          }
          f32x4 un = zero4();
          mma(un, *(const f32x4*)&sm.tt[t2][n16][4 * g4], rhs);
          f32x4 yv = zero4();
#pragma unroll
          for (int bl = 0; bl < NB; ++bl) mma(yv, *(const f32x4*)&sm.po[t2][1][n16][kSC * bl + 4 * g4], uo[bl][a]);
          mma(yv, *(const f32x4*)&sm.aq[t2][n16][4 * g4], un);
          CT* yp = (CT*)p.y + tk.y_base + v;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int i = 4 * g4 + s;
            float out = yv[s];
            if (live) out += sm.qco[t2][i] * sm.kr[t2][kSC + i][vl];
            const int t = cb * kSC + i - p.t0;
            if (t >= 0 && t < T) yp[(size_t)t * tk.y_tok] = from_f<CT>(out);
          }
#pragma unroll
          for (int bl = 0; bl < NB; ++bl)
            if (bl == beta)
#pragma unroll
              for (int s = 0; s < 4; ++s) {
                const int i = 4 * g4 + s;
                if (i >= lo && i < hi) uo[bl][a][s] = un[s];
              }
          if (p.ts_u) {   // training stash: this sub-chunk's net writes
            float* us = p.ts_u + ((size_t)chain * p.nch + cb) * kSC * D + v;
#pragma unroll
            for (int s = 0; s < 4; ++s) us[(size_t)(4 * g4 + s) * D] = un[s];
          }
        }
      }
      if (sa && live) {
        // Kronecker reads of sub-chunk c at this wave's value tiles
#pragma unroll
        for (int a = 0; a < VPW; ++a) {
          if (!vown(a)) continue;
          const int l = w2 + 2 * a;
          Frag bf[D / KS];
#pragma unroll
          for (int kb = 0; kb < D / KS; ++kb) bf[kb] = ld_frag(&sm.skron[l * 16 + n16][kb * KS], g4);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            f32x4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < D / KS; ++kb) mma(acc, ld_frag(&sm.x[s2][rt * 16 + n16][kb * KS], g4), bf[kb]);
#pragma unroll
            for (int s = 0; s < 4; ++s) sm.kr[s2][rt * 16 + 4 * g4 + s][l * 16 + n16] = acc[s];
          }
        }
      }
    }
    // the rows of sub-chunk c + 1 (and the loads of c + 2, which stay in
    // flight across the LDS-only barrier): waves 0, 2, 3 their own, wave 3
    // wave 1's
    if (c + 1 < p.c1) {
      if (wave != 1) {
        commit(raw, c + 1, u_own);
        if (c + 2 < p.c1) fetch(raw, c + 2, u_own);
      }
      if (wave == 3) {
        commit(raw1, c + 1, u_w1);
        if (c + 2 < p.c1) fetch(raw1, c + 2, u_w1);
      }
    }
    lds_barrier();
  }
  if (tid == 0) sm.gfin = gacc;
  __syncthreads();
  // window state out (and the final state after the last sub-chunk): the
  // value columns from their workgroup, the keys and decays from the first
#pragma unroll
  for (int a = 0; a < VPW; ++a) {
    if (!vown(a)) continue;
#pragma unroll
    for (int bl = 0; bl < NB; ++bl)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = bl * kSC + 4 * g4 + s, v = vb * VW + (w2 + 2 * a) * 16 + n16;
        uw[i * D + v] = uo[bl][a][s];
        if (p.last && p.U_out) p.U_out[((size_t)chain * D + v) * P + i] = uo[bl][a][s];
      }
  }
  if (vb != 0) return;
  const float gfin = sm.gfin;
  for (int e = tid; e < P * D; e += kNT) {
    const int j = e / D, d = e % D;
    const float kv = sm.vbd[j][d] * expf(sm.boff[j / kSC]);
    vw[e] = kv;
    if (p.last && p.Vb_out) p.Vb_out[((size_t)chain * D + d) * P + j] = kv;
  }
  if (tid == 0) p.gsum[chain] = gfin;
  if (p.last && !p.complete) {  // no compaction follows: A, B decayed since the last one
    // the workspace holds every chain's A [N][R m], then every chain's B [N][R n]
    const float dk = expf(gfin);
    const float* af = p.ab + (size_t)chain * Ge::R * Ge::m;
    const float* bf = p.ab + (size_t)N * Ge::R * Ge::m + (size_t)chain * Ge::R * Ge::n;
    if (p.A_out)
      for (int e = tid; e < Ge::R * Ge::m; e += kNT) p.A_out[(size_t)chain * Ge::R * Ge::m + e] = af[e] * dk;
    if (p.B_out)
      for (int e = tid; e < Ge::R * Ge::n; e += kNT) p.B_out[(size_t)chain * Ge::R * Ge::n + e] = bf[e] * dk;
  }
}

// ---------------------------------------------------------------------------
// compaction, one chain per block: the chunked forward's step between
// intervals and the gdnx_gdn3_compact entry point
// ---------------------------------------------------------------------------
template <int D, int P>
struct G3CompactSmem {
  G3Compact<D, P> k;
  alignas(16) float ab[kAB];
};

// sum_r A_r (x) B_r as a [D][D] (v, k) matrix for the window kernel's reads,
// from the factors Af [R][m], Bf [R][n] (LDS), ld the row stride of sk.  With
// p = iv a_k + ik running over A_r's entries and q = jv b_k + jk over B_r's,
// S'^T[q][p] = sum_r B_r[q] A_r[p] is a product with K = R = 4: one fp32 MFMA
// (16x16x4) per 16 x 16 tile.  Lane (g, l) supplies B_g[q0 + l] and A_g[p0 + l]
// and holds q = q0 + 4 g + e (e < 4), p = p0 + l: the entries
// (iv b_v + jv, ik b_k + jk .. jk + 3) of S_kron, one 4-element store.  The
// tiles go round the 4 waves.
template <int D, typename CT>
__device__ __forceinline__ void write_skron(CT* sk, const float* Af, const float* Bf, int tid, int ld = D) {
  typedef G3D<D> Ge;
  constexpr int QT = Ge::n / 16, NT = QT * (Ge::m / 16);
  static_assert(Ge::R == 4 && Ge::bk % 4 == 0 && Ge::m % 16 == 0 && Ge::n % 16 == 0 && NT % 4 == 0,
                "K = R = 4 MFMA tiles, runs of 4 jk");
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), g = lane >> 4, l16 = lane & 15;
  // every tile's operands are loaded before the first MFMA
  float ao[NT / 4], bo[NT / 4];
#pragma unroll
  for (int u = 0; u < NT / 4; ++u) {
    const int t = wave + 4 * u, q0 = (t % QT) * 16, p0 = (t / QT) * 16;
    ao[u] = Bf[g * Ge::n + q0 + l16];
    bo[u] = Af[g * Ge::m + p0 + l16];
  }
  // and every MFMA issued before the first store
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc[NT / 4];
#pragma unroll
  for (int u = 0; u < NT / 4; ++u) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(ao[u], bo[u], zero4(), 0, 0, 0);
#pragma unroll
  for (int u = 0; u < NT / 4; ++u) {
    const int t = wave + 4 * u, q0 = (t % QT) * 16, p0 = (t / QT) * 16;
    const int p = p0 + l16, q = q0 + 4 * g;
    const int iv = p / Ge::ak, ik = p % Ge::ak, jv = q / Ge::bk, jk = q % Ge::bk;
    st4(sk + (size_t)(iv * Ge::bv + jv) * ld + ik * Ge::bk + jk, acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
  }
}

// ---------------------------------------------------------------------------
// fused forward for the layer's default regime (a compaction after every
// 16-token window: K_c = P = 16): one workgroup per chain walks all of a
// call's windows, each a window step followed by its compaction, with the
// window state, the factors and the Kronecker matrix in LDS (no launch or
// global round trip between the two)
// ---------------------------------------------------------------------------
template <typename CT, int D>
struct G3FusedSmem {
  static constexpr int P = kSC;
  union alignas(16) Phase {
    G3Compact<D, P, false> cs;          // the compaction's scratch
    struct alignas(16) Win {            // the window step's
      CT x[3 * kSC][D + 8];             // x, u and the scalars first: the next window's commit
      float u[kSC][D + 4];              // writes them while the compaction still uses all of
      float G[kSC], alpha[kSC], lg[kSC], kco[kSC], qco[kSC], gam[kSC], vsc[kSC];   // its LDS but R_mat
      alignas(16) float kr[2 * kSC][D + 4];
      float pp[4][kSC][kSC + 4];
      float po[2][kSC][P + 4];
      CT skron[D][D + 8];               // rebuilt from the factors after every compaction
    } w;
  } ph;
  alignas(16) float ab[kAB];            // A | B of this chain
  alignas(16) float uwin[P][D + 4];     // the window's net writes (slot-major)
  alignas(16) float vbd[P][D + 4];      // its keys, decayed to now
  alignas(16) CT vbx[sizeof(CT) == 4 ? 1 : P][D + 8];
  float boff[1];
};
template <typename CT, int D>
constexpr bool fused_fits() { return sizeof(G3FusedSmem<CT, D>) <= 160 * 1024; }

template <typename CT, int D>
__global__ void __launch_bounds__(kNT) gdn3_fused_kernel(G3FwdArgs p) {
  constexpr int P = kSC;
  typedef G3FusedSmem<CT, D> Sm;
  __shared__ Sm sm;
  static_assert(sizeof(Sm) <= 160 * 1024, "LDS budget");
  typedef G3D<D> Ge;
  constexpr int Rm = Ge::R * Ge::m, Rn = Ge::R * Ge::n, VPW = (D / 16 + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), g4 = lane >> 4, n16 = lane & 15;
  const int N = p.B * p.H * p.M;
  const int chain = xcd_remap(blockIdx.x, N);
  const G3Tok tk(p, chain, D);
  const int DG = D / 8, ui = tid / DG, ud = 8 * (tid % DG);
  const bool has_unit = tid < kSC * DG;

  // the call's sub-chunks, each its own compaction interval
  const long long tend = (long long)p.t0 + p.T;
  const int cg0 = p.t0 / kSC, cg1 = (int)((tend + kSC - 1) / kSC);
  const bool carried = p.A0 != nullptr;
  G3Raw<CT> raw;
  g3_fetch<CT>(p, tk, raw, cg0 * kSC + ui - p.t0, has_unit, ud);

  // initial state: the carried one (A0, B0 [N][R m|n], U0, Vb0 [N][D][P]) or zero
  const size_t cb = (size_t)chain * D * P;
  for (int e = tid; e < Rm; e += kNT) sm.ab[e] = carried ? p.A0[(size_t)chain * Rm + e] : 0.f;
  for (int e = tid; e < Rn; e += kNT) sm.ab[Rm + e] = carried ? p.B0[(size_t)chain * Rn + e] : 0.f;
  for (int e = tid; e < D * P; e += kNT) {
    const int d = e / P, j = e % P;
    const float uv = carried ? p.U0[cb + e] : 0.f, kv = carried ? p.Vb0[cb + e] : 0.f;
    sm.uwin[j][d] = uv;
    sm.vbd[j][d] = kv;
    if constexpr (sizeof(CT) == 2) sm.vbx[j][d] = from_f<CT>(kv);
  }
  if (tid == 0) sm.boff[0] = 0.f;
  __syncthreads();
  if (carried) write_skron<D, CT>(&sm.ph.w.skron[0][0], sm.ab, sm.ab + Rm, tid, D + 8);
  bool live = carried;
  bool committed = false;   // the window's token rows were committed during the last compaction
  typedef typename Sm::Phase::Win WinT;
  constexpr bool kEarly = offsetof(WinT, skron) <= sizeof(sm.ph.cs.rm);   // x .. po inside R_mat's LDS
  G3Raw<CT> raw2;
  float gacc = 0.f;
  int event = 0;
  const G3WinView<CT, D, P> w{sm.ph.w.x, sm.ph.w.u, sm.ph.w.kr, sm.ph.w.pp, sm.ph.w.po, sm.ph.w.skron, sm.vbd,
                              sm.vbx, sm.ph.w.G, sm.ph.w.alpha, sm.ph.w.lg, sm.ph.w.kco, sm.ph.w.qco,
                              sm.ph.w.gam, sm.ph.w.vsc, sm.boff};
  f32x4 uo[1][VPW];
  // the chain's sketch, the same at every compaction, held from here (a load
  // per compaction waited, in order, for the window's output stores before it)
  G3Sketch<D> sk;
  g3_sketch_load<D>(sk, p.sketch + (size_t)chain * Ge::n * (p.cmode ? Ge::R : Ge::q), p.cmode ? Ge::R : Ge::q, tid);
  // (passed through an empty asm here, so that the loop sees register values,
  // not loads it would wait for at every use)
#pragma unroll
  for (int u = 0; u < G3Sketch<D>::N; ++u) sk.v[u] = __int_as_float(opaque(__float_as_int(sk.v[u])));
  for (int c = cg0; c < cg1; ++c) {
    // the window step (its net writes through the registers of their waves)
#pragma unroll
    for (int a = 0; a < VPW; ++a)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int vt = wave + 4 * a;
        uo[0][a][s] = vt < D / 16 ? sm.uwin[4 * g4 + s][vt * 16 + n16] : 0.f;
      }
    g3_window_step<CT, D, P, 1>(w, p, tk, chain, 0, c, true, -1, live, gacc, uo, raw, committed);
#pragma unroll
    for (int a = 0; a < VPW; ++a)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int vt = wave + 4 * a;
        if (vt < D / 16) sm.uwin[4 * g4 + s][vt * 16 + n16] = uo[0][a][s];
      }
    const bool complete = (long long)(c + 1) * kSC <= tend;
    __syncthreads();
    if (!complete) break;   // the tail: no compaction follows
    // its compaction (gdn3/gdn3_upgrade.py:650-719), the factors decayed by e^{gacc}
    const int qs = p.cmode ? Ge::R : Ge::q;
    // the next window's token loads and their commit run in the eigen-solve's
    // shadow when that window's commit targets lie in R_mat's LDS (dead by then)
    const bool pre = kEarly && p.cmode == 0 && c + 1 < cg1;
    // (waves 1..3, all of the next window's state-independent half; nothing
    // is added to the eigen-solve's wave)
    auto issue = [&]() {};
    auto commit = [&]() {
      if (pre && wave > 0) g3_stage_a_shadow<CT, D, P>(w, p, tk, raw, raw2, c + 1, wave, lane);
    };
    g3_compact<D, P>(sm.ph.cs, sm.ab, &sm.uwin[0][0], &sm.vbd[0][0], (size_t)(D + 4), (size_t)1, gacc, p.sdec,
                     p.sketch + (size_t)chain * Ge::n * qs,
                     p.stats ? p.stats + ((size_t)event * N + chain) * 2 : nullptr, tid, p.cmode, issue, commit, &sk);
    __syncthreads();
    if (p.train_states) {   // the factors after every compaction, for the backward
      const G3Stash ts = g3_stash(p.train_states, N, p.nch, p.T / p.Kc, D, kSC, Ge::RMN);
      for (int e = tid; e < Rm + Rn; e += kNT) ts.ab[((size_t)event * N + chain) * Ge::RMN + e] = sm.ab[e];
    }
    ++event;
    gacc = 0.f;
    live = true;
    if (c + 1 < cg1) {   // the next window's loads (under the Kronecker matrix's rebuild), unless committed
      if (!pre) g3_fetch<CT>(p, tk, raw, (c + 1) * kSC + ui - p.t0, has_unit, ud);
      write_skron<D, CT>(&sm.ph.w.skron[0][0], sm.ab, sm.ab + Rm, tid, D + 8);
    }
    committed = pre;
  }
  __syncthreads();
  // the final state: U, Vb [N][D][P]; A, B (decayed since the last compaction)
  const float dk = expf(gacc);
  for (int e = tid; e < D * P; e += kNT) {
    const int d = e / P, j = e % P;
    if (p.U_out) p.U_out[cb + e] = sm.uwin[j][d];
    if (p.Vb_out) p.Vb_out[cb + e] = sm.vbd[j][d];
  }
  if (p.A_out)
    for (int e = tid; e < Rm; e += kNT) p.A_out[(size_t)chain * Rm + e] = sm.ab[e] * dk;
  if (p.B_out)
    for (int e = tid; e < Rn; e += kNT) p.B_out[(size_t)chain * Rn + e] = sm.ab[Rm + e] * dk;
}

// One chain's compaction; bi indexes the statistics (the chain's row in the
// launch).
template <int D, int P, typename CT>
__device__ __forceinline__ void compact_chain(const G3CompactArgs& p, G3CompactSmem<D, P>& sm, int chain, int bi,
                                              int tid) {
  typedef G3D<D> Ge;
  constexpr int Rm = Ge::R * Ge::m, Rn = Ge::R * Ge::n;
  for (int e = tid; e < Rm; e += kNT) sm.ab[e] = p.A[(size_t)chain * Rm + e];
  for (int e = tid; e < Rn; e += kNT) sm.ab[Rm + e] = p.Bf[(size_t)chain * Rn + e];
  const size_t cb = (size_t)chain * D * P;
  const float gacc = p.gsum ? p.gsum[chain] : 0.f;
  __syncthreads();
  const int qs = p.mode ? Ge::R : Ge::q;   // sketch columns
  g3_compact<D, P>(sm.k, sm.ab, p.U + cb, p.Vb + cb, (size_t)p.u_sp, (size_t)p.u_sd, gacc, p.sdec, p.sketch + (size_t)chain * Ge::n * qs,
                   p.stats ? p.stats + (size_t)bi * 2 : nullptr, tid, p.mode);
  for (int e = tid; e < Rm; e += kNT) {
    p.A_out[(size_t)chain * Rm + e] = sm.ab[e];
    if (p.A_fin) p.A_fin[(size_t)chain * Rm + e] = sm.ab[e];
  }
  for (int e = tid; e < Rn; e += kNT) {
    p.B_out[(size_t)chain * Rn + e] = sm.ab[Rm + e];
    if (p.B_fin) p.B_fin[(size_t)chain * Rn + e] = sm.ab[Rm + e];
  }
  if (p.ab_stash)
    for (int e = tid; e < Rm + Rn; e += kNT) p.ab_stash[(size_t)chain * (Rm + Rn) + e] = sm.ab[e];
  if (p.skron) write_skron<D, CT>((CT*)p.skron + (size_t)chain * D * D, sm.ab, sm.ab + Rm, tid);
}

template <int D, int P, typename CT>
__global__ void __launch_bounds__(kNT) gdn3_compact_kernel(G3CompactArgs p) {
  __shared__ G3CompactSmem<D, P> sm;
  static_assert(sizeof(G3CompactSmem<D, P>) <= 160 * 1024, "LDS budget");
  const int tid = threadIdx.x;
  if (!p.pos) {
    compact_chain<D, P, CT>(p, sm, blockIdx.x, blockIdx.x, tid);
    return;
  }
  // decode batch: only the rows whose token closes a compaction interval.
  // The chains are strided over a grid of at most kDecCompactGrid
  // workgroups; a workgroup's threads check up to kNT of its chains at once
  // and list those that compact (the order of the list does not matter:
  // the chains are independent), so a step that closes no interval costs
  // one round of position reads.
  __shared__ int todo[kNT];
  __shared__ int ntodo;
  const int K = (p.N - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;   // this workgroup's chains
  for (int base = 0; base < K; base += kNT) {
    if (tid == 0) ntodo = 0;
    __syncthreads();
    if (base + tid < K) {
      const int bi = blockIdx.x + (base + tid) * gridDim.x;
      const int row = bi / p.hm;
      const int pos = p.pos[row];
      bool go = pos >= 0 && (pos + 1) % p.Kc == 0;   // (a negative position is an empty row)
      if (go && p.slots) {
        const int sl = p.slots[row];
        go = sl >= 0 && sl < p.nslots;
      }
      if (go) todo[atomicAdd(&ntodo, 1)] = bi;
    }
    __syncthreads();
    const int n = ntodo;
    for (int i = 0; i < n; ++i) {
      const int bi = todo[i];
      const int chain = p.slots ? p.slots[bi / p.hm] * p.hm + bi % p.hm : bi;
      compact_chain<D, P, CT>(p, sm, chain, bi, tid);
      __syncthreads();   // the chain's last LDS reads before the next one's loads
    }
  }
}

// The carried state (A0, B0, U0, Vb0 in the output layouts) in the window
// kernel's workspace form: the factors, their Kronecker matrix, the window's
// writes and keys slot-major, and no decay accumulated since the factors.
template <int D, int P, typename CT>
__global__ void __launch_bounds__(kNT) gdn3_state_in_kernel(G3FwdArgs p) {
  typedef G3D<D> Ge;
  constexpr int Rm = Ge::R * Ge::m, Rn = Ge::R * Ge::n;
  __shared__ float ab[Rm + Rn];
  const int tid = threadIdx.x, chain = blockIdx.x;
  const int N = p.B * p.H * p.M;
  for (int e = tid; e < Rm; e += kNT) {
    const float a = p.A0[(size_t)chain * Rm + e];
    ab[e] = a;
    p.ab[(size_t)chain * Rm + e] = a;
  }
  for (int e = tid; e < Rn; e += kNT) {
    const float b = p.B0[(size_t)chain * Rn + e];
    ab[Rm + e] = b;
    p.ab[(size_t)N * Rm + (size_t)chain * Rn + e] = b;
  }
  // [D][P] -> [P][D]: consecutive threads read consecutive (d, slot) entries
  const size_t cb = (size_t)chain * D * P;
  for (int e = tid; e < D * P; e += kNT) {
    const int d = e / P, j = e % P;
    p.uw[cb + (size_t)j * D + d] = p.U0[cb + e];
    p.vw[cb + (size_t)j * D + d] = p.Vb0[cb + e];
  }
  if (tid == 0) p.gsum[chain] = 0.f;
  __syncthreads();
  write_skron<D, CT>((CT*)p.skron + (size_t)chain * D * D, ab, ab + Rm, tid);
}

__global__ void fill_zero_kernel(float* p, long long n) {
  for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (long long)gridDim.x * blockDim.x)
    p[e] = 0.f;
}

// ---------------------------------------------------------------------------
// Kronecker read S x = vec(sum_r A_r X B_r^T) + U (Vb^T x), X = x as [a_k, b_k]
// (gdn3/gdn3_upgrade.py:626-639; identity of gdn3/kernels.py:7-16)
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kNT) kron_read_kernel(KronReadArgs p) {
  __shared__ float xs[D];
  __shared__ float zs[kRMax * kMN];  // Z_r[iv][jk] = sum_ik A_r[iv][ik] X[ik][jk]
  __shared__ float cp[64];           // Vb_p . x
  const int tid = threadIdx.x;
  const int row = blockIdx.x;  // (chain, c)
  const int chain = row / p.C;
  const G3Geom ge = p.ge;
  const int P = p.P;
  const float* x = p.x + (size_t)row * D;
  const float* A = p.A + (size_t)chain * ge.R * ge.m;
  const float* Bf = p.Bf + (size_t)chain * ge.R * ge.n;
  const float* U = p.U + (size_t)chain * D * P;
  const float* Vb = p.Vb + (size_t)chain * D * P;
  if (tid < D) xs[tid] = x[tid];
  __syncthreads();
  const int nz = ge.R * ge.av * ge.bk;
  for (int e = tid; e < nz; e += kNT) {
    const int r = e / (ge.av * ge.bk), rem = e % (ge.av * ge.bk), iv = rem / ge.bk, jk = rem % ge.bk;
    float s = 0.f;
    for (int ik = 0; ik < ge.ak; ++ik) s += A[(r * ge.av + iv) * ge.ak + ik] * xs[ik * ge.bk + jk];
    zs[e] = s;
  }
  for (int pp = tid; pp < P; pp += kNT) {
    float s = 0.f;
    for (int k = 0; k < D; ++k) s += Vb[k * P + pp] * xs[k];
    cp[pp] = s;
  }
  __syncthreads();
  if (tid < D) {
    const int v = tid, iv = v / ge.bv, jv = v % ge.bv;
    float s = 0.f;
    for (int r = 0; r < ge.R; ++r)
      for (int jk = 0; jk < ge.bk; ++jk)
        s += zs[(r * ge.av + iv) * ge.bk + jk] * Bf[(r * ge.bv + jv) * ge.bk + jk];
    for (int pp = 0; pp < P; ++pp) s += U[v * P + pp] * cp[pp];
    p.y[(size_t)row * D + v] = s;
  }
}

// Workgroups of a decode batch's compaction launch (grid-stride over chains).
constexpr int kDecCompactGrid = 2048;

template <int D, int P>
int launch_compact(const G3CompactArgs& a, hipStream_t stream) {
  const int grid = a.pos ? (a.N < kDecCompactGrid ? a.N : kDecCompactGrid) : a.N;
  if (a.skron && a.skron_dtype == GDNX_DTYPE_BF16)
    hipLaunchKernelGGL((gdn3_compact_kernel<D, P, bf16>), dim3(grid), dim3(kNT), 0, stream, a);
  else
    hipLaunchKernelGGL((gdn3_compact_kernel<D, P, float>), dim3(grid), dim3(kNT), 0, stream, a);
  return check_launch("gdn3_compact_kernel");
}

int compact_dispatch(const G3CompactArgs& a, hipStream_t stream) {
  if (a.N == 0) return GDNX_OK;
  if (a.D == 128 && a.P == 16) return launch_compact<128, 16>(a, stream);
  if (a.D == 128 && a.P == 32) return launch_compact<128, 32>(a, stream);
  if (a.D == 128 && a.P == 64) return launch_compact<128, 64>(a, stream);
  if (a.D == 64 && a.P == 16) return launch_compact<64, 16>(a, stream);
  if (a.D == 64 && a.P == 32) return launch_compact<64, 32>(a, stream);
  if (a.D == 64 && a.P == 64) return launch_compact<64, 64>(a, stream);
  return set_error(GDNX_ERR_SHAPE, "gdn3_compact: unsupported head_dim %d / P %d", a.D, a.P);
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// value split: ~512 workgroups, two per CU (NVB workgroups per chain, at
// least one value tile each), or the smallest larger split whose LDS fits
// The pipelined window kernel for intervals of several sub-chunks: the
// value split whose workgroups all run at once (at most two per CU, as LDS
// allows) with the fewest rounds, the widest among equals
int cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

template <typename CT, int D, int P, int NVB>
void pipe_score(int N, int& best_nvb, long long& best_rounds) {
  constexpr size_t lds = pipe_lds<CT, D, P, NVB>();
  if constexpr (lds <= 160 * 1024) {
    const int per_cu = lds <= 80 * 1024 ? 2 : 1;
    const long long cap = (long long)cu_count() * per_cu, wgs = (long long)N * NVB;
    const long long rounds = (wgs + cap - 1) / cap;
    if (rounds <= best_rounds) {
      best_rounds = rounds;
      best_nvb = NVB;
    }
  }
}

template <typename CT, int D, int P, int NVB>
void pipe_launch(const G3FwdArgs& a, int N, hipStream_t stream) {
  if (a.gate_ch > 1)
    hipLaunchKernelGGL((gdn3_window_pipe_kernel<CT, D, P, NVB, 2>), dim3(N * NVB), dim3(kNT), 0, stream, a);
  else
    hipLaunchKernelGGL((gdn3_window_pipe_kernel<CT, D, P, NVB, 1>), dim3(N * NVB), dim3(kNT), 0, stream, a);
}

template <typename CT, int D, int P>
int launch_pipe(const G3FwdArgs& a, int N, hipStream_t stream) {
  constexpr int V2 = D / 16 < 2 ? D / 16 : 2, V4 = D / 16 < 4 ? D / 16 : 4, V8 = D / 16 < 8 ? D / 16 : 8;
  int nvb = 0;
  long long rounds = 1LL << 62;
  pipe_score<CT, D, P, 1>(N, nvb, rounds);
  pipe_score<CT, D, P, V2>(N, nvb, rounds);
  pipe_score<CT, D, P, V4>(N, nvb, rounds);
  pipe_score<CT, D, P, V8>(N, nvb, rounds);
  if constexpr (pipe_lds<CT, D, P, 1>() <= 160 * 1024)
    if (nvb == 1) pipe_launch<CT, D, P, 1>(a, N, stream);
  if constexpr (V2 != 1 && pipe_lds<CT, D, P, V2>() <= 160 * 1024)
    if (nvb == V2) pipe_launch<CT, D, P, V2>(a, N, stream);
  if constexpr (V4 != V2 && pipe_lds<CT, D, P, V4>() <= 160 * 1024)
    if (nvb == V4) pipe_launch<CT, D, P, V4>(a, N, stream);
  if constexpr (V8 != V4 && pipe_lds<CT, D, P, V8>() <= 160 * 1024)
    if (nvb == V8) pipe_launch<CT, D, P, V8>(a, N, stream);
  if (nvb == 0) return set_error(GDNX_ERR_SHAPE, "gdn3: no window split fits LDS");
  return check_launch("gdn3_window_pipe_kernel");
}

template <typename CT, int D, int P>
int launch_window(const G3FwdArgs& a, int N, hipStream_t stream) {
  // intervals of several sub-chunks overlap one sub-chunk's algebra with the
  // next one's grams and inverse
  if (a.c1 - a.c0 >= 3) return launch_pipe<CT, D, P>(a, N, stream);
  constexpr int V2 = D / 16 < 2 ? D / 16 : 2, V4 = D / 16 < 4 ? D / 16 : 4, V8 = D / 16 < 8 ? D / 16 : 8;
  static_assert(win_fits<CT, D, P, V8>(), "the widest split fits");
  const int nvb = N >= 512 ? 1 : N >= 256 ? V2 : N >= 128 ? V4 : V8;
  bool done = false;
  if constexpr (win_fits<CT, D, P, 1>())
    if (!done && nvb <= 1) {
      hipLaunchKernelGGL((gdn3_window_kernel<CT, D, P, 1>), dim3(N), dim3(kNT), 0, stream, a);
      done = true;
    }
  if constexpr (win_fits<CT, D, P, V2>())
    if (!done && nvb <= V2) {
      hipLaunchKernelGGL((gdn3_window_kernel<CT, D, P, V2>), dim3(N * V2), dim3(kNT), 0, stream, a);
      done = true;
    }
  if constexpr (win_fits<CT, D, P, V4>())
    if (!done && nvb <= V4) {
      hipLaunchKernelGGL((gdn3_window_kernel<CT, D, P, V4>), dim3(N * V4), dim3(kNT), 0, stream, a);
      done = true;
    }
  if (!done) hipLaunchKernelGGL((gdn3_window_kernel<CT, D, P, V8>), dim3(N * V8), dim3(kNT), 0, stream, a);
  return check_launch("gdn3_window_kernel");
}

template <typename CT, int D, int P>
int run_gdn3_fwd(G3FwdArgs a, hipStream_t stream) {
  typedef G3D<D> Ge;
  const int N = a.B * a.H * a.M;
  if constexpr (P == kSC && fused_fits<CT, D>()) {
    if (a.Kc == kSC) {   // the layer's default regime: one fused launch for the whole call
      a.nch = (a.T + kSC - 1) / kSC;
      G3Stash ts{nullptr, nullptr, nullptr};
      if (a.train_states) ts = g3_stash(a.train_states, N, a.nch, a.T / a.Kc, D, kSC, Ge::RMN);
      a.ts_u = ts.u;
      a.ts_g = ts.gacc;
      hipLaunchKernelGGL((gdn3_fused_kernel<CT, D>), dim3(N), dim3(kNT), 0, stream, a);
      return check_launch("gdn3_fused_kernel");
    }
  }
  char* w = (char*)a.workspace;
  a.skron = w;
  w += align256((size_t)N * D * D * sizeof(CT));
  a.ab = (float*)w;
  w += align256((size_t)N * Ge::R * (Ge::m + Ge::n) * 4);
  a.uw = (float*)w;
  w += align256((size_t)N * P * D * 4);
  a.vw = (float*)w;
  w += align256((size_t)N * P * D * 4);
  a.gsum = (float*)w;
  const bool carried = a.A0 != nullptr;
  int rc;
  if (carried) {
    hipLaunchKernelGGL((gdn3_state_in_kernel<D, P, CT>), dim3(N), dim3(kNT), 0, stream, a);
    rc = check_launch("gdn3_state_in_kernel");
  } else {
    const long long nab = (long long)N * Ge::R * (Ge::m + Ge::n);
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((nab + 255) / 256 < 4096 ? (nab + 255) / 256 : 4096)),
                       dim3(256), 0, stream, a.ab, nab);
    rc = check_launch("fill_zero_kernel");
  }
  if (rc) return rc;
  // sub-chunks are global: sub-chunk c covers tokens [16 c, 16 c + 16) of
  // the whole sequence, of which this call holds [t0, t0 + T)
  const long long tend = (long long)a.t0 + a.T;
  const int cg0 = a.t0 / kSC, cg1 = (int)((tend + kSC - 1) / kSC);
  a.nch = (a.T + kSC - 1) / kSC;
  G3Stash ts{nullptr, nullptr, nullptr};
  if (a.train_states) ts = g3_stash(a.train_states, N, a.nch, a.T / a.Kc, D, kSC, Ge::RMN);
  a.ts_u = ts.u;
  a.ts_g = ts.gacc;
  const int per = a.Kc / kSC;
  int event = 0;
  bool first = true;
  for (int c0 = cg0; c0 < cg1;) {
    int c1 = (c0 / per + 1) * per;   // the next compaction boundary
    if (c1 > cg1) c1 = cg1;
    a.c0 = c0;
    a.c1 = c1;
    a.first = first && !carried;     // zero window state
    a.live = !first || carried;      // the Kronecker factors may be nonzero
    a.last = c1 == cg1;
    a.complete = (long long)c1 * kSC <= tend && c1 % per == 0;
    if ((rc = launch_window<CT, D, P>(a, N, stream))) return rc;
    if (a.complete) {
      G3CompactArgs ca{};
      ca.A = a.ab;
      ca.Bf = a.ab + (size_t)N * Ge::R * Ge::m;
      ca.U = a.uw;
      ca.Vb = a.vw;
      ca.sketch = a.sketch;
      ca.A_out = a.ab;
      ca.B_out = a.ab + (size_t)N * Ge::R * Ge::m;
      ca.stats = a.stats ? a.stats + (size_t)event * N * 2 : nullptr;
      ca.ge = a.ge;
      ca.N = N;
      ca.D = D;
      ca.P = P;
      ca.sdec = a.sdec;
      ca.u_sp = D;
      ca.u_sd = 1;
      ca.gsum = a.gsum;
      ca.skron = a.skron;
      ca.skron_dtype = a.dtype;
      ca.A_fin = a.last ? a.A_out : nullptr;
      ca.B_fin = a.last ? a.B_out : nullptr;
      ca.ab_stash = ts.ab ? ts.ab + (size_t)event * N * Ge::RMN : nullptr;
      ca.mode = a.cmode;
      if ((rc = compact_dispatch(ca, stream))) return rc;
      ++event;
    }
    first = false;
    c0 = c1;
  }
  return GDNX_OK;
}

}  // namespace

// Static scratch for gdnx_gdn3_chunk_fwd_state_noalloc: the forward's
// workspace (Kronecker matrices, factors, window state) for callers that
// cannot allocate (graph capture, serving loops).  Each device the library
// runs on holds its own copy for the life of the process; host code reaches
// it only through the address hipGetSymbolAddress returns for that device.
static __device__ __align__(256) unsigned char scratch[kG3ScratchBytes];

namespace {
std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int gdn3_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(GDNX_ERR_HIP, "no current HIP device (or device index >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(GDNX_ERR_HIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GDNX_OK;
}

int gdn3_zero_fill(float* p, size_t n, hipStream_t stream) {
  if (n == 0) return GDNX_OK;
  const size_t nb = (n + 255) / 256;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)(nb < 4096 ? nb : 4096)), dim3(256), 0, stream, p,
                     (long long)n);
  return check_launch("fill_zero_kernel");
}

size_t gdn3_workspace_bytes(int N, int D, int P, int dtype) {
  const size_t cb = dtype == GDNX_DTYPE_BF16 ? 2 : 4;
  const int R = 4, mn = D == 128 ? 256 + 64 : 64 + 64;
  return align256((size_t)N * D * D * cb) + align256((size_t)N * R * mn * 4) + 2 * align256((size_t)N * P * D * 4) +
         align256((size_t)N * 4);
}

size_t gdn3_train_states_bytes(int N, int T, int D, int P, int Kc) {
  (void)P;   // the stash is kept per 16-token sub-chunk whatever the window
  const int nch = (T + kSC - 1) / kSC, ncomp = T / Kc;
  const int rmn = D == 128 ? G3D<128>::RMN : G3D<64>::RMN;
  return g3_stash_bytes(N, nch, ncomp, D, kSC, rmn);
}

// whether run_gdn3_fwd runs the call as one fused launch, which uses no
// workspace (the layer's default regime, a compaction after every window)
bool gdn3_fwd_fused(int D, int P, int Kc, int dtype) {
  if (P != kSC || Kc != kSC) return false;
  if (dtype == GDNX_DTYPE_BF16) return D == 128 ? fused_fits<bf16, 128>() : D == 64 && fused_fits<bf16, 64>();
  return D == 128 ? fused_fits<float, 128>() : D == 64 && fused_fits<float, 64>();
}

int gdn3_fwd_dispatch(const G3FwdArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.P == 16) return run_gdn3_fwd<bf16, 128, 16>(a, stream);
    if (a.D == 128 && a.P == 32) return run_gdn3_fwd<bf16, 128, 32>(a, stream);
    if (a.D == 128 && a.P == 64) return run_gdn3_fwd<bf16, 128, 64>(a, stream);
    if (a.D == 64 && a.P == 16) return run_gdn3_fwd<bf16, 64, 16>(a, stream);
    if (a.D == 64 && a.P == 32) return run_gdn3_fwd<bf16, 64, 32>(a, stream);
    if (a.D == 64 && a.P == 64) return run_gdn3_fwd<bf16, 64, 64>(a, stream);
  } else {
    if (a.D == 128 && a.P == 16) return run_gdn3_fwd<float, 128, 16>(a, stream);
    if (a.D == 128 && a.P == 32) return run_gdn3_fwd<float, 128, 32>(a, stream);
    if (a.D == 128 && a.P == 64) return run_gdn3_fwd<float, 128, 64>(a, stream);
    if (a.D == 64 && a.P == 16) return run_gdn3_fwd<float, 64, 16>(a, stream);
    if (a.D == 64 && a.P == 32) return run_gdn3_fwd<float, 64, 32>(a, stream);
    if (a.D == 64 && a.P == 64) return run_gdn3_fwd<float, 64, 64>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "gdn3: unsupported head_dim %d / P %d (64 or 128 / 16, 32 or 64)", a.D, a.P);
}

int gdn3_compact_dispatch(const G3CompactArgs& a, hipStream_t stream) { return compact_dispatch(a, stream); }

int kron_read_dispatch(const KronReadArgs& a, hipStream_t stream) {
  if ((long long)a.N * a.C == 0) return GDNX_OK;
  if (a.D == 128)
    hipLaunchKernelGGL((kron_read_kernel<128>), dim3(a.N * a.C), dim3(kNT), 0, stream, a);
  else if (a.D == 64)
    hipLaunchKernelGGL((kron_read_kernel<64>), dim3(a.N * a.C), dim3(kNT), 0, stream, a);
  else
    return set_error(GDNX_ERR_SHAPE, "kron_read: unsupported head_dim %d", a.D);
  return check_launch("kron_read_kernel");
}

}  // namespace gdnx

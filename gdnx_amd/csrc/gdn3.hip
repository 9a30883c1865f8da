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
#include "delta_common.hpp"
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int kRMax = 4;    // Kronecker rank bound
constexpr int kQ = 8;       // sketch width bound: min(R + 4, m, n) <= 8
constexpr int kMN = 256;    // bound on m = a_v a_k and n = b_v b_k
constexpr int kAB = 1280;   // bound on R (m + n) for m n = d^2, m, n <= 256
constexpr int kNT = 256;

__device__ __forceinline__ float stable_alpha_f(float c) {
  // (1 - e^{-c}) / c with its series near 0 (gdn3/gdn3_upgrade.py:641-648)
  if (fabsf(c) < 1e-6f) return 1.f - 0.5f * c + c * c * (1.f / 6.f);
  return -expm1f(-c) / c;
}

__device__ __forceinline__ float log_decay(float d) {
  // clamp(dec, 0, 1) as a natural-log decay, floored at kLogFloor
  d = fminf(d, 1.f);
  return d > 0.f ? fmaxf(logf(d), kLogFloor) : kLogFloor;
}

// Sum of NV doubles over the 256 threads of the block, in a fixed order;
// every thread receives the totals.  red: 4 * NV doubles of LDS.
template <int NV>
__device__ __forceinline__ void block_sum(double (&v)[NV], double* red, int tid) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int e = 0; e < NV; ++e) v[e] += __shfl_xor(v[e], off, 64);
  if ((tid & 63) == 0)
#pragma unroll
    for (int e = 0; e < NV; ++e) red[(tid >> 6) * NV + e] = v[e];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < NV; ++e) v[e] = (red[e] + red[NV + e]) + (red[2 * NV + e] + red[3 * NV + e]);
  __syncthreads();
}

// LDS of one compaction.
template <int D, int P>
struct G3Compact {
  alignas(16) float rm[D * D + kMN];        // R_mat: m rows of n + 1 floats
  alignas(16) double y[kMN * kQ];           // range basis, rows of kQ
  alignas(16) double z[kMN * kQ];           // R_mat^T Y (rows of kQ), then Bm = Q^T R_mat [kQ][n]
  alignas(16) float gs[kMN * kQ];           // sketch, rows of kQ (zero padded)
  alignas(16) float ut[P][D + 4];           // window net writes U_p
  alignas(16) double us[kRMax][kMN];        // leading left singular vectors of R_mat
  alignas(16) double vs[kRMax][kMN];        // leading right singular vectors
  double red[4 * 64];
  double lmat[kQ * kQ];         // Cholesky factor L (row-major), L^T = R
  double ev[kQ * kQ];           // eigenvectors of Bm Bm^T (columns)
  double lam[kQ];
  double sig[kRMax];
  double amax[4][kRMax];
  double sgn[kRMax];
  int aidx[4][kRMax];
  int order[kQ];
};

// Jacobi rotation zeroing a_pq (Numerical Recipes convention):
// J[p][p] = J[q][q] = c, J[p][q] = s, J[q][p] = -s.
__device__ __forceinline__ void jacobi_rot(double app, double aqq, double apq, double& c, double& s) {
  if (apq == 0.0) {
    c = 1.0;
    s = 0.0;
    return;
  }
  const double th = (aqq - app) / (2.0 * apq);
  double t;
  if (fabs(th) > 1e150) t = 0.5 / th;
  else t = (th >= 0.0 ? 1.0 : -1.0) / (fabs(th) + sqrt(th * th + 1.0));
  c = 1.0 / sqrt(t * t + 1.0);
  s = t * c;
}

// Round-robin (circle method) partner of index x in round st of 7 for 8 indices.
__device__ __forceinline__ int rr_partner(int x, int st) {
  if (x == 7) return st;
  if (x == st) return 7;
  return (2 * st - x + 14) % 7;
}

// Y <- Y R^{-1} with Y^T Y = R^T R (Cholesky QR, applied twice).  Columns
// whose pivot falls below 1e-24 of the largest diagonal are set to zero.
template <int D, int P>
__device__ void orth_rows(G3Compact<D, P>& cs, int m, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int seg = (m + 3) / 4;
  for (int pass = 0; pass < 2; ++pass) {
    {  // Gram, 4 row segments
      const int i = lane >> 3, j = lane & 7;
      const int r0 = wave * seg, r1 = min(m, r0 + seg);
      double s = 0.0;
      for (int row = r0; row < r1; ++row) s += cs.y[row * kQ + i] * cs.y[row * kQ + j];
      cs.red[wave * 64 + lane] = s;
    }
    __syncthreads();
    if (wave == 0) {
      const int i = lane >> 3, j = lane & 7;
      double a = (cs.red[lane] + cs.red[64 + lane]) + (cs.red[128 + lane] + cs.red[192 + lane]);
      double dmax = 0.0;
#pragma unroll
      for (int k = 0; k < kQ; ++k) dmax = fmax(dmax, __shfl(a, 9 * k, 64));
      const double tol = dmax * 1e-24;
#pragma unroll
      for (int k = 0; k < kQ; ++k) {
        const double akk = __shfl(a, 9 * k, 64);
        const double aik = __shfl(a, 8 * i + k, 64);
        const double ajk = __shfl(a, 8 * j + k, 64);
        const double d = (akk > tol && akk > 0.0) ? sqrt(akk) : 0.0;
        const double lik = d > 0.0 ? aik / d : 0.0, ljk = d > 0.0 ? ajk / d : 0.0;
        if (i > k && j > k) a -= lik * ljk;
        if (j == k && i >= k) a = (i == k) ? d : lik;  // column k becomes L[:, k]
      }
      cs.lmat[lane] = (j <= i) ? a : 0.0;  // L[i][j]
    }
    __syncthreads();
    if (tid < m) {
      double yr[kQ], qn[kQ];
#pragma unroll
      for (int j = 0; j < kQ; ++j) yr[j] = cs.y[tid * kQ + j];
      // q R = y with R[i][j] = L[j][i]
#pragma unroll
      for (int j = 0; j < kQ; ++j) {
        double s = yr[j];
#pragma unroll
        for (int i = 0; i < j; ++i) s -= qn[i] * cs.lmat[j * kQ + i];
        const double rjj = cs.lmat[j * kQ + j];
        qn[j] = rjj > 0.0 ? s / rjj : 0.0;
      }
#pragma unroll
      for (int j = 0; j < kQ; ++j) cs.y[tid * kQ + j] = qn[j];
    }
    __syncthreads();
  }
}

// Compaction of one chain (gdn3/gdn3_upgrade.py:650-719) on LDS inputs:
// ab = [A (R x m) | B (R x n)] as stored (the Kronecker part is decayed by
// e^{gacc} per factor), cs.ut = window net writes [P][D], vbd = window keys
// decayed to now [P][D].  Writes the blended A, B back into ab and, from
// thread 0, stats = (|R_mat|^2, sum of the R kept sigma^2).  Sign
// convention: each (u_r, v_r) pair is flipped so that the largest-magnitude
// entry of v_r is positive (first index on ties).
template <int D, int P>
__device__ void g3_compact(G3Compact<D, P>& cs, float* ab, const float (*vbd)[D + 4], const G3Geom& ge,
                           float gacc, float sdec, const float* __restrict__ sketch, double* stats, int tid) {
  const int R = ge.R, m = ge.m, n = ge.n, q = ge.q, av = ge.av, ak = ge.ak, bv = ge.bv, bk = ge.bk;
  const int ldr = n + 1;
  float* A = ab;
  float* Bv = ab + R * m;
  const int lane = tid & 63, wave = tid >> 6;

  for (int e = tid; e < n * kQ; e += kNT) {
    const int c = e / kQ, j = e % kQ;
    cs.gs[e] = j < q ? sketch[c * q + j] : 0.f;
  }
  // residual part rearrange(U Vb^T), 4x4 register blocks over (v, k)
  for (int blk = tid; blk < (D / 4) * (D / 4); blk += kNT) {
    const int v0 = 4 * (blk / (D / 4)), k0 = 4 * (blk % (D / 4));
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = 0.f;
#pragma unroll 4
    for (int p = 0; p < P; ++p) {
      const f32x4 uu = *(const f32x4*)&cs.ut[p][v0];
      const f32x4 kk = *(const f32x4*)&vbd[p][k0];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] += uu[a] * kk[b];
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int v = v0 + a, iv = v / bv, jv = v % bv;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int k = k0 + b, ik = k / bk, jk = k % bk;
        cs.rm[(iv * ak + ik) * ldr + jv * bk + jk] = acc[a][b];
      }
    }
  }
  __syncthreads();
  // Kronecker part (A, B each decayed by e^{gacc}) and the energy |R_mat|^2
  const float sc2 = expf(2.f * gacc);
  double en[1] = {0.0};
  for (int e = tid; e < m * n; e += kNT) {
    const int row = e / n, col = e % n;
    float s = 0.f;
    for (int r = 0; r < R; ++r) s += A[r * m + row] * Bv[r * n + col];
    const float val = cs.rm[row * ldr + col] + sc2 * s;
    cs.rm[row * ldr + col] = val;
    en[0] += (double)val * (double)val;
  }
  block_sum<1>(en, cs.red, tid);

  // range finder with two power iterations; orthonormalising between the
  // products leaves the final basis unchanged (up to column signs)
  auto mul_rm = [&](const double* zsrc) {  // Y = R_mat Z (zsrc) or R_mat G (null)
    for (int row = tid; row < m; row += kNT) {
      double acc[kQ];
#pragma unroll
      for (int j = 0; j < kQ; ++j) acc[j] = 0.0;
      if (zsrc) {
        for (int c = 0; c < n; ++c) {
          const double r = cs.rm[row * ldr + c];
#pragma unroll
          for (int j = 0; j < kQ; ++j) acc[j] += r * zsrc[c * kQ + j];
        }
      } else {
        for (int c = 0; c < n; ++c) {
          const double r = cs.rm[row * ldr + c];
#pragma unroll
          for (int j = 0; j < kQ; ++j) acc[j] += r * (double)cs.gs[c * kQ + j];
        }
      }
#pragma unroll
      for (int j = 0; j < kQ; ++j) cs.y[row * kQ + j] = acc[j];
    }
    __syncthreads();
  };
  mul_rm(nullptr);
  orth_rows(cs, m, tid);
  for (int it = 0; it < 2; ++it) {
    for (int o = tid; o < n * kQ; o += kNT) {
      const int c = o % n, j = o / n;
      double acc = 0.0;
      for (int row = 0; row < m; ++row) acc += (double)cs.rm[row * ldr + c] * cs.y[row * kQ + j];
      cs.z[c * kQ + j] = acc;
    }
    __syncthreads();
    mul_rm(cs.z);
    orth_rows(cs, m, tid);
  }
  // Bm = Q^T R_mat  [kQ][n]
  for (int o = tid; o < n * kQ; o += kNT) {
    const int c = o % n, j = o / n;
    double acc = 0.0;
    for (int row = 0; row < m; ++row) acc += cs.y[row * kQ + j] * (double)cs.rm[row * ldr + c];
    cs.z[j * n + c] = acc;
  }
  __syncthreads();
  // eigen-decomposition of W = Bm Bm^T by cyclic Jacobi in wave 0
  if (wave == 0) {
    const int i = lane >> 3, j = lane & 7;
    double a = 0.0;
    for (int c = 0; c < n; ++c) a += cs.z[i * n + c] * cs.z[j * n + c];
    double vv = (i == j) ? 1.0 : 0.0;
    for (int sweep = 0; sweep < 12; ++sweep) {
      double off = (i != j) ? a * a : 0.0, dia = (i == j) ? a * a : 0.0;
#pragma unroll
      for (int o2 = 32; o2 > 0; o2 >>= 1) {
        off += __shfl_xor(off, o2, 64);
        dia += __shfl_xor(dia, o2, 64);
      }
      if (!(off > 1e-30 * dia)) break;  // uniform across the wave
      for (int st = 0; st < 7; ++st) {
        const int pi = rr_partner(i, st), pj = rr_partner(j, st);
        double ci, si, cj, sj;
        {
          const int p = min(i, pi), qq = max(i, pi);
          jacobi_rot(__shfl(a, 9 * p, 64), __shfl(a, 9 * qq, 64), __shfl(a, 8 * p + qq, 64), ci, si);
        }
        {
          const int p = min(j, pj), qq = max(j, pj);
          jacobi_rot(__shfl(a, 9 * p, 64), __shfl(a, 9 * qq, 64), __shfl(a, 8 * p + qq, 64), cj, sj);
        }
        // J[i][i] = c; J[pi][i] = -s if i < pi else +s
        const double xi = (i < pi) ? -si : si, xj = (j < pj) ? -sj : sj;
        const double a_ipj = __shfl(a, 8 * i + pj, 64);
        const double a_pij = __shfl(a, 8 * pi + j, 64);
        const double a_pipj = __shfl(a, 8 * pi + pj, 64);
        const double v_ipj = __shfl(vv, 8 * i + pj, 64);
        a = ci * cj * a + ci * xj * a_ipj + xi * cj * a_pij + xi * xj * a_pipj;
        vv = vv * cj + v_ipj * xj;
      }
    }
    cs.ev[lane] = vv;  // ev[i][j]: component i of eigenvector j
    if (i == j) cs.lam[i] = a;
  }
  __syncthreads();
  if (tid < kQ) {  // rank of eigenvalue tid, descending, ties by index
    const double li = cs.lam[tid];
    int rk = 0;
    for (int j = 0; j < kQ; ++j) rk += (cs.lam[j] > li || (cs.lam[j] == li && j < tid)) ? 1 : 0;
    cs.order[rk] = tid;
  }
  __syncthreads();
  if (tid < R) {
    const double l = cs.lam[cs.order[tid]];
    cs.sig[tid] = l > 0.0 ? sqrt(l) : 0.0;
  }
  __syncthreads();
  // leading singular vectors: u_r = Q ev_r, v_r = Bm^T ev_r / sigma_r
  for (int row = tid; row < m; row += kNT)
    for (int r = 0; r < R; ++r) {
      const int o = cs.order[r];
      double s = 0.0;
#pragma unroll
      for (int j = 0; j < kQ; ++j) s += cs.y[row * kQ + j] * cs.ev[j * kQ + o];
      cs.us[r][row] = s;
    }
  for (int c = tid; c < n; c += kNT)
    for (int r = 0; r < R; ++r) {
      const int o = cs.order[r];
      const double sg = cs.sig[r];
      double s = 0.0;
#pragma unroll
      for (int j = 0; j < kQ; ++j) s += cs.z[j * n + c] * cs.ev[j * kQ + o];
      cs.vs[r][c] = sg > 0.0 ? s / sg : (c == r ? 1.0 : 0.0);
    }
  __syncthreads();
  // canonical signs: argmax_c |v_r[c]|, first index on ties
  {
    double bv_[kRMax];
    int bi[kRMax];
#pragma unroll
    for (int r = 0; r < kRMax; ++r) {
      bv_[r] = -1.0;
      bi[r] = 0x7fffffff;
    }
    for (int c = tid; c < n; c += kNT)
#pragma unroll
      for (int r = 0; r < kRMax; ++r)
        if (r < R) {
          const double ad = fabs(cs.vs[r][c]);
          if (ad > bv_[r]) {
            bv_[r] = ad;
            bi[r] = c;
          }
        }
#pragma unroll
    for (int r = 0; r < kRMax; ++r) {
#pragma unroll
      for (int o2 = 32; o2 > 0; o2 >>= 1) {
        const double ov = __shfl_xor(bv_[r], o2, 64);
        const int oi = __shfl_xor(bi[r], o2, 64);
        if (ov > bv_[r] || (ov == bv_[r] && oi < bi[r])) {
          bv_[r] = ov;
          bi[r] = oi;
        }
      }
      if (lane == 0) {
        cs.amax[wave][r] = bv_[r];
        cs.aidx[wave][r] = bi[r];
      }
    }
  }
  __syncthreads();
  if (tid < R) {
    double bv_ = cs.amax[0][tid];
    int bi = cs.aidx[0][tid];
    for (int w = 1; w < 4; ++w) {
      const double ov = cs.amax[w][tid];
      const int oi = cs.aidx[w][tid];
      if (ov > bv_ || (ov == bv_ && oi < bi)) {
        bv_ = ov;
        bi = oi;
      }
    }
    cs.sgn[tid] = (bi != 0x7fffffff && cs.vs[tid][bi] < 0.0) ? -1.0 : 1.0;
  }
  __syncthreads();
  // two-timescale blend of the decayed factors with the SVD factors
  const float dk = expf(gacc);
  const float s1 = sdec, s2 = 1.f - sdec;
  for (int e = tid; e < R * m; e += kNT) {
    const int r = e / m, row = e % m;
    const double sv = cs.sgn[r] * cs.sig[r] * cs.us[r][row];
    A[e] = s1 * (A[e] * dk) + s2 * (float)sv;
  }
  for (int e = tid; e < R * n; e += kNT) {
    const int r = e / n, col = e % n;
    const double sv = cs.sgn[r] * cs.vs[r][col];
    Bv[e] = s1 * (Bv[e] * dk) + s2 * (float)sv;
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
template <typename CT, int D, int P>
struct G3Chunk {
  alignas(16) CT x[3 * P][D + 8];      // rows: H (0..P-1), Q (P..2P-1), K (2P..3P-1)
  alignas(16) float u[P][D + 4];       // w (.) v
  alignas(16) float kr[2 * P][D + 4];  // Kronecker reads of H and Q
  alignas(16) float pp[4][P][P + 4];   // H K^T, Q K^T, H Vbd^T, Q Vbd^T -> Lm, Aq, Ho, Qo
};

template <typename CT, int D, int P>
struct G3Smem {
  union {
    G3Chunk<CT, D, P> c;
    G3Compact<D, P> k;
  } w;
  alignas(16) float ab[kAB];           // A (R x m) | B (R x n)
  alignas(16) float vbd[P][D + 4];     // window keys decayed to the chunk start
  alignas(16) CT vbx[P][D + 8];        // the same in the compute dtype
  float G[P], alpha[P], lg[P], kco[P], qco[P], gam[P], vsc[P];
};

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

template <typename CT, int D, int P>
__global__ void __launch_bounds__(kNT) gdn3_fwd_kernel(G3FwdArgs p) {
  __shared__ G3Smem<CT, D, P> sm;
  constexpr int DG = D / 8;  // 8-element load units per token row
  constexpr int UNITS = P * DG;
  constexpr int W16 = W16Of<CT>::value;
  constexpr int KS = FragT<CT>::KSTEP;
  typedef typename FragT<CT>::type Frag;
  static_assert(UNITS <= kNT && UNITS % 64 == 0, "one load unit per thread");
  static_assert(sizeof(G3Smem<CT, D, P>) <= 160 * 1024, "LDS budget");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, n16 = lane & 15;
  const int H = p.H, M = p.M, T = p.T;
  const int N = p.B * H * M;
  const int chain = xcd_remap(blockIdx.x, N);
  const int b = chain / (H * M), hm = chain % (H * M), h = hm / M, m = hm % M;
  const G3Geom ge = p.ge;
  CT* skron = (CT*)p.skron + (size_t)chain * D * D;

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

  struct Raw {
    uint4 k[W16], q[W16], v[W16];
    f32x4 b0, b1, w0, w1;
    float dec;
  };
  auto fetch = [&](Raw& r, int c) {
    const int t = c * P + ui;
    if (has_unit && t < T) {
      const uint4* kp = (const uint4*)((const CT*)p.k + qkv_base + (size_t)t * qkv_tok + ud);
      const uint4* qp = (const uint4*)((const CT*)p.q + qkv_base + (size_t)t * qkv_tok + ud);
      const uint4* vp = (const uint4*)((const CT*)p.v + qkv_base + (size_t)t * qkv_tok + ud);
#pragma unroll
      for (int w = 0; w < W16; ++w) {
        r.k[w] = kp[w];
        r.q[w] = qp[w];
        r.v[w] = vp[w];
      }
      if (gc > 1) {
        const float* bp = p.bg + gate_base + (size_t)t * gate_tok + ud;
        const float* wp = p.wg + gate_base + (size_t)t * gate_tok + ud;
        r.b0 = *(const f32x4*)bp;
        r.b1 = *(const f32x4*)(bp + 4);
        r.w0 = *(const f32x4*)wp;
        r.w1 = *(const f32x4*)(wp + 4);
      } else {
        const float bs = p.bg[gate_base + (size_t)t * gate_tok];
        const float ws = p.wg[gate_base + (size_t)t * gate_tok];
        r.b0 = r.b1 = (f32x4){bs, bs, bs, bs};
        r.w0 = r.w1 = (f32x4){ws, ws, ws, ws};
      }
      r.dec = p.dec[dec_base + (size_t)t * dec_tok];
    } else {
#pragma unroll
      for (int w = 0; w < W16; ++w) r.k[w] = r.q[w] = r.v[w] = make_uint4(0u, 0u, 0u, 0u);
      r.b0 = r.b1 = r.w0 = r.w1 = zero4();
      r.dec = 1.f;
    }
  };
  auto commit = [&](const Raw& r) {
    if (!has_unit) return;
    float kf[8], qf[8], vf[8];
    unpack8(r.k, kf, (const CT*)nullptr);
    unpack8(r.q, qf, (const CT*)nullptr);
    unpack8(r.v, vf, (const CT*)nullptr);
    const float bb[8] = {r.b0[0], r.b0[1], r.b0[2], r.b0[3], r.b1[0], r.b1[1], r.b1[2], r.b1[3]};
    const float ww[8] = {r.w0[0], r.w0[1], r.w0[2], r.w0[3], r.w1[0], r.w1[1], r.w1[2], r.w1[3]};
    float hf[8], uu[8], part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hf[e] = bb[e] * kf[e];
      uu[e] = ww[e] * vf[e];
      part += kf[e] * hf[e];
    }
    store8(&sm.w.c.x[ui][ud], hf);
#pragma unroll
    for (int w = 0; w < W16; ++w) {
      *(uint4*)&sm.w.c.x[P + ui][ud + w * (16 / sizeof(CT))] = r.q[w];
      *(uint4*)&sm.w.c.x[2 * P + ui][ud + w * (16 / sizeof(CT))] = r.k[w];
    }
    *(f32x4*)&sm.w.c.u[ui][ud] = (f32x4){uu[0], uu[1], uu[2], uu[3]};
    *(f32x4*)&sm.w.c.u[ui][ud + 4] = (f32x4){uu[4], uu[5], uu[6], uu[7]};
#pragma unroll
    for (int off = 1; off < DG; off <<= 1) part += __shfl_xor(part, off, 64);
    if (tid % DG == 0) {
      sm.alpha[ui] = stable_alpha_f(part);
      sm.lg[ui] = log_decay(r.dec);
    }
  };

  // state: A = B = 0, empty window
  for (int e = tid; e < kAB; e += kNT) sm.ab[e] = 0.f;
  for (int e = tid; e < P * (D + 4); e += kNT) (&sm.vbd[0][0])[e] = 0.f;
  for (int e = tid; e < P * (D + 8); e += kNT) (&sm.vbx[0][0])[e] = (CT)0.f;
  float uo[P];
#pragma unroll
  for (int i = 0; i < P; ++i) uo[i] = 0.f;
  float gacc = 0.f;
  bool live = false;
  int event = 0;

  const int nchunks = (T + P - 1) / P;
  Raw raw;
  fetch(raw, 0);
  for (int c = 0; c < nchunks; ++c) {
    __syncthreads();
    commit(raw);
    if (c + 1 < nchunks) fetch(raw, c + 1);
    __syncthreads();
    // per-token scalars (wave 0) | grams and Kronecker reads (MFMA)
    if (wave == 0) {
      float gl = lane < P ? sm.lg[lane] : 0.f;
#pragma unroll
      for (int off = 1; off < P; off <<= 1) {
        const float o = __shfl_up(gl, off, 64);
        if (lane >= off) gl += o;
      }
      const float gl_last = __shfl(gl, P - 1, 64);
      if (lane < P) {
        const float e2 = expf(2.f * (gacc + gl));
        sm.G[lane] = gl;
        sm.gam[lane] = expf(gl);
        sm.kco[lane] = sm.alpha[lane] * e2;
        sm.qco[lane] = e2;
        sm.vsc[lane] = expf(gl_last - gl);
      }
    }
    {
      constexpr int NPT = P / 16;
      const CT* arows = &sm.w.c.x[(wave & 1) ? P : 0][0];
      const CT* brows = (wave < 2) ? &sm.w.c.x[2 * P][0] : &sm.vbx[0][0];
#pragma unroll
      for (int ti = 0; ti < NPT * NPT; ++ti) {
        const int it = ti / NPT, jt = ti % NPT;
        const f32x4 acc = tile_nt<CT, D>(arows + (it * 16 + n16) * (D + 8), brows + (jt * 16 + n16) * (D + 8), g4);
#pragma unroll
        for (int s = 0; s < 4; ++s) sm.w.c.pp[wave][it * 16 + 4 * g4 + s][jt * 16 + n16] = acc[s];
      }
    }
    if (live) {
      constexpr int VPW = (D / 16) / 4, NRT = 2 * P / 16;
#pragma unroll
      for (int a = 0; a < VPW; ++a) {
        const int vt = wave * VPW + a;
        const CT* brow = skron + (size_t)(vt * 16 + n16) * D;
        Frag bf[D / KS];
#pragma unroll
        for (int kb = 0; kb < D / KS; ++kb) bf[kb] = ld_frag(brow + kb * KS, g4);
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < D / KS; ++kb) mma(acc, ld_frag(&sm.w.c.x[rt * 16 + n16][kb * KS], g4), bf[kb]);
#pragma unroll
          for (int s = 0; s < 4; ++s) sm.w.c.kr[rt * 16 + 4 * g4 + s][vt * 16 + n16] = acc[s];
        }
      }
    }
    __syncthreads();
    // coefficient matrices
    for (int e = tid; e < P * P; e += kNT) {
      const int i = e / P, j = e % P;
      const float gi = sm.G[i], gj = sm.G[j], al = sm.alpha[i], ga = sm.gam[i];
      const float dij = (j <= i) ? expf(gi - gj) : 0.f;
      sm.w.c.pp[0][i][j] = (j < i) ? al * dij * sm.w.c.pp[0][i][j] : 0.f;
      sm.w.c.pp[1][i][j] = dij * sm.w.c.pp[1][i][j];
      sm.w.c.pp[2][i][j] = (j >= i) ? al * ga * sm.w.c.pp[2][i][j] : 0.f;
      sm.w.c.pp[3][i][j] = (j >= i) ? ga * sm.w.c.pp[3][i][j] : 0.f;
    }
    __syncthreads();
    // net writes by substitution and outputs, one value column per thread
    if (tid < D) {
      const int v = tid;
      float un[P];
#pragma unroll
      for (int i = 0; i < P; ++i) {
        float r = sm.alpha[i] * sm.w.c.u[i][v];
        if (live) r -= sm.kco[i] * sm.w.c.kr[i][v];
#pragma unroll
        for (int q2 = i; q2 < P; ++q2) r -= sm.w.c.pp[2][i][q2] * uo[q2];
#pragma unroll
        for (int j = 0; j < i; ++j) r -= sm.w.c.pp[0][i][j] * un[j];
        un[i] = r;
      }
      CT* yp = (CT*)p.y + y_base + v;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        float yv = live ? sm.qco[i] * sm.w.c.kr[P + i][v] : 0.f;
#pragma unroll
        for (int q2 = i; q2 < P; ++q2) yv += sm.w.c.pp[3][i][q2] * uo[q2];
#pragma unroll
        for (int j = 0; j <= i; ++j) yv += sm.w.c.pp[1][i][j] * un[j];
        const int t = c * P + i;
        if (t < T) yp[(size_t)t * y_tok] = from_f<CT>(yv);
      }
#pragma unroll
      for (int i = 0; i < P; ++i) uo[i] = un[i];
    }
    // window keys for the next chunk: k_j decayed to this chunk's end
    for (int e = tid; e < P * D; e += kNT) {
      const int j = e / D, d = e % D;
      const float kv = to_f(sm.w.c.x[2 * P + j][d]) * sm.vsc[j];
      sm.vbd[j][d] = kv;
      sm.vbx[j][d] = from_f<CT>(kv);
    }
    gacc += sm.G[P - 1];
    const int tend = (c + 1) * P;
    if (tend <= T && tend % p.Kc == 0) {
      __syncthreads();
      if (tid < D)
#pragma unroll
        for (int i = 0; i < P; ++i) sm.w.k.ut[i][tid] = uo[i];
      __syncthreads();
      g3_compact<D, P>(sm.w.k, sm.ab, sm.vbd, ge, gacc, p.sdec, p.sketch + (size_t)chain * ge.n * ge.q,
                       p.stats ? p.stats + ((size_t)event * N + chain) * 2 : nullptr, tid);
      // materialise sum_r A_r (x) B_r as a [D][D] (v, k) matrix for the reads
      const float* Af = sm.ab;
      const float* Bf = sm.ab + ge.R * ge.m;
      for (int e = tid; e < D * D; e += kNT) {
        const int v = e / D, k = e % D;
        const int iv = v / ge.bv, jv = v % ge.bv, ik = k / ge.bk, jk = k % ge.bk;
        float s = 0.f;
        for (int r = 0; r < ge.R; ++r) s += Af[r * ge.m + iv * ge.ak + ik] * Bf[r * ge.n + jv * ge.bk + jk];
        skron[e] = from_f<CT>(s);
      }
      __threadfence_block();
      gacc = 0.f;
      live = true;
      ++event;
    }
  }
  __syncthreads();
  // final state (reference layouts); A, B carry the decay since the last compaction
  const float dk = expf(gacc);
  if (p.A_out)
    for (int e = tid; e < ge.R * ge.m; e += kNT) p.A_out[(size_t)chain * ge.R * ge.m + e] = sm.ab[e] * dk;
  if (p.B_out)
    for (int e = tid; e < ge.R * ge.n; e += kNT)
      p.B_out[(size_t)chain * ge.R * ge.n + e] = sm.ab[ge.R * ge.m + e] * dk;
  if (p.U_out && tid < D)
#pragma unroll
    for (int i = 0; i < P; ++i) p.U_out[((size_t)chain * D + tid) * P + i] = uo[i];
  if (p.Vb_out)
    for (int e = tid; e < D * P; e += kNT) {
      const int k = e / P, i = e % P;
      p.Vb_out[(size_t)chain * D * P + e] = sm.vbd[i][k];
    }
}

// ---------------------------------------------------------------------------
// standalone compaction (reference layouts)
// ---------------------------------------------------------------------------
template <int D, int P>
struct G3CompactSmem {
  G3Compact<D, P> k;
  alignas(16) float ab[kAB];
  alignas(16) float vbd[P][D + 4];
};

template <int D, int P>
__global__ void __launch_bounds__(kNT) gdn3_compact_kernel(G3CompactArgs p) {
  __shared__ G3CompactSmem<D, P> sm;
  static_assert(sizeof(G3CompactSmem<D, P>) <= 160 * 1024, "LDS budget");
  const int tid = threadIdx.x;
  const int chain = blockIdx.x;
  const G3Geom ge = p.ge;
  const int Rm = ge.R * ge.m, Rn = ge.R * ge.n;
  for (int e = tid; e < Rm; e += kNT) sm.ab[e] = p.A[(size_t)chain * Rm + e];
  for (int e = tid; e < Rn; e += kNT) sm.ab[Rm + e] = p.Bf[(size_t)chain * Rn + e];
  for (int e = tid; e < D * P; e += kNT) {
    const int d = e / P, i = e % P;
    sm.k.ut[i][d] = p.U[(size_t)chain * D * P + e];
    sm.vbd[i][d] = p.Vb[(size_t)chain * D * P + e];
  }
  __syncthreads();
  g3_compact<D, P>(sm.k, sm.ab, sm.vbd, ge, 0.f, p.sdec, p.sketch + (size_t)chain * ge.n * ge.q,
                   p.stats ? p.stats + (size_t)chain * 2 : nullptr, tid);
  for (int e = tid; e < Rm; e += kNT) p.A_out[(size_t)chain * Rm + e] = sm.ab[e];
  for (int e = tid; e < Rn; e += kNT) p.B_out[(size_t)chain * Rn + e] = sm.ab[Rm + e];
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

template <typename CT, int D, int P>
int launch_gdn3_fwd(const G3FwdArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((gdn3_fwd_kernel<CT, D, P>), dim3(a.B * a.H * a.M), dim3(kNT), 0, stream, a);
  return check_launch("gdn3_fwd_kernel");
}

}  // namespace

int gdn3_fwd_dispatch(const G3FwdArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.P == 16) return launch_gdn3_fwd<bf16, 128, 16>(a, stream);
    if (a.D == 64 && a.P == 16) return launch_gdn3_fwd<bf16, 64, 16>(a, stream);
    if (a.D == 64 && a.P == 32) return launch_gdn3_fwd<bf16, 64, 32>(a, stream);
  } else {
    if (a.D == 128 && a.P == 16) return launch_gdn3_fwd<float, 128, 16>(a, stream);
    if (a.D == 64 && a.P == 16) return launch_gdn3_fwd<float, 64, 16>(a, stream);
    if (a.D == 64 && a.P == 32) return launch_gdn3_fwd<float, 64, 32>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "gdn3: unsupported head_dim %d / P %d (128/16, 64/16, 64/32)", a.D, a.P);
}

int gdn3_compact_dispatch(const G3CompactArgs& a, hipStream_t stream) {
  if (a.N == 0) return GDNX_OK;
  if (a.D == 128 && a.P == 16)
    hipLaunchKernelGGL((gdn3_compact_kernel<128, 16>), dim3(a.N), dim3(kNT), 0, stream, a);
  else if (a.D == 64 && a.P == 16)
    hipLaunchKernelGGL((gdn3_compact_kernel<64, 16>), dim3(a.N), dim3(kNT), 0, stream, a);
  else if (a.D == 64 && a.P == 32)
    hipLaunchKernelGGL((gdn3_compact_kernel<64, 32>), dim3(a.N), dim3(kNT), 0, stream, a);
  else
    return set_error(GDNX_ERR_SHAPE, "gdn3_compact: unsupported head_dim %d / P %d", a.D, a.P);
  return check_launch("gdn3_compact_kernel");
}

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

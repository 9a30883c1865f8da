// Shared pieces of the GDN3 Kronecker-residual kernels (forward window and
// compaction in gdn3.hip, backward in gdn3_bwd.hip): the layer's Kronecker
// geometry, the exact write coefficient alpha(c) and its derivative, the
// clamped log decay, and the layout of the training stash.
#pragma once
#include "delta_common.hpp"
#include "gdnx_common.hpp"

namespace gdnx {

constexpr int kRMax = 4;    // Kronecker rank bound
constexpr int kQ = 8;       // sketch width bound: min(R + 4, m, n) <= 8
constexpr int kMN = 256;    // bound on m = a_v a_k and n = b_v b_k
constexpr int kAB = 1280;   // bound on R (m + n) for m n = d^2, m, n <= 256
constexpr int kNT = 256;    // threads of every GDN3 block

// Kronecker geometry of the layer (gdn3/gdn3_upgrade.py:73-77: rank 4,
// a_k = 16, b_k = 8, so (a_v, a_k, b_v, b_k) = (16, 16, 8, 8) at head dim 128;
// (8, 8, 8, 8) at head dim 64).  Compile-time, so every loop over the
// factors unrolls and every index split is a shift.
template <int D> struct G3C;
template <> struct G3C<128> { static constexpr int R = 4, av = 16, ak = 16, bv = 8, bk = 8, lbv = 3, lbk = 3; };
template <> struct G3C<64> { static constexpr int R = 4, av = 8, ak = 8, bv = 8, bk = 8, lbv = 3, lbk = 3; };
template <int D> struct G3D : G3C<D> {
  static constexpr int m = G3C<D>::av * G3C<D>::ak, n = G3C<D>::bv * G3C<D>::bk;
  static constexpr int q = (G3C<D>::R + 4 < m ? (G3C<D>::R + 4 < n ? G3C<D>::R + 4 : n) : (m < n ? m : n));
  static constexpr int ln = G3C<D>::lbv + G3C<D>::lbk;
  static constexpr int RMN = G3C<D>::R * (m + n);   // floats of one (A | B) factor set
  static_assert((1 << G3C<D>::lbv) == G3C<D>::bv && (1 << G3C<D>::lbk) == G3C<D>::bk && m <= kMN && n <= kMN &&
                    q <= kQ && G3C<D>::R <= kRMax, "geometry");
};

// sum_r A_r (x) B_r at (v, k), factors as stored: A [R][a_v][a_k], B [R][b_v][b_k]
template <int D>
__device__ __forceinline__ float kron_entry(const float* __restrict__ Af, const float* __restrict__ Bf, int v, int k) {
  typedef G3D<D> Ge;
  const int iv = v >> Ge::lbv, jv = v & (Ge::bv - 1), ik = k >> Ge::lbk, jk = k & (Ge::bk - 1);
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < Ge::R; ++r) s += Af[r * Ge::m + iv * Ge::ak + ik] * Bf[r * Ge::n + jv * Ge::bk + jk];
  return s;
}

__device__ __forceinline__ float stable_alpha_f(float c) {
  // (1 - e^{-c}) / c (gdn3/gdn3_upgrade.py:641-648).  Below |c| = 1/8 its
  // Taylor series to c^5 (truncation c^6 / 5040 < 1e-9); above, from the
  // hardware exponential (1 - e^{-c} then cancels by at most a factor 8.5,
  // a few 1e-7 relative).  The reference's own series branch (|c| < 1e-6)
  // agrees with both to rounding.
  if (fabsf(c) < 0.125f)
    return 1.f - c * (0.5f - c * (1.f / 6.f - c * (1.f / 24.f - c * (1.f / 120.f - c * (1.f / 720.f)))));
  return (1.f - __expf(-c)) / c;
}

// d alpha / dc: (c e^{-c} + expm1(-c)) / c^2, by its Taylor series below
// |c| = 0.05 where the closed form cancels
__device__ __forceinline__ float stable_dalpha_f(float c) {
  if (fabsf(c) < 0.05f) return -0.5f + c * (1.f / 3.f - c * (1.f / 8.f - c * (1.f / 30.f - c * (1.f / 144.f))));
  return (c * expf(-c) + expm1f(-c)) / (c * c);
}

__device__ __forceinline__ float log_decay(float d) {
  // clamp(dec, 0, 1) as a natural-log decay, floored at kLogFloor
  d = fminf(d, 1.f);
  return d > 0.f ? fmaxf(logf(d), kLogFloor) : kLogFloor;
}

// d log_decay(d) / dd where the clamp and the floor pass the value through
__device__ __forceinline__ float dlog_decay(float d) {
  return (d <= 1.f && d > 0.f && logf(d) > kLogFloor) ? 1.f / d : 0.f;
}

// Training stash of the forward (read by the backward), per chain n of N,
// chunk c of nch, compaction e of ncomp:
//   U    [N][nch][P][D] fp32  the chunk's net writes alpha_i r_i
//   gacc [N][nch]       fp32  log decay since the last compaction at the chunk start
//   ab   [ncomp][N][RMN] fp32 the factors (A | B) each compaction leaves
struct G3Stash {
  float* u;
  float* gacc;
  float* ab;
};
__host__ __device__ __forceinline__ size_t g3_align256(size_t x) { return (x + 255) & ~(size_t)255; }
__host__ __device__ __forceinline__ G3Stash g3_stash(void* base, int N, int nch, int ncomp, int D, int P, int rmn) {
  char* w = (char*)base;
  G3Stash s;
  s.u = (float*)w;
  w += g3_align256((size_t)N * nch * P * D * 4);
  s.gacc = (float*)w;
  w += g3_align256((size_t)N * nch * 4);
  s.ab = (float*)w;
  (void)ncomp;
  (void)rmn;
  return s;
}
__host__ __device__ __forceinline__ size_t g3_stash_bytes(int N, int nch, int ncomp, int D, int P, int rmn) {
  return g3_align256((size_t)N * nch * P * D * 4) + g3_align256((size_t)N * nch * 4) +
         g3_align256((size_t)ncomp * N * rmn * 4 + 4);
}

}  // namespace gdnx

// GDN3 dense-regime write coefficient and its backward (gfx950).
//
// With lane-shared keys k [B,T,H,D] and scalar per-lane gates
// beta [B,T,H,M], GDN3's exact-alpha write (gdn3/gdn3_upgrade.py:641-648,
// used at gdn3/_reference_recurrence.py:73-78) reduces to one coefficient per
// token and lane:
//   c = beta |k|^2,   alpha(c) = (1 - exp(-c)) / c  (1 - c/2 + c^2/6 for
//   |c| < 1e-6, the reference's Taylor branch),   a = alpha(c) beta
// which the delta-rule kernels use as both erase and write coefficient.
// Backward, given da (the sum of the erase and write coefficient
// gradients):
//   dbeta = da (alpha + c alpha'(c)),   dk += 2 k sum_m da_m beta_m^2 alpha'(c_m)
// alpha'(c) = (c exp(-c) - (1 - exp(-c))) / c^2 is taken from its series
// -1/2 + c/3 - c^2/8 + c^3/30 - c^4/144 for |c| < 0.05 (where the closed
// form cancels) and from the closed form elsewhere.
//
// Sixteen lanes per (b, t, h) row: each holds 8 (bf16) or 4 (fp32)
// features, the squared norm is reduced across the 16, and lane m < M forms
// lane m's coefficient.
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

__device__ __forceinline__ float alpha_f(float c) {
  if (fabsf(c) < 1e-6f) return 1.f - c * 0.5f + c * c * (1.f / 6.f);
  return -expm1f(-c) / c;
}

__device__ __forceinline__ float dalpha_f(float c) {
  if (fabsf(c) < 0.05f) return -0.5f + c * (1.f / 3.f - c * (1.f / 8.f - c * (1.f / 30.f - c * (1.f / 144.f))));
  return (c * expf(-c) + expm1f(-c)) / (c * c);
}

template <typename IO>
__device__ __forceinline__ void load_row8(const IO* p, float* x);
template <>
__device__ __forceinline__ void load_row8<bf16>(const bf16* p, float* x) {
  const bf16x8 v = *(const bf16x8*)p;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}
template <>
__device__ __forceinline__ void load_row8<float>(const float* p, float* x) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = a[e];
    x[4 + e] = b[e];
  }
}

// 16 lanes x 8 features = 128; D = 64 uses 8 features on lanes 0..7 of each 16
template <typename IO, int D>
__global__ void __launch_bounds__(256) gdn3_coeff_kernel(GCoeffArgs p) {
  constexpr int PER = D / 16;   // features per lane
  const size_t row = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const size_t nrows = (size_t)p.B * p.T * p.H;
  if (row >= nrows) return;
  const IO* kr = (const IO*)p.k + row * D + l * PER;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (PER == 8) {
    load_row8<IO>(kr, x);
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) x[e] = to_f(kr[e]);
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += x[e] * x[e];
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 16);
  if (l < p.M) {
    const float beta = p.beta[row * p.M + l];
    const float c = beta * s;
    p.a[row * p.M + l] = alpha_f(c) * beta;
  }
}

template <typename IO, int D>
__global__ void __launch_bounds__(256) gdn3_coeff_bwd_kernel(GCoeffArgs p) {
  constexpr int PER = D / 16;
  const size_t row = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const size_t nrows = (size_t)p.B * p.T * p.H;
  if (row >= nrows) return;
  const IO* kr = (const IO*)p.k + row * D + l * PER;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (PER == 8) {
    load_row8<IO>(kr, x);
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) x[e] = to_f(kr[e]);
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += x[e] * x[e];
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 16);
  // lane m < M: its coefficient's gradient; g = sum_m da_m beta_m^2 alpha'(c_m)
  float g = 0.f;
  if (l < p.M) {
    const size_t i = row * p.M + l;
    const float beta = p.beta[i];
    const float da = p.da_e[i] + (p.da_w ? p.da_w[i] : 0.f);
    const float c = beta * s;
    const float dal = dalpha_f(c);
    p.dbeta[i] = da * (alpha_f(c) + c * dal);
    g = da * beta * beta * dal;
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) g += __shfl_xor(g, off, 16);
  IO* dkr = (IO*)p.dk + row * D + l * PER;
#pragma unroll
  for (int e = 0; e < PER; ++e) dkr[e] = from_f<IO>(to_f(dkr[e]) + 2.f * g * x[e]);
}

template <typename IO, int D>
static int launch_coeff(const GCoeffArgs& a, bool bwd, hipStream_t stream) {
  const size_t nrows = (size_t)a.B * a.T * a.H;
  const dim3 grid((unsigned)((nrows + 15) / 16));
  if (bwd) {
    hipLaunchKernelGGL((gdn3_coeff_bwd_kernel<IO, D>), grid, dim3(256), 0, stream, a);
    return check_launch("gdn3_coeff_bwd_kernel");
  }
  hipLaunchKernelGGL((gdn3_coeff_kernel<IO, D>), grid, dim3(256), 0, stream, a);
  return check_launch("gdn3_coeff_kernel");
}

int gdn3_coeff_dispatch(const GCoeffArgs& a, bool bwd, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128) return launch_coeff<bf16, 128>(a, bwd, stream);
    if (a.D == 64) return launch_coeff<bf16, 64>(a, bwd, stream);
  } else {
    if (a.D == 128) return launch_coeff<float, 128>(a, bwd, stream);
    if (a.D == 64) return launch_coeff<float, 64>(a, bwd, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "gdn3 coefficient: head_dim %d unsupported", a.D);
}

}  // namespace gdnx

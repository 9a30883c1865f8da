// Lane sums for q, k, v shared by a head's lanes (gfx950).
//
// The reference layer feeds one q, k and v per head to its M lanes through an
// expand (gdn3/gdn3_upgrade.py:785-787), so their gradients are the sums over
// the lanes of the per-lane gradients the recurrence's backward writes.
// gdnx_lane_sum forms such a sum, in lane order, and writes it in the IO
// dtype: one pass over the per-lane fp32 gradients (HBM-bound), where a sum
// to fp32 and a separate cast would read and write the reduced tensor again.
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

// thread e sums the 8 consecutive elements 8 (e mod D/8) .. of row e / (D/8)
template <typename OT>
__global__ void __launch_bounds__(256) lane_sum_kernel(const float* __restrict__ x, OT* __restrict__ out,
                                                      long long rows, int M, int D) {
  const long long units = rows * (D / 8);
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= units) return;
  const long long row = e / (D / 8);
  const int d = 8 * (int)(e % (D / 8));
  const float* xp = x + (size_t)row * M * D + d;
  // the lanes' partials are read once: non-temporal loads
  f32x4 s0 = __builtin_nontemporal_load((const f32x4*)xp), s1 = __builtin_nontemporal_load((const f32x4*)(xp + 4));
  for (int m = 1; m < M; ++m) {
    s0 += __builtin_nontemporal_load((const f32x4*)(xp + (size_t)m * D));
    s1 += __builtin_nontemporal_load((const f32x4*)(xp + (size_t)m * D + 4));
  }
  OT* op = out + (size_t)row * D + d;
  st4(op, s0[0], s0[1], s0[2], s0[3]);
  st4(op + 4, s1[0], s1[1], s1[2], s1[3]);
}

}  // namespace
}  // namespace gdnx

using namespace gdnx;

extern "C" int gdnx_lane_sum(const float* x, void* out, long long rows, int M, int D, int dtype, void* stream) {
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "lane sum: dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (rows < 0 || M < 1 || D < 8 || D % 8 != 0)
    return set_error(GDNX_ERR_SHAPE, "lane sum: rows %lld, M %d, D %d (M >= 1, D a multiple of 8)", rows, M, D);
  if (rows > 0 && (!x || !out)) return set_error(GDNX_ERR_ARG, "lane sum: x and out must be non-null");
  if (((uintptr_t)x | (uintptr_t)out) % 16 != 0)
    return set_error(GDNX_ERR_ARG, "lane sum: x and out must be 16-byte aligned");
  if (rows == 0) return GDNX_OK;
  const long long units = rows * (D / 8);
  const dim3 grid((unsigned)((units + 255) / 256));
  if (dtype == GDNX_DTYPE_BF16)
    hipLaunchKernelGGL(lane_sum_kernel<bf16>, grid, dim3(256), 0, (hipStream_t)stream, x, (bf16*)out, rows, M, D);
  else
    hipLaunchKernelGGL(lane_sum_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream, x, (float*)out, rows, M, D);
  return check_launch("lane_sum_kernel");
}

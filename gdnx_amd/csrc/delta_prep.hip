// Per-chunk operands of the chunked delta rule that do not depend on the
// carried state, computed for every (b, h, chunk) and lane in parallel
// (gfx950).  The sequential forward scan then only carries the state.
//
// For chain (b, h, m) and chunk c with inclusive log-decay prefix G (clamped
// to [kLogFloor, 0] per token, as in the scan):
//   L  = (exp(G_i - G_j) a_e,i k_i . k_j)_{j<i},   T = (I + L)^-1
//   TA = T diag(a_w),  TB = T diag(a_e exp(G)),  Aq = (exp(G_i - G_j) q_i . k_j)_{j<=i}
//   gam = exp(G),  dec = exp(G_last - G)
// (the chunk algebra of the forward kernel; reference chunk structure
// gdn3/gdn3_upgrade.py:467-521, decay ratios replaced by log-space
// differences).  One workgroup per (b, h, chunk) stages K and Q once for the
// M lanes, which share them.
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename CT, int D, int C>
struct alignas(16) PrepSmem {
  typedef Dims<CT, D, C> Dm;
  CT q[C * Dm::LDD];
  CT k[C * Dm::LDD];
  CT ta[C * Dm::LDC];
  CT tb[C * Dm::LDC];
  CT aq[C * Dm::LDC];
  float L[C * Dm::LDF];
  float LT[C * Dm::LDT];
  float Td[C * Dm::LDT];
  float G[C], gam[C], dec[C], ae[C], aw[C];
};

// [C][LDC] LDS tile -> [C][C] global, 16-byte stores
template <typename CT, int C, int LDC>
__device__ __forceinline__ void store_cc(CT* __restrict__ dst, const CT* src, int tid, int nt) {
  constexpr int PER = 16 / sizeof(CT), NU = C * C / PER;
  for (int u = tid; u < NU; u += nt) {
    const int i = (u * PER) / C, j = (u * PER) % C;
    *(uint4*)&dst[(size_t)u * PER] = *(const uint4*)&src[i * LDC + j];
  }
}

template <typename CT, int D, int C>
__global__ void __launch_bounds__((Dims<CT, D, C>::NT)) delta_prep_kernel(DeltaArgs p) {
  typedef Dims<CT, D, C> Dm;
  constexpr int LDC = Dm::LDC, NT = Dm::NT;
  __shared__ PrepSmem<CT, D, C> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int NC = (p.T + C - 1) / C;
  const int nblk = p.B * p.H * NC;
  const int blk = xcd_remap(blockIdx.x, nblk);
  const int c = blk % NC, h = (blk / NC) % p.H, b = blk / (NC * p.H);
  const int t0 = c * C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t st = (size_t)p.H * p.M;
  const PrepPtrs<CT> po = prep_ptrs<CT>(p.prep, (size_t)p.B * p.H * p.M * NC, C);

  for (int i = tid; i < C * LDC; i += NT) {  // never-written upper parts read as zero
    sm.ta[i] = from_f<CT>(0.f);
    sm.tb[i] = from_f<CT>(0.f);
    sm.aq[i] = from_f<CT>(0.f);
  }
  {
    TileRegs rq, rk;
    tile_fetch<CT, D, C>(rq, (const CT*)p.q + qoff, rs, t0, p.T, tid);
    tile_fetch<CT, D, C>(rk, (const CT*)p.k + qoff, rs, t0, p.T, tid);
    tile_commit<CT, D, C>(rq, sm.q, nullptr, tid);
    tile_commit<CT, D, C>(rk, sm.k, nullptr, tid);
  }
  const ChunkScalars cs{sm.G, sm.gam, sm.dec, sm.ae, sm.aw, nullptr};
  for (int m = 0; m < p.M; ++m) {
    const size_t soff = ((size_t)b * p.T * p.H + h) * p.M + m;
    if (wave == 0) prep_scalars<C>(cs, p.ae + soff, p.aw + soff, p.g + soff, st, t0, p.T, lane);
    __syncthreads();
    chunk_grams<CT, D, C>(sm.k, sm.q, sm.L, sm.LT, sm.G, sm.ae, wave, lane,
                          [&](int i, int j0, const float* v) { st4(&sm.aq[i * LDC + j0], v[0], v[1], v[2], v[3]); });
    __syncthreads();
    invert_unit_lower<C>(
        sm.L, sm.LT, sm.Td, wave, lane,
        [&](int j) { return make_float2(sm.aw[j], sm.ae[j] * sm.gam[j]); },
        [&](int i, int j, float t, float2 f) {
          sm.ta[i * LDC + j] = from_f<CT>(t * f.x);
          sm.tb[i * LDC + j] = from_f<CT>(t * f.y);
        });
    __syncthreads();
    const size_t rec = (((size_t)b * p.H + h) * p.M + m) * NC + c;  // chain-major, chunks contiguous
    store_cc<CT, C, LDC>(po.ta + rec * C * C, sm.ta, tid, NT);
    store_cc<CT, C, LDC>(po.tb + rec * C * C, sm.tb, tid, NT);
    store_cc<CT, C, LDC>(po.aq + rec * C * C, sm.aq, tid, NT);
    if (tid < C) {
      po.sc[rec * 2 * C + tid] = sm.gam[tid];
      po.sc[rec * 2 * C + C + tid] = sm.dec[tid];
    }
    __syncthreads();
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
  const size_t es = dtype == GDNX_DTYPE_BF16 ? 2 : 4;
  return NR * (3 * (size_t)C * C * es + 2 * (size_t)C * 4);
}

}  // namespace gdnx

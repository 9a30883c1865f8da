// One-token decode step of the decoupled-erase delta rule (gfx950), on a
// contiguous state per row or on a state pool indexed by a slot per row (a
// decode-state cache: sequences join and leave without moving states).
//
// The reference has no decode path (its layers swallow cache_params,
// gdn3/gdn3_upgrade.py:725); the step is one iteration of the sequential
// oracle, gdn3/_reference_recurrence.py:60-84 (dense regime) and
// research/kernel_ab/ref_scan.py:40-45, on a carried fp32 state:
//
//   g' = exp(min(log_g, 0));  m = g' S^T e;  r = w - m;
//   S <- g' S + k r^T;        y = S^T q = g' S^T q + (k.q) r
//   with e = a_e k, w = a_w v.
// With a decay per key channel (the KMD-2 native scan, research/kernel_ab/
// ref_scan.py:40-45, g [.., d_k]) g' scales the rows of S: m = S^T (g' e),
// y = S^T (g' q) + (k.q) r, S <- diag(g') S + k r^T.
//
// HBM-bound: every step reads and writes each d x d fp32 state once, with
// non-temporal loads and stores (the state is not reused within a step, so
// it bypasses the caches' retention).  One workgroup of TH threads per chain
// holds the chain's state in registers: thread t owns columns 4(t % (d/4))..+3
// of rows t / (d/4) + RG j (RG = TH / (d/4) row groups), so a wave reads and
// writes 1 KB contiguous runs with 16-byte accesses and each element is
// touched exactly once in each direction.  The two contractions over k
// (S^T e, S^T q) are folded across the row groups of a wave with shuffles,
// then across the waves through LDS.  d = 128 uses TH = 1024 (4 rows per
// thread; the short per-thread load chain measured 6% faster than 256
// threads x 16 rows), d = 64 uses TH = 256.
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

template <typename IO, int D, int TH>
__global__ void __launch_bounds__(TH) delta_decode_kernel(DecodeArgs p) {
  constexpr int CG = D / 4;          // column groups of 4
  constexpr int RG = TH / CG;        // row groups
  constexpr int RPT = D / RG;        // rows per thread
  constexpr int NWV = TH / 64;       // waves
  static_assert(RG * RPT == D && TH >= D, "launch shape");
  __shared__ float s_k[D], s_q[D], s_g[D], s_red[2][NWV][D];
  __shared__ float s_kq;

  const int tid = threadIdx.x;
  const int nch = p.NS * p.H * p.M;
  const int chain = xcd_remap(blockIdx.x, nch);
  const int head = chain / p.M;                 // (seq, head) index
  const int cg = tid % CG, rg = tid / CG;
  size_t sidx = chain;                          // this chain's state
  if (p.slots) {                                // state pool: row s uses slot slots[s]
    const int hm = p.H * p.M, sl = p.slots[chain / hm];
    if (sl < 0 || sl >= p.nslots) {             // an empty row: zero output, no state touched
      if (tid < D) ((IO*)p.y)[(size_t)chain * D + tid] = from_f<IO>(0.f);
      return;
    }
    sidx = (size_t)sl * hm + chain % hm;
  }
  const float ae = p.ae[chain], aw = p.aw[chain];
  const float gam = p.chan ? 1.f : __expf(fmaxf(fminf(p.g[chain], 0.f), kLogFloor));
  const IO* kg = (const IO*)p.k + (size_t)head * D;
  const IO* qg = (const IO*)p.q + (size_t)head * D;
  const IO* vg = (const IO*)p.v + (size_t)head * D;
  float* S = p.state + sidx * D * D;

  // state loads first: they are the HBM stream
  f32x4 s[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j)
    s[j] = __builtin_nontemporal_load((const f32x4*)&S[(size_t)(rg + RG * j) * D + 4 * cg]);

  if (tid < D) {
    s_k[tid] = to_f(kg[tid]);
    s_q[tid] = to_f(qg[tid]);
    s_g[tid] = p.chan ? __expf(fmaxf(fminf(p.g[(size_t)chain * D + tid], 0.f), kLogFloor)) : gam;
  }
  __syncthreads();
  if (tid < 64) {
    float kq = 0.f;
    for (int i = tid; i < D; i += 64) kq += s_k[i] * s_q[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kq += __shfl_xor(kq, off, 64);
    if (tid == 0) s_kq = kq;
  }
  f32x4 pe = zero4(), pq = zero4();
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const float gj = p.chan ? s_g[rg + RG * j] : 1.f;
    const float kk = s_k[rg + RG * j] * gj, qq = s_q[rg + RG * j] * gj;
    pe += s[j] * kk;
    pq += s[j] * qq;
  }
  // the 64/CG row groups of one wave sit in lanes l, l ^ CG, ... : fold them
  static_assert(CG == 32 || CG == 16, "head dim 128 or 64");
#pragma unroll
  for (int off = CG; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pe[e] += __shfl_xor(pe[e], off, 64);
      pq[e] += __shfl_xor(pq[e], off, 64);
    }
  // remaining row groups: one partial per wave (lanes < CG) via LDS
  const int lane = tid & 63, wave = tid >> 6;
  if (lane < CG) {
    *(f32x4*)&s_red[0][wave][4 * cg] = pe;
    *(f32x4*)&s_red[1][wave][4 * cg] = pq;
  }
  __syncthreads();
  f32x4 te = zero4(), tq = zero4();
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    te += *(const f32x4*)&s_red[0][w][4 * cg];
    tq += *(const f32x4*)&s_red[1][w][4 * cg];
  }
  // r = a_w v - gamma a_e S^T k ; y = gamma S^T q + (k.q) r
  f32x4 vv;
#pragma unroll
  for (int e = 0; e < 4; ++e) vv[e] = to_f(vg[4 * cg + e]);
  const f32x4 r = aw * vv - (gam * ae) * te;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const float kk = s_k[rg + RG * j];
    const f32x4 o = s_g[rg + RG * j] * s[j] + kk * r;
    __builtin_nontemporal_store(o, (f32x4*)&S[(size_t)(rg + RG * j) * D + 4 * cg]);
  }
  if (rg == 0) {
    const f32x4 y = gam * tq + s_kq * r;
    IO* yg = (IO*)p.y + (size_t)chain * D + 4 * cg;
    st4(yg, y[0], y[1], y[2], y[3]);
  }
}

template <typename IO, int D>
static int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  constexpr int TH = D == 128 ? 1024 : 256;
  hipLaunchKernelGGL((delta_decode_kernel<IO, D, TH>), dim3(a.NS * a.H * a.M), dim3(TH), 0, stream, a);
  return check_launch("delta_decode_kernel");
}

int decode_dispatch(const DecodeArgs& a, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128) return launch_decode<bf16, 128>(a, stream);
    if (a.D == 64) return launch_decode<bf16, 64>(a, stream);
  } else {
    if (a.D == 128) return launch_decode<float, 128>(a, stream);
    if (a.D == 64) return launch_decode<float, 64>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "decode: unsupported head dim %d", a.D);
}

}  // namespace gdnx

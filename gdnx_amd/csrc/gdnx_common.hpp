// Shared device helpers for the gdnx HIP kernels (gfx950 / CDNA4 only).
//
// MFMA conventions (checked on gfx950 with an in-bounds lane-layout probe):
//   v_mfma_f32_16x16x32_bf16 / v_mfma_f32_16x16x4_f32, lane l = 16*g + n:
//     A operand: lane supplies A[m = n][k in set(g)]
//     B operand: lane supplies B[k in set(g)][n]
//     D result : lane holds  D[4g + i][n], i = 0..3
// Every product is written "NT": both operands are stored K-contiguous, and
// the K index set a lane supplies is the same permutation for A and B, so
// the sum over K is exact whatever order the instruction uses internally.
//   bf16 k-step (32): lane holds k = kb + 4g + i (i<4) and kb + 16 + 4g + (i-4)
//   fp32 k-step (16): lane holds k = kb + 4g + s (one instruction per s)
// With this choice an accumulator tile pair (rows kb..kb+31) is directly a
// B/A fragment over k = rows, so state and net writes never leave registers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdnx {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename CT> struct FragT;
template <> struct FragT<bf16> {
  typedef bf16x8 type;
  static constexpr int KSTEP = 32;  // k per MFMA step
  static constexpr int TPS = 2;     // accumulator tiles per k-step
};
template <> struct FragT<float> {
  typedef f32x4 type;
  static constexpr int KSTEP = 16;
  static constexpr int TPS = 1;
};

__device__ __forceinline__ void mma(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const f32x4& a, const f32x4& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
}

// Fragment from a K-contiguous LDS row: p points at element [row][kb].
__device__ __forceinline__ bf16x8 ld_frag(const bf16* p, int g) {
  bf16x4 lo = *(const bf16x4*)(p + 4 * g);
  bf16x4 hi = *(const bf16x4*)(p + 16 + 4 * g);
  return (bf16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ f32x4 ld_frag(const float* p, int g) {
  return *(const f32x4*)(p + 4 * g);
}

// Fragment over k = accumulator rows: tiles t0 (rows kb..kb+15) and t1
// (rows kb+16..kb+31; ignored for fp32), each row scaled by s0[i] / s1[i].
__device__ __forceinline__ bf16x8 acc_frag(bf16*, const f32x4& t0, const f32x4& t1,
                                           const f32x4& s0, const f32x4& s1) {
  return (bf16x8){(bf16)(t0[0] * s0[0]), (bf16)(t0[1] * s0[1]), (bf16)(t0[2] * s0[2]),
                  (bf16)(t0[3] * s0[3]), (bf16)(t1[0] * s1[0]), (bf16)(t1[1] * s1[1]),
                  (bf16)(t1[2] * s1[2]), (bf16)(t1[3] * s1[3])};
}
__device__ __forceinline__ f32x4 acc_frag(float*, const f32x4& t0, const f32x4&,
                                          const f32x4& s0, const f32x4&) {
  return t0 * s0;
}
__device__ __forceinline__ bf16x8 acc_frag(bf16*, const f32x4& t0, const f32x4& t1) {
  return (bf16x8){(bf16)t0[0], (bf16)t0[1], (bf16)t0[2], (bf16)t0[3],
                  (bf16)t1[0], (bf16)t1[1], (bf16)t1[2], (bf16)t1[3]};
}
__device__ __forceinline__ f32x4 acc_frag(float*, const f32x4& t0, const f32x4&) { return t0; }

__device__ __forceinline__ f32x4 zero4() { return (f32x4){0.f, 0.f, 0.f, 0.f}; }

// Workgroup barrier for LDS traffic only.  __syncthreads() is a workgroup
// release/acquire fence, which on CDNA (one vmcnt for loads and stores)
// waits for every outstanding global load, a prefetch issued just before it
// included.  Here only LDS operations complete before s_barrier, so loads
// issued for a later step stay in flight across it; the memory clobber keeps
// the compiler from moving memory accesses across the barrier.  Global
// stores before it are not made visible to the other waves.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The thread index as a value the compiler cannot prove invariant: index
// arithmetic derived from it is recomputed where it is used rather than
// hoisted out of an enclosing loop and held in registers across the loop's
// other phases (where those registers are wanted for loads in flight).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Orders one wave's LDS accesses across its lanes: what a lane wrote before
// this point is what the wave's other lanes read after it.  The hardware
// completes a wave's LDS accesses in issue order; the wavefront-scope fences
// keep the compiler from moving a lane's accesses across this point (to the
// compiler, another lane's write is another thread's, so without them a
// lane's read may be hoisted above a write it does not itself depend on).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 4 consecutive CT values from floats (for 8/16-byte LDS stores).
__device__ __forceinline__ void st4(bf16* p, float a, float b, float c, float d) {
  *(bf16x4*)p = (bf16x4){(bf16)a, (bf16)b, (bf16)c, (bf16)d};
}
__device__ __forceinline__ void st4(float* p, float a, float b, float c, float d) {
  *(f32x4*)p = (f32x4){a, b, c, d};
}

__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f(float x) { return x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }

// Lowest log-decay per token: exp(-60) ~ 9e-27 acts as a reset while keeping
// differences of cumulative log-decays finite.
constexpr float kLogFloor = -60.0f;

// XCD-aware block -> work-item map: the 8 XCDs receive blocks round-robin,
// so consecutive work items (e.g. the lanes of one head, which read the same
// q/k/v) are placed on one XCD and share its L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  return (bid % 8) * (nblocks / 8) + bid / 8;
}

}  // namespace gdnx

// One-token step of the GDN3 Kronecker-residual recurrence on a carried state
// (gfx950), for decode after a prefill through gdnx_gdn3_chunk_fwd_state.
//
// The reference has no decode path (GDN3LinearAttn.forward ignores
// cache_params, gdn3/gdn3_upgrade.py:725); the step is one iteration of the
// frozen oracle's token loop, gdn3/_reference_recurrence.py:60-90, on the
// state in the reference's layouts (:52-55), updated in place:
//
//   gamma = clamp(dec, 0, 1);  A, B, Vb *= gamma
//   h = b (.) k;  u = w (.) v;  S x = vec(sum_r A_r X B_r^T) + U (Vb^T x)
//   r = u - S h;  alpha = alpha(k.h);  y = S q + alpha (k.q) r
//   U[:, p] = alpha r;  Vb[:, p] = k,  p = pos mod P
//
// and, after the tokens with (pos + 1) mod K_c == 0, the compaction of
// gdnx_gdn3_compact on those rows' chains (a second launch that returns at
// once for the other rows).
//
// A chain reads its 21.5 KB state (d = 128, P = 16) and writes back A, B,
// Vb (decayed) and one column of U.  One 256-thread block per chain stages
// the state in LDS with 16-byte loads (non-temporal for the parts rewritten
// in full), forms the two reads S h, S q from LDS (Vb^T x as per-slot
// partial sums over d ranges reduced across lanes, the Kronecker part as
// A_r X, then (A_r X) B_r^T), and writes from the registers it loaded.
// Every product reads its LDS operands as 16-byte vectors and keeps four
// outputs per thread, so the LDS traffic per chain stays a few times the
// state's size (with scalar reads the block was bound by LDS bandwidth,
// not by HBM).
#include "gdn3_common.hpp"
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int kDT = 256;   // threads per chain

template <int D, int P>
struct G3DecSmem {
  typedef G3D<D> Ge;
  static constexpr int LDP = P + 4;   // U / Vb row length: 16-byte aligned rows, 16 lanes' rows on distinct banks
  float A[Ge::R * Ge::m];          // gamma A   [R][a_v][a_k]
  float B[Ge::R * Ge::n];          // gamma B   [R][b_v][b_k]
  float U[D][LDP];                 // U [d][slot]
  float V[D][LDP];                 // gamma Vb
  float x[2][D];                   // h, q
  float k[D], u[D];
  float ax[2][Ge::R][Ge::av][Ge::bk];   // A_r X for X = h, q
  float coef[2][P];                // (gamma Vb)^T h, (gamma Vb)^T q
  float sx[2][D];                  // S h, S q
  float red[2];                    // k.h, k.q
};

// Sum over aligned groups of N consecutive lanes (N = 1 .. 32), in every
// lane of the group: DPP quad permutes, half-row and row mirrors, then the
// 16-lane row swap.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32, "power-of-two group up to 32");
  if constexpr (N >= 2) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
  if constexpr (N >= 4) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
  if constexpr (N >= 8) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));
  if constexpr (N >= 16) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));
  if constexpr (N >= 32) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  return x;
}

template <typename IO, int D, int P>
__global__ void __launch_bounds__(kDT) gdn3_decode_kernel(G3DecArgs p) {
  typedef G3D<D> Ge;
  typedef G3DecSmem<D, P> Sm;
  constexpr int RM = Ge::R * Ge::m, RN = Ge::R * Ge::n, DP = D * P, LDP = Sm::LDP;
  constexpr int NA = (RM / 4 + kDT - 1) / kDT, NB = (RN / 4 + kDT - 1) / kDT, NU = (DP / 4 + kDT - 1) / kDT;
  static_assert(RM % 4 == 0 && RN % 4 == 0 && DP % 4 == 0 && P % 4 == 0, "16-byte units");
  static_assert(Ge::ak % 4 == 0 && Ge::bk % 4 == 0 && 2 * D <= kDT && D % 64 == 0, "decode geometry");
  __shared__ __attribute__((aligned(16))) Sm sm;

  const int tid = threadIdx.x;
  const int hm = p.H * p.M;
  const int chain = blockIdx.x;                 // (row, h, m)
  const int row = chain / hm, ch = chain % hm, h = ch / p.M, m = ch % p.M;
  const int sl = p.slots ? p.slots[row] : row;
  IO* yg = (IO*)p.y + (size_t)chain * D;
  if (p.stats && tid < 2) p.stats[(size_t)chain * 2 + tid] = 0.0;
  const int pos = p.pos[row];
  // an empty row (slot outside the pool, or a negative position, which has
  // no residual slot): zero output, no state touched
  if (sl < 0 || sl >= p.nslots || pos < 0) {
    for (int d = tid; d < D; d += kDT) yg[d] = from_f<IO>(0.f);
    return;
  }
  const size_t sidx = (size_t)sl * hm + ch;
  const int slot = pos % P;
  float* Ag = p.A + sidx * RM;
  float* Bg = p.Bf + sidx * RN;
  float* Ug = p.U + sidx * DP;
  float* Vg = p.Vb + sidx * DP;

  // the token's inputs first (a few scalars per thread), then the state
  // stream: loads retire in order, so staging the inputs below waits only for
  // them, not for the state behind them
  const float gam = fminf(fmaxf(p.dec[chain], 0.f), 1.f);
  const int L = p.qkv_lanes, gc = p.gate_ch;
  const size_t io = (((size_t)row * p.H + h) * L + (L > 1 ? m : 0)) * D;
  const size_t go = (size_t)chain * gc;
  static_assert(D <= kDT, "one input element per thread");
  float in_k = 0.f, in_q = 0.f, in_v = 0.f, in_b = 0.f, in_w = 0.f;
  if (tid < D) {
    in_k = to_f(((const IO*)p.k)[io + tid]);
    in_q = to_f(((const IO*)p.q)[io + tid]);
    in_v = to_f(((const IO*)p.v)[io + tid]);
    in_b = p.bg[go + (gc > 1 ? tid : 0)];
    in_w = p.wg[go + (gc > 1 ? tid : 0)];
  }
  f32x4 ra[NA], rb[NB], ru[NU], rv[NU];
#pragma unroll
  for (int j = 0; j < NA; ++j)
    if (tid + j * kDT < RM / 4) ra[j] = __builtin_nontemporal_load((const f32x4*)Ag + tid + j * kDT);
#pragma unroll
  for (int j = 0; j < NB; ++j)
    if (tid + j * kDT < RN / 4) rb[j] = __builtin_nontemporal_load((const f32x4*)Bg + tid + j * kDT);
#pragma unroll
  for (int j = 0; j < NU; ++j)
    if (tid + j * kDT < DP / 4) {
      ru[j] = ((const f32x4*)Ug)[tid + j * kDT];
      rv[j] = __builtin_nontemporal_load((const f32x4*)Vg + tid + j * kDT);
    }
  if (tid < D) {
    sm.k[tid] = in_k;
    sm.x[0][tid] = in_b * in_k;
    sm.x[1][tid] = in_q;
    sm.u[tid] = in_w * in_v;
  }
#pragma unroll
  for (int j = 0; j < NA; ++j)
    if (tid + j * kDT < RM / 4) {
      ra[j] *= gam;
      *(f32x4*)&sm.A[4 * (tid + j * kDT)] = ra[j];
    }
#pragma unroll
  for (int j = 0; j < NB; ++j)
    if (tid + j * kDT < RN / 4) {
      rb[j] *= gam;
      *(f32x4*)&sm.B[4 * (tid + j * kDT)] = rb[j];
    }
#pragma unroll
  for (int j = 0; j < NU; ++j)
    if (tid + j * kDT < DP / 4) {
      const int e = 4 * (tid + j * kDT), d = e / P, s0 = e % P;
      rv[j] *= gam;
      *(f32x4*)&sm.U[d][s0] = ru[j];
      *(f32x4*)&sm.V[d][s0] = rv[j];
    }
  __syncthreads();

  // k.h and k.q (wave 0)
  if (tid < 64) {
    float kh = 0.f, kq = 0.f;
    for (int d = tid; d < D; d += 64) {
      kh += sm.k[d] * sm.x[0][d];
      kq += sm.k[d] * sm.x[1][d];
    }
    kh = wave_sum(kh);
    kq = wave_sum(kq);
    if (tid == 0) {
      sm.red[0] = kh;
      sm.red[1] = kq;
    }
  }
  // Vb^T h, Vb^T q: a group of TPC lanes per (vector, 4 slots), lane `part`
  // summing rows d = part, part + TPC, ... (consecutive lanes read
  // consecutive rows), then the group's sum
  {
    constexpr int NCB = 2 * (P / 4);           // (vector, slot quad) combinations
    constexpr int TPC = kDT / NCB;             // lanes per combination
    static_assert(TPC >= 1 && TPC <= 32 && (TPC & (TPC - 1)) == 0 && D % TPC == 0, "coef split");
    const int cb = tid / TPC, part = tid % TPC, xi = cb / (P / 4), s0 = 4 * (cb % (P / 4));
    f32x4 acc = zero4();
#pragma unroll 4
    for (int d = part; d < D; d += TPC) acc += *(const f32x4*)&sm.V[d][s0] * sm.x[xi][d];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = group_sum<TPC>(acc[e]);
    if (part == 0) *(f32x4*)&sm.coef[xi][s0] = acc;
  }
  // (A_r X)[iv][jb] = sum_ik A_r[iv][ik] x[ik b_k + jb], four jb per thread
  {
    constexpr int JG = Ge::bk / 4, NO4 = 2 * Ge::R * Ge::av * JG;
#pragma unroll 1
    for (int o = tid; o < NO4; o += kDT) {
      const int jg = o % JG, iv = (o / JG) % Ge::av, r = (o / (JG * Ge::av)) % Ge::R, xi = o / (JG * Ge::av * Ge::R);
      const float* ar = &sm.A[r * Ge::m + iv * Ge::ak];
      const float* xr = &sm.x[xi][4 * jg];
      f32x4 acc = zero4();
#pragma unroll
      for (int i4 = 0; i4 < Ge::ak; i4 += 4) {
        const f32x4 a4 = *(const f32x4*)&ar[i4];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += a4[e] * *(const f32x4*)&xr[(i4 + e) * Ge::bk];
      }
      *(f32x4*)&sm.ax[xi][r][iv][4 * jg] = acc;
    }
  }
  __syncthreads();

  // (S x)[d] at d = iv b_v + jv, one thread per (x, d):
  // sum_r sum_jb (A_r X)[iv][jb] B_r[jv][jb] + sum_p U[d][p] coef[p]
  if (tid < 2 * D) {
    const int xi = tid / D, d = tid % D, iv = d / Ge::bv, jv = d % Ge::bv;
    f32x4 acc = zero4();
#pragma unroll
    for (int r = 0; r < Ge::R; ++r)
#pragma unroll
      for (int j4 = 0; j4 < Ge::bk; j4 += 4)
        acc += *(const f32x4*)&sm.ax[xi][r][iv][j4] * *(const f32x4*)&sm.B[r * Ge::n + jv * Ge::bk + j4];
#pragma unroll
    for (int s4 = 0; s4 < P; s4 += 4) acc += *(const f32x4*)&sm.U[d][s4] * *(const f32x4*)&sm.coef[xi][s4];
    sm.sx[xi][d] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  __syncthreads();
  const float c = sm.red[0], kq = sm.red[1];
  const float alpha = stable_alpha_f(c);
  for (int d = tid; d < D; d += kDT) {
    const float r = sm.u[d] - sm.sx[0][d];
    yg[d] = from_f<IO>(sm.sx[1][d] + alpha * kq * r);
    Ug[(size_t)d * P + slot] = alpha * r;    // the new write; the rest of U is unchanged
  }
  // decayed factors and keys back, the token's key in its slot
#pragma unroll
  for (int j = 0; j < NA; ++j)
    if (tid + j * kDT < RM / 4) __builtin_nontemporal_store(ra[j], (f32x4*)Ag + tid + j * kDT);
#pragma unroll
  for (int j = 0; j < NB; ++j)
    if (tid + j * kDT < RN / 4) __builtin_nontemporal_store(rb[j], (f32x4*)Bg + tid + j * kDT);
#pragma unroll
  for (int j = 0; j < NU; ++j)
    if (tid + j * kDT < DP / 4) {
      const int e = 4 * (tid + j * kDT), d = e / P, s0 = e % P;
      f32x4 o = rv[j];
      if (slot >= s0 && slot < s0 + 4) o[slot - s0] = sm.k[d];
      __builtin_nontemporal_store(o, (f32x4*)Vg + tid + j * kDT);
    }
}

template <typename IO, int D, int P>
int launch_g3_decode(const G3DecArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((gdn3_decode_kernel<IO, D, P>), dim3(a.NS * a.H * a.M), dim3(kDT), 0, stream, a);
  return check_launch("gdn3_decode_kernel");
}

template <typename IO>
int g3_decode_io(const G3DecArgs& a, hipStream_t stream) {
  if (a.D == 128) {
    if (a.P == 16) return launch_g3_decode<IO, 128, 16>(a, stream);
    if (a.P == 32) return launch_g3_decode<IO, 128, 32>(a, stream);
    if (a.P == 64) return launch_g3_decode<IO, 128, 64>(a, stream);
  } else if (a.D == 64) {
    if (a.P == 16) return launch_g3_decode<IO, 64, 16>(a, stream);
    if (a.P == 32) return launch_g3_decode<IO, 64, 32>(a, stream);
    if (a.P == 64) return launch_g3_decode<IO, 64, 64>(a, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "gdn3 decode: unsupported head_dim %d / P %d", a.D, a.P);
}

}  // namespace

int gdn3_decode_dispatch(const G3DecArgs& a, hipStream_t stream) {
  if ((long long)a.NS * a.H * a.M == 0) return GDNX_OK;
  return a.dtype == GDNX_DTYPE_BF16 ? g3_decode_io<bf16>(a, stream) : g3_decode_io<float>(a, stream);
}

}  // namespace gdnx

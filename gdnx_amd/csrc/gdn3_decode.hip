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
// HBM-bound: a chain reads its 21.5 KB state (d = 128, P = 16) and writes
// back A, B, Vb (decayed) and one column of U.  One 256-thread block per
// chain stages the state in LDS with 16-byte loads (non-temporal for the
// parts rewritten in full), forms the two reads S h, S q from LDS
// (Vb^T x as per-slot partial sums folded across lanes, the Kronecker part as
// A_r X, then (A_r X) B_r^T), and writes from the registers it loaded.
#include "gdn3_common.hpp"
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int kDT = 256;   // threads per chain

template <int D, int P>
struct G3DecSmem {
  typedef G3D<D> Ge;
  float A[Ge::R * Ge::m];          // gamma A   [R][a_v][a_k]
  float B[Ge::R * Ge::n];          // gamma B   [R][b_v][b_k]
  float U[D][P + 1];               // U [d][slot] (padded: column reads spread over banks)
  float V[D][P + 1];               // gamma Vb
  float x[2][D];                   // h, q
  float k[D], u[D];
  float ax[2][Ge::R][Ge::av][Ge::bk];   // A_r X for X = h, q
  float coef[2][P];                // (gamma Vb)^T h, (gamma Vb)^T q
  float red[2];                    // k.h, k.q
};

template <typename IO, int D, int P>
__global__ void __launch_bounds__(kDT) gdn3_decode_kernel(G3DecArgs p) {
  typedef G3D<D> Ge;
  constexpr int RM = Ge::R * Ge::m, RN = Ge::R * Ge::n, DP = D * P;
  constexpr int NA = (RM / 4 + kDT - 1) / kDT, NB = (RN / 4 + kDT - 1) / kDT, NU = (DP / 4 + kDT - 1) / kDT;
  static_assert(RM % 4 == 0 && RN % 4 == 0 && DP % 4 == 0 && P % 4 == 0, "16-byte units");
  __shared__ G3DecSmem<D, P> sm;

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

  // the state stream first
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
  const float gam = fminf(fmaxf(p.dec[chain], 0.f), 1.f);
  const int L = p.qkv_lanes, gc = p.gate_ch;
  const size_t io = (((size_t)row * p.H + h) * L + (L > 1 ? m : 0)) * D;
  const size_t go = (size_t)chain * gc;
  for (int d = tid; d < D; d += kDT) {
    const float kk = to_f(((const IO*)p.k)[io + d]);
    const float bb = p.bg[go + (gc > 1 ? d : 0)], ww = p.wg[go + (gc > 1 ? d : 0)];
    sm.k[d] = kk;
    sm.x[0][d] = bb * kk;
    sm.x[1][d] = to_f(((const IO*)p.q)[io + d]);
    sm.u[d] = ww * to_f(((const IO*)p.v)[io + d]);
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
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sm.U[d][s0 + s] = ru[j][s];
        sm.V[d][s0 + s] = rv[j][s];
      }
    }
  __syncthreads();

  // k.h and k.q (wave 0); Vb^T h, Vb^T q as per-slot partials over d ranges
  // folded across the lanes that share a slot; A_r X
  if (tid < 64) {
    float kh = 0.f, kq = 0.f;
    for (int d = tid; d < D; d += 64) {
      kh += sm.k[d] * sm.x[0][d];
      kq += sm.k[d] * sm.x[1][d];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      kh += __shfl_xor(kh, off, 64);
      kq += __shfl_xor(kq, off, 64);
    }
    if (tid == 0) {
      sm.red[0] = kh;
      sm.red[1] = kq;
    }
  }
  {
    constexpr int TPO = kDT / (2 * P);          // threads per (vector, slot) output
    static_assert(TPO >= 1 && (TPO & (TPO - 1)) == 0 && TPO <= 64 && D % TPO == 0, "coef split");
    const int o = tid / TPO, part = tid % TPO, xi = o / P, s = o % P;
    float acc = 0.f;
    for (int d = part; d < D; d += TPO) acc += sm.V[d][s] * sm.x[xi][d];
#pragma unroll
    for (int off = 1; off < TPO; off <<= 1) acc += __shfl_xor(acc, off, 64);
    if (part == 0) sm.coef[xi][s] = acc;
  }
  {
    // (A_r X)[iv][jb] = sum_ik A_r[iv][ik] x[ik b_k + jb]
    constexpr int NO = 2 * Ge::R * Ge::av * Ge::bk;
    for (int o = tid; o < NO; o += kDT) {
      const int jb = o % Ge::bk, iv = (o / Ge::bk) % Ge::av, r = (o / (Ge::bk * Ge::av)) % Ge::R,
                xi = o / (Ge::bk * Ge::av * Ge::R);
      const float* ar = &sm.A[r * Ge::m + iv * Ge::ak];
      float acc = 0.f;
#pragma unroll
      for (int ik = 0; ik < Ge::ak; ++ik) acc += ar[ik] * sm.x[xi][ik * Ge::bk + jb];
      sm.ax[xi][r][iv][jb] = acc;
    }
  }
  __syncthreads();

  // S x at d = iv b_v + jv: sum_r sum_jb (A_r X)[iv][jb] B_r[jv][jb] + sum_p U[d][p] coef[p]
  const float c = sm.red[0], kq = sm.red[1];
  const float alpha = stable_alpha_f(c);
  for (int d = tid; d < D; d += kDT) {
    const int iv = d / Ge::bv, jv = d % Ge::bv;
    float sx[2];
#pragma unroll
    for (int xi = 0; xi < 2; ++xi) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < Ge::R; ++r)
#pragma unroll
        for (int jb = 0; jb < Ge::bk; ++jb) acc += sm.ax[xi][r][iv][jb] * sm.B[r * Ge::n + jv * Ge::bk + jb];
#pragma unroll
      for (int s = 0; s < P; ++s) acc += sm.U[d][s] * sm.coef[xi][s];
      sx[xi] = acc;
    }
    const float r = sm.u[d] - sx[0];
    yg[d] = from_f<IO>(sx[1] + alpha * kq * r);
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

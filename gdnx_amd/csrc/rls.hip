// Rank-r block-Householder delta rule with the RLS T-factor: the recurrence of
// KMD2LinearAttn._scan (gdn3/kmd2.py:166-214) and of the testbed mixer
// (research/testbed_mqar.py:226-262).  Per chain (b, h), state S [dv, dk]
// (value-major, as the reference), per token with R write slots:
//
//   S  <- S diag(a)                          channel decay (key axis)
//   Kt  = Bg * K                             [R, dk] gated erase keys
//   S  <- S - (S Kt^T) (eps I + Kt Kt^T)^-1 Kt
//   S  <- S + (Wg * V)^T K                   rank-R gated write
//   y   = sum_o mix_o S q_o                  RO query slots
//
// The value rows of S evolve independently, so a workgroup holds one chain
// with every lane owning 4 rows x CPL = dk/16 key columns; the 16 lanes of a
// DPP row span the key axis, and all per-row dot products (S Kt^T, S q,
// Kt Kt^T) are DPP reductions inside the row -- no barrier on the token
// path.  Token inputs are staged per chunk of C tokens through LDS, the next
// chunk's global loads in flight while the current one is scanned.
//
// Backward: the forward stores S every CK tokens; the reverse pass reloads a
// checkpoint, recomputes the CK states in registers and runs the adjoint
// token by token.  Per-row gradients (dV, dWg) are written directly; the
// column gradients (dq, dK, dBg, da: sums over the value rows) are reduced
// within the wave by lane swaps, across waves through LDS once per CK tokens,
// in a fixed order (deterministic).
#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int kMaxPre = 4;    // staged float4 per thread per chunk

__device__ __forceinline__ float row_sum16(float x) {
  // rotations 8, 4, 2, 1 inside the DPP row: all 16 lanes form the same sums
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
  return x;
}

// sum over the four DPP rows of the wave (lanes l, l^16, l^32, l^48)
__device__ __forceinline__ float cross_rows4(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

template <int N> __device__ __forceinline__ void lds_vec(const float* p, float* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
      const f32x4 v = *(const f32x4*)(p + j);
      out[j] = v[0];
      out[j + 1] = v[1];
      out[j + 2] = v[2];
      out[j + 3] = v[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = p[j];
  }
}

// (eps I + G)^-1 for the SPD R x R matrix, Gauss-Jordan in registers
template <int R> __device__ __forceinline__ void tfactor(const float G[R][R], float eps, float T[R][R]) {
  if constexpr (R == 1) {
    T[0][0] = 1.0f / (eps + G[0][0]);
  } else {
    float A[R][R];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int j = 0; j < R; ++j) {
        A[i][j] = G[i][j] + (i == j ? eps : 0.0f);
        T[i][j] = i == j ? 1.0f : 0.0f;
      }
#pragma unroll
    for (int p = 0; p < R; ++p) {
      const float inv = 1.0f / A[p][p];
#pragma unroll
      for (int j = 0; j < R; ++j) {
        A[p][j] *= inv;
        T[p][j] *= inv;
      }
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (i == p) continue;
        const float f = A[i][p];
#pragma unroll
        for (int j = 0; j < R; ++j) {
          A[i][j] -= f * A[p][j];
          T[i][j] -= f * T[p][j];
        }
      }
    }
  }
}

struct RlsArgs {
  const float* q;      // [B,T,H,RO,dk]
  const float* K;      // [B,T,H,R,dk]
  const float* V;      // [B,T,H,R,dv]
  const float* Bg;     // [B,T,H,R,dk]
  const float* Wg;     // [B,T,H,R,dv]
  const float* a;      // [B,T,H,dk]
  const float* mix;    // [H,RO] (RO > 1)
  const float* state0; // [B,H,dv,dk] or null
  const float* dy;     // [B,T,H,dv] (backward)
  const float* dstate; // [B,H,dv,dk] gradient of the final state or null (backward)
  float* y;            // [B,T,H,dv]
  float* state_out;    // [B,H,dv,dk] or null
  float* ckpt;         // [B*H, ceil(T/CK), dv, dk]
  float* dq;
  float* dK;
  float* dV;
  float* dBg;
  float* dWg;
  float* da;
  float* dmix;         // [B*H, RO] per chain
  float* dstate0;      // [B,H,dv,dk] or null
  int B, T, H, RO, dk, dv, C, CK;
  float eps;
  int cP, cR, ste;     // testbed compaction: every cP tokens to rank cR (cP = 0: off)
  float cs;            // its slow decay (blend weight of the truncation)
  float* part;         // split backward: per (chain, row block, token) column partials
  float* mixpart;      // split backward: per (chain, token block) out_mix partials
};

// Token record layout in LDS (floats): K [R][dk], Bg [R][dk], a [dk],
// q [RO][dk], V [R][dv], Wg [R][dv], (backward) dy [dv].
struct RecLayout {
  int oK, oBg, oA, oQ, oV, oW, oDy, stride;
  __device__ RecLayout(int R, int RO, int dk, int dv, bool bwd) {
    oK = 0;
    oBg = R * dk;
    oA = 2 * R * dk;
    oQ = oA + dk;
    oV = oQ + RO * dk;
    oW = oV + R * dv;
    oDy = oW + R * dv;
    stride = oDy + (bwd ? dv : 0);
  }
};

// Cooperative chunk staging: global -> registers (issued early) -> LDS.  The
// first kMaxPre float4 per thread are prefetched while the previous chunk is
// scanned; a chunk larger than that is completed synchronously at commit.
struct Stager {
  f32x4 pre[kMaxPre];
  int chain, t0, ntok;
  __device__ f32x4 load(const RlsArgs& g, const RecLayout& L, int R, int f, bool bwd) const {
    const int b = chain / g.H, h = chain % g.H;
    const int U = L.stride / 4;
    const int lens[7] = {R * g.dk, R * g.dk, g.dk, g.RO * g.dk, R * g.dv, R * g.dv, bwd ? g.dv : 0};
    const float* bases[7] = {g.K, g.Bg, g.a, g.q, g.V, g.Wg, g.dy};
    const int tl = f / U;
    int o = 4 * (f - tl * U);
    int arr = 0;
#pragma unroll
    for (int z = 0; z < 6; ++z)
      if (arr == z && o >= lens[z]) {
        o -= lens[z];
        arr = z + 1;
      }
    const float* base = bases[0];
    int len = lens[0];
#pragma unroll
    for (int z = 1; z < 7; ++z)
      if (arr == z) {
        base = bases[z];
        len = lens[z];
      }
    return *(const f32x4*)(base + (((size_t)b * g.T + t0 + tl) * g.H + h) * len + o);
  }
  __device__ void fetch(const RlsArgs& g, const RecLayout& L, int R, int ch, int t, int n, bool bwd) {
    chain = ch;
    t0 = t;
    ntok = n;
    const int U = L.stride / 4, nthr = blockDim.x;
#pragma unroll
    for (int k = 0; k < kMaxPre; ++k) {
      const int f = threadIdx.x + k * nthr;
      pre[k] = f < ntok * U ? load(g, L, R, f, bwd) : zero4();
    }
  }
  __device__ void commit(float* buf, const RlsArgs& g, const RecLayout& L, int R, bool bwd) {
    const int U = L.stride / 4, nthr = blockDim.x;
#pragma unroll
    for (int k = 0; k < kMaxPre; ++k) {
      const int f = threadIdx.x + k * nthr;
      if (f < ntok * U) *(f32x4*)(buf + 4 * f) = pre[k];
    }
    for (int f = threadIdx.x + kMaxPre * nthr; f < ntok * U; f += nthr) *(f32x4*)(buf + 4 * f) = load(g, L, R, f, bwd);
  }
};

// Per-token operands of one lane, read from the staged record.
template <int CPL, int R> struct TokIn {
  float a[CPL], K[R][CPL], Kt[R][CPL], Bg[R][CPL];
  float w[R][4];   // w' = Wg * V of the lane's 4 rows
  float T[R][R];
};

template <int CPL, int R>
__device__ __forceinline__ void load_tok(TokIn<CPL, R>& in, const float* rec, const RecLayout& L, int dk,
                                         int dv, int l16, int rg, float eps) {
  const int c0 = CPL * l16;
  lds_vec<CPL>(rec + L.oA + c0, in.a);
  float G[R][R];
#pragma unroll
  for (int s = 0; s < R; ++s) {
    lds_vec<CPL>(rec + L.oK + s * dk + c0, in.K[s]);
    lds_vec<CPL>(rec + L.oBg + s * dk + c0, in.Bg[s]);
#pragma unroll
    for (int j = 0; j < CPL; ++j) in.Kt[s][j] = in.Bg[s][j] * in.K[s][j];
    float v4[4], g4[4];
    lds_vec<4>(rec + L.oV + s * dv + 4 * rg, v4);
    lds_vec<4>(rec + L.oW + s * dv + 4 * rg, g4);
#pragma unroll
    for (int i = 0; i < 4; ++i) in.w[s][i] = g4[i] * v4[i];
  }
#pragma unroll
  for (int s = 0; s < R; ++s)
#pragma unroll
    for (int u = s; u < R; ++u) {
      float x = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) x += in.Kt[s][j] * in.Kt[u][j];
      G[s][u] = G[u][s] = row_sum16(x);
    }
  tfactor<R>(G, eps, in.T);
}

// One token of the recurrence on the lane's 4 x CPL block; returns p and z
// (the erase projections) for the backward.
template <int CPL, int R>
__device__ __forceinline__ void token_step(float s[4][CPL], const TokIn<CPL, R>& in, float p[R][4], float z[R][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) s[i][j] *= in.a[j];
#pragma unroll
  for (int u = 0; u < R; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) x += s[i][j] * in.Kt[u][j];
      p[u][i] = row_sum16(x);
    }
#pragma unroll
  for (int u = 0; u < R; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = 0.0f;
#pragma unroll
      for (int v = 0; v < R; ++v) x += p[v][i] * in.T[v][u];
      z[u][i] = x;
    }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float x = s[i][j];
#pragma unroll
      for (int u = 0; u < R; ++u) x += in.w[u][i] * in.K[u][j] - z[u][i] * in.Kt[u][j];
      s[i][j] = x;
    }
}


// ---------------------------------------------------------------------------
// Testbed compaction (research/testbed_mqar.py:245-260): after the write of
// every cP-th token, S <- cs S_lr + (1 - cs) S with S_lr the best rank-cR
// approximation of S.  The workgroup writes S to LDS, forms the smaller Gram
// (S S^T or S^T S, m = min(dv, dk) <= 64), diagonalises it by parallel cyclic
// Jacobi (round-robin pairing: m/2 disjoint rotations per round, m - 1 rounds
// per sweep, until the off-diagonal mass is below 1e-12 of the total), keeps
// the eigenvectors of the cR largest eigenvalues and projects.
// ---------------------------------------------------------------------------
__host__ __device__ inline size_t compact_lds_floats(int dk, int dv, int cR, int nthr) {
  const int m = dv <= dk ? dv : dk, n = dv <= dk ? dk : dv;
  return (size_t)dv * dk + 2 * (size_t)m * (m + 1) + m + 2 * m + (size_t)cR * n + nthr + 4;
}

template <int CPL>
__device__ void compact_state(float s[4][CPL], const RlsArgs& g, float* sm, int rg, int c0) {
  const int dk = g.dk, dv = g.dv, nthr = blockDim.x, tid = threadIdx.x;
  const bool vside = dv <= dk;
  const int m = vside ? dv : dk, n = vside ? dk : dv, ld = m + 1, cR = g.cR;
  float* S = sm;                                  // [dv][dk]
  float* A = S + dv * dk;                         // [m][ld]
  float* E = A + m * ld;                          // [m][ld] eigenvectors in columns
  float* rot = E + m * ld;                        // [m/2][2]
  int* sel = (int*)(rot + m);                     // [cR]
  float* Pm = (float*)(sel + 2 * m);              // [cR][n]
  float* red = Pm + cR * n;                       // [nthr]
  int* flag = (int*)(red + nthr);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) S[(4 * rg + i) * dk + c0 + j] = s[i][j];
  __syncthreads();
  float tot = 0.0f;
  for (int e = tid; e < m * m; e += nthr) {
    const int i = e / m, j = e - i * m;
    float x = 0.0f;
    if (vside)
      for (int c = 0; c < n; ++c) x += S[i * dk + c] * S[j * dk + c];
    else
      for (int v = 0; v < n; ++v) x += S[v * dk + i] * S[v * dk + j];
    A[i * ld + j] = x;
    E[i * ld + j] = i == j ? 1.0f : 0.0f;
    tot += x * x;
  }
  red[tid] = tot;
  __syncthreads();
  if (tid == 0) {
    float t = 0.0f;
    for (int k = 0; k < nthr; ++k) t += red[k];
    red[0] = t;
  }
  __syncthreads();
  const float total = red[0];
  __syncthreads();
  const int half = m / 2;
  for (int sweep = 0; sweep < 16; ++sweep) {
    for (int r = 0; r < m - 1; ++r) {
      // round r pairs (r, m-1) and ((r+q) mod (m-1), (r-q) mod (m-1)), q = 1 .. m/2 - 1
      for (int q = tid; q < half; q += nthr) {
        const int p0 = q == 0 ? r : (r + q) % (m - 1);
        const int q0 = q == 0 ? m - 1 : (r - q + (m - 1)) % (m - 1);
        const float app = A[p0 * ld + p0], aqq = A[q0 * ld + q0], apq = A[p0 * ld + q0];
        float c = 1.0f, sn = 0.0f;
        if (fabsf(apq) > 1e-30f && fabsf(apq) > 1e-9f * sqrtf(fabsf(app * aqq))) {
          const float tau = (aqq - app) / (2.0f * apq);
          const float at = fabsf(tau);
          const float t = (tau >= 0.0f ? 1.0f : -1.0f) / (at > 1e15f ? 2.0f * at : at + sqrtf(1.0f + tau * tau));
          c = 1.0f / sqrtf(1.0f + t * t);
          sn = t * c;
        }
        rot[2 * q] = c;
        rot[2 * q + 1] = sn;
      }
      __syncthreads();
      // rows p, q of A <- J^T A
      for (int e = tid; e < half * m; e += nthr) {
        const int q = e / m, j = e - q * m;
        const int p0 = q == 0 ? r : (r + q) % (m - 1);
        const int q0 = q == 0 ? m - 1 : (r - q + (m - 1)) % (m - 1);
        const float c = rot[2 * q], sn = rot[2 * q + 1];
        const float a = A[p0 * ld + j], b = A[q0 * ld + j];
        A[p0 * ld + j] = c * a - sn * b;
        A[q0 * ld + j] = sn * a + c * b;
      }
      __syncthreads();
      // columns p, q of A <- A J, and of the eigenvectors E <- E J
      for (int e = tid; e < half * m; e += nthr) {
        const int q = e / m, i = e - q * m;
        const int p0 = q == 0 ? r : (r + q) % (m - 1);
        const int q0 = q == 0 ? m - 1 : (r - q + (m - 1)) % (m - 1);
        const float c = rot[2 * q], sn = rot[2 * q + 1];
        const float a = A[i * ld + p0], b = A[i * ld + q0];
        A[i * ld + p0] = c * a - sn * b;
        A[i * ld + q0] = sn * a + c * b;
        const float x = E[i * ld + p0], y = E[i * ld + q0];
        E[i * ld + p0] = c * x - sn * y;
        E[i * ld + q0] = sn * x + c * y;
      }
      __syncthreads();
    }
    float off = 0.0f;
    for (int e = tid; e < m * m; e += nthr) {
      const int i = e / m, j = e - i * m;
      if (i != j) off += A[i * ld + j] * A[i * ld + j];
    }
    red[tid] = off;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int k = 0; k < nthr; ++k) t += red[k];
      *flag = t <= 1e-12f * total;
    }
    __syncthreads();
    const bool done = *flag;
    __syncthreads();
    if (done) break;
  }
  // the cR largest eigenvalues (first index on ties)
  if (tid == 0) {
    for (int k = 0; k < cR; ++k) {
      int best = -1;
      float bv = 0.0f;
      for (int i = 0; i < m; ++i) {
        bool used = false;
        for (int u = 0; u < k; ++u) used |= sel[u] == i;
        if (!used && (best < 0 || A[i * ld + i] > bv)) {
          best = i;
          bv = A[i * ld + i];
        }
      }
      sel[k] = best;
    }
  }
  __syncthreads();
  // projection onto the kept eigenvectors: Pm = E_R^T S (value side) or (S E_R)^T (key side)
  for (int e = tid; e < cR * n; e += nthr) {
    const int k = e / n, x = e - k * n, col = sel[k];
    float acc = 0.0f;
    if (vside)
      for (int v = 0; v < m; ++v) acc += E[v * ld + col] * S[v * dk + x];
    else
      for (int c = 0; c < m; ++c) acc += S[x * dk + c] * E[c * ld + col];
    Pm[k * n + x] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int v = 4 * rg + i, c = c0 + j;
      float lr = 0.0f;
      for (int k = 0; k < cR; ++k)
        lr += vside ? E[v * ld + sel[k]] * Pm[k * n + c] : Pm[k * n + v] * E[c * ld + sel[k]];
      s[i][j] = g.cs * lr + (1.0f - g.cs) * s[i][j];
    }
  __syncthreads();
}

template <int CPL, int R, bool COMPACT>
__global__ __launch_bounds__(512) void rls_fwd_kernel(RlsArgs g) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15;
  const int rg = tid >> 4;   // row group: rows 4 rg .. 4 rg + 3
  const int chain = blockIdx.x, h = chain % g.H;
  const int dk = g.dk, dv = g.dv, T = g.T, C = g.C, RO = g.RO;
  const RecLayout L(R, RO, dk, dv, false);
  const int c0 = CPL * l16;
  float mix[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) mix[o] = o < RO ? (RO > 1 ? g.mix[h * RO + o] : 1.0f) : 0.0f;

  float s[4][CPL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      s[i][j] = g.state0 ? g.state0[((size_t)chain * dv + 4 * rg + i) * dk + c0 + j] : 0.0f;

  const int nch = (T + C - 1) / C;
  Stager st;
  if (nch > 0) {
    st.fetch(g, L, R, chain, 0, min(C, T), false);
    st.commit(lds, g, L, R, false);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * C, ntok = min(C, T - t0);
    float* buf = lds + (c & 1) * C * L.stride;
    if (c + 1 < nch) st.fetch(g, L, R, chain, t0 + C, min(C, T - t0 - C), false);
    for (int tl = 0; tl < ntok; ++tl) {
      const int t = t0 + tl;
      if (g.ckpt && t % g.CK == 0) {
        float* ck = g.ckpt + (((size_t)chain * ((T + g.CK - 1) / g.CK + 1) + t / g.CK) * dv + 4 * rg) * dk + c0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < CPL; ++j) ck[(size_t)i * dk + j] = s[i][j];
      }
      const float* rec = buf + tl * L.stride;
      TokIn<CPL, R> in;
      load_tok<CPL, R>(in, rec, L, dk, dv, l16, rg, g.eps);
      float p[R][4], z[R][4];
      token_step<CPL, R>(s, in, p, z);
      if constexpr (COMPACT) {
        if ((t + 1) % g.cP == 0) compact_state<CPL>(s, g, lds + 2 * C * L.stride, rg, c0);
      }
      float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int o = 0; o < 4; ++o) {
        if (o < RO) {
          float qv[CPL];
          lds_vec<CPL>(rec + L.oQ + o * dk + c0, qv);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) x += s[i][j] * qv[j];
            y[i] += mix[o] * row_sum16(x);
          }
        }
      }
      if (l16 == 0)
        *(f32x4*)(g.y + (((size_t)(chain / g.H) * T + t) * g.H + h) * dv + 4 * rg) = (f32x4){y[0], y[1], y[2], y[3]};
    }
    if (c + 1 < nch) st.commit(lds + ((c + 1) & 1) * C * L.stride, g, L, R, false);
    __syncthreads();
  }
  if (g.state_out) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) g.state_out[((size_t)chain * dv + 4 * rg + i) * dk + c0 + j] = s[i][j];
  }
  if (g.ckpt) {   // the final state closes the checkpoint list
    const int nck = (T + g.CK - 1) / g.CK;
    float* ck = g.ckpt + (((size_t)chain * (nck + 1) + nck) * dv + 4 * rg) * dk + c0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) ck[(size_t)i * dk + j] = s[i][j];
  }
}

// ---------------------------------------------------------------------------
// Forward without compaction, rows spread over workgroups.  The value rows of
// S are independent, so a workgroup takes 16 rows of one chain -- one row per
// DPP row, CPL key columns per lane -- and a chain runs on dv / 16
// workgroups: a lane carries CPL state elements instead of 4 CPL, which cuts
// the per-token instruction path (this scan's bound) about 4x.  Token
// operands are staged per chunk through LDS as in rls_fwd_kernel (one copy
// per workgroup, the next chunk's loads in flight); checkpoints and the
// final state use its layout.
// ---------------------------------------------------------------------------
template <int CPL, int R>
__global__ __launch_bounds__(256) void rls_fwd_rb_kernel(RlsArgs g) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15;
  const int nrb = g.dv / 16;
  const int chain = blockIdx.x / nrb, v = 16 * (blockIdx.x % nrb) + (tid >> 4);
  const int b = chain / g.H, h = chain % g.H;
  const int dk = g.dk, dv = g.dv, T = g.T, C = g.C, RO = g.RO;
  const RecLayout L(R, RO, dk, dv, false);
  const int c0 = CPL * l16;
  const int nck = (T + g.CK - 1) / g.CK;
  float mix[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) mix[o] = o < RO ? (RO > 1 ? g.mix[h * RO + o] : 1.0f) : 0.0f;
  float s[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) s[j] = g.state0 ? g.state0[((size_t)chain * dv + v) * dk + c0 + j] : 0.0f;

  const int nch = (T + C - 1) / C;
  Stager st;
  if (nch > 0) {
    st.fetch(g, L, R, chain, 0, min(C, T), false);
    st.commit(lds, g, L, R, false);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * C, ntok = min(C, T - t0);
    const float* buf = lds + (c & 1) * C * L.stride;
    if (c + 1 < nch) st.fetch(g, L, R, chain, t0 + C, min(C, T - t0 - C), false);
    for (int tl = 0; tl < ntok; ++tl) {
      const int t = t0 + tl;
      const float* rec = buf + tl * L.stride;
      if (g.ckpt && t % g.CK == 0) {
        float* ck = g.ckpt + (((size_t)chain * (nck + 1) + t / g.CK) * dv + v) * dk + c0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) ck[j] = s[j];
      }
      float a[CPL], K[R][CPL], Kt[R][CPL], w[R], G[R][R], Tf[R][R];
      lds_vec<CPL>(rec + L.oA + c0, a);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float bg[CPL];
        lds_vec<CPL>(rec + L.oK + r * dk + c0, K[r]);
        lds_vec<CPL>(rec + L.oBg + r * dk + c0, bg);
#pragma unroll
        for (int j = 0; j < CPL; ++j) Kt[r][j] = bg[j] * K[r][j];
        w[r] = rec[L.oW + r * dv + v] * rec[L.oV + r * dv + v];
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int r2 = r; r2 < R; ++r2) {
          float d = 0.0f;
#pragma unroll
          for (int j = 0; j < CPL; ++j) d += Kt[r][j] * Kt[r2][j];
          G[r][r2] = G[r2][r] = row_sum16(d);
        }
      tfactor<R>(G, g.eps, Tf);
#pragma unroll
      for (int j = 0; j < CPL; ++j) s[j] *= a[j];
      float p[R], z[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) d += s[j] * Kt[r][j];
        p[r] = row_sum16(d);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int r2 = 0; r2 < R; ++r2) d += p[r2] * Tf[r2][r];
        z[r] = d;
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float d = s[j];
#pragma unroll
        for (int r = 0; r < R; ++r) d += w[r] * K[r][j] - z[r] * Kt[r][j];
        s[j] = d;
      }
      float y = 0.0f;
#pragma unroll
      for (int o = 0; o < 4; ++o) {
        if (o < RO) {
          float qv[CPL];
          lds_vec<CPL>(rec + L.oQ + o * dk + c0, qv);
          float d = 0.0f;
#pragma unroll
          for (int j = 0; j < CPL; ++j) d += s[j] * qv[j];
          y += mix[o] * row_sum16(d);
        }
      }
      if (l16 == 0) g.y[(((size_t)b * T + t) * g.H + h) * dv + v] = y;
    }
    if (c + 1 < nch) st.commit(lds + ((c + 1) & 1) * C * L.stride, g, L, R, false);
    __syncthreads();
  }
  if (g.state_out) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) g.state_out[((size_t)chain * dv + v) * dk + c0 + j] = s[j];
  }
  if (g.ckpt) {
    float* ck = g.ckpt + (((size_t)chain * (nck + 1) + nck) * dv + v) * dk + c0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) ck[j] = s[j];
  }
}

// Column partials of one token: g = sum_v dy s3 (dk), dK (R dk), dKt (R dk),
// da (dk), then dT (R^2).
__host__ __device__ constexpr int part_len(int R, int dk) { return (2 + 2 * R) * dk + R * R; }

template <int CPL, int R, int CK>
__global__ __launch_bounds__(512) void rls_bwd_kernel(RlsArgs g) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, dr = lane >> 4, wave = tid >> 6;
  const int rg = tid >> 4;
  const int nw = blockDim.x >> 6;
  const int chain = blockIdx.x, b = chain / g.H, h = chain % g.H;
  const int dk = g.dk, dv = g.dv, T = g.T, C = g.C, RO = g.RO;
  const RecLayout L(R, RO, dk, dv, true);
  const int c0 = CPL * l16;
  const int PL = part_len(R, dk);
  float* red = lds + 2 * C * L.stride;        // [nw][CK][PL]
  float* tsh = red + (size_t)nw * CK * PL;    // [CK][R*R] T-factors of the sub-chunk
  float mix[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) mix[o] = o < RO ? (RO > 1 ? g.mix[h * RO + o] : 1.0f) : 0.0f;
  float dmix_acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nck = (T + g.CK - 1) / g.CK;

  float ds[4][CPL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      ds[i][j] = g.dstate ? g.dstate[((size_t)chain * dv + 4 * rg + i) * dk + c0 + j] : 0.0f;

  const int nch = (T + C - 1) / C;
  // checkpoints are visited in decreasing order; the next one is in flight
  // while a sub-chunk is processed
  auto ck_ptr = [&](int k) { return g.ckpt + (((size_t)chain * (nck + 1) + k) * dv + 4 * rg) * dk + c0; };
  float ckn[4][CPL];
  if (nck > 0) {
    const float* ck = ck_ptr(nck - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) ckn[i][j] = ck[(size_t)i * dk + j];
  }
  Stager st;
  if (nch > 0) {
    const int t0 = (nch - 1) * C;
    st.fetch(g, L, R, chain, t0, T - t0, true);
    st.commit(lds + ((nch - 1) & 1) * C * L.stride, g, L, R, true);
  }
  __syncthreads();
  for (int c = nch - 1; c >= 0; --c) {
    const int t0 = c * C, ntok = min(C, T - t0);
    const float* buf = lds + (c & 1) * C * L.stride;
    if (c > 0) st.fetch(g, L, R, chain, t0 - C, C, true);
    const int nsub = (ntok + CK - 1) / CK;
    for (int sc = nsub - 1; sc >= 0; --sc) {
      const int u0 = sc * CK, nu = min(CK, ntok - u0);   // tokens t0 + u0 .. + nu - 1
      // ---- recompute the states before each token of the sub-chunk
      float S0[CK][4][CPL];
      {
        const int k = (t0 + u0) / CK;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < CPL; ++j) S0[0][i][j] = ckn[i][j];
        if (k > 0) {
          const float* ck = ck_ptr(k - 1);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) ckn[i][j] = ck[(size_t)i * dk + j];
        }
      }
#pragma unroll
      for (int u = 1; u < CK; ++u) {
        if (u < nu) {
          TokIn<CPL, R> in;
          load_tok<CPL, R>(in, buf + (u0 + u - 1) * L.stride, L, dk, dv, l16, rg, g.eps);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) S0[u][i][j] = S0[u - 1][i][j];
          float p[R][4], z[R][4];
          token_step<CPL, R>(S0[u], in, p, z);
        }
      }
      // ---- adjoint, last token first
#pragma unroll
      for (int u = CK - 1; u >= 0; --u) {
        if (u < nu) {
          const float* rec = buf + (u0 + u) * L.stride;
          const int t = t0 + u0 + u;
          TokIn<CPL, R> in;
          load_tok<CPL, R>(in, rec, L, dk, dv, l16, rg, g.eps);
          float s1[4][CPL], s3[4][CPL];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) s3[i][j] = S0[u][i][j];
          float p[R][4], z[R][4];
          token_step<CPL, R>(s3, in, p, z);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) s1[i][j] = S0[u][i][j] * in.a[j];
          // read: ds3 += sum_o mix_o dy q_o ; column partial gsum = sum_v dy s3
          float dyv[4];
          lds_vec<4>(rec + L.oDy + 4 * rg, dyv);
          const bool compacted = g.cP && (t + 1) % g.cP == 0;
          if (compacted) {   // the read saw the compacted state: the next checkpoint
            const float* ck = ck_ptr((t + 1) / CK);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int j = 0; j < CPL; ++j) s3[i][j] = ck[(size_t)i * dk + j];
          }
          float gcol[CPL];
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            float x = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) x += dyv[i] * s3[i][j];
            gcol[j] = x;
          }
#pragma unroll
          for (int o = 0; o < 4; ++o) {
            if (o < RO) {
              float qv[CPL];
              lds_vec<CPL>(rec + L.oQ + o * dk + c0, qv);
#pragma unroll
              for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < CPL; ++j) ds[i][j] += mix[o] * dyv[i] * qv[j];
            }
          }
          if (compacted && !g.ste) {   // S_c = cs S_lr + (1 - cs) S, S_lr without gradient
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int j = 0; j < CPL; ++j) ds[i][j] *= 1.0f - g.cs;
          }
          // write: dw'_u = ds3 K_u (rows), column partial dK_u = sum_v w'_u ds3
          float pK[R][CPL], pKt[R][CPL];
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2) {
            float dw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float x = 0.0f;
#pragma unroll
              for (int j = 0; j < CPL; ++j) x += ds[i][j] * in.K[u2][j];
              dw[i] = row_sum16(x);
            }
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
              float x = 0.0f;
#pragma unroll
              for (int i = 0; i < 4; ++i) x += in.w[u2][i] * ds[i][j];
              pK[u2][j] = x;
            }
            if (l16 == 0) {
              float v4[4], g4[4];
              lds_vec<4>(rec + L.oV + u2 * dv + 4 * rg, v4);
              lds_vec<4>(rec + L.oW + u2 * dv + 4 * rg, g4);
              const size_t o = ((((size_t)b * T + t) * g.H + h) * R + u2) * dv + 4 * rg;
              *(f32x4*)(g.dV + o) = (f32x4){dw[0] * g4[0], dw[1] * g4[1], dw[2] * g4[2], dw[3] * g4[3]};
              *(f32x4*)(g.dWg + o) = (f32x4){dw[0] * v4[0], dw[1] * v4[1], dw[2] * v4[2], dw[3] * v4[3]};
            }
          }
          // erase: dz = -ds2 Kt^T (rows), dKt -= sum_v z ds2; dp = dz T; dT = p^T dz
          float dz[R][4];
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float x = 0.0f;
#pragma unroll
              for (int j = 0; j < CPL; ++j) x += ds[i][j] * in.Kt[u2][j];
              dz[u2][i] = -row_sum16(x);
            }
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
              float x = 0.0f;
#pragma unroll
              for (int i = 0; i < 4; ++i) x += z[u2][i] * ds[i][j];
              pKt[u2][j] = -x;
            }
          float dp[R][4];
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float x = 0.0f;
#pragma unroll
              for (int v = 0; v < R; ++v) x += dz[v][i] * in.T[u2][v];
              dp[u2][i] = x;
            }
          float dT[R][R];
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int v = 0; v < R; ++v) {
              float x = 0.0f;
#pragma unroll
              for (int i = 0; i < 4; ++i) x += p[u2][i] * dz[v][i];
              dT[u2][v] = l16 == 0 ? x : 0.0f;   // p, dz are replicated over the DPP row
            }
          // ds1 = ds2 + dp Kt ; dKt += sum_v dp s1 ; da = sum_v ds1 s0 ; ds0 = ds1 a
          float pa[CPL];
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int u2 = 0; u2 < R; ++u2) {
              float x = 0.0f;
#pragma unroll
              for (int i = 0; i < 4; ++i) x += dp[u2][i] * s1[i][j];
              pKt[u2][j] += x;
            }
            float x = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float d1 = ds[i][j];
#pragma unroll
              for (int u2 = 0; u2 < R; ++u2) d1 += dp[u2][i] * in.Kt[u2][j];
              x += d1 * S0[u][i][j];
              ds[i][j] = d1 * in.a[j];
            }
            pa[j] = x;
          }
          // wave partials of the column sums -> LDS
          float* rp = red + ((size_t)wave * CK + u) * PL;
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            const float v0 = cross_rows4(gcol[j]);
            const float v1 = cross_rows4(pa[j]);
            if (dr == 0) {
              rp[c0 + j] = v0;
              rp[(1 + 2 * R) * dk + c0 + j] = v1;
            }
#pragma unroll
            for (int u2 = 0; u2 < R; ++u2) {
              const float w0 = cross_rows4(pK[u2][j]);
              const float w1 = cross_rows4(pKt[u2][j]);
              if (dr == 0) {
                rp[(1 + u2) * dk + c0 + j] = w0;
                rp[(1 + R + u2) * dk + c0 + j] = w1;
              }
            }
          }
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int v = 0; v < R; ++v) {
              // dT summed over the lanes l16 == 0 of the wave's four DPP rows
              const float x = cross_rows4(dT[u2][v]);
              if (lane == 0) rp[(2 + 2 * R) * dk + u2 * R + v] = x;
            }
          if (tid == 0) {
#pragma unroll
            for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
              for (int v = 0; v < R; ++v) tsh[u * R * R + u2 * R + v] = in.T[u2][v];
          }
        }
      }
      __syncthreads();
      // ---- combine the waves' partials: per token and key column
      for (int e = tid; e < nu * dk; e += blockDim.x) {
        const int u = e / dk, col = e - u * dk;
        const int t = t0 + u0 + u;
        const float* rec = buf + (u0 + u) * L.stride;
        float gs = 0.0f, pa = 0.0f, pK[R], pKt[R], dT[R][R];
#pragma unroll
        for (int u2 = 0; u2 < R; ++u2) pK[u2] = pKt[u2] = 0.0f;
#pragma unroll
        for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
          for (int v = 0; v < R; ++v) dT[u2][v] = 0.0f;
        for (int w = 0; w < nw; ++w) {
          const float* rp = red + ((size_t)w * CK + u) * PL;
          gs += rp[col];
          pa += rp[(1 + 2 * R) * dk + col];
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2) {
            pK[u2] += rp[(1 + u2) * dk + col];
            pKt[u2] += rp[(1 + R + u2) * dk + col];
          }
#pragma unroll
          for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
            for (int v = 0; v < R; ++v) dT[u2][v] += rp[(2 + 2 * R) * dk + u2 * R + v];
        }
        // dM = -T dT T (T symmetric); dKt += (dM + dM^T) Kt
        float Tm[R][R], dM[R][R];
#pragma unroll
        for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
          for (int v = 0; v < R; ++v) Tm[u2][v] = tsh[u * R * R + u2 * R + v];
#pragma unroll
        for (int u2 = 0; u2 < R; ++u2)
#pragma unroll
          for (int v = 0; v < R; ++v) {
            float x = 0.0f;
#pragma unroll
            for (int m = 0; m < R; ++m)
#pragma unroll
              for (int n = 0; n < R; ++n) x += Tm[u2][m] * dT[m][n] * Tm[n][v];
            dM[u2][v] = -x;
          }
        const size_t tok = ((size_t)b * T + t) * g.H + h;
#pragma unroll
        for (int u2 = 0; u2 < R; ++u2) {
          float dkt = pKt[u2];
#pragma unroll
          for (int v = 0; v < R; ++v)
            dkt += (dM[u2][v] + dM[v][u2]) * rec[L.oBg + v * dk + col] * rec[L.oK + v * dk + col];
          const float kk = rec[L.oK + u2 * dk + col], bg = rec[L.oBg + u2 * dk + col];
          g.dBg[(tok * R + u2) * dk + col] = dkt * kk;
          g.dK[(tok * R + u2) * dk + col] = pK[u2] + dkt * bg;
        }
#pragma unroll
        for (int o = 0; o < 4; ++o) {
          if (o < RO) {
            g.dq[(tok * RO + o) * dk + col] = mix[o] * gs;
            dmix_acc[o] += rec[L.oQ + o * dk + col] * gs;
          }
        }
        g.da[tok * dk + col] = pa;
      }
      __syncthreads();
    }
    if (c > 0) st.commit(lds + ((c - 1) & 1) * C * L.stride, g, L, R, true);
    __syncthreads();
  }
  if (g.dstate0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) g.dstate0[((size_t)chain * dv + 4 * rg + i) * dk + c0 + j] = ds[i][j];
  }
  // d out_mix of this chain: fixed-order block sum
#pragma unroll
  for (int o = 0; o < 4; ++o) {
    if (o < RO) {
      red[tid] = dmix_acc[o];
      __syncthreads();
      if (tid == 0) {
        float x = 0.0f;
        for (int k = 0; k < (int)blockDim.x; ++k) x += red[k];
        g.dmix[(size_t)chain * RO + o] = x;
      }
      __syncthreads();
    }
  }
}


// ---------------------------------------------------------------------------
// Backward on row blocks (no compaction): a workgroup takes 16 value rows of
// one chain, one row per DPP row, as rls_fwd_rb_kernel does, and a chain runs
// on dv / 16 workgroups.  Row gradients (dV, dWg) are stored directly; each
// workgroup writes its per-token column partials (sum over its 16 rows of
// dy s3, w' ds3, -z ds2 + dp s1, ds1 s0 and p^T dz) to a buffer, and
// rls_bwd_reduce_kernel sums the row blocks in a fixed order and forms dq,
// dK, dBg, da and the out_mix partials.
// ---------------------------------------------------------------------------
template <int CPL, int R, int CK>
__global__ __launch_bounds__(256) void rls_bwd_rb_kernel(RlsArgs g) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, dr = lane >> 4, wave = tid >> 6;
  const int G = g.dv / 16;
  const int chain = blockIdx.x / G, rb = blockIdx.x % G, v = 16 * rb + (tid >> 4);
  const int b = chain / g.H, h = chain % g.H;
  const int dk = g.dk, dv = g.dv, T = g.T, C = g.C, RO = g.RO;
  const RecLayout L(R, RO, dk, dv, true);
  const int c0 = CPL * l16;
  const int PL = part_len(R, dk);
  float* red = lds + 2 * C * L.stride;        // [4 waves][CK][PL]
  float mix[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) mix[o] = o < RO ? (RO > 1 ? g.mix[h * RO + o] : 1.0f) : 0.0f;
  const int nck = (T + CK - 1) / CK;
  float ds[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) ds[j] = g.dstate ? g.dstate[((size_t)chain * dv + v) * dk + c0 + j] : 0.0f;
  auto ck_ptr = [&](int k) { return g.ckpt + (((size_t)chain * (nck + 1) + k) * dv + v) * dk + c0; };
  float ckn[CPL];
  if (nck > 0) {
    const float* ck = ck_ptr(nck - 1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) ckn[j] = ck[j];
  }
  // operands of one token for this lane's row
  struct Tok {
    float a[CPL], K[R][CPL], Kt[R][CPL], w[R], T[R][R];
  };
  auto load = [&](Tok& x, const float* rec) {
    lds_vec<CPL>(rec + L.oA + c0, x.a);
    float G2[R][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float bg[CPL];
      lds_vec<CPL>(rec + L.oK + r * dk + c0, x.K[r]);
      lds_vec<CPL>(rec + L.oBg + r * dk + c0, bg);
#pragma unroll
      for (int j = 0; j < CPL; ++j) x.Kt[r][j] = bg[j] * x.K[r][j];
      x.w[r] = rec[L.oW + r * dv + v] * rec[L.oV + r * dv + v];
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int r2 = r; r2 < R; ++r2) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) d += x.Kt[r][j] * x.Kt[r2][j];
        G2[r][r2] = G2[r2][r] = row_sum16(d);
      }
    tfactor<R>(G2, g.eps, x.T);
  };
  // s (state before the token) -> s after it; p, z the erase projections
  auto step = [&](float st[CPL], const Tok& x, float p[R], float z[R]) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) st[j] *= x.a[j];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) d += st[j] * x.Kt[r][j];
      p[r] = row_sum16(d);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float d = 0.0f;
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2) d += p[r2] * x.T[r2][r];
      z[r] = d;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float d = st[j];
#pragma unroll
      for (int r = 0; r < R; ++r) d += x.w[r] * x.K[r][j] - z[r] * x.Kt[r][j];
      st[j] = d;
    }
  };

  const int nch = (T + C - 1) / C;
  Stager stg;
  if (nch > 0) {
    const int t0 = (nch - 1) * C;
    stg.fetch(g, L, R, chain, t0, T - t0, true);
    stg.commit(lds + ((nch - 1) & 1) * C * L.stride, g, L, R, true);
  }
  __syncthreads();
  for (int c = nch - 1; c >= 0; --c) {
    const int t0 = c * C, ntok = min(C, T - t0);
    const float* buf = lds + (c & 1) * C * L.stride;
    if (c > 0) stg.fetch(g, L, R, chain, t0 - C, C, true);
    const int nsub = (ntok + CK - 1) / CK;
    for (int sc = nsub - 1; sc >= 0; --sc) {
      const int u0 = sc * CK, nu = min(CK, ntok - u0);
      float S0[CK][CPL];
      {
        const int k = (t0 + u0) / CK;
#pragma unroll
        for (int j = 0; j < CPL; ++j) S0[0][j] = ckn[j];
        if (k > 0) {
          const float* ck = ck_ptr(k - 1);
#pragma unroll
          for (int j = 0; j < CPL; ++j) ckn[j] = ck[j];
        }
      }
#pragma unroll
      for (int u = 1; u < CK; ++u) {
        if (u < nu) {
          Tok x;
          load(x, buf + (u0 + u - 1) * L.stride);
#pragma unroll
          for (int j = 0; j < CPL; ++j) S0[u][j] = S0[u - 1][j];
          float p[R], z[R];
          step(S0[u], x, p, z);
        }
      }
#pragma unroll
      for (int u = CK - 1; u >= 0; --u) {
        if (u < nu) {
          const float* rec = buf + (u0 + u) * L.stride;
          const int t = t0 + u0 + u;
          const size_t tok = ((size_t)b * T + t) * g.H + h;
          Tok x;
          load(x, rec);
          float s1[CPL], s3[CPL], p[R], z[R];
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            s1[j] = S0[u][j] * x.a[j];
            s3[j] = S0[u][j];
          }
          step(s3, x, p, z);
          const float dyv = rec[L.oDy + v];
          float gcol[CPL];
#pragma unroll
          for (int j = 0; j < CPL; ++j) gcol[j] = dyv * s3[j];
#pragma unroll
          for (int o = 0; o < 4; ++o) {
            if (o < RO) {
              float qv[CPL];
              lds_vec<CPL>(rec + L.oQ + o * dk + c0, qv);
#pragma unroll
              for (int j = 0; j < CPL; ++j) ds[j] += mix[o] * dyv * qv[j];
            }
          }
          float pK[R][CPL], pKt[R][CPL], dz[R], dp[R], dT[R][R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float d = 0.0f, e = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
              d += ds[j] * x.K[r][j];
              e += ds[j] * x.Kt[r][j];
              pK[r][j] = x.w[r] * ds[j];
              pKt[r][j] = -z[r] * ds[j];
            }
            const float dw = row_sum16(d);
            dz[r] = -row_sum16(e);
            if (l16 == 0) {
              const float vv = rec[L.oV + r * dv + v], gw = rec[L.oW + r * dv + v];
              g.dV[(tok * R + r) * dv + v] = dw * gw;
              g.dWg[(tok * R + r) * dv + v] = dw * vv;
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float d = 0.0f;
#pragma unroll
            for (int r2 = 0; r2 < R; ++r2) d += dz[r2] * x.T[r][r2];
            dp[r] = d;
          }
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int r2 = 0; r2 < R; ++r2) dT[r][r2] = l16 == 0 ? p[r] * dz[r2] : 0.0f;
          float pa[CPL];
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            float d1 = ds[j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              pKt[r][j] += dp[r] * s1[j];
              d1 += dp[r] * x.Kt[r][j];
            }
            pa[j] = d1 * S0[u][j];
            ds[j] = d1 * x.a[j];
          }
          // the wave's four rows -> LDS
          float* rp = red + ((size_t)wave * CK + u) * PL;
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            const float v0 = cross_rows4(gcol[j]);
            const float v1 = cross_rows4(pa[j]);
            if (dr == 0) {
              rp[c0 + j] = v0;
              rp[(1 + 2 * R) * dk + c0 + j] = v1;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const float w0 = cross_rows4(pK[r][j]);
              const float w1 = cross_rows4(pKt[r][j]);
              if (dr == 0) {
                rp[(1 + r) * dk + c0 + j] = w0;
                rp[(1 + R + r) * dk + c0 + j] = w1;
              }
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int r2 = 0; r2 < R; ++r2) {
              const float xx = cross_rows4(dT[r][r2]);
              if (lane == 0) rp[(2 + 2 * R) * dk + r * R + r2] = xx;
            }
        }
      }
      __syncthreads();
      // this row block's partials of the sub-chunk's tokens, waves summed in order
      for (int e = tid; e < nu * PL; e += 256) {
        const int u = e / PL, xi = e - u * PL;
        const float* rp = red + (size_t)u * PL + xi;
        const size_t wstride = (size_t)CK * PL;
        g.part[(((size_t)chain * G + rb) * T + t0 + u0 + u) * PL + xi] =
            (rp[0] + rp[wstride]) + (rp[2 * wstride] + rp[3 * wstride]);
      }
      __syncthreads();
    }
    if (c > 0) stg.commit(lds + ((c - 1) & 1) * C * L.stride, g, L, R, true);
    __syncthreads();
  }
  if (g.dstate0) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) g.dstate0[((size_t)chain * dv + v) * dk + c0 + j] = ds[j];
  }
}

// Column gradients from the row-block partials: one workgroup per (chain,
// block of kRedTok tokens); per token the T-factor is recomputed from K, Bg
// and dT = sum of the blocks' p^T dz turns into dM = -T dT T.
constexpr int kRedTok = 16;

template <int R>
__global__ __launch_bounds__(256) void rls_bwd_reduce_kernel(RlsArgs g) {
  __shared__ float Tm[kRedTok][R * R], dTm[kRedTok][R * R], red[256];
  const int tid = threadIdx.x;
  const int nblk = (g.T + kRedTok - 1) / kRedTok;
  const int chain = blockIdx.x / nblk, blk = blockIdx.x % nblk;
  const int b = chain / g.H, h = chain % g.H;
  const int dk = g.dk, T = g.T, RO = g.RO, G = g.dv / 16;
  const int PL = part_len(R, dk);
  const int t0 = blk * kRedTok, nt = min(kRedTok, T - t0);
  // per token: the Gram of the erase keys and the row blocks' dT
  if (tid < nt) {
    const int t = t0 + tid;
    const size_t tok = ((size_t)b * T + t) * g.H + h;
    float Gm[R][R], Tf[R][R];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int r2 = r; r2 < R; ++r2) {
        float d = 0.0f;
        for (int c = 0; c < dk; ++c) {
          const float x1 = g.Bg[(tok * R + r) * dk + c] * g.K[(tok * R + r) * dk + c];
          const float x2 = g.Bg[(tok * R + r2) * dk + c] * g.K[(tok * R + r2) * dk + c];
          d += x1 * x2;
        }
        Gm[r][r2] = Gm[r2][r] = d;
      }
    tfactor<R>(Gm, g.eps, Tf);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2) {
        float d = 0.0f;
        for (int k = 0; k < G; ++k)
          d += g.part[(((size_t)chain * G + k) * T + t) * PL + (2 + 2 * R) * dk + r * R + r2];
        dTm[tid][r * R + r2] = d;
        Tm[tid][r * R + r2] = Tf[r][r2];
      }
  }
  __syncthreads();
  float mixacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float mixv[4];
#pragma unroll
  for (int o = 0; o < 4; ++o) mixv[o] = o < RO ? (RO > 1 ? g.mix[h * RO + o] : 1.0f) : 0.0f;
  for (int e = tid; e < nt * dk; e += 256) {
    const int u = e / dk, col = e - u * dk;
    const int t = t0 + u;
    const size_t tok = ((size_t)b * T + t) * g.H + h;
    float gs = 0.0f, pa = 0.0f, pK[R], pKt[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pK[r] = pKt[r] = 0.0f;
    for (int k = 0; k < G; ++k) {
      const float* pp = g.part + (((size_t)chain * G + k) * T + t) * PL;
      gs += pp[col];
      pa += pp[(1 + 2 * R) * dk + col];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        pK[r] += pp[(1 + r) * dk + col];
        pKt[r] += pp[(1 + R + r) * dk + col];
      }
    }
    float dM[R][R];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2) {
        float x = 0.0f;
#pragma unroll
        for (int m = 0; m < R; ++m)
#pragma unroll
          for (int n = 0; n < R; ++n) x += Tm[u][r * R + m] * dTm[u][m * R + n] * Tm[u][n * R + r2];
        dM[r][r2] = -x;
      }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float dkt = pKt[r];
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2)
        dkt += (dM[r][r2] + dM[r2][r]) * g.Bg[(tok * R + r2) * dk + col] * g.K[(tok * R + r2) * dk + col];
      const float kk = g.K[(tok * R + r) * dk + col], bg = g.Bg[(tok * R + r) * dk + col];
      g.dBg[(tok * R + r) * dk + col] = dkt * kk;
      g.dK[(tok * R + r) * dk + col] = pK[r] + dkt * bg;
    }
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      if (o < RO) {
        g.dq[(tok * RO + o) * dk + col] = mixv[o] * gs;
        mixacc[o] += g.q[(tok * RO + o) * dk + col] * gs;
      }
    }
    g.da[tok * dk + col] = pa;
  }
#pragma unroll
  for (int o = 0; o < 4; ++o) {
    if (o < RO) {
      red[tid] = mixacc[o];
      __syncthreads();
      if (tid == 0) {
        float x = 0.0f;
        for (int k = 0; k < 256; ++k) x += red[k];
        g.mixpart[((size_t)chain * nblk + blk) * RO + o] = x;
      }
      __syncthreads();
    }
  }
}

__global__ void rls_mix_sum_kernel(RlsArgs g, int nblk) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= g.B * g.H * g.RO) return;
  const int chain = e / g.RO, o = e % g.RO;
  float x = 0.0f;
  for (int k = 0; k < nblk; ++k) x += g.mixpart[((size_t)chain * nblk + k) * g.RO + o];
  g.dmix[e] = x;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// checkpoint interval: the backward keeps CK states per lane in registers; a
// compaction falls on the last token of a CK group (cP a multiple of CK)
int rls_ck(int dk, int R, int cP) {
  const int ck = (dk <= 32 && R <= 3) || (dk == 64 && R == 1) ? 4 : 2;
  return cP % ck == 0 ? ck : 2;
}

struct RlsGeom {
  int C, CK, threads;
  size_t lds;
};

static RlsGeom rls_geom(int R, int RO, int dk, int dv, bool bwd, int cP, int cR) {
  RlsGeom G{};
  G.CK = rls_ck(dk, R, cP);
  G.threads = 4 * dv;
  const int stride = (2 * R + 1 + RO) * dk + 2 * R * dv + (bwd ? dv : 0);
  const int nw = G.threads / 64;
  const size_t red = bwd ? ((size_t)nw * G.CK * part_len(R, dk) + (size_t)G.CK * R * R) * 4
                         : (cP ? compact_lds_floats(dk, dv, cR, G.threads) * 4 : 0);
  const size_t budget = 156 * 1024;
  // largest chunk that fits LDS, preferring one whose loads all prefetch
  G.C = 0;
  for (int pass = 0; pass < 2 && G.C == 0; ++pass)
    for (int C = 32; C >= G.CK; C >>= 1) {
      const size_t lds = (size_t)2 * C * stride * 4 + red;
      if (lds <= budget && (pass == 1 || C * (stride / 4) <= kMaxPre * G.threads)) {
        G.C = C;
        G.lds = lds;
        break;
      }
    }
  return G;
}

template <int CPL, int R>
static int launch_rls(const RlsArgs& a0, bool bwd, hipStream_t stream) {
  RlsArgs a = a0;
  a.CK = rls_ck(a.dk, R, a.cP);
  const unsigned nchains = (unsigned)(a.B * a.H);
  if (!bwd && !a.cP) {
    // the workgroup stages a chunk for 256 threads (16 rows)
    const int stride = (2 * R + 1 + a.RO) * a.dk + 2 * R * a.dv;
    int C = 32;
    while (C > a.CK && ((size_t)2 * C * stride * 4 > 64 * 1024 || C * (stride / 4) > kMaxPre * 256)) C >>= 1;
    if ((size_t)2 * C * stride * 4 > 64 * 1024) return set_error(GDNX_ERR_SHAPE, "RLS scan: record too large for LDS");
    a.C = C;
    const size_t lds = (size_t)2 * C * stride * 4;
    auto k = rls_fwd_rb_kernel<CPL, R>;
    hipLaunchKernelGGL(k, dim3(nchains * (unsigned)(a.dv / 16)), dim3(256), lds, stream, a);
    return check_launch("rls_fwd_rb_kernel");
  }
  if (bwd && !a.cP && a.part) {
    // row blocks of 16 value rows: chunk records + the waves' partials in LDS
    const int strideb = (2 * R + 1 + a.RO) * a.dk + 2 * R * a.dv + a.dv;
    const size_t red = (size_t)4 * a.CK * part_len(R, a.dk) * 4;
    int C = 0;
    size_t lds = 0;
    for (int pass = 0; pass < 2 && C == 0; ++pass)
      for (int c = 32; c >= a.CK; c >>= 1) {
        const size_t l = (size_t)2 * c * strideb * 4 + red;
        if (l <= 156 * 1024 && (pass == 1 || c * (strideb / 4) <= kMaxPre * 256)) {
          C = c;
          lds = l;
          break;
        }
      }
    if (C == 0) return set_error(GDNX_ERR_SHAPE, "RLS backward: record too large for LDS");
    a.C = C;
    const unsigned G = (unsigned)(a.dv / 16);
    if (a.CK == 2) {
      auto k = rls_bwd_rb_kernel<CPL, R, 2>;
      if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return set_error(GDNX_ERR_HIP, "rls_bwd_rb_kernel: cannot reserve %zu bytes of LDS", lds);
      hipLaunchKernelGGL(k, dim3(nchains * G), dim3(256), lds, stream, a);
    } else {
      auto k = rls_bwd_rb_kernel<CPL, R, 4>;
      if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return set_error(GDNX_ERR_HIP, "rls_bwd_rb_kernel: cannot reserve %zu bytes of LDS", lds);
      hipLaunchKernelGGL(k, dim3(nchains * G), dim3(256), lds, stream, a);
    }
    int rc = check_launch("rls_bwd_rb_kernel");
    if (rc != GDNX_OK) return rc;
    const int nblk = (a.T + kRedTok - 1) / kRedTok;
    hipLaunchKernelGGL((rls_bwd_reduce_kernel<R>), dim3(nchains * (unsigned)nblk), dim3(256), 0, stream, a);
    rc = check_launch("rls_bwd_reduce_kernel");
    if (rc != GDNX_OK) return rc;
    hipLaunchKernelGGL(rls_mix_sum_kernel, dim3((nchains * a.RO + 255) / 256), dim3(256), 0, stream, a, nblk);
    return check_launch("rls_mix_sum_kernel");
  }
  const RlsGeom G = rls_geom(R, a0.RO, a0.dk, a0.dv, bwd, a0.cP, a0.cR);
  if (G.C == 0) return set_error(GDNX_ERR_SHAPE, "RLS scan: R=%d, R_out=%d, key_dim=%d, value_dim=%d do not fit LDS",
                                 R, a0.RO, a0.dk, a0.dv);
  a.C = G.C;
  if (!bwd) {
    auto k = a.cP ? rls_fwd_kernel<CPL, R, true> : rls_fwd_kernel<CPL, R, false>;
    if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)G.lds) != hipSuccess)
      return set_error(GDNX_ERR_HIP, "rls_fwd_kernel: cannot reserve %zu bytes of LDS", G.lds);
    hipLaunchKernelGGL(k, dim3(nchains), dim3(G.threads), G.lds, stream, a);
    return check_launch("rls_fwd_kernel");
  }
  if (G.CK == 2) {
    auto k = rls_bwd_kernel<CPL, R, 2>;
    if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)G.lds) != hipSuccess)
      return set_error(GDNX_ERR_HIP, "rls_bwd_kernel: cannot reserve %zu bytes of LDS", G.lds);
    hipLaunchKernelGGL(k, dim3(nchains), dim3(G.threads), G.lds, stream, a);
  } else {
    auto k = rls_bwd_kernel<CPL, R, 4>;
    if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)G.lds) != hipSuccess)
      return set_error(GDNX_ERR_HIP, "rls_bwd_kernel: cannot reserve %zu bytes of LDS", G.lds);
    hipLaunchKernelGGL(k, dim3(nchains), dim3(G.threads), G.lds, stream, a);
  }
  return check_launch("rls_bwd_kernel");
}

template <int CPL>
static int launch_rls_r(const RlsArgs& a, int R, bool bwd, hipStream_t stream) {
  switch (R) {
    case 1: return launch_rls<CPL, 1>(a, bwd, stream);
    case 2: return launch_rls<CPL, 2>(a, bwd, stream);
    case 3: return launch_rls<CPL, 3>(a, bwd, stream);
    default: return launch_rls<CPL, 4>(a, bwd, stream);
  }
}

}  // namespace

size_t rls_bwd_workspace_bytes(int nchains, int T, int R, int dk, int dv) {
  const size_t part = (size_t)nchains * (dv / 16) * T * part_len(R, dk);
  const size_t mix = (size_t)nchains * ((T + kRedTok - 1) / kRedTok) * 4;
  return (part + mix) * sizeof(float) + 256;
}

size_t rls_ckpt_bytes(int nchains, int T, int R, int dk, int dv, int cP) {
  const int CK = rls_ck(dk, R, cP);
  return (size_t)nchains * ((T + CK - 1) / CK + 1) * dv * dk * sizeof(float);
}

int rls_dispatch(const RlsDesc& d, bool bwd, hipStream_t stream) {
  RlsArgs a{};
  a.q = d.q; a.K = d.K; a.V = d.V; a.Bg = d.Bg; a.Wg = d.Wg; a.a = d.a; a.mix = d.mix;
  a.state0 = d.state0; a.dy = d.dy; a.dstate = d.dstate; a.y = d.y; a.state_out = d.state_out;
  a.ckpt = d.ckpt; a.dq = d.dq; a.dK = d.dK; a.dV = d.dV; a.dBg = d.dBg; a.dWg = d.dWg; a.da = d.da;
  a.dmix = d.dmix; a.dstate0 = d.dstate0;
  a.B = d.B; a.T = d.T; a.H = d.H; a.RO = d.RO; a.dk = d.dk; a.dv = d.dv; a.eps = d.eps;
  a.cP = d.cP; a.cR = d.cR; a.cs = d.cs; a.ste = d.ste;
  if (d.workspace && !d.cP) {
    a.part = (float*)d.workspace;
    a.mixpart = a.part + (size_t)(d.B * d.H) * (d.dv / 16) * d.T * part_len(d.R, d.dk);
  }
  if (d.T == 0) return GDNX_OK;
  switch (d.dk) {
    case 32: return launch_rls_r<2>(a, d.R, bwd, stream);
    case 64: return launch_rls_r<4>(a, d.R, bwd, stream);
    default: return launch_rls_r<8>(a, d.R, bwd, stream);
  }
}

}  // namespace gdnx

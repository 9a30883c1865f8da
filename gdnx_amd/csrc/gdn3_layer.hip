// Boundary pre-ops and post-ops of the GDN3 layer, fused.
//
// GDN3LinearAttn.forward (gdn3/gdn3_upgrade.py:785-856) surrounds the
// recurrence with element-wise work that torch runs as ~30 separate kernels
// over lane-expanded [B,T,H,M,*] tensors:
//   prologue  b_gates = sigmoid(b_proj + 0.1 proj_a)              (:799-802)
//             w_gates = sigmoid(w_proj + 0.1 proj_b)              (:804-807)
//             decay   = min(mean_tau exp(-min(softplus(x), 5) rate_tau), clamp)  (:811-822)
//             q_m, k_m = lane RoPE of the lane-shared q, k        (:827-828, :378-401)
//   epilogue  out = normalize(sum_m softmax_m(logits) y_m) sqrt(V) norm   (:842-856)
// Here each direction of each is one pass over HBM that reads every input
// once and writes every output once.  The pre-ops run one workgroup per
// token (b, t): its RoPE angles are staged in LDS once and each wave takes
// one (b, t, h) row at a time, issuing all of the row's loads before any
// use, so a wave keeps the whole row (2.5 KB forward, 10 KB backward at the
// layer shape) in flight; the RoPE partners are read back from the wave's
// own LDS slice.  The post-ops give each row 16 lanes (one DPP row), so a
// wave streams four rows at once and reduces within its DPP rows.  All
// arithmetic is float32.
//
// Lane RoPE (per lane m, d = pairs[m] half-split pairs (x_i, x_{d+i})):
//   x_i'     = x_i cos - x_{d+i} sin
//   x_{d+i}' = x_i' sin + x_{d+i} cos
// The second half reads the UPDATED first half, because the reference writes
// the first half into the tensor that x1/x2 view before it computes the second
// (:396-398); with bf16 IO, x_i' is rounded to bf16 before that use, as the
// in-place write rounds it.  cos/sin come from the caller's [M, T, K/2] tables
// (the reference caches them per (lane, T) on the device, :342-376); a lane
// with pairs[m] = 0 is the identity.
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {
namespace {

constexpr int kWaves = 4;          // waves per workgroup
constexpr int kEpiRows = 16;       // epilogue rows per workgroup (16 lanes each)
constexpr int kEpiMaxParts = 2048; // epilogue backward: partial d_norm rows

template <typename IO> struct Vec4T;
template <> struct Vec4T<bf16> { typedef bf16x4 type; };
template <> struct Vec4T<float> { typedef f32x4 type; };

template <typename IO> __device__ __forceinline__ void st4io(IO* p, const f32x4& x) {
  *(typename Vec4T<IO>::type*)p =
      (typename Vec4T<IO>::type){from_f<IO>(x[0]), from_f<IO>(x[1]), from_f<IO>(x[2]), from_f<IO>(x[3])};
}
template <typename IO> __device__ __forceinline__ float round_io(float x) { return to_f(from_f<IO>(x)); }

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + __expf(-x)); }

// torch softplus (beta 1, threshold 20)
__device__ __forceinline__ float softplusf(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// RoPE output j of lane m from the lane-shared row x (LDS).
template <typename IO>
__device__ __forceinline__ float rope_out(const float* x, int j, int d, const float* cs, const float* sn) {
  if (j < d) return x[j] * cs[j] - x[j + d] * sn[j];
  if (j < 2 * d) {
    const int i = j - d;
    const float x1n = round_io<IO>(x[i] * cs[i] - x[j] * sn[i]);
    return x1n * sn[i] + x[j] * cs[i];
  }
  return x[j];
}

// Gradient of the lane-shared input element j from lane m's output gradient g.
__device__ __forceinline__ float rope_grad(const float* g, int j, int d, const float* cs, const float* sn) {
  if (j < d) return (g[j] + g[j + d] * sn[j]) * cs[j];
  if (j < 2 * d) {
    const int i = j - d;
    const float t = g[i] + g[j] * sn[i];
    return g[j] * cs[i] - t * sn[i];
  }
  return g[j];
}



// Sum over the 16 lanes of each DPP row, left in every lane of the row.  The
// rotations 8, 4, 2, 1 pair lane i with i^8, i^4, i^2, i^1 in value, so all
// sixteen lanes form the same sums in the same order: bitwise equal results.
__device__ __forceinline__ int lane_pairs(const int (&p)[4], int m) {
  return m == 0 ? p[0] : m == 1 ? p[1] : m == 2 ? p[2] : p[3];
}

__device__ __forceinline__ float row_sum16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
  return x;
}

// LDS accesses of one wave to its own slice: order them without a workgroup barrier
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <typename IO> __device__ __forceinline__ f32x4 cvt4(const typename Vec4T<IO>::type& v) {
  return (f32x4){to_f(v[0]), to_f(v[1]), to_f(v[2]), to_f(v[3])};
}

// Stage this token's RoPE angles, [m * half + i] for i < pairs[m].
__device__ __forceinline__ void stage_tables(const G3ProArgs& a, int t, float* tc, float* ts) {
  const int half = a.K >> 1;
  for (int e = threadIdx.x; e < a.M * half; e += 256) {
    const int m = e / half, i = e - m * half;
    if (i < lane_pairs(a.pairs, m)) {
      const size_t o = ((size_t)m * a.T + t) * half + i;
      tc[e] = a.cs[o];
      ts[e] = a.sn[o];
    }
  }
}

// NG: groups of 4 elements per lane covering M*K and M*V (<= 4 * 256)
template <typename IO, int NG>
__global__ __launch_bounds__(256) void g3_prologue_fwd_kernel(G3ProArgs a) {
  typedef typename Vec4T<IO>::type V4;
  __shared__ float tc[4 * 128], ts[4 * 128];
  __shared__ float xs[kWaves][2][256];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int K = a.K, V = a.V, M = a.M, H = a.H, half = K >> 1;
  const long long tok = blockIdx.x;
  const int t = (int)(tok % a.T);
  stage_tables(a, t, tc, ts);
  __syncthreads();
  const IO* __restrict__ gq = (const IO*)a.q;
  const IO* __restrict__ gk = (const IO*)a.k;
  const IO* __restrict__ gbp = (const IO*)a.bp;
  const IO* __restrict__ gwp = (const IO*)a.wp;
  const IO* __restrict__ gdp = (const IO*)a.dp;
  for (int h = wv; h < H; h += kWaves) {
    const long long r = tok * H + h;
    // every load of the row first
    V4 xq = {}, xk = {}, b[NG], w[NG], dp = {};
    if (4 * lane < K) {
      xq = *(const V4*)(gq + r * K + 4 * lane);
      xk = *(const V4*)(gk + r * K + 4 * lane);
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int e = 4 * lane + 256 * g;
      b[g] = e < M * K ? *(const V4*)(gbp + r * M * K + e) : V4{};
      w[g] = e < M * V ? *(const V4*)(gwp + r * M * V + e) : V4{};
    }
    if (lane < M) dp = *(const V4*)(gdp + (r * M + lane) * 4);
    const float pa = to_f(((const IO*)a.pa)[r]) * 0.1f, pb = to_f(((const IO*)a.pb)[r]) * 0.1f;

    if (4 * lane < K) {
      *(f32x4*)&xs[wv][0][4 * lane] = cvt4<IO>(xq);
      *(f32x4*)&xs[wv][1][4 * lane] = cvt4<IO>(xk);
    }
    wave_lds_sync();
    IO* qr = (IO*)a.qr + r * M * K;
    IO* kr = (IO*)a.kr + r * M * K;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int e = 4 * lane + 256 * g;
      if (e < M * K) {
        const int m = e / K, j0 = e - m * K;
        const int d = lane_pairs(a.pairs, m);
        f32x4 oq, ok;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          oq[c] = rope_out<IO>(xs[wv][0], j0 + c, d, tc + m * half, ts + m * half);
          ok[c] = rope_out<IO>(xs[wv][1], j0 + c, d, tc + m * half, ts + m * half);
        }
        st4io(qr + e, oq);
        st4io(kr + e, ok);
        const f32x4 x = cvt4<IO>(b[g]);
        *(f32x4*)(a.bg + r * M * K + e) =
            (f32x4){sigmoidf(x[0] + pa), sigmoidf(x[1] + pa), sigmoidf(x[2] + pa), sigmoidf(x[3] + pa)};
      }
      if (e < M * V) {
        const f32x4 x = cvt4<IO>(w[g]);
        *(f32x4*)(a.wg + r * M * V + e) =
            (f32x4){sigmoidf(x[0] + pb), sigmoidf(x[1] + pb), sigmoidf(x[2] + pb), sigmoidf(x[3] + pb)};
      }
    }
    if (lane < M) {
      const f32x4 x = cvt4<IO>(dp);
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) s += expf(-fminf(softplusf(x[c]), 5.0f) * a.rates[c]);
      a.dec[r * M + lane] = fminf(s / 4.0f, a.clamp);
    }
    wave_lds_sync();   // the next row's staging must follow this row's reads
  }
}

template <typename IO, int NG>
__global__ __launch_bounds__(256) void g3_prologue_bwd_kernel(G3ProArgs a) {
  typedef typename Vec4T<IO>::type V4;
  __shared__ float tc[4 * 128], ts[4 * 128];
  __shared__ float gs[kWaves][2][4 * 256];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int K = a.K, V = a.V, M = a.M, H = a.H, half = K >> 1;
  const long long tok = blockIdx.x;
  const int t = (int)(tok % a.T);
  stage_tables(a, t, tc, ts);
  __syncthreads();
  const IO* __restrict__ gbp = (const IO*)a.bp;
  const IO* __restrict__ gwp = (const IO*)a.wp;
  const IO* __restrict__ gdp = (const IO*)a.dp;
  for (int h = wv; h < H; h += kWaves) {
    const long long r = tok * H + h;
    // every load of the row first
    f32x4 gq[NG], gk[NG], db[NG], dw[NG];
    V4 b[NG], w[NG], dp = {};
    float dd = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int e = 4 * lane + 256 * g;
      const bool ik = e < M * K, iv = e < M * V;
      gq[g] = ik ? *(const f32x4*)(a.dqr + r * M * K + e) : zero4();
      gk[g] = ik ? *(const f32x4*)(a.dkr + r * M * K + e) : zero4();
      db[g] = ik ? *(const f32x4*)(a.dbg + r * M * K + e) : zero4();
      b[g] = ik ? *(const V4*)(gbp + r * M * K + e) : V4{};
      dw[g] = iv ? *(const f32x4*)(a.dwg + r * M * V + e) : zero4();
      w[g] = iv ? *(const V4*)(gwp + r * M * V + e) : V4{};
    }
    if (lane < M) {
      dp = *(const V4*)(gdp + (r * M + lane) * 4);
      dd = a.ddec[r * M + lane];
    }
    const float pa = to_f(((const IO*)a.pa)[r]) * 0.1f, pb = to_f(((const IO*)a.pb)[r]) * 0.1f;

#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int e = 4 * lane + 256 * g;
      if (e < M * K) {
        *(f32x4*)&gs[wv][0][e] = gq[g];
        *(f32x4*)&gs[wv][1][e] = gk[g];
      }
    }
    wave_lds_sync();
    if (4 * lane < K) {
      const int j0 = 4 * lane;
      f32x4 aq = zero4(), ak = zero4();
      for (int m = 0; m < M; ++m) {
        const int d = lane_pairs(a.pairs, m);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          aq[c] += rope_grad(&gs[wv][0][m * K], j0 + c, d, tc + m * half, ts + m * half);
          ak[c] += rope_grad(&gs[wv][1][m * K], j0 + c, d, tc + m * half, ts + m * half);
        }
      }
      *(f32x4*)(a.dq + r * K + j0) = aq;
      *(f32x4*)(a.dk + r * K + j0) = ak;
    }
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int e = 4 * lane + 256 * g;
      if (e < M * K) {
        const f32x4 x = cvt4<IO>(b[g]);
        f32x4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float s = sigmoidf(x[c] + pa);
          o[c] = db[g][c] * ((1.0f - s) * s);
        }
        *(f32x4*)(a.dbp + r * M * K + e) = o;
        sa += (o[0] + o[1]) + (o[2] + o[3]);
      }
      if (e < M * V) {
        const f32x4 x = cvt4<IO>(w[g]);
        f32x4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float s = sigmoidf(x[c] + pb);
          o[c] = dw[g][c] * ((1.0f - s) * s);
        }
        *(f32x4*)(a.dwp + r * M * V + e) = o;
        sb += (o[0] + o[1]) + (o[2] + o[3]);
      }
    }
    sa = wave_sum(sa) * 0.1f;
    sb = wave_sum(sb) * 0.1f;
    if (lane == 0) {
      a.dpa[r] = sa;
      a.dpb[r] = sb;
    }
    if (lane < M) {
      const f32x4 x = cvt4<IO>(dp);
      f32x4 sp, ex;
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sp[c] = softplusf(x[c]);
        ex[c] = expf(-fminf(sp[c], 5.0f) * a.rates[c]);
        s += ex[c];
      }
      // clamp passes the gradient where its input is <= the bound (torch)
      const float dm = s / 4.0f <= a.clamp ? dd * 0.25f : 0.0f;
      f32x4 dx;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float dsp = sp[c] <= 5.0f ? -dm * ex[c] * a.rates[c] : 0.0f;
        const float z = expf(x[c]);
        dx[c] = x[c] > 20.0f ? dsp : dsp * z / (z + 1.0f);
      }
      *(f32x4*)(a.ddp + (r * M + lane) * 4) = dx;
    }
    wave_lds_sync();
  }
}

constexpr float kNormEps = 1e-6f;   // F.normalize eps (:851)

// One row's epilogue operands in the 16 lanes of a DPP row: lane l16 holds
// v = 4 (l16 + 16 c) .. +3 for c < NC (V <= 64 NC).
template <int NC> struct EpiRow {
  float w[4];
  f32x4 u[NC];        // routed
  f32x4 y[4][NC];
  float n, rn;        // max(|u|, eps), |u|
};

template <typename IO, int NC>
__device__ __forceinline__ void epi_load(EpiRow<NC>& s, const G3EpiArgs& a, long long r, int l16) {
  typedef typename Vec4T<IO>::type V4;
  const int M = a.M, V = a.V;
  const IO* __restrict__ lg = (const IO*)a.lg + r * M;
  const IO* __restrict__ y = (const IO*)a.y + r * M * V;
  // every per-lane array is indexed by unrolled constants (no scratch)
  V4 raw[4][NC];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int v = 4 * (l16 + 16 * c);
      raw[m][c] = (m < M && v < V) ? *(const V4*)(y + m * V + v) : V4{};
    }
  float l[4], mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    l[m] = m < M ? to_f(lg[m]) : -INFINITY;
    mx = fmaxf(mx, l[m]);
  }
  float den = 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    s.w[m] = m < M ? expf(l[m] - mx) : 0.0f;
    den += s.w[m];
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) s.w[m] /= den;
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    s.u[c] = zero4();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      s.y[m][c] = cvt4<IO>(raw[m][c]);
      s.u[c] += s.w[m] * s.y[m][c];
    }
    ss += (s.u[c][0] * s.u[c][0] + s.u[c][1] * s.u[c][1]) + (s.u[c][2] * s.u[c][2] + s.u[c][3] * s.u[c][3]);
  }
  s.rn = sqrtf(row_sum16(ss));
  s.n = fmaxf(s.rn, kNormEps);
}

template <typename IO, int NC>
__global__ __launch_bounds__(256) void g3_epilogue_fwd_kernel(G3EpiArgs a) {
  const int l16 = threadIdx.x & 15;
  const float sv = sqrtf((float)a.V);
  for (long long r = (long long)blockIdx.x * kEpiRows + (threadIdx.x >> 4); r < a.rows;
       r += (long long)gridDim.x * kEpiRows) {
    EpiRow<NC> s;
    epi_load<IO, NC>(s, a, r, l16);
    IO* out = (IO*)a.out + r * a.V;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int v = 4 * (l16 + 16 * c);
      if (v < a.V) {
        const f32x4 nm = *(const f32x4*)(a.norm + v);
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = s.u[c][e] / s.n * sv * nm[e];
        st4io(out + v, o);
      }
    }
  }
}

template <typename IO, int NC>
__global__ __launch_bounds__(256) void g3_epilogue_bwd_kernel(G3EpiArgs a) {
  typedef typename Vec4T<IO>::type V4;
  __shared__ float red[kEpiRows][256];
  const int l16 = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int M = a.M, V = a.V;
  const float sv = sqrtf((float)V);
  f32x4 dn[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dn[c] = zero4();
  for (long long r = (long long)blockIdx.x * kEpiRows + grp; r < a.rows; r += (long long)gridDim.x * kEpiRows) {
    f32x4 d[NC], nm[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int v = 4 * (l16 + 16 * c);
      d[c] = v < V ? cvt4<IO>(*(const V4*)((const IO*)a.dout + r * V + v)) : zero4();
      nm[c] = v < V ? *(const f32x4*)(a.norm + v) : zero4();
    }
    EpiRow<NC> s;
    epi_load<IO, NC>(s, a, r, l16);
    f32x4 g[NC];
    float gu = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      dn[c] += d[c] * (s.u[c] / s.n * sv);
      g[c] = d[c] * nm[c] * sv;
      gu += (g[c][0] * s.u[c][0] + g[c][1] * s.u[c][1]) + (g[c][2] * s.u[c][2] + g[c][3] * s.u[c][3]);
    }
    gu = row_sum16(gu);
    // d(u / n)/du with n = max(|u|, eps): the |u| branch carries u / |u|
    const float k2 = s.rn >= kNormEps ? gu / (s.n * s.n) / s.rn : 0.0f;
    float dmy[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float duu = 0.0f;
    IO* dy = (IO*)a.dy + r * M * V;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int v = 4 * (l16 + 16 * c);
      const f32x4 du = g[c] / s.n - k2 * s.u[c];
      duu += (du[0] * s.u[c][0] + du[1] * s.u[c][1]) + (du[2] * s.u[c][2] + du[3] * s.u[c][3]);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        dmy[m] += (du[0] * s.y[m][c][0] + du[1] * s.y[m][c][1]) + (du[2] * s.y[m][c][2] + du[3] * s.y[m][c][3]);
        if (m < M && v < V) st4io(dy + m * V + v, s.w[m] * du);
      }
    }
    duu = row_sum16(duu);
    float dl = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < M) {
        const float tm = s.w[m] * (row_sum16(dmy[m]) - duu);
        if (l16 == m) dl = tm;
      }
    }
    if (l16 < M) a.dlg[r * M + l16] = dl;
  }
  // block partial of d_norm over its 16 row slots, in a fixed order
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int v = 4 * (l16 + 16 * c);
    if (v < V) *(f32x4*)&red[grp][v] = dn[c];
  }
  __syncthreads();
  for (int v = threadIdx.x; v < V; v += 256) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < kEpiRows; ++q) s += red[q][v];
    a.part[(size_t)blockIdx.x * V + v] = s;
  }
}

// d_norm[v] = sum over the partial rows, one workgroup per column, fixed order
__global__ __launch_bounds__(256) void g3_epilogue_norm_kernel(G3EpiArgs a, int nparts) {
  __shared__ float red[256];
  const int v = blockIdx.x;
  float s = 0.0f;
  for (int p = threadIdx.x; p < nparts; p += 256) s += a.part[(size_t)p * a.V + v];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.dnorm[v] = red[0];
}

int epi_blocks(long long rows, int cap) {
  const long long b = (rows + kEpiRows - 1) / kEpiRows;
  return (int)(b < cap ? b : cap);
}

template <typename IO, int NG>
void launch_prologue(const G3ProArgs& a, bool bwd, hipStream_t stream) {
  const dim3 grid((unsigned)(a.rows / a.H)), block(256);
  if (bwd) hipLaunchKernelGGL((g3_prologue_bwd_kernel<IO, NG>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((g3_prologue_fwd_kernel<IO, NG>), grid, block, 0, stream, a);
}

template <typename IO>
void launch_prologue_ng(const G3ProArgs& a, bool bwd, hipStream_t stream) {
  const int n = a.M * (a.K > a.V ? a.K : a.V);
  const int ng = (n + 255) / 256;
  if (ng <= 1) launch_prologue<IO, 1>(a, bwd, stream);
  else if (ng == 2) launch_prologue<IO, 2>(a, bwd, stream);
  else if (ng == 3) launch_prologue<IO, 3>(a, bwd, stream);
  else launch_prologue<IO, 4>(a, bwd, stream);
}

template <typename IO, int NC>
void launch_epilogue(const G3EpiArgs& a, bool bwd, int nb, hipStream_t stream) {
  if (bwd) hipLaunchKernelGGL((g3_epilogue_bwd_kernel<IO, NC>), dim3(nb), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((g3_epilogue_fwd_kernel<IO, NC>), dim3(nb), dim3(256), 0, stream, a);
}

template <typename IO>
void launch_epilogue_nc(const G3EpiArgs& a, bool bwd, int nb, hipStream_t stream) {
  const int nc = (a.V + 63) / 64;
  if (nc <= 1) launch_epilogue<IO, 1>(a, bwd, nb, stream);
  else if (nc == 2) launch_epilogue<IO, 2>(a, bwd, nb, stream);
  else if (nc == 3) launch_epilogue<IO, 3>(a, bwd, nb, stream);
  else launch_epilogue<IO, 4>(a, bwd, nb, stream);
}

}  // namespace

// Lane RoPE pairs by the reference's rule (gdn3/gdn3_upgrade.py:181-182,
// :342-376): d = floor(K f_m / 2); a lane with scale 1 whose d exceeds the
// layer's table width floor(K/4)/2 is left unchanged (0 here).
void gdn3_lane_pairs(int M, int K, int pairs[4]) {
  static const double frac[4] = {0.50, 0.25, 0.50, 0.50};
  static const double scale[4] = {1.0, 0.3, 0.5, 0.2};
  const int width = (int)(K * 0.25) / 2;
  for (int m = 0; m < 4; ++m) {
    int d = m < M ? (int)(K * frac[m] / 2.0) : 0;
    if (d < 1 || (scale[m] == 1.0 && d > width)) d = 0;
    pairs[m] = d;
  }
}

size_t gdn3_epilogue_workspace_bytes(long long rows, int V) {
  return (size_t)epi_blocks(rows, kEpiMaxParts) * V * sizeof(float);
}

int gdn3_prologue_dispatch(const G3ProArgs& a, bool bwd, int dtype, hipStream_t stream) {
  if (a.rows == 0) return GDNX_OK;
  if (a.rows / a.H > 0x7fffffffLL) return set_error(GDNX_ERR_SHAPE, "B * T too large");
  if (dtype == GDNX_DTYPE_BF16) launch_prologue_ng<bf16>(a, bwd, stream);
  else launch_prologue_ng<float>(a, bwd, stream);
  return check_launch(bwd ? "g3_prologue_bwd_kernel" : "g3_prologue_fwd_kernel");
}

int gdn3_epilogue_dispatch(const G3EpiArgs& a, bool bwd, int dtype, hipStream_t stream) {
  if (a.rows == 0) {
    if (!bwd) return GDNX_OK;
    hipLaunchKernelGGL(g3_epilogue_norm_kernel, dim3(a.V), dim3(256), 0, stream, a, 0);
    return check_launch("g3_epilogue_norm_kernel");
  }
  const int nb = epi_blocks(a.rows, bwd ? kEpiMaxParts : 16384);
  if (dtype == GDNX_DTYPE_BF16) launch_epilogue_nc<bf16>(a, bwd, nb, stream);
  else launch_epilogue_nc<float>(a, bwd, nb, stream);
  int rc = check_launch(bwd ? "g3_epilogue_bwd_kernel" : "g3_epilogue_fwd_kernel");
  if (rc != GDNX_OK || !bwd) return rc;
  hipLaunchKernelGGL(g3_epilogue_norm_kernel, dim3(a.V), dim3(256), 0, stream, a, nb);
  return check_launch("g3_epilogue_norm_kernel");
}

}  // namespace gdnx

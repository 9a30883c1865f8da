// Checkpointed gradient kernel of the chunked delta rule (gfx950): the
// backward's second stage when the forward kept one state per 256-token
// segment (bf16 IO, 32- or 64-token scan chunks, at most 4 lanes per head).
//
// Per chain (b, h, m) and 32-token sub-chunk, with S the state entering the
// sub-chunk and dS the gradient of the state leaving it (see delta_bwd.hip
// for the full list):
//   P1 = dY S^T, P2 = dB S^T, P3 = R dS^T
//   dQ += diag(exp G) P1,  dK += diag(dec) P3 - diag(a_e exp G) P2,  dV += diag(a_w) dB
//   dAq = dY R^T (j <= i), dL = -dB R^T (j < i) -> dQK, dKK and the per-token
//   decay / erase gradients
//   S  <- gamma_C S  + K^T diag(dec) R                      (next sub-chunk's S)
//   dS <- gamma_C dS + Q^T diag(exp G) dY - K^T diag(a_e exp G) dB   (previous one's dS)
// R (the net writes) and dB are per-token quantities, stashed by the scans
// whatever their chunking, so states and state gradients at 32-token
// boundaries follow from the segment's two end points by the last two lines.
// The reference differentiates this chunk graph with torch autograd
// (gdn3/gdn3_upgrade.py:467-521; its trainer recomputes the layer's forward
// under gradient checkpointing, train/train_gdn3_distill.py:263-266).
//
// One workgroup per (b, h, segment) holds the M lanes that share q/k/v, so
// their dq/dk/dv are summed on chip (fixed order, no atomics).  Wave w owns
// key tile w: its columns of a lane's S^T (dS^T) as fp32 accumulator tiles
// [value rows][key columns], which are directly MFMA fragments over
// k = value, and whose update is a product over the sub-chunk's tokens with
// no other wave's data.  The products with them are formed transposed
// (P1^T = S dY^T: key rows, token columns), so a lane holds four keys of one
// token: the per-token sums over keys (q.P1, k.P2, k.P3) are three in-lane
// adds and two lane-group swaps, and dq / dk / dv accumulate as [key][token]
// tiles that are stored without a transpose.  Two lanes' states are resident at a
// time (four would leave too few of the 256 registers a wave has at two
// waves per SIMD: the compiler spilled ~200 per lane), so the workgroup
// runs the two passes below once per pair of lanes and carries a pair's
// dq, dk and dv sums to the next through a float32 scratch of its own in
// the workspace.  Two passes:
//   F (sub-chunks in order, lanes inside): S from the segment's checkpoint;
//     P1, P2, the C x C gram gradients; dq complete; dk's P2 and gram part to
//     a float32 scratch in the workspace; per-token partial dG, da_e.
//   B (sub-chunks in reverse, lanes inside): dS from the checkpoint the
//     reverse scan kept at the segment's end; P3; dk complete; dv, da_w;
//     dG finished and dlog_g as its suffix sums.
// The chunk-end decay term of a sub-chunk c is E_{c+1} = <dS_{c+1}, S_{c+1}>
// (gamma_C <dS_{c+1}, S_c> plus the decay of the sub-chunk's own writes).
// E obeys E_c = E_{c+1} + sum_i (exp G_i q_i.P1_i - a_e,i exp G_i k_i.P2_i
// - dec_i k_i.P3_i), so pass B starts from E at the segment's end, formed
// directly from the checkpoint and pass F's last state, and walks it back
// with the row sums it forms anyway.
#include "delta_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

namespace {

constexpr int kLaneCap = 4;   // lanes per head this kernel takes
constexpr int kRes = 2;       // lanes whose states are resident at a time

template <int D>
struct SegDims {
  static constexpr int C = 32;                           // sub-chunk (tokens)
  static constexpr int NSUB = kSegTokens / C;            // sub-chunks per segment
  static constexpr int NW = D / 16;                      // waves; wave w owns key (and value) tile w
  static constexpr int NT = 64 * NW;
  static constexpr int NDT = D / 16;
  static constexpr int NKB = D / 32;                     // bf16 k-steps over a feature dim
  static constexpr int NCT = C / 16;                     // token tiles per sub-chunk
  static constexpr int LDD = D + 4;                      // [token][D] rows
  static constexpr int LDC = C + 4;                      // [D][token] rows
  static constexpr int NP = NCT * (NCT + 1) / 2;         // lower 16x16 tile pairs
  static constexpr int NTASK = (2 * NP + NW - 1) / NW;   // C x C tile tasks per wave
  static constexpr int SW = NW - 1;                      // the wave that forms the per-token scalars
  static constexpr int NRQ = 2;                          // row-sum quantities per pass
  static constexpr int RLD = NRQ * NW + 4;               // red row length
  static_assert(C * D == 8 * NT, "one 16-byte unit of a [C][D] tile per thread");
  static_assert(NCT == 2, "pair32: two token tiles");
};

// per-step token scalars: log decay prefix, exp G, decay to the sub-chunk's
// end, a_e, a_w, the unclamped log decay, a_e exp G and its negation
enum { kG = 0, kGam, kDec, kAe, kAw, kRaw, kAeg, kNaeg, kNumScal };

template <int D>
struct alignas(16) SegLaneF {   // pass F: one lane's tiles
  typedef SegDims<D> Sd;
  bf16 dy[Sd::C * Sd::LDD];
  bf16 dx[Sd::C * Sd::LDD];
  bf16 r[Sd::C * Sd::LDD];
  bf16 rt[D * Sd::LDC];
};
template <int D>
struct alignas(16) SegLaneB {   // pass B
  typedef SegDims<D> Sd;
  bf16 r[Sd::C * Sd::LDD];
  bf16 dx[Sd::C * Sd::LDD];
  bf16 dyt[D * Sd::LDC];
  bf16 dxt[D * Sd::LDC];
};
template <int D>
union alignas(16) SegLane {
  SegLaneF<D> f;
  SegLaneB<D> b;
};

template <int D>
struct alignas(16) SegSmem {
  typedef SegDims<D> Sd;
  static constexpr int C = Sd::C;
  bf16 q[C * Sd::LDD];      // Q rows (pass F)
  bf16 k[C * Sd::LDD];      // K rows
  bf16 v[C * Sd::LDD];      // V rows (pass B)
  bf16 qt[D * Sd::LDC];     // Q^T
  bf16 kt[D * Sd::LDC];     // K^T
  SegLane<D> ln[2];         // lane tiles, by step parity
  float sc[3][kNumScal][C]; // per step (mod 3): token scalars
  float red[3][C][Sd::RLD]; // per step: per-wave row sums
  float tri[3][Sd::NP][5][16];   // per step: row / column sums of the C x C gradient terms
  bf16 A1[C * Sd::LDC];     // dQK (lower incl. diagonal)
  bf16 A2[C * Sd::LDC];     // dQK^T
  bf16 A3[C * Sd::LDC];     // dKK + dKK^T
  float dgp[Sd::NSUB][kRes][C];   // pass F's part of dG per token
  float incf[Sd::NSUB][kRes];     // pass F's part of E_c - E_{c+1}
  float ean[Sd::NW][kRes];        // per-wave parts of E at the segment's end
  float E[kRes];                  // E_{c+1} of the sub-chunk pass B is at
};

// One 16-byte unit of a sub-chunk's [C][D] tile region in the scans' raw
// accumulator-tile layout (unit u: tile u / 32 = (token tile, value tile),
// lanes 2 (u % 32) and 2 (u % 32) + 1): 4 consecutive tokens of two
// adjacent value columns.
struct TileUnit {
  int tok, col;   // first token (within the sub-chunk), first column
};
template <int D>
__device__ __forceinline__ TileUnit tile_unit_of(int u) {
  constexpr int NDT = D / 16;
  const int tl = u >> 5, lp = u & 31;
  const int it = tl / NDT, V = tl % NDT, g = lp >> 3, n0 = 2 * (lp & 7);
  return TileUnit{16 * it + 4 * g, 16 * V + n0};
}
// rows [tok + i][col], [tok + i][col + 1], i = 0..3 (two bf16 per store)
template <int LD>
__device__ __forceinline__ void unit_commit_rows(bf16* dst, const uint4& x, TileUnit t) {
  const unsigned w[4] = {x.x, x.y, x.z, x.w};   // x.x, x.y: column col, tokens 0..3; x.z, x.w: column col + 1
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned a = (w[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    const unsigned b = (w[2 + (i >> 1)] >> ((i & 1) * 16)) & 0xffffu;
    *(unsigned*)&dst[(t.tok + i) * LD + t.col] = a | (b << 16);
  }
}
// transposed: [col][tok .. tok + 3], [col + 1][tok .. tok + 3]
template <int LD>
__device__ __forceinline__ void unit_commit_tr(bf16* dst, const uint4& x, TileUnit t) {
  *(uint2*)&dst[t.col * LD + t.tok] = make_uint2(x.x, x.y);
  *(uint2*)&dst[(t.col + 1) * LD + t.tok] = make_uint2(x.z, x.w);
}
// Lower 16x16 tile pair p of a 32-token sub-chunk: (0,0), (1,0), (1,1)
// (closed form: no loop on the wave's task index).
__device__ __forceinline__ void pair32(int p, int& it, int& jt) {
  it = p > 0 ? 1 : 0;
  jt = p > 1 ? 1 : 0;
}

// 16x16 NT tile product over K (both operands K-contiguous LDS rows), every
// operand read before the first MFMA.
template <int K>
__device__ __forceinline__ f32x4 tile_nt_pf(const bf16* arow, const bf16* brow, int g4) {
  bf16x8 a[K / 32], b[K / 32];
#pragma unroll
  for (int kb = 0; kb < K / 32; ++kb) {
    a[kb] = ld_frag(arow + kb * 32, g4);
    b[kb] = ld_frag(brow + kb * 32, g4);
  }
  f32x4 acc = zero4();
#pragma unroll
  for (int kb = 0; kb < K / 32; ++kb) mma(acc, a[kb], b[kb]);
  return acc;
}

// Row-major [C][D] tiles (q, k, v, dy) are staged one 16-byte unit per
// thread: token tid % 32, features 8 (tid / 32) .. + 7.  A wave's 64 lanes
// then cover the 32 tokens of two feature groups, so the 2-byte stores of a
// transposed commit spread over every bank (the tokens' row offset in the
// [D][C + 4] array moves a lane pair to the next bank).
__device__ __forceinline__ int row_unit_tok(int tid) { return tid & 31; }
__device__ __forceinline__ int row_unit_d0(int tid) { return (tid >> 5) * 8; }

// Sum of x over the four 16-lane rows of the wave, in every lane (gfx950
// permlane swaps: lane l is added to l ^ 16, then to l ^ 32).
__device__ __forceinline__ float sum_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// one row-major unit (8 consecutive features of one token) transposed: [d][tok]
template <int LD>
__device__ __forceinline__ void row_commit_tr(bf16* dst, const uint4& x, int tok, int d0) {
  const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const unsigned short v = (unsigned short)((w[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
    *(unsigned short*)&dst[(d0 + e) * LD + tok] = v;
  }
}
template <int LD>
__device__ __forceinline__ void row_commit_nat(bf16* dst, const uint4& x, int tok, int d0) {
  uint2* d = (uint2*)&dst[tok * LD + d0];
  d[0] = make_uint2(x.x, x.y);
  d[1] = make_uint2(x.z, x.w);
}

template <int D>
__global__ void __launch_bounds__(SegDims<D>::NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
delta_grad_seg_kernel(DeltaBwdArgs p) {
  typedef SegDims<D> Sd;
  typedef bf16x8 Frag;
  constexpr int C = Sd::C, NW = Sd::NW, NDT = Sd::NDT, NKB = Sd::NKB, NCT = Sd::NCT, NP = Sd::NP;
  constexpr int LDD = Sd::LDD, LDC = Sd::LDC, NTASK = Sd::NTASK, SW = Sd::SW, NSUB = Sd::NSUB, RLD = Sd::RLD;
  __shared__ SegSmem<D> sm;

  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  // the wave that fetches and stages each step's token scalars: one of the
  // waves with no C x C tile task at D = 128 (and not the scalar wave), so
  // the staging does not lengthen the busiest waves' steps (15 % faster than
  // staging them on wave 0)
  constexpr int SCW = NW - 2;
  const int BH = p.B * p.H, M = p.M;
  const int s = blockIdx.x / BH, bh = blockIdx.x % BH, b = bh / p.H, h = bh % p.H;
  const int N = BH * M;
  const int NSEG = (p.T + kSegTokens - 1) / kSegTokens;
  const int t_seg = s * kSegTokens;
  const int nsub = min(NSUB, (p.T - t_seg + C - 1) / C);
  const int CS = p.C;   // the scans' chunk (32 or 64 tokens): the stash's record length
  const StashGeom sg = stash_geom(N, p.T, D, CS, p.cps);
  const bf16* sck = (const bf16*)p.s_stash;   // state records, then the net writes R
  const bf16* rst = sck + sg.states;
  const bf16* dsck = (const bf16*)p.ds_stash; // state-gradient records, then dB
  const bf16* dxst = dsck + sg.states;
  // this workgroup's float32 scratch: dq, dk, dv sums of the lane pairs so far
  // (and dk's pass-F part), [3][sub-chunk][wave][token tile][64 lanes][4]
  float* scr = (float*)((char*)p.ds_stash + ((sg.states + sg.tiles) * sizeof(bf16) + 255) / 256 * 256) +
               ((size_t)bh * NSEG + s) * 3 * kSegTokens * D;
  float* const dqs = scr;
  float* const dks = scr + kSegTokens * D;
  float* const dvs = scr + 2 * kSegTokens * D;
  const size_t rs = (size_t)p.H * D;                  // q/k/v token stride
  const size_t rsy = (size_t)p.H * M * D;             // dy token stride
  const size_t st = (size_t)p.H * M;                  // scalar token stride
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const unsigned rsb = (unsigned)(rs * sizeof(bf16)), ysb = (unsigned)(rsy * sizeof(bf16));
  auto chain_of = [&](int m) { return (size_t)bh * M + m; };
  auto rows_left = [&](int t0) { return min(C, p.T - t0); };
  auto scr_off = [&](int c, int it, int lane) { return (size_t)c * C * D + ((wave * NCT + it) * 64 + lane) * 4; };

  // ---- per-step prefetch registers: one 16-byte unit of each [C][D] tile
  // per thread, and (wave SCW, lanes < C) the token scalars; m is the lane's
  // index in its head ----
  struct Pf {
    uint4 y, r, x;
    ScalarRegs sc;
  };
  auto tile_src = [&](const bf16* region, int c, int m) {
    const int t0 = t_seg + c * C, cs = t0 / CS, j = (t0 % CS) / C;
    return region + rec_index(chain_of(m), cs, (size_t)N) * CS * D + (size_t)j * C * D;
  };
  auto fetch_step = [&](Pf& f, int c, int m, int tid) {
    const int t0 = t_seg + c * C;
    f.r = *(const uint4*)(tile_src(rst, c, m) + 8 * tid);
    f.x = *(const uint4*)(tile_src(dxst, c, m) + 8 * tid);
    const bf16* yb = (const bf16*)p.dy + (((size_t)b * p.T + t0) * p.H + h) * M * D + (size_t)m * D;
    const __amdgpu_buffer_rsrc_t yr = buf_rsrc(yb, (unsigned)rows_left(t0) * ysb);
    f.y = buf_load16(yr, (unsigned)row_unit_tok(tid) * ysb + row_unit_d0(tid) * sizeof(bf16));
    if (wave == SCW) {
      const size_t so = ((size_t)b * p.T * p.H + h) * M + m;
      scal_fetch_all<C>(f.sc, p.ae + so, p.aw + so, p.g + so, st, t0, p.T, tid & 63);
    }
  };
  auto commit_scalars = [&](const ScalarRegs& r, float (*sc)[C], int lane) {
    const float G = lane_prefix<C>(fmaxf(fminf(r.g, 0.f), kLogFloor), lane);
    const float Glast = lane_value(G, C - 1);
    if (lane < C) {
      const float gam = __expf(G);
      sc[kG][lane] = G;
      sc[kGam][lane] = gam;
      sc[kDec][lane] = __expf(Glast - G);
      sc[kAe][lane] = r.ae;
      sc[kAw][lane] = r.aw;
      sc[kRaw][lane] = r.g;
      sc[kAeg][lane] = r.ae * gam;
      sc[kNaeg][lane] = -r.ae * gam;
    }
  };
  // sub-chunk tiles q, k, v: one row-major unit each per thread
  struct SubPf {
    uint4 q, k, v;
  };
  auto fetch_sub = [&](SubPf& f, int c, int tid) {
    const int t0 = t_seg + max(min(c, nsub - 1), 0) * C;   // (out-of-range prefetches refetch an end)
    const unsigned nb = (unsigned)rows_left(t0) * rsb;
    const unsigned off = (unsigned)row_unit_tok(tid) * rsb + row_unit_d0(tid) * sizeof(bf16);
    f.q = buf_load16(buf_rsrc((const bf16*)p.q + qoff + (size_t)t0 * rs, nb), off);
    f.k = buf_load16(buf_rsrc((const bf16*)p.k + qoff + (size_t)t0 * rs, nb), off);
    f.v = buf_load16(buf_rsrc((const bf16*)p.v + qoff + (size_t)t0 * rs, nb), off);
  };

  const int NG = (M + kRes - 1) / kRes;   // lane pairs
  for (int lg = 0; lg < NG; ++lg) {
    const int mb = lg * kRes, ML = min(kRes, M - mb);   // lanes mb .. mb + ML - 1
    const bool first = lg == 0, last = lg == NG - 1;
    if (!first) __syncthreads();   // the previous pair's last readers of the shared tiles are done

    // ---- the pair's states entering the segment, S^T (key tile `wave`) ----
    f32x4 Sacc[kRes][NDT];
    {
      const int lane = tid0 & 63;
#pragma unroll
      for (int m = 0; m < kRes; ++m) {
        // one lane's tiles at a time (loads, then transposes): S^T[16 vt + 4 g + e][16 wave + n]
        bf16x4 raw[NDT];
        const bf16* rec = sck + ((size_t)s * N + chain_of(mb + min(m, ML - 1))) * D * D;
#pragma unroll
        for (int vt = 0; vt < NDT; ++vt) raw[vt] = *(const bf16x4*)(rec + stash_tile_offset<bf16, D>(wave, vt, lane));
#pragma unroll
        for (int vt = 0; vt < NDT; ++vt) Sacc[m][vt] = m < ML ? tile_transpose_raw(raw[vt], lane) : zero4();
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // =========================== pass F ===========================
    {
      Pf pf;
      SubPf spf;
      f32x4 dQacc[NCT], dKacc[NCT], gram[NTASK], dgram[NTASK];
      fetch_sub(spf, 0, tid0);
      fetch_step(pf, 0, mb, tid0);
      auto commit_sub = [&](const SubPf& f, int tid) {
        const int row = row_unit_tok(tid), col = row_unit_d0(tid);
        row_commit_nat<LDD>(sm.q, f.q, row, col);
        row_commit_nat<LDD>(sm.k, f.k, row, col);
        row_commit_tr<LDC>(sm.qt, f.q, row, col);
        row_commit_tr<LDC>(sm.kt, f.k, row, col);
        for (int e = tid; e < C * LDC; e += Sd::NT) {
          sm.A1[e] = (bf16)0.f;
          sm.A2[e] = (bf16)0.f;
          sm.A3[e] = (bf16)0.f;
        }
      };
      auto commit_step = [&](const Pf& f, SegLaneF<D>& L, float (*sc)[C], int tid) {
        const TileUnit tu = tile_unit_of<D>(tid);
        unit_commit_rows<LDD>(L.r, f.r, tu);
        unit_commit_tr<LDC>(L.rt, f.r, tu);
        unit_commit_rows<LDD>(L.dx, f.x, tu);
        row_commit_nat<LDD>(L.dy, f.y, row_unit_tok(tid), row_unit_d0(tid));
        if (wave == SCW) commit_scalars(f.sc, sc, tid & 63);
      };
      // per-token scalars of step (c, m) (wave SW): da_e, pass F's part of dG and of E
      auto scalars_F = [&](int c, int m, int j3) {
        const int lane = tid0 & 63;
        const float(*sc)[C] = sm.sc[j3];
        float dGF = 0.f, inc = 0.f;
        if (lane < C) {
          const int i = lane, ib = i >> 4, ir = i & 15;
          float r0 = 0.f, r1 = 0.f;
#pragma unroll
          for (int w = 0; w < NW; w += 4) {
            const f32x4 a = *(const f32x4*)&sm.red[j3][i][w];
            const f32x4 e = *(const f32x4*)&sm.red[j3][i][NW + w];
            r0 += (a[0] + a[1]) + (a[2] + a[3]);
            r1 += (e[0] + e[1]) + (e[2] + e[3]);
          }
          inc = sc[kGam][i] * r0 - sc[kAeg][i] * r1;
          dGF = inc;
          float dae = -sc[kGam][i] * r1;
          for (int bj = 0; bj <= ib; ++bj) {
            const int pr = ib * (ib + 1) / 2 + bj;
            dGF += sm.tri[j3][pr][0][ir] + sm.tri[j3][pr][3][ir];
            dae += sm.tri[j3][pr][2][ir];
          }
          for (int bi = ib; bi < NCT; ++bi) {
            const int pr = bi * (bi + 1) / 2 + ib;
            dGF -= sm.tri[j3][pr][1][ir] + sm.tri[j3][pr][4][ir];
          }
          sm.dgp[c][m][i] = dGF;
          const int t = t_seg + c * C + i;
          if (t < p.T) p.dae[(((size_t)b * p.T + t) * p.H + h) * M + mb + m] = dae;
        }
        inc = wave_sum(inc);
        if (lane == 0) sm.incf[c][m] = inc;
      };

      commit_sub(spf, tid0);
      commit_step(pf, sm.ln[0].f, sm.sc[0], tid0);
      {
        const int j1 = min(1, nsub * ML - 1);
        fetch_step(pf, j1 / ML, mb + j1 % ML, tid0);
      }

      for (int c = 0; c < nsub; ++c) {
        const int tid = opaque(tid0);
        const int lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          dQacc[it] = first ? zero4() : *(const f32x4*)(dqs + scr_off(c, it, lane));   // earlier pairs' sums
          dKacc[it] = first ? zero4() : *(const f32x4*)(dks + scr_off(c, it, lane));
        }
#pragma unroll
        for (int m = 0; m < kRes; ++m) {
          if (m >= ML) break;
          const int j = c * ML + m, j3 = j % 3;
          __syncthreads();   // step j's tiles committed; step j - 1's sums complete
          if (m == 0) {
            // the sub-chunk's raw grams (q_i.k_j, k_i.k_j) in the registers of
            // the wave that owns each C x C tile task
#pragma unroll
            for (int jj = 0; jj < NTASK; ++jj) {
              const int task = wave + NW * jj;
              gram[jj] = dgram[jj] = zero4();
              if (task < 2 * NP) {
                const bool isL = task >= NP;
                int it, jt;
                pair32(isL ? task - NP : task, it, jt);
                const bf16* arow = isL ? &sm.k[(it * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
                gram[jj] = tile_nt_pf<D>(arow, &sm.k[(jt * 16 + n16) * LDD], g4);
              }
            }
          }
          if (m > 0 && wave == SW) scalars_F(c, m - 1, (j - 1) % 3);   // (a sub-chunk's last step: in its epilogue)
          if (m == ML - 1) fetch_sub(spf, c + 1, tid);   // the next sub-chunk's q, k through this step
          const SegLaneF<D>& L = sm.ln[j & 1].f;
          const float(*sc)[C] = sm.sc[j3];
          // ---- P1^T = S dY^T, P2^T = S dB^T on this wave's key tile: lane
          // (g, n) holds keys 16 wave + 4 g + e of token 16 it + n ----
          f32x4 P1[NCT], P2[NCT];
#pragma unroll
          for (int it = 0; it < NCT; ++it) P1[it] = P2[it] = zero4();
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            Frag ay[NCT], ax[NCT];
#pragma unroll
            for (int it = 0; it < NCT; ++it) {
              ay[it] = ld_frag(&L.dy[(it * 16 + n16) * LDD + kb * 32], g4);
              ax[it] = ld_frag(&L.dx[(it * 16 + n16) * LDD + kb * 32], g4);
            }
            const Frag sf = acc_frag((bf16*)nullptr, Sacc[m][2 * kb], Sacc[m][2 * kb + 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int it = 0; it < NCT; ++it) {
              mma(P1[it], sf, ay[it]);
              mma(P2[it], sf, ax[it]);
            }
          }
          // ---- dq, dk parts and the token sums q.P1, k.P2 over this wave's keys ----
#pragma unroll
          for (int it = 0; it < NCT; ++it) {
            const float gi = sc[kGam][it * 16 + n16], ei = sc[kAeg][it * 16 + n16];
            dQacc[it] += gi * P1[it];
            dKacc[it] -= ei * P2[it];
            const bf16x4 q4 = *(const bf16x4*)&sm.q[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
            const bf16x4 k4 = *(const bf16x4*)&sm.k[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
            float r0 = 0.f, r1 = 0.f;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              r0 += P1[it][ii] * (float)q4[ii];
              r1 += P2[it][ii] * (float)k4[ii];
            }
            r0 = sum_rows4(r0);
            r1 = sum_rows4(r1);
            if (g4 == 0) {
              sm.red[j3][it * 16 + n16][wave] = r0;
              sm.red[j3][it * 16 + n16][NW + wave] = r1;
            }
          }
          // ---- dAq = dY R^T (j <= i) and dL = -dB R^T (j < i) on this wave's
          // C x C tile tasks: the lane sums dQK, dKK and the per-token terms ----
#pragma unroll
          for (int jj = 0; jj < NTASK; ++jj) {
            const int task = wave + NW * jj;
            if (task >= 2 * NP) continue;
            const bool isL = task >= NP;
            const int pidx = isL ? task - NP : task;
            int it, jt;
            pair32(pidx, it, jt);
            const bf16* arow = isL ? &L.dx[(it * 16 + n16) * LDD] : &L.dy[(it * 16 + n16) * LDD];
            const f32x4 acc = tile_nt_pf<D>(arow, &L.r[(jt * 16 + n16) * LDD], g4);
            const int jc = jt * 16 + n16;
            const float Gj = sc[kG][jc];
            float xm[4], xa[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int i = it * 16 + 4 * g4 + ii;
              xm[ii] = 0.f;
              xa[ii] = 0.f;
              const float Dij = __expf(sc[kG][i] - Gj);
              if (!isL && jc <= i) {
                const float dqk = acc[ii] * Dij;
                dgram[jj][ii] += dqk;
                xm[ii] = dqk * gram[jj][ii];
              } else if (isL && jc < i) {
                const float dl = -acc[ii];
                const float kk = gram[jj][ii];
                const float dkk = dl * Dij * sc[kAe][i];
                dgram[jj][ii] += dkk;
                xm[ii] = dkk * kk;
                xa[ii] = dl * Dij * kk;
              }
            }
            const int slot = isL ? 3 : 0;
            float rx[4], ra[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              rx[ii] = row_prefix16(xm[ii]);
              ra[ii] = row_prefix16(xa[ii]);
            }
            if (n16 == 15) {
#pragma unroll
              for (int ii = 0; ii < 4; ++ii) {
                sm.tri[j3][pidx][slot][4 * g4 + ii] = rx[ii];
                if (isL) sm.tri[j3][pidx][2][4 * g4 + ii] = ra[ii];
              }
            }
            float cx = (xm[0] + xm[1]) + (xm[2] + xm[3]);
            cx += __shfl_xor(cx, 16, 64);
            cx += __shfl_xor(cx, 32, 64);
            if (g4 == 0) sm.tri[j3][pidx][slot + 1][n16] = cx;
            __builtin_amdgcn_sched_barrier(0);
          }
          // ---- S^T <- gamma_C S^T + R^T diag(dec) K (key tile `wave`) ----
          {
            const float gl = sc[kGam][C - 1];
            const Frag bk = frag_scale(ld_frag(&sm.kt[(wave * 16 + n16) * LDC], g4), &sc[kDec][0], g4);
#pragma unroll
            for (int v2 = 0; v2 < NDT; v2 += 2) {
              const Frag a0 = ld_frag(&L.rt[(v2 * 16 + n16) * LDC], g4);
              const Frag a1 = ld_frag(&L.rt[(v2 * 16 + 16 + n16) * LDC], g4);
              Sacc[m][v2] *= gl;
              Sacc[m][v2 + 1] *= gl;
              mma(Sacc[m][v2], a0, bk);
              mma(Sacc[m][v2 + 1], a1, bk);
            }
          }
          // ---- the next step's tiles into the other buffer; the one after it in flight ----
          {
            const int jn = j + 1;
            if (jn < nsub * ML) commit_step(pf, sm.ln[jn & 1].f, sm.sc[jn % 3], tid);
            const int j2 = min(j + 2, nsub * ML - 1);
            fetch_step(pf, j2 / ML, mb + j2 % ML, tid);
          }
        }
        // ---- sub-chunk epilogue: gram-gradient products, dq and dk's part out ----
        __syncthreads();   // every lane's tile tasks and sums done
        if (wave == SW) scalars_F(c, ML - 1, (c * ML + ML - 1) % 3);
#pragma unroll
        for (int jj = 0; jj < NTASK; ++jj) {
          const int task = wave + NW * jj;
          if (task >= 2 * NP) continue;
          const bool isL = task >= NP;
          int it, jt;
          pair32(isL ? task - NP : task, it, jt);
          const int jc = jt * 16 + n16;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = it * 16 + 4 * g4 + ii;
            const bf16 x = (bf16)dgram[jj][ii];
            if (!isL) {
              if (jc <= i) {
                sm.A1[i * LDC + jc] = x;
                sm.A2[jc * LDC + i] = x;
              }
            } else if (jc < i) {
              sm.A3[i * LDC + jc] = x;
              sm.A3[jc * LDC + i] = x;
            }
          }
        }
        __syncthreads();
        {
          const Frag bkt = ld_frag(&sm.kt[(wave * 16 + n16) * LDC], g4);
          const Frag bqt = ld_frag(&sm.qt[(wave * 16 + n16) * LDC], g4);
#pragma unroll
          for (int it = 0; it < NCT; ++it) {   // dQ^T += K^T dQK^T, dK^T += Q^T dQK + K^T (dKK + dKK^T)
            mma(dQacc[it], bkt, ld_frag(&sm.A1[(it * 16 + n16) * LDC], g4));
            mma(dKacc[it], bqt, ld_frag(&sm.A2[(it * 16 + n16) * LDC], g4));
            mma(dKacc[it], bkt, ld_frag(&sm.A3[(it * 16 + n16) * LDC], g4));
          }
        }
        {
          bf16* dq = (bf16*)p.dq;
#pragma unroll
          for (int it = 0; it < NCT; ++it) {
            *(f32x4*)(dks + scr_off(c, it, lane)) = dKacc[it];
            if (!last) {
              *(f32x4*)(dqs + scr_off(c, it, lane)) = dQacc[it];
            } else {   // lane (g, n): token 16 it + n, keys 16 wave + 4 g ..
              const int t = t_seg + c * C + it * 16 + n16;
              if (t < p.T) {
                const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + wave * 16 + 4 * g4;
                st4(dq + off, dQacc[it][0], dQacc[it][1], dQacc[it][2], dQacc[it][3]);
              }
            }
          }
        }
        if (c + 1 < nsub) {
          __syncthreads();   // every wave done with this sub-chunk's q / k tiles
          commit_sub(spf, tid);
        }
      }
    }

    // =========================== pass B ===========================
    {
      Pf pf;
      SubPf spf;
      f32x4 dKacc[NCT], dVacc[NCT];
      const int jlast = nsub * ML - 1;   // pass B's step j is sub-chunk nsub - 1 - j / ML, lane mb + j % ML
      auto cm_of = [&](int j, int& c, int& m) {
        c = nsub - 1 - j / ML;
        m = j % ML;
      };
      auto commit_sub = [&](const SubPf& f, int tid) {
        const int row = row_unit_tok(tid), col = row_unit_d0(tid);
        row_commit_nat<LDD>(sm.k, f.k, row, col);
        row_commit_nat<LDD>(sm.v, f.v, row, col);
        row_commit_tr<LDC>(sm.qt, f.q, row, col);
        row_commit_tr<LDC>(sm.kt, f.k, row, col);
      };
      auto commit_step = [&](const Pf& f, SegLaneB<D>& L, float (*sc)[C], int tid) {
        const TileUnit tu = tile_unit_of<D>(tid);
        unit_commit_rows<LDD>(L.r, f.r, tu);
        unit_commit_rows<LDD>(L.dx, f.x, tu);
        unit_commit_tr<LDC>(L.dxt, f.x, tu);
        row_commit_tr<LDC>(L.dyt, f.y, row_unit_tok(tid), row_unit_d0(tid));
        if (wave == SCW) commit_scalars(f.sc, sc, tid & 63);
      };
      // dG finished and dlog_g, da_w of step (c, m) (wave SW); E walked back
      auto scalars_B = [&](int c, int m, int j3) {
        const int lane = tid0 & 63;
        const float(*sc)[C] = sm.sc[j3];
        wave_lds_sync();
        const float E = sm.E[m];
        float dG = 0.f, dec3 = 0.f, daw = 0.f;
        if (lane < C) {
          const int i = lane;
          float r3 = 0.f;
#pragma unroll
          for (int w = 0; w < NW; w += 4) {
            const f32x4 a = *(const f32x4*)&sm.red[j3][i][w];
            const f32x4 e = *(const f32x4*)&sm.red[j3][i][NW + w];
            r3 += (a[0] + a[1]) + (a[2] + a[3]);
            daw += (e[0] + e[1]) + (e[2] + e[3]);
          }
          dec3 = sc[kDec][i] * r3;
          dG = sm.dgp[c][m][i] - dec3;
          if (i == C - 1) dG += E;
        }
        const float incb = wave_sum(dec3);
        const float sfx = lane_suffix<C>(lane < C ? dG : 0.f, lane);
        const int t = t_seg + c * C + lane;
        if (lane < C && t < p.T) {
          const size_t si = (((size_t)b * p.T + t) * p.H + h) * M + mb + m;
          const float raw = sc[kRaw][lane];
          p.dg[si] = (raw <= 0.f && raw >= kLogFloor) ? sfx : 0.f;
          p.daw[si] = daw;
        }
        wave_lds_sync();
        if (lane == 0) sm.E[m] = E + sm.incf[c][m] - incb;
      };

      {
        int c0, m0;
        cm_of(0, c0, m0);
        fetch_sub(spf, c0, tid0);
        fetch_step(pf, c0, mb + m0, tid0);
      }
      // ---- dS at the segment's end (checkpoint) replaces S; E there from both ----
      {
        const int lane = tid0 & 63;
        float part[kRes];
#pragma unroll
        for (int m = 0; m < kRes; ++m) {
          part[m] = 0.f;
          bf16x4 raw[NDT];
          const bf16* rec = dsck + ((size_t)s * N + chain_of(mb + min(m, ML - 1))) * D * D;
#pragma unroll
          for (int vt = 0; vt < NDT; ++vt) raw[vt] = *(const bf16x4*)(rec + stash_tile_offset<bf16, D>(wave, vt, lane));
#pragma unroll
          for (int vt = 0; vt < NDT; ++vt) {
            const f32x4 d = m < ML ? tile_transpose_raw(raw[vt], lane) : zero4();
            part[m] += (d[0] * Sacc[m][vt][0] + d[1] * Sacc[m][vt][1]) + (d[2] * Sacc[m][vt][2] + d[3] * Sacc[m][vt][3]);
            Sacc[m][vt] = d;
          }
          part[m] = wave_sum(part[m]);
          __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();   // pass F's last readers of the shared tiles are done
        if (lane == 0) {
#pragma unroll
          for (int m = 0; m < kRes; ++m) sm.ean[wave][m] = part[m];
        }
        commit_sub(spf, tid0);
        commit_step(pf, sm.ln[0].b, sm.sc[0], tid0);
        if (jlast >= 1) {
          int c1, m1;
          cm_of(1, c1, m1);
          fetch_step(pf, c1, mb + m1, tid0);
        }
        __syncthreads();
        if (wave == SW && lane < kRes) {
          float e = 0.f;
          for (int w = 0; w < NW; ++w) e += sm.ean[w][lane];
          sm.E[lane] = e;
        }
      }

      for (int ci = 0; ci < nsub; ++ci) {
        const int c = nsub - 1 - ci;
        const int tid = opaque(tid0);
        const int lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          dKacc[it] = *(const f32x4*)(dks + scr_off(c, it, lane));   // pass F's part (and earlier pairs')
          dVacc[it] = first ? zero4() : *(const f32x4*)(dvs + scr_off(c, it, lane));
        }
#pragma unroll
        for (int m = 0; m < kRes; ++m) {
          if (m >= ML) break;
          const int j = ci * ML + m, j3 = j % 3;
          if (m > 0) {
            __syncthreads();   // step j's tiles committed; step j - 1's sums complete
            if (wave == SW) scalars_B(c, m - 1, (j - 1) % 3);   // (a sub-chunk's last step: in its epilogue)
          }
          if (m == ML - 1) fetch_sub(spf, c - 1, tid);   // the next sub-chunk's q, k, v through this step
          const SegLaneB<D>& L = sm.ln[j & 1].b;
          const float(*sc)[C] = sm.sc[j3];
          // ---- P3^T = dS R^T on this wave's key tile (lane (g, n): keys
          // 16 wave + 4 g + e of token 16 it + n) ----
          f32x4 P3[NCT];
#pragma unroll
          for (int it = 0; it < NCT; ++it) P3[it] = zero4();
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            Frag ar[NCT];
#pragma unroll
            for (int it = 0; it < NCT; ++it) ar[it] = ld_frag(&L.r[(it * 16 + n16) * LDD + kb * 32], g4);
            const Frag sf = acc_frag((bf16*)nullptr, Sacc[m][2 * kb], Sacc[m][2 * kb + 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int it = 0; it < NCT; ++it) mma(P3[it], sf, ar[it]);
          }
          // ---- dk's P3 part, dv (value tile `wave`), and the token sums k.P3, v.dB ----
#pragma unroll
          for (int it = 0; it < NCT; ++it) {
            const float di = sc[kDec][it * 16 + n16], wi = sc[kAw][it * 16 + n16];
            dKacc[it] += di * P3[it];
            const bf16x4 k4 = *(const bf16x4*)&sm.k[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
            const bf16x4 v4 = *(const bf16x4*)&sm.v[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
            const bf16x4 x4 = *(const bf16x4*)&L.dx[(it * 16 + n16) * LDD + wave * 16 + 4 * g4];
            float r3 = 0.f, rv = 0.f;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              dVacc[it][ii] += wi * (float)x4[ii];
              r3 += P3[it][ii] * (float)k4[ii];
              rv += (float)x4[ii] * (float)v4[ii];
            }
            r3 = sum_rows4(r3);
            rv = sum_rows4(rv);
            if (g4 == 0) {
              sm.red[j3][it * 16 + n16][wave] = r3;
              sm.red[j3][it * 16 + n16][NW + wave] = rv;
            }
          }
          // ---- dS^T <- gamma_C dS^T + dY^T diag(exp G) Q - dB^T diag(a_e exp G) K ----
          {
            const float gl = sc[kGam][C - 1];
            const Frag bq = frag_scale(ld_frag(&sm.qt[(wave * 16 + n16) * LDC], g4), &sc[kGam][0], g4);
            const Frag bk = frag_scale(ld_frag(&sm.kt[(wave * 16 + n16) * LDC], g4), &sc[kNaeg][0], g4);
#pragma unroll
            for (int v2 = 0; v2 < NDT; v2 += 2) {
              const Frag ay0 = ld_frag(&L.dyt[(v2 * 16 + n16) * LDC], g4);
              const Frag ax0 = ld_frag(&L.dxt[(v2 * 16 + n16) * LDC], g4);
              const Frag ay1 = ld_frag(&L.dyt[(v2 * 16 + 16 + n16) * LDC], g4);
              const Frag ax1 = ld_frag(&L.dxt[(v2 * 16 + 16 + n16) * LDC], g4);
              Sacc[m][v2] *= gl;
              Sacc[m][v2 + 1] *= gl;
              mma(Sacc[m][v2], ay0, bq);
              mma(Sacc[m][v2 + 1], ay1, bq);
              mma(Sacc[m][v2], ax0, bk);
              mma(Sacc[m][v2 + 1], ax1, bk);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
          // ---- the next step's tiles into the other buffer (whatever its
          // sub-chunk: the lane tiles are double-buffered), the one after it in flight ----
          {
            const int jn = j + 1;
            if (jn <= jlast) commit_step(pf, sm.ln[jn & 1].b, sm.sc[jn % 3], tid);
            if (jn + 1 <= jlast) {
              int c2, m2;
              cm_of(jn + 1, c2, m2);
              fetch_step(pf, c2, mb + m2, tid);
            }
          }
        }
        // ---- sub-chunk epilogue: dk, dv out (or to the scratch for the next pair) ----
        {
          bf16* dk = (bf16*)p.dk;
          bf16* dv = (bf16*)p.dv;
#pragma unroll
          for (int it = 0; it < NCT; ++it) {
            if (!last) {
              *(f32x4*)(dks + scr_off(c, it, lane)) = dKacc[it];
              *(f32x4*)(dvs + scr_off(c, it, lane)) = dVacc[it];
            } else {   // lane (g, n): token 16 it + n, keys / values 16 wave + 4 g ..
              const int t = t_seg + c * C + it * 16 + n16;
              if (t < p.T) {
                const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + wave * 16 + 4 * g4;
                st4(dk + off, dKacc[it][0], dKacc[it][1], dKacc[it][2], dKacc[it][3]);
                st4(dv + off, dVacc[it][0], dVacc[it][1], dVacc[it][2], dVacc[it][3]);
              }
            }
          }
        }
        __syncthreads();   // every wave done with this sub-chunk's tiles; its last step's sums complete
        if (wave == SW) scalars_B(c, ML - 1, (ci * ML + ML - 1) % 3);
        if (c > 0) {
          commit_sub(spf, tid);
          __syncthreads();   // the next sub-chunk's tiles visible
        }
      }
    }
  }
}

}  // namespace

int delta_grad_seg_dispatch(const DeltaBwdArgs& a, hipStream_t stream) {
  const int NSEG = (a.T + kSegTokens - 1) / kSegTokens;
  const unsigned grid = (unsigned)(a.B * a.H * NSEG);
  if (a.M > kLaneCap) return set_error(GDNX_ERR_SHAPE, "checkpointed backward: at most %d lanes per head", kLaneCap);
  if (a.D == 128) {
    static_assert(sizeof(SegSmem<128>) <= 160 * 1024, "LDS budget");
    hipLaunchKernelGGL((delta_grad_seg_kernel<128>), dim3(grid), dim3(SegDims<128>::NT), 0, stream, a);
  } else if (a.D == 64) {
    hipLaunchKernelGGL((delta_grad_seg_kernel<64>), dim3(grid), dim3(SegDims<64>::NT), 0, stream, a);
  } else {
    return set_error(GDNX_ERR_SHAPE, "checkpointed backward: unsupported head dim %d", a.D);
  }
  return check_launch("delta_grad_seg_kernel");
}

}  // namespace gdnx

// Checkpointed gradient kernel of the chunked delta rule (gfx950): the
// backward's last stage when the forward kept one state per 256-token
// segment (bf16 IO, 32-token scan chunks, at most 4 lanes per head).
//
// Per chain (b, h, m) and 32-token sub-chunk, with S the state entering the
// sub-chunk and dS the gradient of the state leaving it (see delta_bwd.hip
// for the full list):
//   P1 = dY S^T, P2 = dB S^T, P3 = R dS^T
//   dQ += diag(exp G) P1,  dK += diag(dec) P3 - diag(a_e exp G) P2,  dV += diag(a_w) dB
//   dAq = dY R^T (j <= i), dL = -dB R^T (j < i) -> dQK, dKK and the per-token
//   decay / erase gradients
//   S  <- gamma_C S  + K^T diag(dec) R                      (next sub-chunk's S)
// R (the net writes) and dB are per-token quantities, stashed by the scans
// whatever their chunking, so the states at 32-token boundaries follow from
// the segment's checkpoint by the last line.  P3 needs the state gradient
// at every chunk end: the reverse scan, which holds it, forms P3 and stashes
// it as bf16 tiles in the layout this kernel's dk accumulators have.
// The reference differentiates this chunk graph with torch autograd
// (gdn3/gdn3_upgrade.py:467-521; its trainer recomputes the layer's forward
// under gradient checkpointing, train/train_gdn3_distill.py:263-266).
//
// One workgroup per (b, h, segment) takes the M lanes that share q/k/v, so
// their dq/dk/dv are summed in a fixed order with no atomics: two lanes'
// states are resident at a time, the lane pairs run one after the other
// over the segment's sub-chunks, and a pair's float32 dq/dk/dv sums go to
// the next pair through the workspace.  Wave w
// owns key tile w: its columns of a lane's S^T as fp32 accumulator tiles
// [value rows][key columns], which are directly MFMA fragments over
// k = value, and whose update is a product over the sub-chunk's tokens with
// no other wave's data.  The products with them are formed transposed
// (P1^T = S dY^T: key rows, token columns), so a lane holds four keys of one
// token: the per-token sums over keys (q.P1, k.P2, k.P3) are three in-lane
// adds and two lane-group swaps, and dq / dk / dv accumulate as [key][token]
// tiles that are stored without a transpose.
//
// The chunk-end decay term of a sub-chunk c is E_{c+1} = <dS_{c+1}, S_{c+1}>.
// E obeys E_c = E_{c+1} + sum_i (exp G_i q_i.P1_i - a_e,i exp G_i k_i.P2_i
// - dec_i k_i.P3_i), so after the pass the kernel forms E at the segment's
// end from the state-gradient checkpoint and the walked state, and walks it
// back over the sub-chunks' sums to finish dlog_g.
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
  static constexpr int NRQ = 2;                          // row sums per step: q.P1, k.P2
  static constexpr int RLD = NRQ * NW + 4;               // red row length
  static_assert(C * D == 8 * NT, "one 16-byte unit of a [C][D] tile per thread");
  static_assert(NCT == 2, "pair32: two token tiles");
};

// per-step token scalars: log decay prefix, exp G, decay to the sub-chunk's
// end, a_e, a_w, a_e exp G, k.P3 (formed by the reverse scan in float32)
enum { kG = 0, kGam, kDec, kAe, kAw, kAeg, kK3, kNumScal };

template <int D>
struct alignas(16) SegLane {   // one lane's step tiles
  typedef SegDims<D> Sd;
  bf16 dy[Sd::C * Sd::LDD];
  bf16 dx[Sd::C * Sd::LDD];   // dB rows
  bf16 r[Sd::C * Sd::LDD];
  bf16 rt[D * Sd::LDC];
  bf16 p3[Sd::C * D];         // P3 tiles as stashed (lane-order fragments of the dk accumulators)
};

template <int D>
struct alignas(16) SegSmem {
  typedef SegDims<D> Sd;
  static constexpr int C = Sd::C;
  bf16 q[C * Sd::LDD];      // Q rows
  bf16 k[C * Sd::LDD];      // K rows
  bf16 v[C * Sd::LDD];      // V rows
  bf16 qt[D * Sd::LDC];     // Q^T
  bf16 kt[D * Sd::LDC];     // K^T
  SegLane<D> ln[2];         // lane tiles, by step parity
  float sc[3][kNumScal][C]; // per step (mod 3): token scalars
  float red[3][C][Sd::RLD]; // per step: per-wave row sums
  float tri[3][Sd::NP][5][16];   // per step: row / column sums of the C x C gradient terms
  bf16 A1[C * Sd::LDC];     // dQK (lower incl. diagonal)
  bf16 A2[C * Sd::LDC];     // dQK^T
  bf16 A3[C * Sd::LDC];     // dKK + dKK^T
  float dgp[Sd::NSUB][kLaneCap][C];   // dG per token, but the chunk-end term
  float inc[Sd::NSUB][kLaneCap];      // E_c - E_{c+1}
  float ean[Sd::NW][kRes];            // per-wave parts of E at the segment's end (the resident lanes)
};

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

// a 16-byte unit of a record read once (non-temporal)
__device__ __forceinline__ uint4 nt_load16(const bf16* p) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int D>
__global__ void __launch_bounds__(SegDims<D>::NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
delta_grad_seg_kernel(DeltaBwdArgs p) {
  typedef SegDims<D> Sd;
  typedef bf16x8 Frag;
  constexpr int C = Sd::C, NW = Sd::NW, NDT = Sd::NDT, NKB = Sd::NKB, NCT = Sd::NCT, NP = Sd::NP;
  constexpr int LDD = Sd::LDD, LDC = Sd::LDC, NTASK = Sd::NTASK, SW = Sd::SW;
  __shared__ SegSmem<D> sm;

  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  // the wave that fetches and stages each step's token scalars: one of the
  // waves with no C x C tile task at D = 128 (and not the scalar wave), so
  // the staging does not lengthen the busiest waves' steps
  constexpr int SCW = NW - 2;
  const int BH = p.B * p.H, M = p.M;
  const int s = blockIdx.x / BH, bh = blockIdx.x % BH, b = bh / p.H, h = bh % p.H;
  const int N = BH * M;
  const int t_seg = s * kSegTokens;
  const int nsub = min(Sd::NSUB, (p.T - t_seg + C - 1) / C);
  // the scans' chunk, which is the stash's record length and the sub-chunk
  // (dispatch rejects any other p.C), so record offsets are shifts
  constexpr int CS = C;
  const StashGeom sg = stash_geom(N, p.T, D, CS, p.cps);
  const bf16* sck = (const bf16*)p.s_stash;   // state records, then the net writes R
  const bf16* rst = sck + sg.states;
  const bf16* dsck = (const bf16*)p.ds_stash; // state-gradient records, then dB, then P3
  const bf16* dxst = dsck + sg.states;
  const bf16* p3st = dxst + sg.tiles;
  const float* k3st = (const float*)(p3st + sg.tiles);   // k.P3 per token
  // this workgroup's float32 carry of the dq, dk, dv sums from one lane pair
  // to the next, [3][sub-chunk][wave][token tile][64 lanes][4]
  const int NSEG = (p.T + kSegTokens - 1) / kSegTokens;
  float* const dqs = (float*)((char*)p.ds_stash + delta_seg_carry_offset(N, p.T, D, CS, p.cps)) +
                     ((size_t)bh * NSEG + s) * 3 * kSegTokens * D;
  float* const dks = dqs + kSegTokens * D;
  float* const dvs = dqs + 2 * kSegTokens * D;
  const size_t rs = (size_t)p.H * D;                  // q/k/v token stride
  const size_t rsy = (size_t)p.H * M * D;             // dy token stride
  const size_t st = (size_t)p.H * M;                  // scalar token stride
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const unsigned rsb = (unsigned)(rs * sizeof(bf16)), ysb = (unsigned)(rsy * sizeof(bf16));
  auto chain_of = [&](int m) { return (size_t)bh * M + m; };
  auto rows_left = [&](int t0) { return min(C, p.T - t0); };
  auto scr_off = [&](int c, int it, int lane) { return (size_t)c * C * D + ((wave * NCT + it) * 64 + lane) * 4; };
  int mb = 0, ML = min(kRes, M);   // the resident lanes mb .. mb + ML - 1

  // ---- per-step prefetch registers: one 16-byte unit of each [C][D] tile
  // per thread, this lane's P3 fragments, and (wave SCW, lanes < C) the
  // token scalars; step j of a lane pair is sub-chunk j / ML, lane mb + j % ML ----
  struct Pf {
    uint4 y, r, x, p3;
    ScalarRegs sc;   // raw (a clamped token's), masked at commit
    float k3;
    bool ok;         // the lane's token is in the sub-chunk and before T
  };
  auto tile_src = [&](const bf16* region, int c, int m) {
    const int t0 = t_seg + c * C, cs = t0 / CS, j = (t0 % CS) / C;
    return region + rec_index(chain_of(m), cs, (size_t)N) * CS * D + (size_t)j * C * D;
  };
  // Loads retire in order and a wait counts every older load, so nothing
  // here uses a loaded value: the scalars are issued first and masked at
  // commit, and the tiles stay in flight through the next step.
  auto fetch_step = [&](Pf& f, int j, int tid) {
    static_assert(kRes == 2, "one or two resident lanes: step j splits by a shift");
    const int c = ML == 2 ? j >> 1 : j, m = mb + (ML == 2 ? (j & 1) : 0);
    const int t0 = t_seg + c * C;
    if (wave == SCW) {
      const int lane = tid & 63, cs = t0 / CS, jj = (t0 % CS) / C;
      const size_t so = ((size_t)b * p.T * p.H + h) * M + m + (size_t)min(t0 + lane, p.T - 1) * st;
      f.sc.ae = p.ae[so];
      f.sc.aw = p.aw[so];
      f.sc.g = p.g[so];
      f.k3 = k3st[rec_index(chain_of(m), cs, (size_t)N) * CS + jj * C + min(lane, C - 1)];
      f.ok = lane < C && t0 + lane < p.T;
    }
    f.r = nt_load16(tile_src(rst, c, m) + 8 * tid);
    f.x = nt_load16(tile_src(dxst, c, m) + 8 * tid);
    f.p3 = nt_load16(tile_src(p3st, c, m) + 8 * tid);
    const bf16* yb = (const bf16*)p.dy + (((size_t)b * p.T + t0) * p.H + h) * M * D + (size_t)m * D;
    const __amdgpu_buffer_rsrc_t yr = buf_rsrc(yb, (unsigned)rows_left(t0) * ysb);
    f.y = buf_load16(yr, (unsigned)row_unit_tok(tid) * ysb + row_unit_d0(tid) * sizeof(bf16));
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
      sc[kAeg][lane] = r.ae * gam;
    }
  };
  auto commit_step = [&](const Pf& f, SegLane<D>& L, float (*sc)[C], int tid) {
    const TileUnit tu = tile_unit_of<D>(tid);
    unit_commit_rows<LDD>(L.r, f.r, tu);
    unit_commit_tr<LDC>(L.rt, f.r, tu);
    unit_commit_rows<LDD>(L.dx, f.x, tu);
    row_commit_nat<LDD>(L.dy, f.y, row_unit_tok(tid), row_unit_d0(tid));
    *(uint4*)&L.p3[8 * tid] = f.p3;
    if (wave == SCW) {
      const ScalarRegs r{f.ok ? f.sc.ae : 0.f, f.ok ? f.sc.aw : 0.f, f.ok ? f.sc.g : 0.f};
      commit_scalars(r, sc, tid & 63);
      if ((tid & 63) < C) sc[kK3][tid & 63] = f.ok ? f.k3 : 0.f;
    }
  };
  // sub-chunk tiles q, k, v: one row-major unit each per thread
  struct SubPf {
    uint4 q, k, v;
  };
  auto fetch_sub = [&](SubPf& f, int c, int tid) {
    const int t0 = t_seg + min(c, nsub - 1) * C;   // (the prefetch past the last sub-chunk refetches it)
    const unsigned nb = (unsigned)rows_left(t0) * rsb;
    const unsigned off = (unsigned)row_unit_tok(tid) * rsb + row_unit_d0(tid) * sizeof(bf16);
    f.q = buf_load16(buf_rsrc((const bf16*)p.q + qoff + (size_t)t0 * rs, nb), off);
    f.k = buf_load16(buf_rsrc((const bf16*)p.k + qoff + (size_t)t0 * rs, nb), off);
    f.v = buf_load16(buf_rsrc((const bf16*)p.v + qoff + (size_t)t0 * rs, nb), off);
  };
  auto commit_sub = [&](const SubPf& f, int tid) {
    const int row = row_unit_tok(tid), col = row_unit_d0(tid);
    row_commit_nat<LDD>(sm.q, f.q, row, col);
    row_commit_nat<LDD>(sm.k, f.k, row, col);
    row_commit_nat<LDD>(sm.v, f.v, row, col);
    row_commit_tr<LDC>(sm.qt, f.q, row, col);
    row_commit_tr<LDC>(sm.kt, f.k, row, col);
    for (int e = tid; e < C * LDC; e += Sd::NT) {
      sm.A1[e] = (bf16)0.f;
      sm.A2[e] = (bf16)0.f;
      sm.A3[e] = (bf16)0.f;
    }
  };
  // per-token results of step (c, m) (wave SW): da_e, dG but the chunk-end
  // term, and the step's part of E_c - E_{c+1}
  auto scalars = [&](int c, int m, int j3) {
    const int lane = tid0 & 63;
    const float(*sc)[C] = sm.sc[j3];
    float dG = 0.f, inc = 0.f;
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
      inc = sc[kGam][i] * r0 - sc[kAeg][i] * r1 - sc[kDec][i] * sc[kK3][i];
      dG = inc;
      float dae = -sc[kGam][i] * r1;
      for (int bj = 0; bj <= ib; ++bj) {
        const int pr = ib * (ib + 1) / 2 + bj;
        dG += sm.tri[j3][pr][0][ir] + sm.tri[j3][pr][3][ir];
        dae += sm.tri[j3][pr][2][ir];
      }
      for (int bi = ib; bi < NCT; ++bi) {
        const int pr = bi * (bi + 1) / 2 + ib;
        dG -= sm.tri[j3][pr][1][ir] + sm.tri[j3][pr][4][ir];
      }
      sm.dgp[c][m][i] = dG;
      const int t = t_seg + c * C + i;
      if (t < p.T) {
        const size_t si = (((size_t)b * p.T + t) * p.H + h) * M + m;
        p.dae[si] = dae;
      }
    }
    inc = wave_sum(inc);
    if (lane == 0) sm.inc[c][m] = inc;
  };

  const int NG = (M + kRes - 1) / kRes;   // lane pairs
  for (int lg = 0; lg < NG; ++lg) {
  mb = lg * kRes;
  ML = min(kRes, M - mb);
  const bool first = lg == 0, last = lg == NG - 1;
  const int nstep = nsub * ML;
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

  Pf pf;
  SubPf spf;
  f32x4 dQacc[NCT], dKacc[NCT], dVacc[NCT], gram[NTASK], dgram[NTASK];
  fetch_sub(spf, 0, tid0);
  fetch_step(pf, 0, tid0);
  commit_sub(spf, tid0);
  commit_step(pf, sm.ln[0], sm.sc[0], tid0);
  fetch_step(pf, min(1, nstep - 1), tid0);

  for (int c = 0; c < nsub; ++c) {
    const int tid = opaque(tid0);
    const int lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
#pragma unroll
    for (int it = 0; it < NCT; ++it) dQacc[it] = dKacc[it] = dVacc[it] = zero4();
#pragma unroll
    for (int mm = 0; mm < kRes; ++mm) {
      if (mm >= ML) break;
      const int m = mb + mm, j = c * ML + mm, j3 = j % 3;
      __syncthreads();   // step j's tiles committed; step j - 1's sums complete
      if (mm == 0) {
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
      if (mm > 0 && wave == SW) scalars(c, m - 1, (j - 1) % 3);   // (a sub-chunk's last step: in its epilogue)
      const SegLane<D>& L = sm.ln[j & 1];
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
        const Frag sf = acc_frag((bf16*)nullptr, Sacc[mm][2 * kb], Sacc[mm][2 * kb + 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          mma(P1[it], sf, ay[it]);
          mma(P2[it], sf, ax[it]);
        }
      }
      // ---- dq, dk, dv parts and the token sums q.P1, k.P2 (this wave's keys) ----
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        const int tok = it * 16 + n16;
        const float gi = sc[kGam][tok], ei = sc[kAeg][tok], di = sc[kDec][tok], wi = sc[kAw][tok];
        const bf16x4 p3 = *(const bf16x4*)&L.p3[stash_tile_offset<bf16, D>(it, wave, lane)];
        const f32x4 P3 = (f32x4){(float)p3[0], (float)p3[1], (float)p3[2], (float)p3[3]};
        dQacc[it] += gi * P1[it];
        dKacc[it] += di * P3 - ei * P2[it];
        const bf16x4 q4 = *(const bf16x4*)&sm.q[tok * LDD + wave * 16 + 4 * g4];
        const bf16x4 k4 = *(const bf16x4*)&sm.k[tok * LDD + wave * 16 + 4 * g4];
        const bf16x4 x4 = *(const bf16x4*)&L.dx[tok * LDD + wave * 16 + 4 * g4];
        float r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          r0 += P1[it][ii] * (float)q4[ii];
          r1 += P2[it][ii] * (float)k4[ii];
          dVacc[it][ii] += wi * (float)x4[ii];
        }
        r0 = sum_rows4(r0);
        r1 = sum_rows4(r1);
        if (g4 == 0) {
          sm.red[j3][tok][wave] = r0;
          sm.red[j3][tok][NW + wave] = r1;
        }
      }
      if (wave == SW) {
        // da_w = dB.v per token: the diagonals of the two 16 x 16 tiles of
        // dB V^T on MFMA (at D = 128 the scalar wave has no C x C tile
        // task; the staging wave, which has none either, measured slower
        // with it).  Lane (g, n)
        // holds rows 4 g .. 4 g + 3 of column n, so the diagonal entry of
        // token 16 it + n sits in lane (n / 4, n) at row n % 4.
#pragma unroll
        for (int it = 0; it < NCT; ++it) {
          const f32x4 acc = tile_nt_pf<D>(&L.dx[(it * 16 + n16) * LDD], &sm.v[(it * 16 + n16) * LDD], g4);
          const int ii = n16 & 3;
          const float x = ii == 0 ? acc[0] : ii == 1 ? acc[1] : ii == 2 ? acc[2] : acc[3];
          const int t = t_seg + c * C + it * 16 + n16;
          if ((n16 >> 2) == g4 && t < p.T) p.daw[(((size_t)b * p.T + t) * p.H + h) * M + m] = x;
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
          Sacc[mm][v2] *= gl;
          Sacc[mm][v2 + 1] *= gl;
          mma(Sacc[mm][v2], a0, bk);
          mma(Sacc[mm][v2 + 1], a1, bk);
        }
      }
      // ---- the next step's tiles into the other buffer; the one after it in flight ----
      if (j + 1 < nstep) commit_step(pf, sm.ln[(j + 1) & 1], sm.sc[(j + 1) % 3], tid);
      fetch_step(pf, min(j + 2, nstep - 1), tid);
    }
    // ---- sub-chunk epilogue: gram-gradient products; dq, dk, dv out ----
    // the earlier pairs' sums, loaded here (after the steps' prefetches, whose
    // waits they would otherwise join) and added before the stores
    f32x4 cq[NCT], ck[NCT], cv[NCT];
    if (!first) {
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        cq[it] = *(const f32x4*)(dqs + scr_off(c, it, lane));
        ck[it] = *(const f32x4*)(dks + scr_off(c, it, lane));
        cv[it] = *(const f32x4*)(dvs + scr_off(c, it, lane));
      }
    }
    __syncthreads();   // every lane's tile tasks and sums done
    // the next sub-chunk's q / k / v, in flight through the epilogue (every
    // wave is past its last read of this sub-chunk's row tiles)
    if (c + 1 < nsub) fetch_sub(spf, c + 1, tid);
    if (wave == SW) scalars(c, mb + ML - 1, (c * ML + ML - 1) % 3);
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
    if (!first) {
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        dQacc[it] += cq[it];
        dKacc[it] += ck[it];
        dVacc[it] += cv[it];
      }
    }
    if (!last) {   // the sums so far to the next pair
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        *(f32x4*)(dqs + scr_off(c, it, lane)) = dQacc[it];
        *(f32x4*)(dks + scr_off(c, it, lane)) = dKacc[it];
        *(f32x4*)(dvs + scr_off(c, it, lane)) = dVacc[it];
      }
    } else {
      // lane (g, n): token 16 it + n, keys / values 16 wave + 4 g ..
      bf16* dq = (bf16*)p.dq;
      bf16* dk = (bf16*)p.dk;
      bf16* dv = (bf16*)p.dv;
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        const int t = t_seg + c * C + it * 16 + n16;
        if (t < p.T) {
          const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + wave * 16 + 4 * g4;
          st4(dq + off, dQacc[it][0], dQacc[it][1], dQacc[it][2], dQacc[it][3]);
          st4(dk + off, dKacc[it][0], dKacc[it][1], dKacc[it][2], dKacc[it][3]);
          st4(dv + off, dVacc[it][0], dVacc[it][1], dVacc[it][2], dVacc[it][3]);
        }
      }
    }
    if (c + 1 < nsub) {
      __syncthreads();   // every wave done with this sub-chunk's q / k / v tiles
      commit_sub(spf, tid);
    }
  }

  // ---- E at the segment's end: <dS, S> with dS from the reverse scan's
  // checkpoint and S the walked state ----
  {
    const int lane = tid0 & 63;
    float part[kRes];
#pragma unroll
    for (int m = 0; m < kRes; ++m) {
      part[m] = 0.f;
      if (m >= ML) continue;
      bf16x4 raw[NDT];
      const bf16* rec = dsck + ((size_t)s * N + chain_of(mb + m)) * D * D;
#pragma unroll
      for (int vt = 0; vt < NDT; ++vt) raw[vt] = *(const bf16x4*)(rec + stash_tile_offset<bf16, D>(wave, vt, lane));
#pragma unroll
      for (int vt = 0; vt < NDT; ++vt) {
        const f32x4 d = tile_transpose_raw(raw[vt], lane);
        part[m] += (d[0] * Sacc[m][vt][0] + d[1] * Sacc[m][vt][1]) + (d[2] * Sacc[m][vt][2] + d[3] * Sacc[m][vt][3]);
      }
      part[m] = wave_sum(part[m]);
    }
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < kRes; ++m) sm.ean[wave][m] = part[m];
    }
  }
  __syncthreads();   // the per-wave parts of E, every step's dG and E increments
  // ---- dlog_g: per sub-chunk, the suffix sums of dG with E_{c+1} at its
  // last token; wave w walks lane mb + w's E back over the sub-chunks ----
  if (wave < ML) {
    const int m = mb + wave, lane = tid0 & 63;
    float E = 0.f;
    for (int w = 0; w < NW; ++w) E += sm.ean[w][wave];
    for (int c = nsub - 1; c >= 0; --c) {
      float dG = lane < C ? sm.dgp[c][m][lane] : 0.f;
      if (lane == C - 1) dG += E;
      const float sfx = lane_suffix<C>(dG, lane);
      const int t = t_seg + c * C + lane;
      if (lane < C && t < p.T) {
        const size_t si = (((size_t)b * p.T + t) * p.H + h) * M + m;
        const float raw = p.g[si];
        p.dg[si] = (raw <= 0.f && raw >= kLogFloor) ? sfx : 0.f;
      }
      E += sm.inc[c][m];
    }
  }
  }   // lane pairs
}

}  // namespace

int delta_grad_seg_dispatch(const DeltaBwdArgs& a, hipStream_t stream) {
  const int NSEG = (a.T + kSegTokens - 1) / kSegTokens;
  const unsigned grid = (unsigned)(a.B * a.H * NSEG);
  if (a.M > kLaneCap) return set_error(GDNX_ERR_SHAPE, "checkpointed backward: at most %d lanes per head", kLaneCap);
  if (a.C != SegDims<128>::C) return set_error(GDNX_ERR_SHAPE, "checkpointed backward: %d-token chunks only", SegDims<128>::C);
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

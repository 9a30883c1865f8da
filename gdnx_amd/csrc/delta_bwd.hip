// Chunked decoupled-erase delta rule, backward (gfx950).
//
// Forward per chunk (see delta_fwd.hip): R = T (W - diag(exp G) E S0),
// Y = diag(exp G) Q S0 + Aq R, S_C = gamma_C S0 + K^T diag(dec) R with
// E = diag(a_e) K, W = diag(a_w) V.  Given dY and dS_C:
//
//   dR   = diag(dec) K dS_C + Aq^T dY            dB = T^T dR
//   dS0  = gamma_C dS_C + (diag(exp G) Q)^T dY - (diag(a_e exp G) K)^T dB
//   dV   = diag(a_w) dB                          da_w = rowsum(dB o V)
//   dAq  = dY R^T (j<=i),  dL = -dB R^T (j<i)    (then through D, a_e, grams)
//   dQ   = diag(exp G) dY S0^T + dQK K
//   dK   = diag(dec) R dS_C^T - diag(a_e exp G) dB S0^T + dQK^T Q + (dKK + dKK^T) K
//   dG_i = exp(G_i) q_i.(dY S0^T)_i - a_e,i exp(G_i) k_i.(dB S0^T)_i + mask terms
//          + chunk-end terms; dg = reverse cumulative sum of dG in the chunk.
//
// Two stages:
//   delta_scan_bwd_kernel (delta_scan.hip)  the reverse scan: value-split
//     workgroups per chain walk the chunks in reverse with dS in registers,
//     reading the forward's prep records (T, Aq, decays), and stash dS_C and
//     dB of every chunk.  Needs no S0.
//   delta_bwd_grads_kernel  one workgroup per (batch, head, chunk), looping
//     over the M lanes that share q/k/v: reads S0, R (forward stash) and
//     dS_C, dB (reverse-scan stash), runs the contractions over value columns
//     with the state rows read straight from the row-major stashes, and sums
//     the lanes' dq/dk/dv in registers (fixed order, no atomics), so the lane
//     expansion of the reference (gdn3/gdn3_upgrade.py:785-787) costs no
//     extra memory traffic.
// The reference differentiates its chunk graph with torch autograd
// (gdn3/gdn3_upgrade.py:467-521) and its KMD-2 TRSM by hand
// (gdn3/kmd2_fast_scan.py:143-160).
#include "delta_common.hpp"

namespace gdnx {

// ---------------------------------------------------------------------------
// per-chunk gradients, lanes summed in-block
// ---------------------------------------------------------------------------
// Wave w owns one 16-column tile of the key dimension (and the same tile of
// the value dimension): its rows of S0 / dS_C, its dq/dk/dv tiles and its
// share of the P products stay in registers.
//   C <= 32: one workgroup of D/16 waves per (b, h, chunk), two waves per SIMD.
//   C = 64: the per-wave arrays double (the chunk's 64 rows) and need ~370
//   registers, so a workgroup has four waves, one per SIMD with the whole
//   512-entry register file, and covers 64 key columns: KH = D/64 workgroups
//   per (b, h, chunk) split the key (and value) columns.  Each reads only its
//   rows of the states (the dominant traffic) and computes the lane-shared
//   C x C gram gradients itself; the per-token scalar gradients are linear in
//   the key-split row sums, so each workgroup writes a partial and a second
//   kernel adds them (the pair runs side by side on one XCD, so the chunk
//   tiles both read come from L2 the second time).
template <typename CT, int D, int C>
struct GradDims {
  static constexpr int KT = 1;                          // key tiles per wave
  static constexpr int NW = C >= 64 ? 4 : D / 16;       // waves per workgroup
  static constexpr int KH = D / (16 * NW);              // workgroups per (b, h, chunk)
  static constexpr int NT = 64 * NW;
  static constexpr int WPE = C >= 64 ? 1 : 2;           // waves per SIMD the kernel is compiled for
};

// Small per-lane arrays, double-buffered by lane parity: the per-token
// scalar gradients of lane m are formed (by one wave) while the workgroup
// computes lane m + 1.
template <int C, int NW, int NP>
struct alignas(16) GradLaneBuf {
  float G[C], gam[C], dec[C], ae[C], aw[C], graw[C];
  // [row][quantity * NW + wave]: q.P1, k.P2, k.P3, v.dB partial sums; rows padded by 4
  // floats so that one row per lane reads conflict-free as 16-byte vectors
  float red[C][4 * NW + 4];
  float tri[NP][5][16];  // per tile pair: row and column sums of Xm (dAq part), row sums of AE,
                         // row and column sums of Xm (dL part)
  float scal[NW];        // per-wave partial <dS_C, S0>
};

template <typename CT, int D, int C>
struct alignas(16) BwdGradSmem {
  typedef Dims<CT, D, C> Dm;
  static constexpr int LDD = Dm::LDD, LDC = Dm::LDC, NW = GradDims<CT, D, C>::NW;
  static constexpr int NP = (C / 16) * (C / 16 + 1) / 2;  // lower 16x16 tile pairs
  CT q[C * LDD];
  CT k[C * LDD];
  CT v[C * LDD];
  // (the grams q_i.k_j, k_i.k_j and their lane-summed gradients live in the
  // registers of the wave that owns each 16x16 tile)
  union alignas(16) U {
    struct alignas(16) {  // one lane's chunk tiles, rows [token][v]
      CT dy[C * LDD], R[C * LDD], dB[C * LDD];
    } ln;
    struct alignas(16) {  // after the lanes: transposed Q, K and the gram-gradient factors
      CT qt[D * LDC], kt[D * LDC], A1[C * LDC], A2[C * LDC], A3[C * LDC];
    } fin;
  } u;
  GradLaneBuf<C, NW, NP> lb[2];
};

// One lane's inputs to the gradient kernel, fetched a lane ahead: this
// wave's rows of S0 and dS_C (raw tiles, one per 16 value columns, for each
// of its key tiles), this thread's share of the R / dB tiles and of dY (all
// value columns: the workgroup's NW waves take value tiles wave + NW j), and
// (scalar wave) the per-token coefficients.
template <typename CT, int D, int C>
struct GradPrefetch {
  typedef typename Vec4T<CT>::type V4;
  static constexpr int KT = GradDims<CT, D, C>::KT;
  static constexpr int NVL = D / 16 / GradDims<CT, D, C>::NW;   // value tiles loaded per wave
  static constexpr int NDT = D / 16, NCT = C / 16, NT = GradDims<CT, D, C>::NT;
  static constexpr int VEC = 16 / sizeof(CT);
  static constexpr int NDY = (C * D / VEC + NT - 1) / NT;
  V4 s[KT][NDT], ds[KT][NDT];
  V4 r[NVL][NCT], db[NVL][NCT];
  uint4 dy[NDY];
  ScalarRegs sc;
};

// Gradient kernel: one workgroup per (batch, head, chunk), looping over the M
// lanes that share q/k/v.  Per lane it reads the stashed S0, R (forward) and
// dS_C, dB (reverse scan) and forms, wave w owning key columns d and value
// columns v in its KT tiles:
//   P1 = dY S0^T, P2 = dB S0^T, P3 = R dS_C^T      (S0 / dS_C rows of this wave
//                                                   as fragments over k = v)
//   dQ += diag(exp G) P1,  dK += diag(dec) P3 - diag(a_e exp G) P2
//   dV += diag(a_w) dB,    da_w = rowsum(dB o V)
//   dAq = dY R^T (j<=i),   dL = -dB R^T (j<i)  -> dQK, dKK (lane sums) and the
//   per-token decay / erase gradients.
// After the lanes: dQ += dQK K, dK += dQK^T Q + (dKK + dKK^T) K.
template <typename CT, int D, int C>
__global__ void __launch_bounds__((GradDims<CT, D, C>::NT))
__attribute__((amdgpu_waves_per_eu(GradDims<CT, D, C>::WPE, GradDims<CT, D, C>::WPE)))
delta_bwd_grads_kernel(DeltaBwdArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  typedef BwdGradSmem<CT, D, C> Sm;
  typedef GradPrefetch<CT, D, C> Pf;
  typedef GradLaneBuf<C, GradDims<CT, D, C>::NW, Sm::NP> LB;
  typedef typename Vec4T<CT>::type V4;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NCT = Dm::NCT, NDT = Dm::NDT, LDD = Dm::LDD, LDC = Dm::LDC;
  constexpr int NW = GradDims<CT, D, C>::NW, NT = GradDims<CT, D, C>::NT, KT = GradDims<CT, D, C>::KT;
  constexpr int NKV = D / KS, NP = Sm::NP;
  constexpr int SW = NW - 1;  // the wave that forms the per-token scalar gradients
  __shared__ Sm sm;

  const int tid0 = threadIdx.x;
  const int tid = tid0;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  constexpr int KH = GradDims<CT, D, C>::KH;
  const int NC = (p.T + C - 1) / C;
  const int nblocks = p.B * p.H * NC * KH;
  const int work = xcd_remap(blockIdx.x, nblocks);
  // key halves fastest (the pair lands on one XCD), then chunks in ascending
  // order over all heads: the records the reverse scan wrote last (low
  // chunks) are read first, some still from the memory-side cache (measured
  // 4 % faster than head-major order)
  const int kh = work % KH, blk = work / KH;
  const int c = blk / (p.B * p.H);
  const int h = (blk % (p.B * p.H)) % p.H;
  const int b = (blk % (p.B * p.H)) / p.H;
  const int tile0 = (kh * NW + wave) * KT;   // this wave's first key (and value) tile
  const int t0 = c * C;
  const size_t rs = (size_t)p.H * D;
  const size_t qoff = ((size_t)b * p.T * p.H + h) * D;
  const size_t rsy = (size_t)p.H * p.M * D;
  const size_t st = (size_t)p.H * p.M;
  const size_t nrec = (size_t)p.B * p.H * p.M * NC;
  const CT* s_st = (const CT*)p.s_stash;     // [nrec] stash_state: states entering each chunk
  const CT* r_st = s_st + nrec * D * D;      // [nrec] stash_tiles: net writes R
  const CT* ds_st = (const CT*)p.ds_stash;   // [nrec] stash_state: state gradients at chunk ends
  const CT* db_st = ds_st + nrec * D * D;    // [nrec] stash_tiles: dB

  // ---- lane mm's inputs, fetched into registers a lane ahead in two parts:
  // the chunk tiles (dY, R, dB, scalars) at the start of the previous lane,
  // and this wave's state rows (S0, dS_C) spread through the previous lane's
  // P products, so the loads stream while the lanes compute.  Every load is
  // unconditional (dY's tail tokens go through a buffer resource) ----
  const unsigned ysb = (unsigned)(rsy * sizeof(CT));
  auto rec_of = [&](int mm) { return rec_index(((size_t)b * p.H + h) * p.M + mm, c, (size_t)p.B * p.H * p.M); };
  auto prefetch_tiles = [&](Pf& f, int mm, int tid_) {
    const int lane_ = tid_ & 63;
    const size_t rec = rec_of(mm);
#pragma unroll
    for (int j = 0; j < Pf::NVL; ++j)
#pragma unroll
      for (int it = 0; it < NCT; ++it) {  // tile (it, V = wave + NW j) of R and dB
        const size_t off = rec * C * D + stash_tile_offset<CT, D>(it, wave + NW * j, lane_);
        f.r[j][it] = *(const V4*)(r_st + off);
        f.db[j][it] = *(const V4*)(db_st + off);
      }
    const CT* yb = (const CT*)p.dy + (((size_t)b * p.T * p.H + h) * p.M + mm) * D + (size_t)t0 * rsy;
    const __amdgpu_buffer_rsrc_t yr = buf_rsrc(yb, (unsigned)min(C, p.T - t0) * ysb);
#pragma unroll
    for (int j = 0; j < Pf::NDY; ++j) {
      const int qv = tid_ + j * NT, row = qv / (D / Pf::VEC), col = (qv % (D / Pf::VEC)) * Pf::VEC;
      f.dy[j] = buf_load16(yr, (unsigned)row * ysb + col * sizeof(CT));
    }
    const size_t soff = ((size_t)b * p.T * p.H + h) * p.M + mm;
    scal_fetch_all<C>(f.sc, p.ae + soff, p.aw + soff, p.g + soff, st, t0, p.T, lane_);
  };
  auto prefetch_state = [&](Pf& f, int mm, int V, int tid_) {
    const size_t rec = rec_of(mm);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f.s[kt][V] = *(const V4*)stash_state_ptr<CT, D, C>(s_st + rec * D * D, tile0 + kt, V, tid_ & 63);
      f.ds[kt][V] = *(const V4*)stash_state_ptr<CT, D, C>(ds_st + rec * D * D, tile0 + kt, V, tid_ & 63);
    }
  };

  // ---- per-token scalar gradients of lane mm (wave SW, one token per lane) ----
  auto scalar_grads = [&](int mm, const LB& q) {
    float dGi = 0.f, daei = 0.f, dawi = 0.f, r3d = 0.f;
    if (lane < C) {
      const int i = lane, ib = i >> 4, ir = i & 15;
      float rs[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) {   // this row's NW partials (16-byte vectors when NW % 4 == 0)
        rs[a] = 0.f;
        if constexpr (NW % 4 == 0) {
#pragma unroll
          for (int w = 0; w < NW; w += 4) {
            const f32x4 x = *(const f32x4*)&q.red[i][a * NW + w];
            rs[a] += (x[0] + x[1]) + (x[2] + x[3]);
          }
        } else {
#pragma unroll
          for (int w = 0; w < NW; ++w) rs[a] += q.red[i][a * NW + w];
        }
      }
      dawi = rs[3];
      dGi = q.gam[i] * rs[0] - q.gam[i] * q.ae[i] * rs[1] - q.dec[i] * rs[2];
      daei = -q.gam[i] * rs[1];
      // Xm row i lives in tiles (ib, jt <= ib); column i in tiles (it >= ib, ib)
      // (every key part has them: the first one adds them)
      if (kh == 0) {
        for (int bj = 0; bj <= ib; ++bj) {
          const int pr = ib * (ib + 1) / 2 + bj;
          dGi += q.tri[pr][0][ir] + q.tri[pr][3][ir];
          daei += q.tri[pr][2][ir];
        }
        for (int bi = ib; bi < NCT; ++bi) {
          const int pr = bi * (bi + 1) / 2 + ib;
          dGi -= q.tri[pr][1][ir] + q.tri[pr][4][ir];
        }
      }
      r3d = q.dec[i] * rs[2];
    }
    // chunk-end decay: d/dG_last of gamma_C <dS_C, S0> and of the dec factors
    r3d = wave_sum(r3d);
    if (lane == C - 1) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s += q.scal[w];
      dGi += s * q.gam[C - 1] + r3d;
    }
    // dg_s = sum_{i >= s} dG_i (suffix sum within the chunk)
    const float sfx = lane_suffix<C>((lane < C) ? dGi : 0.f, lane);
    const int t = t0 + lane;
    if (lane < C && t < p.T) {
      const size_t si = ((size_t)(b * p.T + t) * p.H + h) * p.M + mm;
      const float raw = q.graw[lane];
      const float dgv = (raw <= 0.f && raw >= kLogFloor) ? sfx : 0.f;
      if constexpr (KH == 1) {
        p.dae[si] = daei;
        p.daw[si] = dawi;
        p.dg[si] = dgv;
      } else {   // this key part's share, [KH][3][rows] after dS and dB in the workspace
        const size_t rows = (size_t)p.B * p.T * p.H * p.M;
        float* part = (float*)(db_st + nrec * C * D) + (size_t)kh * 3 * rows;
        part[si] = daei;
        part[rows + si] = dawi;
        part[2 * rows + si] = dgv;
      }
    }
  };

  // q, k, v of the chunk first, then lane 0's inputs: the staging commit
  // below waits only for its own loads
  Pf pf;
  {
    Stage<CT, C, D, 1, NT> sq, sk, sv;
    const unsigned rsb = (unsigned)(rs * sizeof(CT)), nb = (unsigned)min(C, p.T - t0) * rsb;
    sq.fetch(buf_rsrc((const CT*)p.q + qoff + (size_t)t0 * rs, nb), rsb, tid);
    sk.fetch(buf_rsrc((const CT*)p.k + qoff + (size_t)t0 * rs, nb), rsb, tid);
    sv.fetch(buf_rsrc((const CT*)p.v + qoff + (size_t)t0 * rs, nb), rsb, tid);
    prefetch_tiles(pf, 0, tid);
#pragma unroll
    for (int V = 0; V < NDT; ++V) prefetch_state(pf, 0, V, tid);
    sq.template commit_nat<LDD>(sm.q, tid);
    sk.template commit_nat<LDD>(sm.k, tid);
    sv.template commit_nat<LDD>(sm.v, tid);
  }
  f32x4 dQacc[KT][NCT], dKacc[KT][NCT], dVacc[KT][NCT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int it = 0; it < NCT; ++it) dQacc[kt][it] = dKacc[kt][it] = dVacc[kt][it] = zero4();
  __syncthreads();
  // raw grams (shared by the lanes) in the registers of the wave that owns the
  // tile: task pidx < NP is tile pair pidx of Q K^T (with the gradient dQK),
  // NP + pidx the same pair of K K^T (with dKK); wave w owns tasks w + NW j
  constexpr int NTASK = (2 * NP + NW - 1) / NW;
  f32x4 gram[NTASK], dgram[NTASK];
#pragma unroll
  for (int j = 0; j < NTASK; ++j) {
    const int task = wave + NW * j;
    gram[j] = dgram[j] = zero4();
    if (task < 2 * NP) {
      const bool isL = task >= NP;
      int it, jt;
      tri_pair(isL ? task - NP : task, it, jt);
      const CT* arow = isL ? &sm.k[(it * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
      gram[j] = tile_nt<CT, D>(arow, &sm.k[(jt * 16 + n16) * LDD], g4);
    }
  }

  for (int m = 0; m < p.M; ++m) {
    // per-thread indices re-derived each lane: keeps the compiler from hoisting
    // (and spilling) every loop-invariant per-thread address out of the loop
    const int tid = opaque(tid0);
    const int lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
    LB& lb = sm.lb[m & 1];
    __syncthreads();  // lane m-1 done with the lane tiles; lane m-2's scalar pass done with lb
    if constexpr (C >= 64) {
      if (m > 0) prefetch_tiles(pf, m, tid);   // (C = 64: no registers to hold them a lane ahead)
    }
    // ---- commit lane m's prefetched inputs ----
#pragma unroll
    for (int j = 0; j < Pf::NDY; ++j) {
      const int qv = tid + j * NT, row = qv / (D / Pf::VEC), col = (qv % (D / Pf::VEC)) * Pf::VEC;
      if (qv < C * D / Pf::VEC) {
        uint2* d2 = (uint2*)&sm.u.ln.dy[row * LDD + col];
        d2[0] = make_uint2(pf.dy[j].x, pf.dy[j].y);
        d2[1] = make_uint2(pf.dy[j].z, pf.dy[j].w);
      }
    }
#pragma unroll
    for (int j = 0; j < Pf::NVL; ++j)
#pragma unroll
      for (int it = 0; it < NCT; ++it)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int col = (wave + NW * j) * 16 + n16;
          sm.u.ln.R[(it * 16 + 4 * g4 + i) * LDD + col] = pf.r[j][it][i];
          sm.u.ln.dB[(it * 16 + 4 * g4 + i) * LDD + col] = pf.db[j][it][i];
        }
    if (wave == SW) {
      const ChunkScalars cs{lb.G, lb.gam, lb.dec, lb.ae, lb.aw, lb.graw};
      scal_commit<C>(cs, pf.sc, lane);
    }
    const int mn = min(m + 1, p.M - 1);   // (the last lane refetches itself, unused)
    if constexpr (C < 64) prefetch_tiles(pf, mn, tid);   // the tile registers are free again: the next lane's
    __syncthreads();
    if (m > 0 && wave == SW) scalar_grads(m - 1, sm.lb[(m - 1) & 1]);

    // ---- dAq = dY R^T (j <= i) and dL = -dB R^T (j < i), lower tiles: task
    // pidx < NP is tile pair pidx of dAq, NP + pidx the same pair of dL ----
#pragma unroll
    for (int jj = 0; jj < NTASK; ++jj) {
      const int task = wave + NW * jj;
      if (task >= 2 * NP) continue;
      const bool isL = task >= NP;
      const int pidx = isL ? task - NP : task;
      int it, jt;
      tri_pair(pidx, it, jt);
      const CT* arow = isL ? &sm.u.ln.dB[(it * 16 + n16) * LDD] : &sm.u.ln.dy[(it * 16 + n16) * LDD];
      const f32x4 acc = tile_nt<CT, D>(arow, &sm.u.ln.R[(jt * 16 + n16) * LDD], g4);
      const int j = jt * 16 + n16;
      const float Gj = lb.G[j];
      float xm[4], xa[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = it * 16 + 4 * g4 + ii;
        xm[ii] = 0.f;
        xa[ii] = 0.f;
        const float Dij = __expf(lb.G[i] - Gj);
        if (!isL && j <= i) {
          const float dqk = acc[ii] * Dij;
          dgram[jj][ii] += dqk;
          xm[ii] = dqk * gram[jj][ii];
        } else if (isL && j < i) {
          const float dl = -acc[ii];
          const float kk = gram[jj][ii];
          const float dkk = dl * Dij * lb.ae[i];
          dgram[jj][ii] += dkk;
          xm[ii] = dkk * kk;
          xa[ii] = dl * Dij * kk;
        }
      }
      // row sums (over the 16 columns j, lane 15 of each row) and column sums (over the 16 rows i)
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
          lb.tri[pidx][slot][4 * g4 + ii] = rx[ii];
          if (isL) lb.tri[pidx][2][4 * g4 + ii] = ra[ii];
        }
      }
      float cx = (xm[0] + xm[1]) + (xm[2] + xm[3]);
      cx += __shfl_xor(cx, 16, 64);
      cx += __shfl_xor(cx, 32, 64);
      if (g4 == 0) lb.tri[pidx][slot + 1][n16] = cx;
      __builtin_amdgcn_sched_barrier(0);   // one task's fragments in flight at a time
    }

    // ---- P1 = dY S0^T, P2 = dB S0^T, P3 = R dS^T on this wave's key tiles:
    // this wave's rows of S0 / dS_C (fetched during the previous lane) become
    // fragments over k = v once, and their registers are refilled with the
    // next lane's rows right away, so those loads stream through the
    // products; then per row tile (one tile's P products live at a time) the
    // products, dV, da_w and the row sums ----
    Frag Sf[KT][NKV], dSf[KT][NKV];
    float sdot = 0.f;   // <dS_C, S0> over this wave's rows
#pragma unroll
    for (int kb = 0; kb < NKV; ++kb) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        f32x4 ys[TPS], yd[TPS];
#pragma unroll
        for (int hh = 0; hh < TPS; ++hh) {
          ys[hh] = tile_transpose_raw(pf.s[kt][kb * TPS + hh], lane);
          yd[hh] = tile_transpose_raw(pf.ds[kt][kb * TPS + hh], lane);
        }
        Sf[kt][kb] = acc_frag((CT*)nullptr, ys[0], ys[TPS - 1]);
        dSf[kt][kb] = acc_frag((CT*)nullptr, yd[0], yd[TPS - 1]);
#pragma unroll
        for (int e = 0; e < FragLen<CT>::value; ++e) sdot += to_f(Sf[kt][kb][e]) * to_f(dSf[kt][kb][e]);
      }
    }
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      f32x4 P1[KT], P2[KT], P3[KT];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) P1[kt] = P2[kt] = P3[kt] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKV; ++kb) {
        const Frag fy = ld_frag(&sm.u.ln.dy[(it * 16 + n16) * LDD + kb * KS], g4);
        const Frag fb = ld_frag(&sm.u.ln.dB[(it * 16 + n16) * LDD + kb * KS], g4);
        const Frag fr = ld_frag(&sm.u.ln.R[(it * 16 + n16) * LDD + kb * KS], g4);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          mma(P1[kt], fy, Sf[kt][kb]);
          mma(P2[kt], fb, Sf[kt][kb]);
          mma(P3[kt], fr, dSf[kt][kb]);
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the fragment loads of one k-step at a time in flight
      }
      // this lane's columns of q, k, v, dB, then 16 independent DPP row-sum
      // chains (summed over the wave's key tiles), then one masked block of stores
      const f32x4 gi = *(const f32x4*)&lb.gam[it * 16 + 4 * g4];
      const f32x4 ei = *(const f32x4*)&lb.ae[it * 16 + 4 * g4];
      const f32x4 di = *(const f32x4*)&lb.dec[it * 16 + 4 * g4];
      const f32x4 wi = *(const f32x4*)&lb.aw[it * 16 + 4 * g4];
      float part[4][4];   // [ii][q.P1, k.P2, k.P3, v.dB] over this wave's columns
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) part[ii][q4] = 0.f;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int dcol = (tile0 + kt) * 16 + n16;
        float xq[4], xk[4], xb[4], xv[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = it * 16 + 4 * g4 + ii;
          xb[ii] = to_f(sm.u.ln.dB[i * LDD + dcol]);
          xk[ii] = to_f(sm.k[i * LDD + dcol]);
          xq[ii] = to_f(sm.q[i * LDD + dcol]);
          xv[ii] = to_f(sm.v[i * LDD + dcol]);
        }
        dQacc[kt][it] += gi * P1[kt];
        dKacc[kt][it] += di * P3[kt] - ei * gi * P2[kt];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          dVacc[kt][it][ii] += wi[ii] * xb[ii];
          part[ii][0] += P1[kt][ii] * xq[ii];
          part[ii][1] += P2[kt][ii] * xk[ii];
          part[ii][2] += P3[kt][ii] * xk[ii];
          part[ii][3] += xb[ii] * xv[ii];
        }
      }
      float rsum[4][4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) rsum[ii][q4] = row_prefix16(part[ii][q4]);
      if (n16 == 15) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) lb.red[it * 16 + 4 * g4 + ii][q4 * NW + wave] = rsum[ii][q4];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next lane's state rows: in flight through this lane's reductions and
    // the next lane's commit and C x C tiles
#pragma unroll
    for (int V = 0; V < NDT; ++V) prefetch_state(pf, mn, V, tid);
    sdot = wave_sum(sdot);
    if (lane == 0) lb.scal[wave] = sdot;
  }
  __syncthreads();  // lane tiles dead: the union becomes Q^T, K^T and the gram-gradient factors
  if (wave == SW) scalar_grads(p.M - 1, sm.lb[(p.M - 1) & 1]);

  // ---- gram gradient products, shared over lanes: A1 = dQK (lower incl.
  // diagonal), A2 = dQK^T, A3 = dKK + dKK^T, written from the owning waves'
  // registers (the masked entries of a tile are zero) over zeroed matrices ----
  for (int idx = tid; idx < C * LDC; idx += NT) {
    sm.u.fin.A1[idx] = from_f<CT>(0.f);
    sm.u.fin.A2[idx] = from_f<CT>(0.f);
    sm.u.fin.A3[idx] = from_f<CT>(0.f);
  }
  for (int idx = tid; idx < C * D; idx += NT) {
    const int i = idx / D, d = idx % D;
    sm.u.fin.qt[d * LDC + i] = sm.q[i * LDD + d];
    sm.u.fin.kt[d * LDC + i] = sm.k[i * LDD + d];
  }
  __syncthreads();
#pragma unroll
  for (int jj = 0; jj < NTASK; ++jj) {
    const int task = wave + NW * jj;
    if (task >= 2 * NP) continue;
    const bool isL = task >= NP;
    int it, jt;
    tri_pair(isL ? task - NP : task, it, jt);
    const int j = jt * 16 + n16;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = it * 16 + 4 * g4 + ii;
      const CT x = from_f<CT>(dgram[jj][ii]);
      if (!isL) {
        if (j <= i) {
          sm.u.fin.A1[i * LDC + j] = x;
          sm.u.fin.A2[j * LDC + i] = x;
        }
      } else if (j < i) {
        sm.u.fin.A3[i * LDC + j] = x;
        sm.u.fin.A3[j * LDC + i] = x;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int dcol = (tile0 + kt) * 16 + n16;
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      dQacc[kt][it] += tile_nt<CT, C>(&sm.u.fin.A1[(it * 16 + n16) * LDC], &sm.u.fin.kt[dcol * LDC], g4);
      dKacc[kt][it] += tile_nt<CT, C>(&sm.u.fin.A2[(it * 16 + n16) * LDC], &sm.u.fin.qt[dcol * LDC], g4);
      dKacc[kt][it] += tile_nt<CT, C>(&sm.u.fin.A3[(it * 16 + n16) * LDC], &sm.u.fin.kt[dcol * LDC], g4);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // stores: transposed tiles, lane (g, n) holds row it*16+n, columns 16*tile + 4g..4g+3
  CT* dq = (CT*)p.dq;
  CT* dk = (CT*)p.dk;
  CT* dv = (CT*)p.dv;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      const int t = t0 + it * 16 + n16;
      const f32x4 xq = tile_transpose((CT*)nullptr, dQacc[kt][it], lane);
      const f32x4 xk = tile_transpose((CT*)nullptr, dKacc[kt][it], lane);
      const f32x4 xv = tile_transpose((CT*)nullptr, dVacc[kt][it], lane);
      if (t < p.T) {
        const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + (tile0 + kt) * 16 + 4 * g4;
        st4(dq + off, xq[0], xq[1], xq[2], xq[3]);
        st4(dk + off, xk[0], xk[1], xk[2], xk[3]);
        st4(dv + off, xv[0], xv[1], xv[2], xv[3]);
      }
    }
}

// the per-token scalar gradients of the KH key parts, added in a fixed order
template <int KH>
__global__ void __launch_bounds__(256) delta_bwd_parts_kernel(const float* __restrict__ part, float* dae,
                                                              float* daw, float* dg, long long rows) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < rows; i += (long long)gridDim.x * 256) {
    float s[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KH; ++k)
#pragma unroll
      for (int q = 0; q < 3; ++q) s[q] += part[((size_t)k * 3 + q) * rows + i];
    dae[i] = s[0];
    daw[i] = s[1];
    dg[i] = s[2];
  }
}

// stages: bit 0 = reverse state scan, bit 1 = gradient kernel
template <typename CT, int D, int C>
static int launch_bwd(const DeltaBwdArgs& a, int stages, hipStream_t stream) {
  const int NC = (a.T + C - 1) / C;
  if (stages & 1) {
    const int rc = delta_scan_bwd_dispatch(a, stream);
    if (rc) return rc;
  }
  if ((stages & 2) && a.cps > 1) return delta_grad_seg_dispatch(a, stream);   // checkpointed stash
  if (stages & 2) {
    constexpr int KH = GradDims<CT, D, C>::KH;
    hipLaunchKernelGGL((delta_bwd_grads_kernel<CT, D, C>), dim3(a.B * a.H * NC * KH), dim3(GradDims<CT, D, C>::NT),
                       0, stream, a);
    int rc = check_launch("delta_bwd_grads_kernel");
    if (rc || KH == 1) return rc;
    const size_t nrec = (size_t)a.B * a.H * a.M * NC, esz = sizeof(CT);
    const float* part = (const float*)((const char*)a.ds_stash + nrec * ((size_t)a.D * a.D + (size_t)C * a.D) * esz);
    const long long rows = (long long)a.B * a.T * a.H * a.M;
    const long long nb = (rows + 255) / 256;
    hipLaunchKernelGGL((delta_bwd_parts_kernel<KH>), dim3((unsigned)(nb < 2048 ? nb : 2048)), dim3(256), 0, stream,
                       part, a.dae, a.daw, a.dg, rows);
    return check_launch("delta_bwd_parts_kernel");
  }
  return GDNX_OK;
}

int delta_bwd_dispatch(const DeltaBwdArgs& a, int stages, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
    if (a.D == 128 && a.C == 64) return launch_bwd<bf16, 128, 64>(a, stages, stream);
    if (a.D == 64 && a.C == 64) return launch_bwd<bf16, 64, 64>(a, stages, stream);
    if (a.D == 128 && a.C == 32) return launch_bwd<bf16, 128, 32>(a, stages, stream);
    if (a.D == 64 && a.C == 32) return launch_bwd<bf16, 64, 32>(a, stages, stream);
  } else {
    if (a.D == 128 && a.C == 16) return launch_bwd<float, 128, 16>(a, stages, stream);
    if (a.D == 64 && a.C == 16) return launch_bwd<float, 64, 16>(a, stages, stream);
    if (a.D == 64 && a.C == 32) return launch_bwd<float, 64, 32>(a, stages, stream);
  }
  return set_error(GDNX_ERR_SHAPE, "backward: unsupported head dim %d / chunk %d for this dtype (use "
                   "gdnx_delta_train_chunk_size)", a.D, a.C);
}

}  // namespace gdnx

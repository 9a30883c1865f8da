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
#ifndef GDNX_GRADS_WAVES_PER_EU
#define GDNX_GRADS_WAVES_PER_EU 2
#endif
// One wave per 16-column tile of the key dimension (D/16 waves): each wave
// keeps only its own rows of S0 / dS_C and its dq/dk/dv tiles in registers.
template <typename CT, int D>
struct GradDims {
  static constexpr int NW = D / 16;
  static constexpr int NT = 64 * NW;
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
  static constexpr int LDD = Dm::LDD, LDC = Dm::LDC, LDF = Dm::LDF, NW = GradDims<CT, D>::NW;
  static constexpr int NP = (C / 16) * (C / 16 + 1) / 2;  // lower 16x16 tile pairs
  CT q[C * LDD];
  CT k[C * LDD];
  CT v[C * LDD];
  float KK[C * LDF];   // k_i . k_j  (lower)
  float QK[C * LDF];   // q_i . k_j  (lower incl. diagonal)
  float dQK[C * LDF];  // sum over lanes of dL/d(q_i.k_j)
  float dKK[C * LDF];  // sum over lanes of dL/d(k_i.k_j), j < i
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

// The value unchanged, but opaque to the optimizer.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// One lane's inputs to the gradient kernel, fetched a lane ahead: this
// wave's rows of S0 and dS_C (raw tiles, one per 16 value columns), this
// thread's share of the R / dB tiles and of dY, and (scalar wave) the
// per-token coefficients.
template <typename CT, int D, int C>
struct GradPrefetch {
  typedef typename Vec4T<CT>::type V4;
  static constexpr int NDT = D / 16, NCT = C / 16, NT = GradDims<CT, D>::NT;
  static constexpr int VEC = 16 / sizeof(CT);
  static constexpr int NDY = (C * D / VEC + NT - 1) / NT;
  V4 s[NDT], ds[NDT];
  V4 r[NCT], db[NCT];
  uint4 dy[NDY];
  ScalarRegs sc;
};

// Gradient kernel: one workgroup per (batch, head, chunk), looping over the M
// lanes that share q/k/v.  Per lane it reads the stashed S0, R (forward) and
// dS_C, dB (reverse scan) and forms, wave w owning key columns d and value
// columns v in [16w, 16w+16):
//   P1 = dY S0^T, P2 = dB S0^T, P3 = R dS_C^T      (S0 / dS_C rows of this wave
//                                                   as fragments over k = v)
//   dQ += diag(exp G) P1,  dK += diag(dec) P3 - diag(a_e exp G) P2
//   dV += diag(a_w) dB,    da_w = rowsum(dB o V)
//   dAq = dY R^T (j<=i),   dL = -dB R^T (j<i)  -> dQK, dKK (lane sums) and the
//   per-token decay / erase gradients.
// After the lanes: dQ += dQK K, dK += dQK^T Q + (dKK + dKK^T) K.
template <typename CT, int D, int C>
__global__ void __launch_bounds__((GradDims<CT, D>::NT)) __attribute__((amdgpu_waves_per_eu(GDNX_GRADS_WAVES_PER_EU)))
delta_bwd_grads_kernel(DeltaBwdArgs p) {
  typedef Dims<CT, D, C> Dm;
  typedef typename Dm::Frag Frag;
  typedef BwdGradSmem<CT, D, C> Sm;
  typedef GradPrefetch<CT, D, C> Pf;
  typedef GradLaneBuf<C, GradDims<CT, D>::NW, Sm::NP> LB;
  typedef typename Vec4T<CT>::type V4;
  constexpr int KS = Dm::KS, TPS = Dm::TPS, NCT = Dm::NCT, NDT = Dm::NDT, LDD = Dm::LDD, LDC = Dm::LDC;
  constexpr int LDF = Dm::LDF, NW = GradDims<CT, D>::NW, NT = GradDims<CT, D>::NT, NKV = D / KS, NP = Sm::NP;
  constexpr int SW = NW - 1;  // the wave that forms the per-token scalar gradients
  __shared__ Sm sm;

  const int tid0 = threadIdx.x;
  const int tid = tid0;
  const int wave = tid >> 6, lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
  const int dcol = wave * 16 + n16;  // this lane's key (and value) column
  const int NC = (p.T + C - 1) / C;
  const int nblocks = p.B * p.H * NC;
  const int blk = xcd_remap(blockIdx.x, nblocks);
  const int c = blk % NC;
  const int h = (blk / NC) % p.H;
  const int b = blk / (NC * p.H);
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
    for (int it = 0; it < NCT; ++it) {  // tile (it, V = wave) of R and dB
      const size_t off = rec * C * D + stash_tile_offset<CT, D>(it, wave, lane_);
      f.r[it] = *(const V4*)(r_st + off);
      f.db[it] = *(const V4*)(db_st + off);
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
    f.s[V] = *(const V4*)stash_state_ptr<CT, D, C>(s_st + rec * D * D, wave, V, tid_ & 63);
    f.ds[V] = *(const V4*)stash_state_ptr<CT, D, C>(ds_st + rec * D * D, wave, V, tid_ & 63);
  };

  // ---- per-token scalar gradients of lane mm (wave SW, one token per lane) ----
  auto scalar_grads = [&](int mm, const LB& q) {
    float dGi = 0.f, daei = 0.f, dawi = 0.f, r3d = 0.f;
    if (lane < C) {
      const int i = lane, ib = i >> 4, ir = i & 15;
      float rs[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) {   // this row's NW partials, read as 16-byte vectors
        rs[a] = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w += 4) {
          const f32x4 x = *(const f32x4*)&q.red[i][a * NW + w];
          rs[a] += (x[0] + x[1]) + (x[2] + x[3]);
        }
      }
      dawi = rs[3];
      dGi = q.gam[i] * rs[0] - q.gam[i] * q.ae[i] * rs[1] - q.dec[i] * rs[2];
      daei = -q.gam[i] * rs[1];
      // Xm row i lives in tiles (ib, jt <= ib); column i in tiles (it >= ib, ib);
      // compile-time tile loops, predicated on the lane's row block
#pragma unroll
      for (int bi = 0; bi < NCT; ++bi) {
#pragma unroll
        for (int bj = 0; bj <= bi; ++bj) {
          const int pr = bi * (bi + 1) / 2 + bj;
          if (bi == ib) {
            dGi += q.tri[pr][0][ir] + q.tri[pr][3][ir];
            daei += q.tri[pr][2][ir];
          }
          if (bj == ib) dGi -= q.tri[pr][1][ir] + q.tri[pr][4][ir];
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
      p.dae[si] = daei;
      p.daw[si] = dawi;
      p.dg[si] = (raw <= 0.f && raw >= kLogFloor) ? sfx : 0.f;
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
  for (int i = tid; i < C * LDF; i += NT) {
    sm.dQK[i] = 0.f;
    sm.dKK[i] = 0.f;
  }
  f32x4 dQacc[NCT], dKacc[NCT], dVacc[NCT];
#pragma unroll
  for (int it = 0; it < NCT; ++it) dQacc[it] = dKacc[it] = dVacc[it] = zero4();
  __syncthreads();
  // raw grams (shared by the lanes)
  for (int task = wave; task < 2 * NP; task += NW) {
    int it, jt;
    tri_pair(task >> 1, it, jt);
    const CT* arow = ((task & 1) == 0) ? &sm.k[(it * 16 + n16) * LDD] : &sm.q[(it * 16 + n16) * LDD];
    const f32x4 acc = tile_nt<CT, D>(arow, &sm.k[(jt * 16 + n16) * LDD], g4);
    float* dst = ((task & 1) == 0) ? sm.KK : sm.QK;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) dst[(it * 16 + 4 * g4 + ii) * LDF + jt * 16 + n16] = acc[ii];
  }

  for (int m = 0; m < p.M; ++m) {
    // per-thread indices re-derived each lane: keeps the compiler from hoisting
    // (and spilling) every loop-invariant per-thread address out of the loop
    const int tid = opaque(tid0);
    const int lane = tid & 63, g4 = lane >> 4, n16 = lane & 15;
    const int dcol = wave * 16 + n16;
    LB& lb = sm.lb[m & 1];
    __syncthreads();  // lane m-1 done with the lane tiles; lane m-2's scalar pass done with lb
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
    for (int it = 0; it < NCT; ++it)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sm.u.ln.R[(it * 16 + 4 * g4 + i) * LDD + dcol] = pf.r[it][i];
        sm.u.ln.dB[(it * 16 + 4 * g4 + i) * LDD + dcol] = pf.db[it][i];
      }
    if (wave == SW) {
      const ChunkScalars cs{lb.G, lb.gam, lb.dec, lb.ae, lb.aw, lb.graw};
      scal_commit<C>(cs, pf.sc, lane);
    }
    const int mn = min(m + 1, p.M - 1);   // (the last lane refetches itself, unused)
    prefetch_tiles(pf, mn, tid);          // the tile registers are free again: fetch the next lane's
    __syncthreads();
    if (m > 0 && wave == SW) scalar_grads(m - 1, sm.lb[(m - 1) & 1]);

    // ---- dAq = dY R^T (j <= i) and dL = -dB R^T (j < i), lower tiles: task
    // pidx < NP is tile pair pidx of dAq, NP + pidx the same pair of dL ----
    for (int task = wave; task < 2 * NP; task += NW) {
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
          sm.dQK[i * LDF + j] += dqk;
          xm[ii] = dqk * sm.QK[i * LDF + j];
        } else if (isL && j < i) {
          const float dl = -acc[ii];
          const float kk = sm.KK[i * LDF + j];
          const float dkk = dl * Dij * lb.ae[i];
          sm.dKK[i * LDF + j] += dkk;
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
    }

    // ---- P1 = dY S0^T, P2 = dB S0^T, P3 = R dS^T on this wave's d tile, k-step
    // outer: this wave's rows of S0 / dS_C (fetched during the previous lane)
    // become fragments over k = v one k-step at a time, and their registers
    // are refilled with the next lane's rows right away, so those loads stream
    // through the products; then dV, da_w and the row sums ----
    f32x4 P1[NCT], P2[NCT], P3[NCT];
#pragma unroll
    for (int it = 0; it < NCT; ++it) P1[it] = P2[it] = P3[it] = zero4();
    float sdot = 0.f;   // <dS_C, S0> over this wave's rows
#pragma unroll
    for (int kb = 0; kb < NKV; ++kb) {
      f32x4 ys[TPS], yd[TPS];
#pragma unroll
      for (int hh = 0; hh < TPS; ++hh) {
        ys[hh] = tile_transpose_raw(pf.s[kb * TPS + hh], lane);
        yd[hh] = tile_transpose_raw(pf.ds[kb * TPS + hh], lane);
      }
      const Frag Sf = acc_frag((CT*)nullptr, ys[0], ys[TPS - 1]);
      const Frag dSf = acc_frag((CT*)nullptr, yd[0], yd[TPS - 1]);
#pragma unroll
      for (int e = 0; e < FragLen<CT>::value; ++e) sdot += to_f(Sf[e]) * to_f(dSf[e]);
#pragma unroll
      for (int hh = 0; hh < TPS; ++hh) prefetch_state(pf, mn, kb * TPS + hh, tid);
#pragma unroll
      for (int it = 0; it < NCT; ++it) {
        mma(P1[it], ld_frag(&sm.u.ln.dy[(it * 16 + n16) * LDD + kb * KS], g4), Sf);
        mma(P2[it], ld_frag(&sm.u.ln.dB[(it * 16 + n16) * LDD + kb * KS], g4), Sf);
        mma(P3[it], ld_frag(&sm.u.ln.R[(it * 16 + n16) * LDD + kb * KS], g4), dSf);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // per row tile: this lane's column of q, k, v, dB read first, then 16
    // independent DPP row-sum chains, then one masked block of stores
#pragma unroll
    for (int it = 0; it < NCT; ++it) {
      float xq[4], xk[4], xv[4], xb[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = it * 16 + 4 * g4 + ii;
        xb[ii] = to_f(sm.u.ln.dB[i * LDD + dcol]);
        xk[ii] = to_f(sm.k[i * LDD + dcol]);
        xq[ii] = to_f(sm.q[i * LDD + dcol]);
        xv[ii] = to_f(sm.v[i * LDD + dcol]);
      }
      const f32x4 gi = *(const f32x4*)&lb.gam[it * 16 + 4 * g4];
      const f32x4 ei = *(const f32x4*)&lb.ae[it * 16 + 4 * g4];
      const f32x4 di = *(const f32x4*)&lb.dec[it * 16 + 4 * g4];
      const f32x4 wi = *(const f32x4*)&lb.aw[it * 16 + 4 * g4];
      dQacc[it] += gi * P1[it];
      dKacc[it] += di * P3[it] - ei * gi * P2[it];
      float rsum[4][4];   // [ii][q.P1, k.P2, k.P3, v.dB]
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        dVacc[it][ii] += wi[ii] * xb[ii];
        rsum[ii][0] = row_prefix16(P1[it][ii] * xq[ii]);
        rsum[ii][1] = row_prefix16(P2[it][ii] * xk[ii]);
        rsum[ii][2] = row_prefix16(P3[it][ii] * xk[ii]);
        rsum[ii][3] = row_prefix16(xb[ii] * xv[ii]);
      }
      if (n16 == 15) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) lb.red[it * 16 + 4 * g4 + ii][q4 * NW + wave] = rsum[ii][q4];
      }
    }
    sdot = wave_sum(sdot);
    if (lane == 0) lb.scal[wave] = sdot;
  }
  __syncthreads();  // lane tiles dead: the union becomes Q^T, K^T and the gram-gradient factors
  if (wave == SW) scalar_grads(p.M - 1, sm.lb[(p.M - 1) & 1]);

  // ---- gram gradient products, shared over lanes ----
  for (int idx = tid; idx < C * C; idx += NT) {
    const int i = idx / C, j = idx % C;
    sm.u.fin.A1[i * LDC + j] = from_f<CT>((j <= i) ? sm.dQK[i * LDF + j] : 0.f);
    sm.u.fin.A2[i * LDC + j] = from_f<CT>((i <= j) ? sm.dQK[j * LDF + i] : 0.f);
    const float s = (j < i) ? sm.dKK[i * LDF + j] : ((i < j) ? sm.dKK[j * LDF + i] : 0.f);
    sm.u.fin.A3[i * LDC + j] = from_f<CT>(s);
  }
  for (int idx = tid; idx < C * D; idx += NT) {
    const int i = idx / D, d = idx % D;
    sm.u.fin.qt[d * LDC + i] = sm.q[i * LDD + d];
    sm.u.fin.kt[d * LDC + i] = sm.k[i * LDD + d];
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < NCT; ++it) {
    dQacc[it] += tile_nt<CT, C>(&sm.u.fin.A1[(it * 16 + n16) * LDC], &sm.u.fin.kt[dcol * LDC], g4);
    dKacc[it] += tile_nt<CT, C>(&sm.u.fin.A2[(it * 16 + n16) * LDC], &sm.u.fin.qt[dcol * LDC], g4);
    dKacc[it] += tile_nt<CT, C>(&sm.u.fin.A3[(it * 16 + n16) * LDC], &sm.u.fin.kt[dcol * LDC], g4);
  }
  // stores: transposed tiles, lane (g, n) holds row it*16+n, columns 16*wave + 4g..4g+3
  CT* dq = (CT*)p.dq;
  CT* dk = (CT*)p.dk;
  CT* dv = (CT*)p.dv;
#pragma unroll
  for (int it = 0; it < NCT; ++it) {
    const int t = t0 + it * 16 + n16;
    const f32x4 xq = tile_transpose((CT*)nullptr, dQacc[it], lane);
    const f32x4 xk = tile_transpose((CT*)nullptr, dKacc[it], lane);
    const f32x4 xv = tile_transpose((CT*)nullptr, dVacc[it], lane);
    if (t < p.T) {
      const size_t off = ((size_t)(b * p.T + t) * p.H + h) * D + wave * 16 + 4 * g4;
      st4(dq + off, xq[0], xq[1], xq[2], xq[3]);
      st4(dk + off, xk[0], xk[1], xk[2], xk[3]);
      st4(dv + off, xv[0], xv[1], xv[2], xv[3]);
    }
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
  if (stages & 2) {
    hipLaunchKernelGGL((delta_bwd_grads_kernel<CT, D, C>), dim3(a.B * a.H * NC), dim3(GradDims<CT, D>::NT), 0, stream, a);
    return check_launch("delta_bwd_grads_kernel");
  }
  return GDNX_OK;
}

int delta_bwd_dispatch(const DeltaBwdArgs& a, int stages, hipStream_t stream) {
  if (a.dtype == GDNX_DTYPE_BF16) {
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

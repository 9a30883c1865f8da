// Internal (non-ABI) declarations shared by the gdnx translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/gdnx.h"

namespace gdnx {

struct DeltaArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  const float* s0;
  void* y;
  float* s_out;
  void* chunk_states;
  int B, T, H, M, D, C, dtype;
  float* r_norm;  // [B,T,H,M] |net write| per token, or null
  void* prep;     // per-chunk operand records (delta_prep_kernel), or null
  int cps;        // chunks per stashed state record (delta_stash_cps)
};

struct DeltaBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  const void* dy;
  const float* ds_final;
  const void* s_stash;   // the forward's chunk_states: states, net writes, prep records
  void* ds_stash;         // state gradients at chunk ends, then dB
  void* dq;
  void* dk;
  void* dv;
  float* dae;
  float* daw;
  float* dg;
  float* ds0;
  int B, T, H, M, D, C, dtype;
  int cps;                // chunks per stashed state record (delta_stash_cps)
};

struct GCoeffArgs {
  const void* k;       // [B,T,H,D] io dtype
  const float* beta;   // [B,T,H,M]
  float* a;            // [B,T,H,M] (forward)
  const float* da_e;   // [B,T,H,M] (backward)
  const float* da_w;   // [B,T,H,M] or null (backward)
  void* dk;            // [B,T,H,D] io dtype, accumulated in place (backward)
  float* dbeta;        // [B,T,H,M] (backward)
  int B, T, H, M, D, dtype;
};

// Per-key-channel decay (one chain per head): float32 tensors, q/k/v/y/lg
// [B,T,H,D], be/bw [B,T,H], states [B,H,D,D].
struct ChanArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* be;
  const float* bw;
  const float* lg;     // natural-log decay per key channel
  const float* s0;
  float* y;
  float* s_out;
  void* chunk_states;
  float* r_norm;
  int B, T, H, D;
  void* workspace;     // forward operand records when chunk_states is null
  float* frec;         // (set by the dispatcher) forward / backward operand records
  float* brec;
};

struct ChanBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* be;
  const float* bw;
  const float* lg;
  const float* dy;
  const float* ds_final;
  const void* s_stash;   // the forward's chunk_states
  void* ds_stash;        // workspace: state gradients, then dB
  float* dq;
  float* dk;
  float* dv;
  float* dbe;
  float* dbw;
  float* dlg;
  float* ds0;
  int B, T, H, D;
};

// Opt-in non-finite detection (finite.hip): with gdnx_set_check_finite(1),
// finite_outputs scans the buffers, synchronises the stream and returns
// GDNX_ERR_NONFINITE if any element is NaN or infinite; otherwise GDNX_OK
// at no cost.
struct FiniteBuf {
  const void* p;
  size_t n;
  int dtype;   // GDNX_DTYPE_*
};
bool check_finite_on();
int finite_check(const FiniteBuf* bufs, int nbuf, hipStream_t stream);
int finite_outputs(const FiniteBuf* bufs, int nbuf, hipStream_t stream);

// Record an error message for gdnx_last_error(); returns code.
int set_error(int code, const char* fmt, ...);
// Check hipGetLastError() after a launch.
int check_launch(const char* what);

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* ae;
  const float* aw;
  const float* g;
  float* state;
  void* y;
  int NS, H, M, D, dtype;
  const int* slots;    // [NS] state-pool slot of each row, or null (row s uses state s)
  int nslots;
  int chan;            // 1: g is a log decay per key channel, [NS, H, M, D]
};

// One-token step of the GDN3 Kronecker-residual state (gdn3_decode.hip).
// Row s of the batch advances state index slots[s] (or s) of every (h, m).
struct G3DecArgs {
  const void* q;       // [NS, H, qkv_lanes, D] io dtype
  const void* k;
  const void* v;
  const float* bg;     // [NS, H, M, gate_ch]
  const float* wg;
  const float* dec;    // [NS, H, M]
  float* A;            // [n_slots, H, M, R, a_v, a_k] (updated in place)
  float* Bf;           // [n_slots, H, M, R, b_v, b_k]
  float* U;            // [n_slots, H, M, D, P]
  float* Vb;           // [n_slots, H, M, D, P]
  const int* slots;    // [NS] or null
  const int* pos;      // [NS] global token index of the row's token
  void* y;             // [NS, H, M, D] io dtype
  double* stats;       // [NS, H, M, 2] or null (zeroed; a compaction overwrites its chain's)
  int NS, nslots, H, M, D, P, qkv_lanes, gate_ch, dtype;
};

// Kronecker-residual geometry: state S = sum_r A_r (x) B_r + U Vb^T with
// A_r [a_v, a_k], B_r [b_v, b_k]; m = a_v a_k, n = b_v b_k, q = sketch width.
// The factors of a power-of-two head dim are powers of two; l* are their
// base-2 logarithms.
struct G3Geom {
  int R, av, ak, bv, bk, m, n, q;
  int lav, lak, lbv, lbk;
};

struct G3FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* bg;     // erase gates, [B,T,H,M,D] or [B,T,H,M]
  const float* wg;     // write gates, same layout
  const float* dec;    // multiplicative decay [B,T,H,M]
  const float* sketch; // [N, n, q]
  void* y;             // [B,T,H,M,D]
  float* A_out;        // [N,R,a_v,a_k] or null
  float* B_out;        // [N,R,b_v,b_k] or null
  float* U_out;        // [N,D,P] or null
  float* Vb_out;       // [N,D,P] or null
  double* stats;       // [T/Kc, N, 2] (energy, kept) or null
  void* workspace;     // carved by the dispatcher into the fields below
  void* train_states;  // training stash for the backward (layout G3Stash) or null
  G3Geom ge;
  int B, T, H, M, D, P, Kc, qkv_lanes, gate_ch, dtype;
  float sdec;
  // carried state: token 0 of this call is global token t0 (it writes slot
  // t0 mod P; compactions follow global tokens t with (t + 1) mod Kc == 0);
  // A0/B0/U0/Vb0 in the output layouts, or all null for a zero state
  int t0;
  int cmode;           // compaction mode (G3CompactArgs::mode)
  const float* A0;
  const float* B0;
  const float* U0;
  const float* Vb0;
  float* ts_u;         // (set by the dispatcher from train_states)
  float* ts_g;
  int nch;
  // per launch (set by the dispatcher)
  void* skron;         // [N, D, D] compute dtype: sum_r A_r (x) B_r
  float* ab;           // [N, R (m + n)]: A | B as of the last compaction
  float* uw;           // [N, P, D] window net writes
  float* vw;           // [N, P, D] window keys decayed to the window end
  float* gsum;         // [N] log decay since the last compaction
  int c0, c1, first, live, last, complete;
};

struct G3CompactArgs {
  const float* A;
  const float* Bf;
  const float* U;      // net writes: element (chain, slot p, feature d) at chain*D*P + p*u_sp + d*u_sd
  const float* Vb;     // keys, same layout
  const float* sketch; // [N, n, q]
  float* A_out;
  float* B_out;
  double* stats;       // [N, 2] or null
  G3Geom ge;
  int N, D, P;
  float sdec;
  int u_sp, u_sd;
  const float* gsum;   // [N] log decay of A and B since they were stored, or null
  void* skron;         // materialised [N, D, D] Kronecker matrix out, or null
  int skron_dtype;
  float* A_fin;        // optional second copy of the result, or null
  float* B_fin;
  float* ab_stash;     // [N][R (m + n)] copy of the result (A | B) for the backward, or null
  // decode: block n is chain n of a batch of rows (hm = H M chains per row);
  // it compacts only when (pos[row] + 1) % Kc == 0, on state index
  // slots[row] * hm + n % hm (or n without slots; a slot outside
  // [0, nslots) is an empty row).  pos null: every block compacts chain n.
  const int* pos;
  const int* slots;
  int hm, Kc, nslots;
  int mode;            // 0: 'svd' (range finder + SVD), 1: 'sketch' (normalised sketch, no SVD)
};

// Backward of the Kronecker-residual regime (gdn3_bwd.hip)
struct G3BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* bg;
  const float* wg;
  const float* dec;
  const void* dy;             // [B,T,H,M,D] compute dtype
  const void* train_states;   // the forward's stash (layout G3Stash)
  float* dq;                  // [B,T,H,M,D] per lane
  float* dk;
  float* dv;
  float* dbg;                 // gate layout ([.., D] or [..])
  float* dwg;
  float* ddec;                // [B,T,H,M]
  int B, T, H, M, D, P, Kc, qkv_lanes, gate_ch, dtype;
};

struct KronReadArgs {
  const float* A;
  const float* Bf;
  const float* U;   // [N, D, P]
  const float* Vb;  // [N, D, P]
  const float* x;   // [N, C, D]
  float* y;         // [N, C, D]
  G3Geom ge;
  int N, C, D, P;
};

struct G3ProArgs {
  const void* q;
  const void* k;
  const void* bp;   // [rows, M, K]
  const void* pa;   // [rows]
  const void* wp;   // [rows, M, V]
  const void* pb;   // [rows]
  const void* dp;   // [rows, M, 4]
  const float* rates;
  const float* cs;  // [M, T, K/2]
  const float* sn;
  void* qr;         // [rows, M, K]
  void* kr;
  float* bg;
  float* wg;
  float* dec;       // [rows, M]
  const float* dqr; // backward inputs, float32, forward-output layouts
  const float* dkr;
  const float* dbg;
  const float* dwg;
  const float* ddec;
  float* dq;        // backward outputs, float32, forward-input layouts
  float* dk;
  float* dbp;
  float* dpa;
  float* dwp;
  float* dpb;
  float* ddp;
  long long rows;
  int T, H, M, K, V;
  int pairs[4];
  float clamp;
};

struct G3EpiArgs {
  const void* y;     // [rows, M, V]
  const void* lg;    // [rows, M]
  const float* norm; // [V]
  void* out;         // [rows, V]
  const void* dout;  // backward: [rows, V]
  void* dy;          // [rows, M, V]
  float* dlg;        // [rows, M]
  float* part;       // [gridDim.x, V] partial d_norm
  float* dnorm;      // [V]
  long long rows;
  int M, V;
};

int gdn3_fwd_dispatch(const G3FwdArgs& a, hipStream_t stream);
bool gdn3_fwd_fused(int D, int P, int Kc, int dtype);
// bytes of the static scratch of gdnx_gdn3_chunk_fwd_state_noalloc (per device)
constexpr size_t kG3ScratchBytes = (size_t)64 << 20;
// that scratch's address on the current device (resolved once per device)
int gdn3_scratch(void** out);
// p[0, n) = 0 on the stream (a fill kernel: safe inside graph capture)
int gdn3_zero_fill(float* p, size_t n, hipStream_t stream);
size_t gdn3_workspace_bytes(int N, int D, int P, int dtype);
size_t gdn3_train_states_bytes(int N, int T, int D, int P, int Kc);
int gdn3_bwd_dispatch(const G3BwdArgs& a, hipStream_t stream);
int gdn3_compact_dispatch(const G3CompactArgs& a, hipStream_t stream);
int kron_read_dispatch(const KronReadArgs& a, hipStream_t stream);
int decode_dispatch(const DecodeArgs& a, hipStream_t stream);
int gdn3_decode_dispatch(const G3DecArgs& a, hipStream_t stream);
int delta_fwd_dispatch(const DeltaArgs& a, hipStream_t stream);
int delta_prep_dispatch(const DeltaArgs& a, hipStream_t stream);
int delta_scan_fwd_dispatch(const DeltaArgs& a, hipStream_t stream);
int delta_scan_bwd_dispatch(const DeltaBwdArgs& a, hipStream_t stream);
size_t delta_prep_bytes(int nchains, int T, int C, int dtype);
// Tokens per recompute segment of the checkpointed backward: the forward
// keeps the state entering every segment, the reverse scan the state
// gradient leaving it, and the gradient kernel rebuilds the states and state
// gradients in between.
constexpr int kSegTokens = 256;
// Chunks per stashed state record: 1 (the state entering every chunk and the
// state gradient leaving it, read by delta_bwd_grads_kernel) or, for bf16 IO
// with 32-token chunks and at most 4 lanes per head, one record per
// kSegTokens-token segment (read by delta_grad_seg_kernel, which recomputes
// the rest in 32-token sub-chunks: the reverse scan's P3 = R dS^T is taken
// at its chunk ends, so its chunk must be the sub-chunk).
__host__ __device__ inline int delta_stash_cps(int D, int C, int dtype, int M) {
  return (dtype == GDNX_DTYPE_BF16 && C == 32 && M >= 1 && M <= 4 && (D == 64 || D == 128)) ? kSegTokens / C : 1;
}
// Per-chain stash geometry: NC chunks; a state record every cps chunks.
struct StashGeom {
  size_t nsrec;   // state records (ceil(NC / cps) per chain)
  size_t nrec;    // chunk records (NC per chain)
  size_t states;  // compute-dtype elements of the state region (nsrec D^2)
  size_t tiles;   // compute-dtype elements of the tile region (R or dB: nrec C D)
};
__host__ __device__ inline StashGeom stash_geom(int nchains, int T, int D, int C, int cps) {
  const size_t NC = (size_t)((T + C - 1) / C);
  StashGeom g;
  g.nsrec = (size_t)nchains * ((NC + cps - 1) / cps);
  g.nrec = (size_t)nchains * NC;
  g.states = g.nsrec * D * D;
  g.tiles = g.nrec * C * D;
  return g;
}
// The checkpointed backward's workspace (bf16 IO): the state gradients at
// segment ends, dB and P3 = R dS^T per token (bf16), k.P3 per token
// (float32), then, with more than two lanes per head, the float32 carry of
// the dq / dk / dv sums between lane pairs ([B H segments][3][kSegTokens][D]).
__host__ __device__ inline size_t delta_seg_carry_offset(int nchains, int T, int D, int C, int cps) {
  const StashGeom g = stash_geom(nchains, T, D, C, cps);
  return ((g.states + 2 * g.tiles) * 2 + g.nrec * C * sizeof(float) + 255) / 256 * 256;
}
// bytes of the state + net-write stash (the prep records follow it in chunk_states)
inline size_t delta_stash_bytes(int nchains, int T, int D, int C, int dtype, int cps) {
  const StashGeom g = stash_geom(nchains, T, D, C, cps);
  return (g.states + g.tiles) * (dtype == GDNX_DTYPE_BF16 ? 2 : 4);
}
// bytes of the backward's workspace: state gradients and dB like the
// forward's stash, then (checkpointed form) the gradient kernel's float32
// dq / dk / dv sums, [B, H, segments][3][kSegTokens][D], or (64-token
// chunks in the per-chunk form) the key halves' per-token partials
size_t delta_bwd_workspace_bytes(int B, int T, int H, int M, int D, int C, int dtype);
int delta_bwd_dispatch(const DeltaBwdArgs& a, int stages, hipStream_t stream);
// the gradient kernel of the checkpointed form (a.cps > 1, delta_grad_seg.hip)
int delta_grad_seg_dispatch(const DeltaBwdArgs& a, hipStream_t stream);
int gdn3_coeff_dispatch(const GCoeffArgs& a, bool bwd, hipStream_t stream);
// Rank-r RLS T-factor scan (rls.hip); all tensors float32
struct RlsDesc {
  const float* q;
  const float* K;
  const float* V;
  const float* Bg;
  const float* Wg;
  const float* a;
  const float* mix;
  const float* state0;
  const float* dy;
  const float* dstate;
  float* y;
  float* state_out;
  float* ckpt;
  float* dq;
  float* dK;
  float* dV;
  float* dBg;
  float* dWg;
  float* da;
  float* dmix;
  float* dstate0;
  int B, T, H, R, RO, dk, dv;
  float eps;
  int cP, cR, ste;   // testbed compaction (cP = 0: off)
  float cs;
  void* workspace;   // backward without compaction: row-block partials (or null)
};
size_t rls_ckpt_bytes(int nchains, int T, int R, int dk, int dv, int cP);
size_t rls_bwd_workspace_bytes(int nchains, int T, int R, int dk, int dv);
int rls_dispatch(const RlsDesc& d, bool bwd, hipStream_t stream);

void gdn3_lane_pairs(int M, int K, int pairs[4]);
size_t gdn3_epilogue_workspace_bytes(long long rows, int V);
int gdn3_prologue_dispatch(const G3ProArgs& a, bool bwd, int dtype, hipStream_t stream);
int gdn3_epilogue_dispatch(const G3EpiArgs& a, bool bwd, int dtype, hipStream_t stream);
int chan_fwd_dispatch(const ChanArgs& a, hipStream_t stream);
int chan_bwd_dispatch(const ChanBwdArgs& a, hipStream_t stream);
size_t chan_states_bytes(int nchains, int T, int D);
size_t chan_fwd_workspace_bytes(int nchains, int T, int D);
int delta_chunk_size(int D, int dtype);
int delta_train_chunk_size(int D, int dtype);

}  // namespace gdnx

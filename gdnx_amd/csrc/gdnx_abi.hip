// C-ABI entry points of libgdnx: argument validation, then dispatch.
#include <initializer_list>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "gdnx_internal.hpp"

namespace gdnx {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(GDNX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return GDNX_OK;
}

int delta_chunk_size(int D, int dtype) {
  if (D != 64 && D != 128) return 0;
  return dtype == GDNX_DTYPE_BF16 ? 64 : 32;
}

// chunk used when the forward stashes states for the backward: 32 for bf16
// (with at most 4 lanes per head the stash keeps one state per 256-token
// segment and the backward recomputes the rest), 16 for float32.  The
// 64-token bf16 chunk stays selectable in the per-chunk stash form: its
// scans hold one chunk's tiles in LDS instead of two (no overlap of the next
// chunk's staging), spill registers, and measured 1.5-2x slower on the
// config-2 step.
int delta_train_chunk_size(int D, int dtype) {
  if (D != 64 && D != 128) return 0;
  return dtype == GDNX_DTYPE_BF16 ? 32 : 16;
}

size_t delta_bwd_workspace_bytes(int B, int T, int H, int M, int D, int C, int dtype) {
  const int cps = delta_stash_cps(D, C, dtype, M);
  if (cps > 1) {   // see delta_seg_carry_offset
    const size_t nseg = (size_t)((T + kSegTokens - 1) / kSegTokens);
    return delta_seg_carry_offset(B * H * M, T, D, C, cps) +
           (M > 2 ? 3 * (size_t)B * H * nseg * kSegTokens * D * sizeof(float) : 0);
  }
  size_t n = delta_stash_bytes(B * H * M, T, D, C, dtype, cps);
  if (dtype == GDNX_DTYPE_BF16 && C == 64) {
    n += 2 * 3 * (size_t)B * T * H * M * sizeof(float);   // the two key halves' per-token partials
  }
  return n;
}

static bool valid_chunk(int D, int dtype, int C) {
  if (dtype == GDNX_DTYPE_BF16) return C == 32 || C == 64;
  return C == 16 || C == 32;
  (void)D;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Whether every factor is >= 0 and their product is at most limit (checked
// without forming a product that could overflow).
static bool prod_le(long long limit, std::initializer_list<long long> xs) {
  long long p = 1;
  for (long long x : xs) {
    if (x < 0) return false;
    if (x != 0 && p > limit / x) return false;
    p *= x;
  }
  return true;
}
// The sizes a size query accepts: at most 2^30 chains (B * H * M) and 2^40
// token-chains (B * T * H * M), so that every byte count below fits in 63 bits.
static bool query_sizes_ok(int B, int T, int H, int M) {
  return prod_le(1LL << 30, {B, H, M}) && prod_le(1LL << 40, {B, T, H, M});
}

static int check_common(const void* q, const void* k, const void* v, int B, int T, int H, int M,
                        int D, int dtype) {
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (D != 64 && D != 128) return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", D);
  if (B < 1 || T < 0 || H < 1 || M < 1)
    return set_error(GDNX_ERR_SHAPE, "bad sizes B=%d T=%d H=%d M=%d", B, T, H, M);
  if ((long long)B * H * M > (1LL << 30)) return set_error(GDNX_ERR_SHAPE, "too many chains");
  // in-chunk tile offsets (64 tokens x the lane-expanded token stride) are 32-bit
  if ((long long)H * M * D * 64 >= (1LL << 31)) return set_error(GDNX_ERR_SHAPE, "H * M too large");
  if (!q || !k || !v) return set_error(GDNX_ERR_ARG, "q, k, v must be non-null");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v))
    return set_error(GDNX_ERR_ARG, "q, k, v must be 16-byte aligned");
  return GDNX_OK;
}

}  // namespace gdnx

using namespace gdnx;

extern "C" int gdnx_abi_version(void) { return GDNX_ABI_VERSION; }

extern "C" const char* gdnx_last_error(void) { return g_err; }

extern "C" int gdnx_delta_chunk_size(int head_dim, int dtype) { return delta_chunk_size(head_dim, dtype); }

extern "C" int gdnx_delta_train_chunk_size(int head_dim, int dtype) {
  return delta_train_chunk_size(head_dim, dtype);
}

extern "C" long long gdnx_delta_chunk_states_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                                   int dtype) {
  const int C = chunk ? chunk : delta_chunk_size(head_dim, dtype);
  if (C == 0 || !valid_chunk(head_dim, dtype, C) || B < 1 || T < 0 || H < 1 || M < 1 ||
      (head_dim != 64 && head_dim != 128) || !query_sizes_ok(B, T, H, M))
    return -1;
  const int cps = delta_stash_cps(head_dim, C, dtype, M);
  return (long long)(delta_stash_bytes(B * H * M, T, head_dim, C, dtype, cps) +
                     delta_prep_bytes(B * H * M, T, C, dtype));
}

extern "C" long long gdnx_delta_bwd_workspace_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                                    int dtype) {
  const int C = chunk ? chunk : delta_train_chunk_size(head_dim, dtype);
  if (C == 0 || !valid_chunk(head_dim, dtype, C) || B < 1 || T < 0 || H < 1 || M < 1 ||
      (head_dim != 64 && head_dim != 128) || !query_sizes_ok(B, T, H, M))
    return -1;
  return (long long)delta_bwd_workspace_bytes(B, T, H, M, head_dim, C, dtype);
}

static int fwd_common(const void* q, const void* k, const void* v, const float* a_e, const float* a_w,
                      const float* log_g, const float* state0, void* y, float* state_out, void* chunk_states,
                      float* r_norm, void* workspace, int B, int T, int H, int M, int head_dim, int chunk,
                      int dtype, void* stream) {
  g_err[0] = 0;
  int rc = check_common(q, k, v, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  if (!a_e || !a_w || !log_g || !y) return set_error(GDNX_ERR_ARG, "a_e, a_w, log_g, y must be non-null");
  if (chunk_states && ((uintptr_t)chunk_states & 15u))
    return set_error(GDNX_ERR_ARG, "chunk_states must be 16-byte aligned");
  if (workspace && ((uintptr_t)workspace & 15u)) return set_error(GDNX_ERR_ARG, "workspace must be 16-byte aligned");
  const int C = chunk ? chunk : delta_chunk_size(head_dim, dtype);
  if (!valid_chunk(head_dim, dtype, C)) return set_error(GDNX_ERR_SHAPE, "chunk %d invalid for this dtype", chunk);
  if (T == 0) return GDNX_OK;
  DeltaArgs a{q, k, v, a_e, a_w, log_g, state0, y, state_out, chunk_states, B, T, H, M, head_dim, C, dtype,
              r_norm, workspace, delta_stash_cps(head_dim, C, dtype, M)};
  if ((rc = delta_fwd_dispatch(a, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H * M, D = head_dim;
  const FiniteBuf outs[] = {{y, rows * D, dtype}, {state_out, (size_t)B * H * M * D * D, GDNX_DTYPE_F32},
                            {r_norm, rows, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 3, (hipStream_t)stream);
}

extern "C" long long gdnx_delta_fwd_workspace_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                                    int dtype) {
  const int C = chunk ? chunk : delta_chunk_size(head_dim, dtype);
  if (C == 0 || !valid_chunk(head_dim, dtype, C) || B < 1 || T < 0 || H < 1 || M < 1 ||
      (head_dim != 64 && head_dim != 128) || !query_sizes_ok(B, T, H, M))
    return -1;
  return (long long)delta_prep_bytes(B * H * M, T, C, dtype);
}

extern "C" int gdnx_delta_chunk_prep(const void* q, const void* k, const float* a_e, const float* a_w,
                                     const float* log_g, void* workspace, int B, int T, int H, int M,
                                     int head_dim, int chunk, int dtype, void* stream) {
  g_err[0] = 0;
  int rc = check_common(q, k, k, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  if (!a_e || !a_w || !log_g) return set_error(GDNX_ERR_ARG, "a_e, a_w, log_g must be non-null");
  if (!workspace) return set_error(GDNX_ERR_WORKSPACE, "workspace is required");
  if ((uintptr_t)workspace & 15u) return set_error(GDNX_ERR_ARG, "workspace must be 16-byte aligned");
  const int C = chunk ? chunk : delta_chunk_size(head_dim, dtype);
  if (!valid_chunk(head_dim, dtype, C)) return set_error(GDNX_ERR_SHAPE, "chunk %d invalid for this dtype", chunk);
  if (T == 0) return GDNX_OK;
  DeltaArgs a{q, k, nullptr, a_e, a_w, log_g, nullptr, nullptr, nullptr, nullptr, B, T, H, M, head_dim, C, dtype,
              nullptr, workspace, 1};
  return delta_prep_dispatch(a, (hipStream_t)stream);
}

extern "C" int gdnx_delta_chunk_fwd(const void* q, const void* k, const void* v, const float* a_e,
                                    const float* a_w, const float* log_g, const float* state0, void* y,
                                    float* state_out, void* chunk_states, void* workspace, int B, int T, int H,
                                    int M, int head_dim, int chunk, int dtype, void* stream) {
  return fwd_common(q, k, v, a_e, a_w, log_g, state0, y, state_out, chunk_states, nullptr, workspace, B, T, H, M,
                    head_dim, chunk, dtype, stream);
}

extern "C" int gdnx_delta_chunk_fwd_scored(const void* q, const void* k, const void* v, const float* a_e,
                                           const float* a_w, const float* log_g, const float* state0, void* y,
                                           float* state_out, void* chunk_states, float* r_norm, void* workspace,
                                           int B, int T, int H, int M, int head_dim, int chunk, int dtype,
                                           void* stream) {
  if (!r_norm) return set_error(GDNX_ERR_ARG, "r_norm must be non-null");
  return fwd_common(q, k, v, a_e, a_w, log_g, state0, y, state_out, chunk_states, r_norm, workspace, B, T, H, M,
                    head_dim, chunk, dtype, stream);
}

static int bwd_common(const void* q, const void* k, const void* v, const float* a_e, const float* a_w,
                      const float* log_g, const void* dy, const float* dstate_out, const void* chunk_states,
                      void* workspace, void* dq, void* dk, void* dv, float* da_e, float* da_w,
                      float* dlog_g, float* dstate0, int B, int T, int H, int M, int head_dim, int chunk,
                      int dtype, int stages, void* stream) {
  g_err[0] = 0;
  int rc = check_common(q, k, v, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  if (!a_e || !log_g || !dy) return set_error(GDNX_ERR_ARG, "a_e, log_g, dy must be non-null");
  if ((stages & 2) && (!a_w || !dq || !dk || !dv || !da_e || !da_w || !dlog_g))
    return set_error(GDNX_ERR_ARG, "a_w and the gradient outputs must be non-null");
  if (!workspace || !chunk_states)
    return set_error(GDNX_ERR_WORKSPACE, "chunk_states (from the forward) and workspace are required");
  if (((uintptr_t)chunk_states & 15u) || ((uintptr_t)workspace & 15u) || !aligned16(dy))
    return set_error(GDNX_ERR_ARG, "chunk_states, workspace and dy must be 16-byte aligned");
  const int C = chunk ? chunk : delta_train_chunk_size(head_dim, dtype);
  if (!valid_chunk(head_dim, dtype, C)) return set_error(GDNX_ERR_SHAPE, "chunk %d invalid for this dtype", chunk);
  if (T == 0) return GDNX_OK;
  DeltaBwdArgs a{q,  k,  v,  a_e,  a_w,  log_g, dy,      dstate_out, chunk_states, workspace, dq, dk,
                 dv, da_e, da_w, dlog_g, dstate0, B, T, H, M, head_dim, C, dtype,
                 delta_stash_cps(head_dim, C, dtype, M)};
  if ((rc = delta_bwd_dispatch(a, stages, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H * M, D = head_dim, tok = (size_t)B * T * H * D;
  const bool g = (stages & 2) != 0;
  const FiniteBuf outs[] = {{g ? dq : nullptr, tok, dtype}, {g ? dk : nullptr, tok, dtype},
                            {g ? dv : nullptr, tok, dtype}, {g ? da_e : nullptr, rows, GDNX_DTYPE_F32},
                            {g ? da_w : nullptr, rows, GDNX_DTYPE_F32}, {g ? dlog_g : nullptr, rows, GDNX_DTYPE_F32},
                            {dstate0, (size_t)B * H * M * D * D, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 7, (hipStream_t)stream);
}

extern "C" int gdnx_delta_chunk_bwd(const void* q, const void* k, const void* v, const float* a_e,
                                    const float* a_w, const float* log_g, const void* dy,
                                    const float* dstate_out, const void* chunk_states, void* workspace,
                                    void* dq, void* dk, void* dv, float* da_e, float* da_w, float* dlog_g,
                                    float* dstate0, int B, int T, int H, int M, int head_dim, int chunk,
                                    int dtype, void* stream) {
  return bwd_common(q, k, v, a_e, a_w, log_g, dy, dstate_out, chunk_states, workspace, dq, dk, dv, da_e,
                    da_w, dlog_g, dstate0, B, T, H, M, head_dim, chunk, dtype, 3, stream);
}

extern "C" int gdnx_delta_chunk_bwd_state(const void* q, const void* k, const float* a_e,
                                          const float* log_g, const void* dy, const float* dstate_out,
                                          const void* chunk_states, void* workspace, float* dstate0, int B,
                                          int T, int H, int M, int head_dim, int chunk, int dtype,
                                          void* stream) {
  return bwd_common(q, k, k, a_e, nullptr, log_g, dy, dstate_out, chunk_states, workspace, nullptr, nullptr,
                    nullptr, nullptr, nullptr, nullptr, dstate0, B, T, H, M, head_dim, chunk, dtype, 1,
                    stream);
}

extern "C" int gdnx_delta_chunk_bwd_grads(const void* q, const void* k, const void* v, const float* a_e,
                                          const float* a_w, const float* log_g, const void* dy,
                                          const void* chunk_states, void* workspace, void* dq,
                                          void* dk, void* dv, float* da_e, float* da_w, float* dlog_g,
                                          int B, int T, int H, int M, int head_dim, int chunk, int dtype,
                                          void* stream) {
  return bwd_common(q, k, v, a_e, a_w, log_g, dy, nullptr, chunk_states, workspace, dq, dk, dv,
                    da_e, da_w, dlog_g, nullptr, B, T, H, M, head_dim, chunk, dtype, 2, stream);
}

extern "C" int gdnx_delta_decode_step(const void* q, const void* k, const void* v, const float* a_e,
                                      const float* a_w, const float* log_g, float* state, void* y, int NS,
                                      int H, int M, int head_dim, int dtype, void* stream) {
  g_err[0] = 0;
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (head_dim != 64 && head_dim != 128)
    return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", head_dim);
  if (NS < 1 || H < 1 || M < 1 || (long long)NS * H * M > (1LL << 30))
    return set_error(GDNX_ERR_SHAPE, "bad sizes NS=%d H=%d M=%d", NS, H, M);
  if (!q || !k || !v || !a_e || !a_w || !log_g || !state || !y)
    return set_error(GDNX_ERR_ARG, "all pointers must be non-null");
  if ((uintptr_t)state & 15u) return set_error(GDNX_ERR_ARG, "state must be 16-byte aligned");
  DecodeArgs a{q, k, v, a_e, a_w, log_g, state, y, NS, H, M, head_dim, dtype, nullptr, 0};
  const int rc = decode_dispatch(a, (hipStream_t)stream);
  if (rc) return rc;
  const FiniteBuf outs[] = {{y, (size_t)NS * H * M * head_dim, dtype}};
  return finite_outputs(outs, 1, (hipStream_t)stream);
}

extern "C" int gdnx_delta_decode_step_slots(const void* q, const void* k, const void* v, const float* a_e,
                                            const float* a_w, const float* log_g, float* state_pool,
                                            const int* slots, void* y, int NS, int n_slots, int H, int M,
                                            int head_dim, int dtype, void* stream) {
  g_err[0] = 0;
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (head_dim != 64 && head_dim != 128)
    return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", head_dim);
  if (NS < 1 || n_slots < 1 || H < 1 || M < 1 || (long long)NS * H * M > (1LL << 30) ||
      (long long)n_slots * H * M > (1LL << 30))
    return set_error(GDNX_ERR_SHAPE, "bad sizes NS=%d n_slots=%d H=%d M=%d", NS, n_slots, H, M);
  if (!q || !k || !v || !a_e || !a_w || !log_g || !state_pool || !slots || !y)
    return set_error(GDNX_ERR_ARG, "all pointers must be non-null");
  if ((uintptr_t)state_pool & 15u) return set_error(GDNX_ERR_ARG, "state_pool must be 16-byte aligned");
  DecodeArgs a{q, k, v, a_e, a_w, log_g, state_pool, y, NS, H, M, head_dim, dtype, slots, n_slots};
  const int rc = decode_dispatch(a, (hipStream_t)stream);
  if (rc) return rc;
  const FiniteBuf outs[] = {{y, (size_t)NS * H * M * head_dim, dtype}};
  return finite_outputs(outs, 1, (hipStream_t)stream);
}

extern "C" int gdnx_delta_decode_step_chan(const void* q, const void* k, const void* v, const float* a_e,
                                           const float* a_w, const float* log_g, float* state_pool,
                                           const int* slots, void* y, int NS, int n_slots, int H, int M,
                                           int head_dim, int dtype, void* stream) {
  g_err[0] = 0;
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (head_dim != 64 && head_dim != 128)
    return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", head_dim);
  if (!slots) n_slots = NS;
  if (NS < 1 || n_slots < 1 || H < 1 || M < 1 || (long long)NS * H * M > (1LL << 30) ||
      (long long)n_slots * H * M > (1LL << 30))
    return set_error(GDNX_ERR_SHAPE, "bad sizes NS=%d n_slots=%d H=%d M=%d", NS, n_slots, H, M);
  if (!q || !k || !v || !a_e || !a_w || !log_g || !state_pool || !y)
    return set_error(GDNX_ERR_ARG, "all pointers but slots must be non-null");
  if ((uintptr_t)state_pool & 15u) return set_error(GDNX_ERR_ARG, "state_pool must be 16-byte aligned");
  DecodeArgs a{q, k, v, a_e, a_w, log_g, state_pool, y, NS, H, M, head_dim, dtype, slots, n_slots, 1};
  const int rc = decode_dispatch(a, (hipStream_t)stream);
  if (rc) return rc;
  const FiniteBuf outs[] = {{y, (size_t)NS * H * M * head_dim, dtype}};
  return finite_outputs(outs, 1, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// GDN3 Kronecker-residual path
// ---------------------------------------------------------------------------
namespace gdnx {

static int g3_geom(int D, int R, int av, int ak, int bv, int bk, G3Geom& ge) {
  if (D != 64 && D != 128) return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", D);
  if (R < 1 || R > 4) return set_error(GDNX_ERR_SHAPE, "Kronecker rank R=%d unsupported (1..4)", R);
  if (av < 1 || ak < 1 || bv < 1 || bk < 1 || av * bv != D || ak * bk != D)
    return set_error(GDNX_ERR_SHAPE, "factors (a_v=%d, a_k=%d, b_v=%d, b_k=%d) need a_v*b_v = a_k*b_k = %d",
                     av, ak, bv, bk, D);
  const int m = av * ak, n = bv * bk;
  if (m > 256 || n > 256) return set_error(GDNX_ERR_SHAPE, "a_v*a_k=%d and b_v*b_k=%d must be <= 256", m, n);
  if (av * bk > 256) return set_error(GDNX_ERR_SHAPE, "a_v*b_k=%d must be <= 256", av * bk);
  int q = R + 4;
  if (m < q) q = m;
  if (n < q) q = n;
  auto lg2 = [](int x) {
    int l = 0;
    while ((1 << l) < x) ++l;
    return l;
  };
  ge = G3Geom{R, av, ak, bv, bk, m, n, q, lg2(av), lg2(ak), lg2(bv), lg2(bk)};
  return GDNX_OK;
}

static bool g3_window_ok(int D, int P) { return (D == 128 || D == 64) && (P == 16 || P == 32 || P == 64); }

// the fused forward and the compaction are compiled for the layer's
// geometry: rank 4 with (16, 16, 8, 8) at head dim 128, (8, 8, 8, 8) at 64
static int g3_layer_geom(int D, const G3Geom& ge) {
  const bool ok = ge.R == 4 && ((D == 128 && ge.av == 16 && ge.ak == 16 && ge.bv == 8 && ge.bk == 8) ||
                                (D == 64 && ge.av == 8 && ge.ak == 8 && ge.bv == 8 && ge.bk == 8));
  if (!ok)
    return set_error(GDNX_ERR_SHAPE,
                     "compiled for R=4 with factors (16,16,8,8) at head_dim 128 or (8,8,8,8) at 64; got R=%d "
                     "(%d,%d,%d,%d) at %d",
                     ge.R, ge.av, ge.ak, ge.bv, ge.bk, D);
  return GDNX_OK;
}

}  // namespace gdnx

extern "C" long long gdnx_gdn3_workspace_bytes(int B, int H, int M, int head_dim, int P, int dtype) {
  if (B < 1 || H < 1 || M < 1 || !g3_window_ok(head_dim, P) ||
      (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16) || !query_sizes_ok(B, 1, H, M))
    return -1;
  return (long long)gdn3_workspace_bytes(B * H * M, head_dim, P, dtype);
}

extern "C" int gdnx_gdn3_num_compactions(int T, int P, int compact_every) {
  if (T < 0 || P < 1 || compact_every < P || compact_every % P != 0) return -1;
  return T / compact_every;
}

extern "C" long long gdnx_gdn3_train_states_bytes(int B, int T, int H, int M, int head_dim, int P,
                                                  int compact_every) {
  if (B < 1 || T < 0 || H < 1 || M < 1 || !g3_window_ok(head_dim, P) || compact_every < P ||
      compact_every % P != 0 || !query_sizes_ok(B, T, H, M))
    return -1;
  return (long long)gdn3_train_states_bytes(B * H * M, T, head_dim, P, compact_every);
}

namespace gdnx {
// validation and argument packing shared by the two GDN3 forward entry points
static int g3_fwd_args(G3FwdArgs& a, const void* q, const void* k, const void* v, int qkv_lanes,
                       const float* b_gates, const float* w_gates, int gate_channels, const float* decay,
                       const float* sketch, void* y, float* A_out, float* B_out, float* U_out, float* Vb_out,
                       double* comp_stats, void* workspace, int B, int T, int H, int M, int head_dim, int R,
                       int P, int compact_every, int a_v, int a_k, int b_v, int b_k, float slow_decay,
                       int dtype, int compact_mode, bool need_workspace = true) {
  int rc = check_common(q, k, v, B, T, H, M, head_dim, dtype);
  if (compact_mode != 0 && compact_mode != 1)
    return set_error(GDNX_ERR_ARG, "compact_mode %d is not 0 (svd) or 1 (sketch)", compact_mode);
  if (rc) return rc;
  G3Geom ge;
  if ((rc = g3_geom(head_dim, R, a_v, a_k, b_v, b_k, ge))) return rc;
  if ((rc = g3_layer_geom(head_dim, ge))) return rc;
  if (!g3_window_ok(head_dim, P))
    return set_error(GDNX_ERR_SHAPE, "residual window P=%d unsupported for head_dim %d (16, 32 or 64)",
                     P, head_dim);
  if (compact_every < P || compact_every % P != 0)
    return set_error(GDNX_ERR_SHAPE, "compact_every=%d must be a positive multiple of P=%d", compact_every, P);
  if (qkv_lanes != 1 && qkv_lanes != M)
    return set_error(GDNX_ERR_SHAPE, "qkv_lanes=%d must be 1 (shared) or M=%d", qkv_lanes, M);
  if (gate_channels != 1 && gate_channels != head_dim)
    return set_error(GDNX_ERR_SHAPE, "gate_channels=%d must be 1 or head_dim=%d", gate_channels, head_dim);
  if (!b_gates || !w_gates || !decay || !sketch || !y || (need_workspace && !workspace))
    return set_error(GDNX_ERR_ARG, "gates, decay, sketch, y and workspace must be non-null");
  if (gate_channels > 1 && (!aligned16(b_gates) || !aligned16(w_gates)))
    return set_error(GDNX_ERR_ARG, "per-channel gates must be 16-byte aligned");
  if (need_workspace && !aligned16(workspace)) return set_error(GDNX_ERR_ARG, "workspace must be 16-byte aligned");
  if (!(slow_decay >= 0.f && slow_decay <= 1.f))
    return set_error(GDNX_ERR_ARG, "slow_decay must lie in [0, 1]");
  a = G3FwdArgs{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.bg = b_gates;
  a.wg = w_gates;
  a.dec = decay;
  a.sketch = sketch;
  a.y = y;
  a.A_out = A_out;
  a.B_out = B_out;
  a.U_out = U_out;
  a.Vb_out = Vb_out;
  a.stats = comp_stats;
  a.workspace = workspace;
  a.ge = ge;
  a.B = B;
  a.T = T;
  a.H = H;
  a.M = M;
  a.D = head_dim;
  a.P = P;
  a.Kc = compact_every;
  a.qkv_lanes = qkv_lanes;
  a.gate_ch = gate_channels;
  a.dtype = dtype;
  a.sdec = slow_decay;
  a.cmode = compact_mode;
  return GDNX_OK;
}

// the GDN3 forward dispatch, then (when checking is on) its outputs' scan
static int g3_fwd_run(const G3FwdArgs& a, hipStream_t stream) {
  int rc = gdn3_fwd_dispatch(a, stream);
  if (rc || !check_finite_on()) return rc;
  const size_t N = (size_t)a.B * a.H * a.M, D = a.D;
  const size_t nev = (size_t)((a.t0 + a.T) / a.Kc - a.t0 / a.Kc);
  const FiniteBuf outs[] = {{a.y, (size_t)a.B * a.T * a.H * a.M * D, a.dtype},
                            {a.A_out, N * a.ge.R * a.ge.m, GDNX_DTYPE_F32},
                            {a.B_out, N * a.ge.R * a.ge.n, GDNX_DTYPE_F32},
                            {a.U_out, N * D * a.P, GDNX_DTYPE_F32},
                            {a.Vb_out, N * D * a.P, GDNX_DTYPE_F32},
                            {a.stats, nev * N * 2, GDNX_DTYPE_F64}};
  return finite_check(outs, 6, stream);
}
}  // namespace gdnx

extern "C" int gdnx_gdn3_chunk_fwd(const void* q, const void* k, const void* v, int qkv_lanes,
                                   const float* b_gates, const float* w_gates, int gate_channels,
                                   const float* decay, const float* sketch, void* y, float* A_out,
                                   float* B_out, float* U_out, float* Vb_out, double* comp_stats,
                                   void* workspace, void* train_states, int B, int T, int H, int M,
                                   int head_dim, int R, int P,
                                   int compact_every, int a_v, int a_k, int b_v, int b_k, float slow_decay,
                                   int dtype, int compact_mode, void* stream) {
  g_err[0] = 0;
  G3FwdArgs a;
  int rc = g3_fwd_args(a, q, k, v, qkv_lanes, b_gates, w_gates, gate_channels, decay, sketch, y, A_out, B_out,
                       U_out, Vb_out, comp_stats, workspace, B, T, H, M, head_dim, R, P, compact_every, a_v, a_k,
                       b_v, b_k, slow_decay, dtype, compact_mode);
  if (rc) return rc;
  if (train_states && !aligned16(train_states)) return set_error(GDNX_ERR_ARG, "train_states must be 16-byte aligned");
  if (T == 0) {   // the final state of an empty run is the zero initial state
    const int N = B * H * M;
    const size_t n[4] = {(size_t)N * R * a_v * a_k, (size_t)N * R * b_v * b_k, (size_t)N * head_dim * P,
                         (size_t)N * head_dim * P};
    float* outs[4] = {A_out, B_out, U_out, Vb_out};
    for (int i = 0; i < 4; ++i)
      if (outs[i] && (rc = gdn3_zero_fill(outs[i], n[i], (hipStream_t)stream))) return rc;
    return GDNX_OK;
  }
  a.train_states = train_states;
  return g3_fwd_run(a, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_num_compactions_from(int t0, int T, int P, int compact_every) {
  if (t0 < 0 || T < 0 || P < 1 || compact_every < P || compact_every % P != 0 ||
      (long long)t0 + T > 0x7fffffffLL)
    return -1;
  return (t0 + T) / compact_every - t0 / compact_every;
}

namespace gdnx {
// the carried-state forward once its arguments are checked: the initial
// state's pass-through for T = 0, else the dispatch (workspace set by caller
// unless T = 0)
static int g3_state_check(const float* A0, const float* B0, const float* U0, const float* Vb0, int t0, int T) {
  const int nin = (A0 != nullptr) + (B0 != nullptr) + (U0 != nullptr) + (Vb0 != nullptr);
  if (nin != 0 && nin != 4) return set_error(GDNX_ERR_ARG, "A0, B0, U0, Vb0 must all be given or all be null");
  if (t0 < 0 || (long long)t0 + T > 0x7fffffffLL) return set_error(GDNX_ERR_SHAPE, "bad start position t0=%d", t0);
  return GDNX_OK;
}

static int g3_state_passthrough(const float* A0, const float* B0, const float* U0, const float* Vb0, float* A_out,
                                float* B_out, float* U_out, float* Vb_out, int N, int R, int a_v, int a_k, int b_v,
                                int b_k, int D, int P, hipStream_t stream) {
  const size_t n[4] = {(size_t)N * R * a_v * a_k, (size_t)N * R * b_v * b_k, (size_t)N * D * P, (size_t)N * D * P};
  const float* ins[4] = {A0, B0, U0, Vb0};
  float* outs[4] = {A_out, B_out, U_out, Vb_out};
  for (int i = 0; i < 4; ++i) {
    if (!outs[i] || outs[i] == ins[i]) continue;
    if (!ins[i]) {
      const int rc = gdn3_zero_fill(outs[i], n[i], stream);
      if (rc) return rc;
    } else if (hipMemcpyAsync(outs[i], ins[i], n[i] * 4, hipMemcpyDeviceToDevice, stream) != hipSuccess) {
      return set_error(GDNX_ERR_HIP, "gdn3 forward: passing the state through failed");
    }
  }
  return GDNX_OK;
}
}  // namespace gdnx

extern "C" int gdnx_gdn3_chunk_fwd_state(const void* q, const void* k, const void* v, int qkv_lanes,
                                         const float* b_gates, const float* w_gates, int gate_channels,
                                         const float* decay, const float* sketch, const float* A0,
                                         const float* B0, const float* U0, const float* Vb0, int t0, void* y,
                                         float* A_out, float* B_out, float* U_out, float* Vb_out,
                                         double* comp_stats, void* workspace, int B, int T, int H, int M,
                                         int head_dim, int R, int P, int compact_every, int a_v, int a_k,
                                         int b_v, int b_k, float slow_decay, int dtype, int compact_mode,
                                         void* stream) {
  g_err[0] = 0;
  G3FwdArgs a;
  int rc = g3_fwd_args(a, q, k, v, qkv_lanes, b_gates, w_gates, gate_channels, decay, sketch, y, A_out, B_out,
                       U_out, Vb_out, comp_stats, workspace, B, T, H, M, head_dim, R, P, compact_every, a_v, a_k,
                       b_v, b_k, slow_decay, dtype, compact_mode);
  if (rc) return rc;
  if ((rc = g3_state_check(A0, B0, U0, Vb0, t0, T))) return rc;
  if (T == 0)
    return g3_state_passthrough(A0, B0, U0, Vb0, A_out, B_out, U_out, Vb_out, B * H * M, R, a_v, a_k, b_v, b_k,
                                head_dim, P, (hipStream_t)stream);
  a.t0 = t0;
  a.A0 = A0;
  a.B0 = B0;
  a.U0 = U0;
  a.Vb0 = Vb0;
  return g3_fwd_run(a, (hipStream_t)stream);
}

extern "C" long long gdnx_gdn3_noalloc_scratch_bytes(void) { return (long long)kG3ScratchBytes; }

extern "C" int gdnx_gdn3_chunk_fwd_state_noalloc(const void* q, const void* k, const void* v, int qkv_lanes,
                                                 const float* b_gates, const float* w_gates, int gate_channels,
                                                 const float* decay, const float* sketch, const float* A0,
                                                 const float* B0, const float* U0, const float* Vb0, int t0,
                                                 void* y, float* A_out, float* B_out, float* U_out, float* Vb_out,
                                                 double* comp_stats, int B, int T, int H, int M, int head_dim,
                                                 int R, int P, int compact_every, int a_v, int a_k, int b_v,
                                                 int b_k, float slow_decay, int dtype, int compact_mode,
                                                 void* stream) {
  g_err[0] = 0;
  G3FwdArgs a;
  int rc = g3_fwd_args(a, q, k, v, qkv_lanes, b_gates, w_gates, gate_channels, decay, sketch, y, A_out, B_out,
                       U_out, Vb_out, comp_stats, nullptr, B, T, H, M, head_dim, R, P, compact_every, a_v, a_k,
                       b_v, b_k, slow_decay, dtype, compact_mode, /*need_workspace=*/false);
  if (rc) return rc;
  if ((rc = g3_state_check(A0, B0, U0, Vb0, t0, T))) return rc;
  // (the layer's default regime runs as one fused launch and needs no scratch)
  const size_t need = gdn3_fwd_fused(head_dim, P, compact_every, dtype)
                          ? 0 : gdn3_workspace_bytes(B * H * M, head_dim, P, dtype);
  if (need > kG3ScratchBytes)
    return set_error(GDNX_ERR_WORKSPACE,
                     "gdn3 no-alloc forward: %d chains need %zu bytes of scratch; the library's static scratch "
                     "holds %zu (use gdnx_gdn3_chunk_fwd_state with a workspace, or fewer chains per call)",
                     B * H * M, need, kG3ScratchBytes);
  if (T == 0)
    return g3_state_passthrough(A0, B0, U0, Vb0, A_out, B_out, U_out, Vb_out, B * H * M, R, a_v, a_k, b_v, b_k,
                                head_dim, P, (hipStream_t)stream);
  void* ws = nullptr;
  if ((rc = gdn3_scratch(&ws))) return rc;
  a.workspace = ws;
  a.t0 = t0;
  a.A0 = A0;
  a.B0 = B0;
  a.U0 = U0;
  a.Vb0 = Vb0;
  return g3_fwd_run(a, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_decode_step(const void* q, const void* k, const void* v, int qkv_lanes,
                                     const float* b_gates, const float* w_gates, int gate_channels,
                                     const float* decay, const float* sketch, float* A, float* Bf, float* U,
                                     float* Vb, const int* slots, const int* pos, void* y, double* comp_stats,
                                     int NS, int n_slots, int H, int M, int head_dim, int R, int P,
                                     int compact_every, int a_v, int a_k, int b_v, int b_k, float slow_decay,
                                     int dtype, int compact_mode, void* stream) {
  g_err[0] = 0;
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (compact_mode != 0 && compact_mode != 1)
    return set_error(GDNX_ERR_ARG, "compact_mode %d is not 0 (svd) or 1 (sketch)", compact_mode);
  G3Geom ge;
  int rc = g3_geom(head_dim, R, a_v, a_k, b_v, b_k, ge);
  if (rc) return rc;
  if ((rc = g3_layer_geom(head_dim, ge))) return rc;
  if (!g3_window_ok(head_dim, P))
    return set_error(GDNX_ERR_SHAPE, "residual window P=%d unsupported for head_dim %d", P, head_dim);
  if (compact_every < P || compact_every % P != 0)
    return set_error(GDNX_ERR_SHAPE, "compact_every=%d must be a positive multiple of P=%d", compact_every, P);
  if (!slots) n_slots = NS;
  if (NS < 1 || n_slots < 1 || H < 1 || M < 1 || (long long)NS * H * M > (1LL << 30) ||
      (long long)n_slots * H * M > (1LL << 30))
    return set_error(GDNX_ERR_SHAPE, "bad sizes NS=%d n_slots=%d H=%d M=%d", NS, n_slots, H, M);
  if (qkv_lanes != 1 && qkv_lanes != M)
    return set_error(GDNX_ERR_SHAPE, "qkv_lanes=%d must be 1 (shared) or M=%d", qkv_lanes, M);
  if (gate_channels != 1 && gate_channels != head_dim)
    return set_error(GDNX_ERR_SHAPE, "gate_channels=%d must be 1 or head_dim=%d", gate_channels, head_dim);
  if (!q || !k || !v || !b_gates || !w_gates || !decay || !sketch || !A || !Bf || !U || !Vb || !pos || !y)
    return set_error(GDNX_ERR_ARG, "inputs, state, pos and y must be non-null (slots may be null)");
  if (!aligned16(A) || !aligned16(Bf) || !aligned16(U) || !aligned16(Vb))
    return set_error(GDNX_ERR_ARG, "A, Bf, U, Vb must be 16-byte aligned");
  if (!(slow_decay >= 0.f && slow_decay <= 1.f))
    return set_error(GDNX_ERR_ARG, "slow_decay must lie in [0, 1]");
  G3DecArgs a{q, k, v, b_gates, w_gates, decay, A, Bf, U, Vb, slots, pos, y, comp_stats,
              NS, n_slots, H, M, head_dim, P, qkv_lanes, gate_channels, dtype};
  if ((rc = gdn3_decode_dispatch(a, (hipStream_t)stream))) return rc;
  // the rows whose token closes a compaction interval: the compaction of
  // gdnx_gdn3_compact on their chains, in place (the others return at once)
  G3CompactArgs ca{};
  ca.A = A;
  ca.Bf = Bf;
  ca.U = U;
  ca.Vb = Vb;
  ca.sketch = sketch;
  ca.A_out = A;
  ca.B_out = Bf;
  ca.stats = comp_stats;
  ca.ge = ge;
  ca.N = NS * H * M;
  ca.D = head_dim;
  ca.P = P;
  ca.sdec = slow_decay;
  ca.u_sp = 1;
  ca.u_sd = P;
  ca.pos = pos;
  ca.slots = slots;
  ca.hm = H * M;
  ca.Kc = compact_every;
  ca.nslots = n_slots;
  ca.mode = compact_mode;
  if ((rc = gdn3_compact_dispatch(ca, (hipStream_t)stream))) return rc;
  const size_t nch = (size_t)NS * H * M;
  const FiniteBuf outs[] = {{y, nch * head_dim, dtype}, {comp_stats, nch * 2, GDNX_DTYPE_F64}};
  return finite_outputs(outs, 2, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_chunk_bwd(const void* q, const void* k, const void* v, int qkv_lanes,
                                   const float* b_gates, const float* w_gates, int gate_channels,
                                   const float* decay, const void* dy, const void* train_states, float* dq,
                                   float* dk, float* dv, float* db_gates, float* dw_gates, float* ddecay, int B,
                                   int T, int H, int M, int head_dim, int R, int P, int compact_every, int a_v,
                                   int a_k, int b_v, int b_k, int dtype, void* stream) {
  g_err[0] = 0;
  int rc = check_common(q, k, v, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  G3Geom ge;
  if ((rc = g3_geom(head_dim, R, a_v, a_k, b_v, b_k, ge))) return rc;
  if ((rc = g3_layer_geom(head_dim, ge))) return rc;
  if (!g3_window_ok(head_dim, P))
    return set_error(GDNX_ERR_SHAPE, "gdn3 backward: residual window P=%d unsupported (16, 32 or 64)", P);
  if (compact_every < P || compact_every % P != 0)
    return set_error(GDNX_ERR_SHAPE, "compact_every=%d must be a positive multiple of P=%d", compact_every, P);
  if (qkv_lanes != 1 && qkv_lanes != M)
    return set_error(GDNX_ERR_SHAPE, "qkv_lanes=%d must be 1 (shared) or M=%d", qkv_lanes, M);
  if (gate_channels != 1 && gate_channels != head_dim)
    return set_error(GDNX_ERR_SHAPE, "gate_channels=%d must be 1 or head_dim=%d", gate_channels, head_dim);
  if (!b_gates || !w_gates || !decay || !dy || !dq || !dk || !dv || !db_gates || !dw_gates || !ddecay)
    return set_error(GDNX_ERR_ARG, "gates, decay, dy and the gradient outputs must be non-null");
  if (!train_states) return set_error(GDNX_ERR_WORKSPACE, "train_states (from the forward) is required");
  if (!aligned16(dy) || !aligned16(train_states) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
      (gate_channels > 1 && (!aligned16(b_gates) || !aligned16(w_gates) || !aligned16(dw_gates))))
    return set_error(GDNX_ERR_ARG, "dy, train_states, the key-sized outputs and per-channel gates must be "
                     "16-byte aligned");
  if (T == 0) return GDNX_OK;
  G3BwdArgs a{q, k, v, b_gates, w_gates, decay, dy, train_states, dq, dk, dv, db_gates, dw_gates, ddecay,
              B, T, H, M, head_dim, P, compact_every, qkv_lanes, gate_channels, dtype};
  if ((rc = gdn3_bwd_dispatch(a, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H * M;
  const FiniteBuf outs[] = {{dq, rows * head_dim, GDNX_DTYPE_F32}, {dk, rows * head_dim, GDNX_DTYPE_F32},
                            {dv, rows * head_dim, GDNX_DTYPE_F32}, {db_gates, rows * gate_channels, GDNX_DTYPE_F32},
                            {dw_gates, rows * gate_channels, GDNX_DTYPE_F32}, {ddecay, rows, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 6, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_compact(const float* A, const float* Bf, const float* U, const float* Vb,
                                 const float* sketch, float* A_out, float* B_out, double* comp_stats, int N,
                                 int head_dim, int R, int P, int a_v, int a_k, int b_v, int b_k,
                                 float slow_decay, int compact_mode, void* stream) {
  g_err[0] = 0;
  if (compact_mode != 0 && compact_mode != 1)
    return set_error(GDNX_ERR_ARG, "compact_mode %d is not 0 (svd) or 1 (sketch)", compact_mode);
  G3Geom ge;
  int rc = g3_geom(head_dim, R, a_v, a_k, b_v, b_k, ge);
  if (rc) return rc;
  if ((rc = g3_layer_geom(head_dim, ge))) return rc;
  if (N < 0 || N > (1 << 30)) return set_error(GDNX_ERR_SHAPE, "bad chain count N=%d", N);
  if (!g3_window_ok(head_dim, P))
    return set_error(GDNX_ERR_SHAPE, "residual window P=%d unsupported for head_dim %d", P, head_dim);
  if (!A || !Bf || !U || !Vb || !sketch || !A_out || !B_out)
    return set_error(GDNX_ERR_ARG, "state, sketch and output pointers must be non-null");
  if (!(slow_decay >= 0.f && slow_decay <= 1.f))
    return set_error(GDNX_ERR_ARG, "slow_decay must lie in [0, 1]");
  G3CompactArgs a{};
  a.A = A;
  a.Bf = Bf;
  a.U = U;
  a.Vb = Vb;
  a.sketch = sketch;
  a.A_out = A_out;
  a.B_out = B_out;
  a.stats = comp_stats;
  a.ge = ge;
  a.N = N;
  a.D = head_dim;
  a.P = P;
  a.sdec = slow_decay;
  a.u_sp = 1;  // reference layout [d][p]
  a.u_sd = P;
  a.mode = compact_mode;
  return gdn3_compact_dispatch(a, (hipStream_t)stream);
}

extern "C" int gdnx_kron_read(const float* A, const float* Bf, const float* U, const float* Vb, const float* x,
                              float* y, int N, int C, int head_dim, int R, int P, int a_v, int a_k, int b_v,
                              int b_k, void* stream) {
  g_err[0] = 0;
  G3Geom ge;
  int rc = g3_geom(head_dim, R, a_v, a_k, b_v, b_k, ge);
  if (rc) return rc;
  if (N < 0 || C < 0 || (long long)N * C > (1LL << 30)) return set_error(GDNX_ERR_SHAPE, "bad sizes N=%d C=%d", N, C);
  if (P < 0 || P > 64) return set_error(GDNX_ERR_SHAPE, "residual slots P=%d unsupported (0..64)", P);
  if (!A || !Bf || !x || !y || (P > 0 && (!U || !Vb)))
    return set_error(GDNX_ERR_ARG, "pointers must be non-null");
  KronReadArgs a{A, Bf, U, Vb, x, y, ge, N, C, head_dim, P};
  return kron_read_dispatch(a, (hipStream_t)stream);
}

static int coeff_common(const void* k, const float* beta, int B, int T, int H, int M, int head_dim, int dtype) {
  g_err[0] = 0;
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (head_dim != 64 && head_dim != 128) return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", head_dim);
  if (B < 1 || T < 0 || H < 1 || M < 1 || M > 16) return set_error(GDNX_ERR_SHAPE, "bad sizes B=%d T=%d H=%d M=%d", B, T, H, M);
  if (!k || !beta) return set_error(GDNX_ERR_ARG, "k and beta must be non-null");
  if (!aligned16(k)) return set_error(GDNX_ERR_ARG, "k must be 16-byte aligned");
  return GDNX_OK;
}

extern "C" int gdnx_gdn3_coeff(const void* k, const float* beta, float* a, int B, int T, int H, int M, int head_dim,
                               int dtype, void* stream) {
  int rc = coeff_common(k, beta, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  if (!a) return set_error(GDNX_ERR_ARG, "a must be non-null");
  if (T == 0) return GDNX_OK;
  GCoeffArgs ga{k, beta, a, nullptr, nullptr, nullptr, nullptr, B, T, H, M, head_dim, dtype};
  return gdn3_coeff_dispatch(ga, false, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_coeff_bwd(const void* k, const float* beta, const float* da_e, const float* da_w, void* dk,
                                   float* dbeta, int B, int T, int H, int M, int head_dim, int dtype, void* stream) {
  int rc = coeff_common(k, beta, B, T, H, M, head_dim, dtype);
  if (rc) return rc;
  if (!da_e || !dk || !dbeta) return set_error(GDNX_ERR_ARG, "da_e, dk and dbeta must be non-null");
  if (!aligned16(dk)) return set_error(GDNX_ERR_ARG, "dk must be 16-byte aligned");
  if (T == 0) return GDNX_OK;
  GCoeffArgs ga{k, beta, nullptr, da_e, da_w, dk, dbeta, B, T, H, M, head_dim, dtype};
  return gdn3_coeff_dispatch(ga, true, (hipStream_t)stream);
}

static int chan_common(const float* q, const float* k, const float* v, const float* be, const float* lg, int B, int T,
                       int H, int D) {
  g_err[0] = 0;
  if (D != 64 && D != 128) return set_error(GDNX_ERR_SHAPE, "head_dim %d unsupported (64 or 128)", D);
  if (B < 1 || T < 0 || H < 1 || (long long)B * H > (1LL << 30)) return set_error(GDNX_ERR_SHAPE, "bad sizes B=%d T=%d H=%d", B, T, H);
  if ((long long)H * D * 16 * 4 >= (1LL << 31)) return set_error(GDNX_ERR_SHAPE, "H too large");
  if (!q || !k || !v || !be || !lg) return set_error(GDNX_ERR_ARG, "q, k, v, beta_e, log_g must be non-null");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(lg))
    return set_error(GDNX_ERR_ARG, "q, k, v, log_g must be 16-byte aligned");
  return GDNX_OK;
}

extern "C" long long gdnx_delta_chan_states_bytes(int B, int T, int H, int head_dim) {
  if (B < 1 || T < 0 || H < 1 || (head_dim != 64 && head_dim != 128) || !query_sizes_ok(B, T, H, 1)) return -1;
  return (long long)chan_states_bytes(B * H, T, head_dim);
}

extern "C" long long gdnx_delta_chan_fwd_workspace_bytes(int B, int T, int H, int head_dim) {
  if (B < 1 || T < 0 || H < 1 || (head_dim != 64 && head_dim != 128) || !query_sizes_ok(B, T, H, 1)) return -1;
  return (long long)chan_fwd_workspace_bytes(B * H, T, head_dim);
}

extern "C" int gdnx_delta_chan_fwd(const float* q, const float* k, const float* v, const float* beta_e,
                                   const float* beta_w, const float* log_g, const float* state0, float* y,
                                   float* state_out, void* chunk_states, void* workspace, float* r_norm, int B,
                                   int T, int H, int head_dim, void* stream) {
  int rc = chan_common(q, k, v, beta_e, log_g, B, T, H, head_dim);
  if (rc) return rc;
  if (!beta_w || !y) return set_error(GDNX_ERR_ARG, "beta_w and y must be non-null");
  if (!chunk_states && !workspace)
    return set_error(GDNX_ERR_WORKSPACE, "chunk_states (training) or workspace (inference) is required");
  if (!aligned16(y) || (chunk_states && !aligned16(chunk_states)) || (workspace && !aligned16(workspace)))
    return set_error(GDNX_ERR_ARG, "y, chunk_states and workspace must be 16-byte aligned");
  if (T == 0) return GDNX_OK;
  ChanArgs a{q, k, v, beta_e, beta_w, log_g, state0, y, state_out, chunk_states, r_norm, B, T, H, head_dim,
             workspace, nullptr, nullptr};
  if ((rc = chan_fwd_dispatch(a, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H;
  const FiniteBuf outs[] = {{y, rows * head_dim, GDNX_DTYPE_F32},
                            {state_out, (size_t)B * H * head_dim * head_dim, GDNX_DTYPE_F32},
                            {r_norm, rows, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 3, (hipStream_t)stream);
}

extern "C" int gdnx_delta_chan_bwd(const float* q, const float* k, const float* v, const float* beta_e,
                                   const float* beta_w, const float* log_g, const float* dy,
                                   const float* dstate_out, const void* chunk_states, void* workspace, float* dq,
                                   float* dk, float* dv, float* dbeta_e, float* dbeta_w, float* dlog_g,
                                   float* dstate0, int B, int T, int H, int head_dim, void* stream) {
  int rc = chan_common(q, k, v, beta_e, log_g, B, T, H, head_dim);
  if (rc) return rc;
  if (!beta_w || !dy || !dq || !dk || !dv || !dbeta_e || !dbeta_w || !dlog_g)
    return set_error(GDNX_ERR_ARG, "beta_w, dy and the gradient outputs must be non-null");
  if (!chunk_states || !workspace)
    return set_error(GDNX_ERR_WORKSPACE, "chunk_states (from the forward) and workspace are required");
  if (!aligned16(dy) || !aligned16(chunk_states) || !aligned16(workspace) || !aligned16(dq) || !aligned16(dk) ||
      !aligned16(dv) || !aligned16(dlog_g))
    return set_error(GDNX_ERR_ARG, "dy, chunk_states, workspace and the key-sized outputs must be 16-byte aligned");
  if (T == 0) return GDNX_OK;
  ChanBwdArgs a{q, k, v, beta_e, beta_w, log_g, dy, dstate_out, chunk_states, workspace, dq, dk, dv,
                dbeta_e, dbeta_w, dlog_g, dstate0, B, T, H, head_dim};
  if ((rc = chan_bwd_dispatch(a, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H, tok = rows * head_dim;
  const FiniteBuf outs[] = {{dq, tok, GDNX_DTYPE_F32},     {dk, tok, GDNX_DTYPE_F32},
                            {dv, tok, GDNX_DTYPE_F32},     {dlog_g, tok, GDNX_DTYPE_F32},
                            {dbeta_e, rows, GDNX_DTYPE_F32}, {dbeta_w, rows, GDNX_DTYPE_F32},
                            {dstate0, (size_t)B * H * head_dim * head_dim, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 7, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// GDN3 layer boundary: fused pre-ops / post-ops
// ---------------------------------------------------------------------------
namespace gdnx {

static int layer_sizes(int B, int T, int H, int M, int K, int V, int dtype, bool need_k) {
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16", dtype);
  if (B < 1 || T < 0 || H < 1 || M < 1 || M > 4)
    return set_error(GDNX_ERR_SHAPE, "bad sizes B=%d T=%d H=%d M=%d (lanes 1..4)", B, T, H, M);
  if (need_k && (K < 4 || K > 256 || K % 4))
    return set_error(GDNX_ERR_SHAPE, "key_dim %d unsupported (multiple of 4, <= 256)", K);
  if (V < 4 || V > 256 || V % 4) return set_error(GDNX_ERR_SHAPE, "value_dim %d unsupported (multiple of 4, <= 256)", V);
  return GDNX_OK;
}

static bool all_aligned(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (!p || !aligned16(p)) return false;
  return true;
}

}  // namespace gdnx

extern "C" int gdnx_gdn3_lane_rope_pairs(int M, int key_dim, int* pairs) {
  g_err[0] = 0;
  if (M < 1 || M > 4 || key_dim < 1 || !pairs || ((uintptr_t)pairs & 3u))
    return set_error(GDNX_ERR_ARG, "need 1 <= M <= 4, key_dim >= 1 and an aligned host int pairs array");
  int p[4];
  gdn3_lane_pairs(M, key_dim, p);
  for (int m = 0; m < M; ++m) pairs[m] = p[m];
  return GDNX_OK;
}

extern "C" int gdnx_gdn3_prologue_fwd(const void* q, const void* k, const void* b_proj, const void* proj_a,
                                      const void* w_proj, const void* proj_b, const void* decay_proj,
                                      const float* rates, const float* rope_cos, const float* rope_sin,
                                      void* q_rope, void* k_rope, float* b_gates, float* w_gates, float* decay,
                                      int B, int T, int H, int M, int key_dim, int value_dim, float decay_clamp,
                                      int dtype, void* stream) {
  g_err[0] = 0;
  int rc = layer_sizes(B, T, H, M, key_dim, value_dim, dtype, true);
  if (rc != GDNX_OK) return rc;
  if (!all_aligned({q, k, b_proj, w_proj, decay_proj, q_rope, k_rope, b_gates, w_gates}) || !proj_a ||
      !proj_b || !rates || !rope_cos || !rope_sin || !decay)
    return set_error(GDNX_ERR_ARG, "pointers must be non-null; tensors 16-byte aligned");
  G3ProArgs a{};
  a.q = q; a.k = k; a.bp = b_proj; a.pa = proj_a; a.wp = w_proj; a.pb = proj_b; a.dp = decay_proj;
  a.rates = rates; a.cs = rope_cos; a.sn = rope_sin;
  a.qr = q_rope; a.kr = k_rope; a.bg = b_gates; a.wg = w_gates; a.dec = decay;
  a.rows = (long long)B * T * H;
  a.T = T; a.H = H; a.M = M; a.K = key_dim; a.V = value_dim; a.clamp = decay_clamp;
  gdn3_lane_pairs(M, key_dim, a.pairs);
  return gdn3_prologue_dispatch(a, false, dtype, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_prologue_bwd(const void* b_proj, const void* proj_a, const void* w_proj,
                                      const void* proj_b, const void* decay_proj, const float* rates,
                                      const float* rope_cos, const float* rope_sin, const float* d_q_rope,
                                      const float* d_k_rope, const float* d_b_gates, const float* d_w_gates,
                                      const float* d_decay, float* dq, float* dk, float* d_b_proj,
                                      float* d_proj_a, float* d_w_proj, float* d_proj_b, float* d_decay_proj,
                                      int B, int T, int H, int M, int key_dim, int value_dim, float decay_clamp,
                                      int dtype, void* stream) {
  g_err[0] = 0;
  int rc = layer_sizes(B, T, H, M, key_dim, value_dim, dtype, true);
  if (rc != GDNX_OK) return rc;
  if (!all_aligned({b_proj, w_proj, decay_proj, d_q_rope, d_k_rope, d_b_gates, d_w_gates, dq, dk, d_b_proj,
                    d_w_proj, d_decay_proj}) ||
      !proj_a || !proj_b || !rates || !rope_cos || !rope_sin || !d_decay || !d_proj_a || !d_proj_b)
    return set_error(GDNX_ERR_ARG, "pointers must be non-null; tensors 16-byte aligned");
  G3ProArgs a{};
  a.bp = b_proj; a.pa = proj_a; a.wp = w_proj; a.pb = proj_b; a.dp = decay_proj;
  a.rates = rates; a.cs = rope_cos; a.sn = rope_sin;
  a.dqr = d_q_rope; a.dkr = d_k_rope; a.dbg = d_b_gates; a.dwg = d_w_gates; a.ddec = d_decay;
  a.dq = dq; a.dk = dk; a.dbp = d_b_proj; a.dpa = d_proj_a; a.dwp = d_w_proj; a.dpb = d_proj_b;
  a.ddp = d_decay_proj;
  a.rows = (long long)B * T * H;
  a.T = T; a.H = H; a.M = M; a.K = key_dim; a.V = value_dim; a.clamp = decay_clamp;
  gdn3_lane_pairs(M, key_dim, a.pairs);
  return gdn3_prologue_dispatch(a, true, dtype, (hipStream_t)stream);
}

extern "C" long long gdnx_gdn3_epilogue_workspace_bytes(int B, int T, int H, int value_dim) {
  if (B < 1 || T < 0 || H < 1 || value_dim < 1 || !query_sizes_ok(B, T, H, 1) || value_dim > (1 << 16)) return -1;
  return (long long)gdn3_epilogue_workspace_bytes((long long)B * T * H, value_dim);
}

extern "C" int gdnx_gdn3_epilogue_fwd(const void* y, const void* router_logits, const float* norm, void* out,
                                      int B, int T, int H, int M, int value_dim, int dtype, void* stream) {
  g_err[0] = 0;
  int rc = layer_sizes(B, T, H, M, 0, value_dim, dtype, false);
  if (rc != GDNX_OK) return rc;
  if (!all_aligned({y, out, norm}) || !router_logits)
    return set_error(GDNX_ERR_ARG, "pointers must be non-null; y, norm and out 16-byte aligned");
  G3EpiArgs a{};
  a.y = y; a.lg = router_logits; a.norm = norm; a.out = out;
  a.rows = (long long)B * T * H; a.M = M; a.V = value_dim;
  return gdn3_epilogue_dispatch(a, false, dtype, (hipStream_t)stream);
}

extern "C" int gdnx_gdn3_epilogue_bwd(const void* y, const void* router_logits, const float* norm,
                                      const void* d_out, void* d_y, float* d_router_logits, float* d_norm,
                                      void* workspace, int B, int T, int H, int M, int value_dim, int dtype,
                                      void* stream) {
  g_err[0] = 0;
  int rc = layer_sizes(B, T, H, M, 0, value_dim, dtype, false);
  if (rc != GDNX_OK) return rc;
  if (!all_aligned({y, norm, d_out, d_y, workspace}) || !router_logits || !d_router_logits || !d_norm)
    return set_error(GDNX_ERR_ARG, "pointers must be non-null; y, norm, d_out, d_y, workspace 16-byte aligned");
  G3EpiArgs a{};
  a.y = y; a.lg = router_logits; a.norm = norm; a.dout = d_out; a.dy = d_y; a.dlg = d_router_logits;
  a.dnorm = d_norm; a.part = (float*)workspace;
  a.rows = (long long)B * T * H; a.M = M; a.V = value_dim;
  return gdn3_epilogue_dispatch(a, true, dtype, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Rank-r RLS T-factor scan
// ---------------------------------------------------------------------------
namespace gdnx {

static int rls_sizes(int B, int T, int H, int R, int RO, int dk, int dv, float eps) {
  if (B < 1 || T < 0 || H < 1) return set_error(GDNX_ERR_SHAPE, "bad sizes B=%d T=%d H=%d", B, T, H);
  if (R < 1 || R > 4 || RO < 1 || RO > 4) return set_error(GDNX_ERR_SHAPE, "slots R=%d, R_out=%d (1..4)", R, RO);
  if (dk != 32 && dk != 64 && dk != 128) return set_error(GDNX_ERR_SHAPE, "key_dim %d unsupported (32, 64, 128)", dk);
  if (dv < 16 || dv > 128 || dv % 16) return set_error(GDNX_ERR_SHAPE, "value_dim %d unsupported (multiple of 16, <= 128)", dv);
  if (!(eps > 0.0f)) return set_error(GDNX_ERR_ARG, "eps must be positive");
  if ((long long)B * H > (1LL << 30)) return set_error(GDNX_ERR_SHAPE, "too many chains");
  return GDNX_OK;
}

static int rls_compact_args(int dk, int dv, int cP, int cR, float sd) {
  if (cP == 0) return GDNX_OK;
  if (cP < 0 || cP % 2) return set_error(GDNX_ERR_ARG, "compact_P=%d must be 0 or a positive even count", cP);
  const int m = dv < dk ? dv : dk;
  if (m > 64 || dk * dv > 4096)
    return set_error(GDNX_ERR_SHAPE, "compaction needs min(key_dim, value_dim) <= 64 and key_dim*value_dim <= 4096");
  if (cR < 1 || cR > m) return set_error(GDNX_ERR_ARG, "compact_R=%d must be in 1..%d", cR, m);
  if (!(sd >= 0.0f && sd <= 1.0f)) return set_error(GDNX_ERR_ARG, "slow_decay must be in [0, 1]");
  return GDNX_OK;
}

static bool aligned_or_null(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && !aligned16(p)) return false;
  return true;
}

}  // namespace gdnx

extern "C" long long gdnx_rls_ckpt_bytes(int B, int T, int H, int R, int key_dim, int value_dim, int compact_P) {
  if (rls_sizes(B, T, H, R, 1, key_dim, value_dim, 1.0f) != GDNX_OK) return -1;
  if (compact_P < 0 || compact_P % 2) return -1;
  return (long long)rls_ckpt_bytes(B * H, T, R, key_dim, value_dim, compact_P);
}

extern "C" long long gdnx_rls_bwd_workspace_bytes(int B, int T, int H, int R, int key_dim, int value_dim) {
  if (rls_sizes(B, T, H, R, 1, key_dim, value_dim, 1.0f) != GDNX_OK) return -1;
  return (long long)rls_bwd_workspace_bytes(B * H, T, R, key_dim, value_dim);
}

extern "C" int gdnx_rls_fwd(const float* q, const float* K, const float* V, const float* Bg, const float* Wg,
                            const float* a, const float* out_mix, const float* state0, float* y, float* state_out,
                            float* ckpt, int B, int T, int H, int R, int R_out, int key_dim, int value_dim,
                            float eps, int compact_P, int compact_R, float slow_decay, void* stream) {
  g_err[0] = 0;
  int rc = rls_sizes(B, T, H, R, R_out, key_dim, value_dim, eps);
  if (rc == GDNX_OK) rc = rls_compact_args(key_dim, value_dim, compact_P, compact_R, slow_decay);
  if (rc != GDNX_OK) return rc;
  if (!all_aligned({q, K, V, Bg, Wg, a, y}) || (R_out > 1 && !out_mix) ||
      !aligned_or_null({state0, state_out, ckpt}))
    return set_error(GDNX_ERR_ARG, "q, K, V, Bg, Wg, a, y (and out_mix when R_out > 1) must be non-null; "
                                   "all tensors 16-byte aligned");
  RlsDesc d{};
  d.q = q; d.K = K; d.V = V; d.Bg = Bg; d.Wg = Wg; d.a = a; d.mix = out_mix; d.state0 = state0;
  d.y = y; d.state_out = state_out; d.ckpt = ckpt;
  d.B = B; d.T = T; d.H = H; d.R = R; d.RO = R_out; d.dk = key_dim; d.dv = value_dim; d.eps = eps;
  d.cP = compact_P; d.cR = compact_R; d.cs = slow_decay;
  if ((rc = rls_dispatch(d, false, (hipStream_t)stream))) return rc;
  const FiniteBuf outs[] = {{y, (size_t)B * T * H * value_dim, GDNX_DTYPE_F32},
                            {state_out, (size_t)B * H * value_dim * key_dim, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 2, (hipStream_t)stream);
}

extern "C" int gdnx_rls_bwd(const float* q, const float* K, const float* V, const float* Bg, const float* Wg,
                            const float* a, const float* out_mix, const float* ckpt, const float* dy,
                            const float* d_state, float* dq, float* dK, float* dV, float* dBg, float* dWg,
                            float* da, float* d_out_mix_seq, float* d_state0, int B, int T, int H, int R,
                            int R_out, int key_dim, int value_dim, float eps, int compact_P, int compact_R,
                            float slow_decay, int straight_through, void* workspace, void* stream) {
  g_err[0] = 0;
  int rc = rls_sizes(B, T, H, R, R_out, key_dim, value_dim, eps);
  if (rc == GDNX_OK) rc = rls_compact_args(key_dim, value_dim, compact_P, compact_R, slow_decay);
  if (rc != GDNX_OK) return rc;
  if (!ckpt) return set_error(GDNX_ERR_WORKSPACE, "the backward needs the forward's checkpoints (ckpt)");
  if (!all_aligned({q, K, V, Bg, Wg, a, ckpt, dy, dq, dK, dV, dBg, dWg, da, d_out_mix_seq}) ||
      (R_out > 1 && !out_mix) || !aligned_or_null({d_state, d_state0}))
    return set_error(GDNX_ERR_ARG, "inputs, checkpoints and gradient outputs must be non-null and 16-byte aligned");
  RlsDesc d{};
  d.q = q; d.K = K; d.V = V; d.Bg = Bg; d.Wg = Wg; d.a = a; d.mix = out_mix; d.ckpt = const_cast<float*>(ckpt);
  d.dy = dy; d.dstate = d_state; d.dq = dq; d.dK = dK; d.dV = dV; d.dBg = dBg; d.dWg = dWg; d.da = da;
  d.dmix = d_out_mix_seq; d.dstate0 = d_state0;
  d.B = B; d.T = T; d.H = H; d.R = R; d.RO = R_out; d.dk = key_dim; d.dv = value_dim; d.eps = eps;
  d.cP = compact_P; d.cR = compact_R; d.cs = slow_decay; d.ste = straight_through != 0;
  if (workspace && !aligned16(workspace)) return set_error(GDNX_ERR_ARG, "workspace must be 16-byte aligned");
  d.workspace = workspace;
  if ((rc = rls_dispatch(d, true, (hipStream_t)stream))) return rc;
  const size_t rows = (size_t)B * T * H;
  const FiniteBuf outs[] = {{dq, rows * R_out * key_dim, GDNX_DTYPE_F32},  {dK, rows * R * key_dim, GDNX_DTYPE_F32},
                            {dV, rows * R * value_dim, GDNX_DTYPE_F32},    {dBg, rows * R * key_dim, GDNX_DTYPE_F32},
                            {dWg, rows * R * value_dim, GDNX_DTYPE_F32},   {da, rows * key_dim, GDNX_DTYPE_F32},
                            {d_out_mix_seq, (size_t)B * H * R_out, GDNX_DTYPE_F32},
                            {d_state0, (size_t)B * H * value_dim * key_dim, GDNX_DTYPE_F32}};
  return finite_outputs(outs, 8, (hipStream_t)stream);
}

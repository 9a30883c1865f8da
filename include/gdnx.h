/* gdnx -- MI355X-native chunked GDN3 / KMD-2 recurrence, C ABI.
 *
 * All entry points are asynchronous on the given HIP stream (passed as
 * void*), allocate nothing, use no float atomics (results are bitwise
 * deterministic) and return an int status: 0 on success, a negative
 * GDNX_ERR_* code otherwise (message via gdnx_last_error(), per thread).
 * Pointers are device pointers to contiguous row-major tensors; the caller
 * owns every buffer.  No C++ exception crosses this boundary.
 *
 * Layouts (b batch, t token, h head, m lane, d/v feature):
 *   q, k, v      [B, T, H, D]        io dtype; shared by the M lanes of a head
 *   a_e, a_w, g  [B, T, H, M]        float32 per-token erase / write
 *                                    coefficients and natural-log decay
 *   y, dy        [B, T, H, M, D]     io dtype
 *   state        [B, H, M, D, D]     float32, key-major [d_k][d_v]
 */
#ifndef GDNX_H
#define GDNX_H

#ifdef __cplusplus
extern "C" {
#endif

#define GDNX_ABI_VERSION 1

enum { GDNX_DTYPE_F32 = 0, GDNX_DTYPE_BF16 = 1 };

enum {
  GDNX_OK = 0,
  GDNX_ERR_ARG = -1,       /* null / misaligned pointer, bad enum */
  GDNX_ERR_SHAPE = -2,     /* unsupported or inconsistent sizes */
  GDNX_ERR_WORKSPACE = -3, /* workspace missing or too small */
  GDNX_ERR_HIP = -4        /* HIP launch or runtime error */
};

/* Version of this ABI (GDNX_ABI_VERSION). */
int gdnx_abi_version(void);

/* Message of the last error on the calling thread ("" if none). */
const char* gdnx_last_error(void);

/* Default chunk length (tokens) of the forward for head_dim / dtype
 * (64 for bf16, 32 for float32). */
int gdnx_delta_chunk_size(int head_dim, int dtype);

/* Chunk length to use when the forward stashes states for the backward
 * (32 for bf16, 16 for float32). */
int gdnx_delta_train_chunk_size(int head_dim, int dtype);

/* Bytes of the per-chunk state stash (one d x d state per chain per chunk,
 * in the compute dtype) for the given chunk (0 = default); -1 if invalid.
 * The backward's workspace has the same size. */
long long gdnx_delta_chunk_states_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                        int dtype);

/* Chunked decoupled-erase delta rule, forward.
 * Replaces the sequential token loop of
 *   GDN3LinearAttn._gdn3_recurrent_state  (reference gdn3/gdn3_upgrade.py:403-531,
 *   frozen oracle gdn3/_reference_recurrence.py:33-94) in its dense regime, and
 *   the KMD-2 scan core (gdn3/kmd2_fast_scan.py:163-260; oracle
 *   research/kernel_ab/ref_scan.py:24-48) with scalar decay.
 * Per chain (b, h, m), token t:  S <- exp(min(g,0)) S;  r = a_w v - a_e S^T k;
 *   S <- S + k r^T;  y = S^T q.
 * state0 / state_out / chunk_states may be NULL.  chunk_states (size from
 * gdnx_delta_chunk_states_bytes) receives the state entering every chunk,
 * which gdnx_delta_chunk_bwd needs. */
int gdnx_delta_chunk_fwd(const void* q, const void* k, const void* v,
                         const float* a_e, const float* a_w, const float* log_g,
                         const float* state0, void* y, float* state_out,
                         void* chunk_states, int B, int T, int H, int M,
                         int head_dim, int chunk, int dtype, void* stream);

/* Backward of gdnx_delta_chunk_fwd.  Replaces torch autograd through the
 * reference's chunk graph (gdn3/gdn3_upgrade.py:467-521) and its hand
 * backward of the KMD-2 TRSM (gdn3/kmd2_fast_scan.py:143-160).
 * chunk_states: the forward's stash, made with the same chunk (0 = train
 * default).  workspace: gdnx_delta_chunk_states_bytes bytes.  dstate_out:
 * gradient w.r.t. the final state (or NULL).  Outputs: dq, dk, dv [B,T,H,D]
 * (summed over the M lanes), da_e, da_w, dlog_g [B,T,H,M] float32, dstate0
 * [B,H,M,D,D] float32 (or NULL).  dlog_g is zero where the forward clamped. */
int gdnx_delta_chunk_bwd(const void* q, const void* k, const void* v,
                         const float* a_e, const float* a_w, const float* log_g,
                         const void* dy, const float* dstate_out,
                         const void* chunk_states, void* workspace,
                         void* dq, void* dk, void* dv,
                         float* da_e, float* da_w, float* dlog_g, float* dstate0,
                         int B, int T, int H, int M, int head_dim, int chunk,
                         int dtype, void* stream);

/* The two stages of gdnx_delta_chunk_bwd, callable separately (e.g. to
 * time or overlap them).  Stage 1 runs the reverse state scan and fills
 * workspace with dS at every chunk end (plus dstate0); stage 2 reads the
 * forward's chunk_states and that workspace and writes every input gradient.
 * Same arguments and layouts as gdnx_delta_chunk_bwd. */
int gdnx_delta_chunk_bwd_state(const void* q, const void* k, const float* a_e,
                               const float* log_g, const void* dy, const float* dstate_out,
                               void* workspace, float* dstate0,
                               int B, int T, int H, int M, int head_dim, int chunk,
                               int dtype, void* stream);
int gdnx_delta_chunk_bwd_grads(const void* q, const void* k, const void* v,
                               const float* a_e, const float* a_w, const float* log_g,
                               const void* dy, const void* chunk_states, const void* workspace,
                               void* dq, void* dk, void* dv,
                               float* da_e, float* da_w, float* dlog_g,
                               int B, int T, int H, int M, int head_dim, int chunk,
                               int dtype, void* stream);

/* One-token decode step, state updated in place.  The reference has no
 * decode path (GDN3LinearAttn.forward ignores cache_params,
 * gdn3/gdn3_upgrade.py:725); this is one iteration of the sequential oracle
 * (gdn3/_reference_recurrence.py:60-84 dense regime, research/kernel_ab/
 * ref_scan.py:40-45) on carried state, i.e. gdnx_delta_chunk_fwd with T=1.
 * q, k, v [NS, H, D] (io dtype, shared by the M chains of a head: lanes x
 * decay timescales); a_e, a_w, log_g [NS, H, M] float32; state
 * [NS, H, M, D, D] float32 key-major, read and written once; y [NS, H, M, D]
 * io dtype. */
int gdnx_delta_decode_step(const void* q, const void* k, const void* v,
                           const float* a_e, const float* a_w, const float* log_g,
                           float* state, void* y, int NS, int H, int M, int head_dim,
                           int dtype, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GDNX_H */

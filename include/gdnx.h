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

#define GDNX_ABI_VERSION 12

enum { GDNX_DTYPE_F32 = 0, GDNX_DTYPE_BF16 = 1, GDNX_DTYPE_F64 = 2 /* gdnx_check_finite only */ };

enum {
  GDNX_OK = 0,
  GDNX_ERR_ARG = -1,       /* null / misaligned pointer, bad enum */
  GDNX_ERR_SHAPE = -2,     /* unsupported or inconsistent sizes */
  GDNX_ERR_WORKSPACE = -3, /* workspace missing or too small */
  GDNX_ERR_HIP = -4,       /* HIP launch or runtime error */
  GDNX_ERR_NONFINITE = -5  /* NaN or infinity in the outputs (checking on) */
};

/* Version of this ABI (GDNX_ABI_VERSION). */
int gdnx_abi_version(void);

/* Message of the last error on the calling thread ("" if none). */
const char* gdnx_last_error(void);

/* Non-finite checking, the counterpart of the reference trainer's NaN/inf
 * guard (train/train_gdn3_distill.py:329-354), which drops a step whose loss
 * or gradient norm is not finite.  Off by default.  When on (process-wide),
 * the recurrence entry points (delta, per-channel, GDN3 and RLS forwards and
 * backwards, the decode steps) scan the outputs they wrote, synchronise their
 * stream and return GDNX_ERR_NONFINITE if any is NaN or infinite.  Returns
 * the previous setting.  Limits while on: each checked call holds one of 64
 * per-device flag words until its stream has synchronised (a 65th concurrent
 * checked call on a device returns GDNX_ERR_HIP), and a checked call on a
 * stream under HIP graph capture returns GDNX_ERR_ARG (the check reads the
 * flag back and synchronises, which capture forbids). */
int gdnx_set_check_finite(int on);

/* Scans x[0, n) (GDNX_DTYPE_F32, _BF16 or _F64) on the stream and waits for
 * it: GDNX_OK if every element is finite, else GDNX_ERR_NONFINITE. */
int gdnx_check_finite(const void* x, long long n, int dtype, void* stream);

/* Default chunk length (tokens) of the forward for head_dim / dtype
 * (64 for bf16, 32 for float32). */
int gdnx_delta_chunk_size(int head_dim, int dtype);

/* Chunk length to use when the forward stashes states for the backward
 * (32 for bf16, 16 for float32; the backward also takes 64 for bf16). */
int gdnx_delta_train_chunk_size(int head_dim, int dtype);

/* Bytes of the stash for the given chunk (0 = default; -1 if invalid).  In
 * order: the d x d states (compute dtype, MFMA-fragment tile order), then
 * every chunk's C x d net writes R (same order), then the chunk's
 * state-independent operands (T = (I + L)^-1 and the decay-masked Q K^T as
 * C x C compute-dtype matrices, and four float32 per-token factors), which
 * the backward's reverse scan reuses.  The states are the one entering every
 * chunk, except for bf16 IO with 32-token chunks and at most 4 lanes per head
 * (the training default): there only the state entering every 256-token
 * segment is kept, and the backward recomputes the others from the net
 * writes (checkpointed form). */
long long gdnx_delta_chunk_states_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                        int dtype);

/* Bytes of the backward's workspace for the given chunk (0 = train default;
 * -1 if invalid, or beyond 2^30 chains or 2^40 token-chains): the state
 * gradients leaving every chunk (every 256-token segment in the checkpointed
 * form) and dB = T^T dR of every chunk, laid out as the forward's stash; in
 * the checkpointed form then P3 = R dS^T of every chunk (bf16, the gradient
 * kernel's dk tile layout) and k.P3 per token (float32), and with more than
 * two lanes per head the gradient kernel's float32 carry of the dq, dk and dv
 * sums between lane pairs, 3 x 256 x head_dim floats per (batch, head,
 * segment).  Changed in ABI 12 (P3 and k.P3 added): query it, do not cache
 * sizes across versions. */
long long gdnx_delta_bwd_workspace_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                         int dtype);

/* Chunked decoupled-erase delta rule, forward.
 * Replaces the sequential token loop of
 *   GDN3LinearAttn._gdn3_recurrent_state  (reference gdn3/gdn3_upgrade.py:403-531,
 *   frozen oracle gdn3/_reference_recurrence.py:33-94) in its dense regime, and
 *   the KMD-2 scan core (gdn3/kmd2_fast_scan.py:163-260; oracle
 *   research/kernel_ab/ref_scan.py:24-48) with scalar decay.
 * Per chain (b, h, m), token t:  S <- exp(min(g,0)) S;  r = a_w v - a_e S^T k;
 *   S <- S + k r^T;  y = S^T q.
 * state0 / state_out / chunk_states / workspace may be NULL.  chunk_states
 * (size from gdnx_delta_chunk_states_bytes) receives what
 * gdnx_delta_chunk_bwd needs (the state entering every chunk, the net writes
 * and the chunk operands).  With chunk_states or workspace (size from
 * gdnx_delta_fwd_workspace_bytes) the forward runs as a fully parallel
 * per-chunk operand pass plus a value-split state scan; with neither, as one
 * fused scan.  Results agree up to rounding order. */
int gdnx_delta_chunk_fwd(const void* q, const void* k, const void* v,
                         const float* a_e, const float* a_w, const float* log_g,
                         const float* state0, void* y, float* state_out,
                         void* chunk_states, void* workspace, int B, int T, int H, int M,
                         int head_dim, int chunk, int dtype, void* stream);

/* Bytes of the optional forward workspace (-1 if invalid): room for every
 * chunk's state-independent operands (T = (I + L)^-1, the decay-masked
 * Q K^T and the per-token decay and coefficient factors), which a fully
 * parallel pass computes before the value-split state scan.  Not needed
 * when chunk_states is given (the operands then go there). */
long long gdnx_delta_fwd_workspace_bytes(int B, int T, int H, int M, int head_dim, int chunk,
                                         int dtype);

/* The intra-chunk phase alone: every chunk's state-independent operands
 * (the decay-masked grams, T = (I + L)^-1 by 16x16 blocks, Aq and the
 * per-token factors; the per-chunk part of the reference's chunk loop,
 * gdn3/gdn3_upgrade.py:467-521) into workspace (gdnx_delta_fwd_workspace_bytes
 * bytes), the records the parallel forward pass writes before its state
 * scan.  Reads q, k, a_e, a_w, log_g. */
int gdnx_delta_chunk_prep(const void* q, const void* k, const float* a_e, const float* a_w,
                          const float* log_g, void* workspace, int B, int T, int H, int M,
                          int head_dim, int chunk, int dtype, void* stream);

/* gdnx_delta_chunk_fwd that also writes r_norm [B, T, H, M] float32, the
 * norm of each token's net write |r_t| = |a_w v - a_e S_bar^T k|; the KMD-2
 * update-norm score is |k_t| |r_t| (scan_with_update_norm,
 * gdn3/kmd2_fast_scan.py:282; reference score research/kmd2_ablation/
 * exact_cache.py:1231-1295). */
int gdnx_delta_chunk_fwd_scored(const void* q, const void* k, const void* v,
                                const float* a_e, const float* a_w, const float* log_g,
                                const float* state0, void* y, float* state_out,
                                void* chunk_states, float* r_norm, void* workspace, int B, int T,
                                int H, int M, int head_dim, int chunk, int dtype, void* stream);

/* Backward of gdnx_delta_chunk_fwd.  Replaces torch autograd through the
 * reference's chunk graph (gdn3/gdn3_upgrade.py:467-521) and its hand
 * backward of the KMD-2 TRSM (gdn3/kmd2_fast_scan.py:143-160).
 * chunk_states: the forward's stash, made with the same chunk (0 = train
 * default).  workspace: gdnx_delta_bwd_workspace_bytes bytes.  dstate_out:
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
 * time or overlap them).  Stage 1 runs the reverse state scan on the
 * forward's chunk operands (in chunk_states) and fills workspace with dS at
 * every chunk end (every segment end in the checkpointed form), dB and, in
 * the checkpointed form, P3 and k.P3 (plus dstate0); stage 2 reads the
 * forward's chunk_states and that workspace and writes every input gradient
 * (in the checkpointed form it also uses the workspace's float32 tail as the
 * lane pairs' carry, so the workspace is not const).  Same arguments and
 * layouts as gdnx_delta_chunk_bwd. */
int gdnx_delta_chunk_bwd_state(const void* q, const void* k, const float* a_e,
                               const float* log_g, const void* dy, const float* dstate_out,
                               const void* chunk_states, void* workspace, float* dstate0,
                               int B, int T, int H, int M, int head_dim, int chunk,
                               int dtype, void* stream);
int gdnx_delta_chunk_bwd_grads(const void* q, const void* k, const void* v,
                               const float* a_e, const float* a_w, const float* log_g,
                               const void* dy, const void* chunk_states, void* workspace,
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

/* The same step on a decode-state cache: state_pool [n_slots, H, M, D, D]
 * float32 holds one state per slot, and row s of the batch (q, k, v, the
 * coefficients and y as above) updates slot slots[s] (int32 [NS], device
 * memory).  A row whose slot lies outside [0, n_slots) is empty: its y is
 * zero and no state is read or written.  No counterpart in the reference
 * (it keeps no recurrent cache); for serving loops whose sequences join and
 * leave the batch without moving their states.  Rows sharing a slot race. */
int gdnx_delta_decode_step_slots(const void* q, const void* k, const void* v,
                                 const float* a_e, const float* a_w, const float* log_g,
                                 float* state_pool, const int* slots, void* y, int NS,
                                 int n_slots, int H, int M, int head_dim, int dtype, void* stream);

/* The decode step with a decay per key channel, for the KMD-2 native state
 * (one step of research/kernel_ab/ref_scan.py:40-45 and of
 * gdn3/kmd2_native.py:109-132; the reference has no decode path):
 * S <- diag(g) S;  r = a_w v - a_e S^T k;  S <- S + k r^T;  y = S^T q, with
 * log_g [NS, H, M, D] float32 (natural log, clamped to <= 0, per key
 * channel).  Other arguments as gdnx_delta_decode_step_slots; slots may be
 * NULL (row s updates state s; n_slots ignored).  KMD-2's query slots enter
 * as their mixed query sum_r out_mix[h, r] q_r (the read is linear in q). */
int gdnx_delta_decode_step_chan(const void* q, const void* k, const void* v,
                                const float* a_e, const float* a_w, const float* log_g,
                                float* state_pool, const int* slots, void* y, int NS,
                                int n_slots, int H, int M, int head_dim, int dtype, void* stream);

/* ---- Per-key-channel decay (the general KMD-2 scan) -----------------------
 * One chain per (batch, head), float32:  S <- diag(g_t) S (g per key
 * channel, log_g = natural log, clamped to <= 0);  r = beta_w v -
 * beta_e S^T k;  S <- S + k r^T;  y = S^T q.  Replaces the chunked KMD-2 scan
 * with a per-channel decay (gdn3/kmd2_fast_scan.py:163-260; oracle
 * research/kernel_ab/ref_scan.py:24-48 and gdn3/kmd2_native.py:109-132,
 * where g = exp(g_head + decay_chan) [B,T,H,dk]).  Chunks of 16 tokens with
 * the decay-weighted grams formed exactly per channel.
 *   q, k, v, y, log_g, dq, dk, dv, dlog_g  [B, T, H, D] float32
 *   beta_e, beta_w, dbeta_e, dbeta_w       [B, T, H] float32
 *   state0, state_out, dstate_out, dstate0 [B, H, D, D] float32 (may be NULL)
 *   r_norm [B, T, H] float32 or NULL: |r_t| (the KMD-2 update score is
 *   |k_t| |r_t|)
 * chunk_states (forward, for the backward: state stash plus each chunk's
 * operand records) and the backward's workspace are
 * gdnx_delta_chan_states_bytes bytes each; a forward without chunk_states
 * needs workspace (gdnx_delta_chan_fwd_workspace_bytes) for the records. */
long long gdnx_delta_chan_states_bytes(int B, int T, int H, int head_dim);
long long gdnx_delta_chan_fwd_workspace_bytes(int B, int T, int H, int head_dim);
int gdnx_delta_chan_fwd(const float* q, const float* k, const float* v, const float* beta_e,
                        const float* beta_w, const float* log_g, const float* state0, float* y,
                        float* state_out, void* chunk_states, void* workspace, float* r_norm, int B,
                        int T, int H, int head_dim, void* stream);
/* Backward of gdnx_delta_chan_fwd; dlog_g is zero where the log-decay was
 * clamped. */
int gdnx_delta_chan_bwd(const float* q, const float* k, const float* v, const float* beta_e,
                        const float* beta_w, const float* log_g, const float* dy,
                        const float* dstate_out, const void* chunk_states, void* workspace,
                        float* dq, float* dk, float* dv, float* dbeta_e, float* dbeta_w,
                        float* dlog_g, float* dstate0, int B, int T, int H, int head_dim,
                        void* stream);

/* GDN3 exact-alpha write coefficient in the dense regime (lane-shared keys,
 * one scalar gate per lane): a = alpha(beta |k|^2) beta with
 * alpha(c) = (1 - exp(-c)) / c (Taylor 1 - c/2 + c^2/6 below |c| = 1e-6).
 * Replaces _stable_alpha_vec and its use in the recurrence
 * (gdn3/gdn3_upgrade.py:641-648; gdn3/_reference_recurrence.py:73-78) for the
 * b = w = beta case, where erase and write coefficients coincide.
 * k [B, T, H, D] io dtype; beta, a [B, T, H, M] float32; M <= 16. */
int gdnx_gdn3_coeff(const void* k, const float* beta, float* a, int B, int T, int H, int M,
                    int head_dim, int dtype, void* stream);

/* Backward of gdnx_gdn3_coeff: with da = da_e + da_w (da_w may be NULL),
 * writes dbeta [B, T, H, M] and adds the coefficient's key gradient into
 * dk [B, T, H, D] (io dtype, in place). */
int gdnx_gdn3_coeff_bwd(const void* k, const float* beta, const float* da_e, const float* da_w,
                        void* dk, float* dbeta, int B, int T, int H, int M, int head_dim,
                        int dtype, void* stream);


/* ---- GDN3 Kronecker-residual regime --------------------------------------
 * State per chain n = (b, h, m):  S = sum_r A_r (x) B_r + U Vb^T  (d_v x d_k),
 * A [R, a_v, a_k], B [R, b_v, b_k] (a_v b_v = a_k b_k = head_dim), and a
 * P-slot residual buffer U [d_v, P] (net writes), Vb [d_k, P] (keys).  The
 * reference layouts of gdn3/gdn3_upgrade.py:444-448.  All state float32. */

/* Bytes of the gdnx_gdn3_chunk_fwd workspace: per chain the materialised
 * Kronecker matrix (d x d, compute dtype), A and B, and the P-slot window
 * carried between compaction intervals; -1 if invalid. */
long long gdnx_gdn3_workspace_bytes(int B, int H, int M, int head_dim, int P, int dtype);

/* Number of compactions gdnx_gdn3_chunk_fwd runs over T tokens (rows of
 * comp_stats): T / compact_every; -1 if invalid. */
int gdnx_gdn3_num_compactions(int T, int P, int compact_every);

/* GDN3 recurrence forward with residual window and periodic compaction.
 * Replaces GDN3LinearAttn._gdn3_recurrent_state (gdn3/gdn3_upgrade.py:403-531)
 * with the semantics of its frozen oracle gdn3/_reference_recurrence.py:33-94:
 * per token gamma = clamp(dec, 0, 1) decays A, B and Vb; h = b.k, u = w.v;
 * r = u - S h; alpha = alpha(k.h); y = S q + alpha (k.q) r; slot t mod P
 * receives (alpha r, k); after token t with (t+1) % compact_every == 0 the
 * compaction of gdnx_gdn3_compact runs (no gradient).  Initial state zero.
 *   q, k, v      [B, T, H, qkv_lanes, D] io dtype (qkv_lanes 1: shared by
 *                the M lanes; M: per lane)
 *   b_gates, w_gates [B, T, H, M, gate_channels] float32 (gate_channels 1:
 *                a scalar gate per lane; head_dim: per channel)
 *   decay        [B, T, H, M] float32 multiplicative decay
 *   sketch       [B*H*M, b_v*b_k, q] float32, q = min(R+4, a_v*a_k, b_v*b_k)
 *                for compact_mode 0, q = R for compact_mode 1
 *   compact_mode 0: 'svd' (randomized range finder + SVD, the default of
 *                gdn3/gdn3_upgrade.py:81); 1: 'sketch' / 'sketch_noqr' (the
 *                two names run one branch, :579-592): R_mat G column-normalised
 *                to Q, Bm = Q^T R_mat row-normalised; reports no error
 *   y            [B, T, H, M, D] io dtype
 *   A_out, B_out, U_out, Vb_out  final state in the layouts above (each
 *                may be NULL), for any T: U / Vb slot t mod P holds the write
 *                and key of the last token t that used it
 *   comp_stats   [T / compact_every, B*H*M, 2] float64 (|R_mat|^2, kept
 *                sigma^2 per chain and compaction) or NULL; the reference's
 *                comp_err is sum over compactions of max(0, sum_n energy -
 *                sum_n kept)
 *   workspace    gdnx_gdn3_workspace_bytes bytes
 *   train_states gdnx_gdn3_train_states_bytes bytes receiving what
 *                gdnx_gdn3_chunk_bwd reads (net writes and accumulated log
 *                decay per window, the factors after every compaction), or
 *                NULL for inference
 * Supported: head_dim 128 or 64 with P = 16, 32 or 64 (GDN3_P,
 * gdn3/gdn3_upgrade.py:74); the layer's Kronecker geometry (R = 4 with
 * factors (16, 16, 8, 8) at head_dim 128, (8, 8, 8, 8) at 64);
 * compact_every a multiple of P. */
int gdnx_gdn3_chunk_fwd(const void* q, const void* k, const void* v, int qkv_lanes,
                        const float* b_gates, const float* w_gates, int gate_channels,
                        const float* decay, const float* sketch, void* y, float* A_out,
                        float* B_out, float* U_out, float* Vb_out, double* comp_stats,
                        void* workspace, void* train_states, int B, int T, int H, int M,
                        int head_dim, int R, int P, int compact_every, int a_v, int a_k, int b_v,
                        int b_k, float slow_decay, int dtype, int compact_mode, void* stream);

/* Number of compactions a call over global tokens [t0, t0 + T) runs (rows
 * of its comp_stats): those after tokens t with (t + 1) % compact_every == 0;
 * -1 if invalid. */
int gdnx_gdn3_num_compactions_from(int t0, int T, int P, int compact_every);

/* gdnx_gdn3_chunk_fwd on a carried state, for prefill and continuation (no
 * counterpart in the reference, whose recurrence always starts from zero
 * state at slot 0: gdn3/_reference_recurrence.py:52-56; its layer ignores
 * cache_params, gdn3/gdn3_upgrade.py:725).  Token t of the call is global
 * token t0 + t of the sequence: it writes slot (t0 + t) % P, and a
 * compaction follows it when (t0 + t + 1) % compact_every == 0, so two calls
 * over [0, T1) and [T1, T) (the second from the first's final state, t0 = T1)
 * equal one call over [0, T).  A0 [N,R,a_v,a_k], B0 [N,R,b_v,b_k],
 * U0 [N,D,P], Vb0 [N,D,P] (N = B H M, all four or none; none = zero state)
 * as a previous call returned them; t0 is the same for every chain.  The
 * final state may alias the initial one.  comp_stats has
 * gdnx_gdn3_num_compactions_from(t0, T, P, compact_every) rows.  Inference
 * only (no training stash); other arguments as gdnx_gdn3_chunk_fwd. */
int gdnx_gdn3_chunk_fwd_state(const void* q, const void* k, const void* v, int qkv_lanes,
                              const float* b_gates, const float* w_gates, int gate_channels,
                              const float* decay, const float* sketch, const float* A0, const float* B0,
                              const float* U0, const float* Vb0, int t0, void* y, float* A_out,
                              float* B_out, float* U_out, float* Vb_out, double* comp_stats,
                              void* workspace, int B, int T, int H, int M, int head_dim, int R, int P,
                              int compact_every, int a_v, int a_k, int b_v, int b_k, float slow_decay,
                              int dtype, int compact_mode, void* stream);

/* gdnx_gdn3_chunk_fwd_state without a workspace argument: it allocates
 * nothing and takes no caller memory beyond inputs and outputs.  No
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * workspace lives in a static device array of
 * gdnx_gdn3_noalloc_scratch_bytes() bytes (64 MiB) that each GPU the library
 * runs on holds until the process ends; calls needing more
 * (gdnx_gdn3_workspace_bytes > that: about 1,250 chains in bf16, 780 in
 * float32 at head_dim 128) return GDNX_ERR_WORKSPACE before any launch.  All
 * calls on one GPU share its array: calls that overlap on one GPU (other
 * streams or threads) race.  Results equal gdnx_gdn3_chunk_fwd_state's. */
long long gdnx_gdn3_noalloc_scratch_bytes(void);
int gdnx_gdn3_chunk_fwd_state_noalloc(const void* q, const void* k, const void* v, int qkv_lanes,
                                      const float* b_gates, const float* w_gates, int gate_channels,
                                      const float* decay, const float* sketch, const float* A0,
                                      const float* B0, const float* U0, const float* Vb0, int t0, void* y,
                                      float* A_out, float* B_out, float* U_out, float* Vb_out,
                                      double* comp_stats, int B, int T, int H, int M, int head_dim, int R,
                                      int P, int compact_every, int a_v, int a_k, int b_v, int b_k,
                                      float slow_decay, int dtype, int compact_mode, void* stream);

/* One-token GDN3 decode step on a carried Kronecker-residual state, updated
 * in place.  One iteration of the frozen oracle's token loop
 * (gdn3/_reference_recurrence.py:60-90; the reference itself has no decode
 * path): gamma = clamp(dec, 0, 1) decays A, B, Vb; r = w.v - S (b.k);
 * y = S q + alpha(k.b.k) (k.q) r; slot pos % P receives (alpha r, k); after a
 * token with (pos + 1) % compact_every == 0 the compaction of
 * gdnx_gdn3_compact runs on that row's chains (same sign convention).
 *   q, k, v      [NS, H, qkv_lanes, D] io dtype (qkv_lanes 1 or M)
 *   b_gates, w_gates [NS, H, M, gate_channels] float32; decay [NS, H, M]
 *   A [n_slots,H,M,R,a_v,a_k], Bf [n_slots,H,M,R,b_v,b_k], U, Vb
 *                [n_slots,H,M,D,P] float32: the state, in place
 *   sketch       [n_slots*H*M, b_v*b_k, q] float32 (rows by state index)
 *   slots        [NS] int32 device: row s advances state slots[s] (a slot
 *                outside [0, n_slots) is an empty row: y = 0, nothing
 *                touched); NULL: row s advances state s (n_slots ignored)
 *   pos          [NS] int32 device, >= 0: global index of row s's token
 *   y            [NS, H, M, D] io dtype
 *   comp_stats   [NS, H, M, 2] float64 or NULL: (|R_mat|^2, kept sigma^2)
 *                for chains compacted by this step, zero for the others
 * Rows that name the same slot race.  Supported shapes as gdnx_gdn3_chunk_fwd. */
int gdnx_gdn3_decode_step(const void* q, const void* k, const void* v, int qkv_lanes,
                          const float* b_gates, const float* w_gates, int gate_channels,
                          const float* decay, const float* sketch, float* A, float* Bf, float* U,
                          float* Vb, const int* slots, const int* pos, void* y, double* comp_stats,
                          int NS, int n_slots, int H, int M, int head_dim, int R, int P,
                          int compact_every, int a_v, int a_k, int b_v, int b_k, float slow_decay,
                          int dtype, int compact_mode, void* stream);

/* Bytes of the gdnx_gdn3_chunk_fwd training stash; -1 if invalid. */
long long gdnx_gdn3_train_states_bytes(int B, int T, int H, int M, int head_dim, int P,
                                       int compact_every);

/* Backward of gdnx_gdn3_chunk_fwd.  Replaces torch autograd through
 * GDN3LinearAttn._gdn3_recurrent_state (gdn3/gdn3_upgrade.py:403-531) with
 * the gradient semantics of its frozen oracle (gdn3/_reference_recurrence.py:
 * 60-90): the factors A, B a compaction leaves carry no gradient (it runs
 * under no_grad); the residual slots U, Vb keep theirs across compactions.
 * Inputs as in the forward, dy [B, T, H, M, D] io dtype, train_states as
 * filled by the forward with the same arguments.  Outputs, float32:
 *   dq, dk, dv   [B, T, H, M, D] per lane (for shared q/k/v the caller sums
 *                over the M lanes)
 *   db_gates, dw_gates  the gates' layout ([..., gate_channels])
 *   ddecay       [B, T, H, M] (zero where the decay was clamped)
 * Supported: P = 16, 32 or 64, head_dim 128 or 64, the layer's Kronecker
 * geometry. */
int gdnx_gdn3_chunk_bwd(const void* q, const void* k, const void* v, int qkv_lanes,
                        const float* b_gates, const float* w_gates, int gate_channels,
                        const float* decay, const void* dy, const void* train_states, float* dq,
                        float* dk, float* dv, float* db_gates, float* dw_gates, float* ddecay, int B,
                        int T, int H, int M, int head_dim, int R, int P, int compact_every, int a_v,
                        int a_k, int b_v, int b_k, int dtype, void* stream);

/* Lane sum: out[r][d] = sum over m = 0 .. M-1, in that order, of x[r][m][d]
 * (x float32 [rows][M][D]; out [rows][D] in dtype GDNX_DTYPE_F32 or _BF16;
 * D a multiple of 8, both 16-byte aligned).  The gradient of q, k or v
 * shared by a head's lanes: it replaces the backward of the reference's
 * lane expand (gdn3/gdn3_upgrade.py:785-787), applied to the per-lane
 * gradients gdnx_gdn3_chunk_bwd writes, and the cast to the IO dtype. */
int gdnx_lane_sum(const float* x, void* out, long long rows, int M, int D, int dtype, void* stream);

/* Rearrangement-SVD compaction with two-timescale blend, one chain per
 * block.  Replaces GDN3LinearAttn._compact_vec (gdn3/gdn3_upgrade.py:650-719)
 * and the 'svd' mode of _compact_fast (:565-624):
 *   R_mat = sum_r vec(A_r) vec(B_r)^T + rearrange(U Vb^T)   [a_v a_k, b_v b_k]
 *   randomized range finder (sketch, two power iterations), SVD of the
 *   projection; A <- s A + (1-s) sigma_r u_r, B <- s B + (1-s) v_r (top R).
 * Signs: each (u_r, v_r) is flipped so that the largest-magnitude entry of
 * v_r is positive (first index on ties); the reference keeps whatever its
 * SVD backend returns.  A, Bf, U, Vb as in the state layout above; sketch
 * [N, b_v*b_k, q] (q as in gdnx_gdn3_chunk_fwd); comp_stats [N, 2]
 * (|R_mat|^2, kept; kept = |R_mat|^2 for compact_mode 1) or NULL.  U and Vb
 * are left unchanged (as the reference does). */
int gdnx_gdn3_compact(const float* A, const float* Bf, const float* U, const float* Vb,
                      const float* sketch, float* A_out, float* B_out, double* comp_stats, int N,
                      int head_dim, int R, int P, int a_v, int a_k, int b_v, int b_k,
                      float slow_decay, int compact_mode, void* stream);

/* Read of the Kronecker-residual state, y = S x for C vectors per chain:
 * vec(sum_r A_r X B_r^T) + U (Vb^T x), X = x viewed as [a_k, b_k].  Replaces
 * _kron_read_vec (gdn3/gdn3_upgrade.py:626-639) and the Triton
 * kron_read_chunk_triton (gdn3/triton_kernels.py:146-175).  x, y [N, C, D]
 * float32; P in 0..64 (U, Vb may be NULL when P = 0). */
int gdnx_kron_read(const float* A, const float* Bf, const float* U, const float* Vb, const float* x,
                   float* y, int N, int C, int head_dim, int R, int P, int a_v, int a_k, int b_v,
                   int b_k, void* stream);

/* ---- GDN3 layer boundary: the element-wise pre-ops and post-ops of
 * GDN3LinearAttn.forward (gdn3/gdn3_upgrade.py:785-856), each direction one
 * pass over HBM.  The reference runs them in line as torch ops (no function
 * boundary); these entry points replace lines 796-828 (prologue) and 842-851
 * (epilogue).  Rows are (b, t, h) in [B, T, H] order; IO tensors are in
 * `dtype`, everything else float32.  Lanes M <= 4 (the reference's lane RoPE
 * table lists four lanes, :181-182); key_dim and value_dim multiples of 4,
 * <= 256. */

/* Lane RoPE pairs d_m by the reference's rule (gdn3/gdn3_upgrade.py:342-376):
 * d = floor(key_dim f_m / 2), f = (0.5, 0.25, 0.5, 0.5); 0 (identity) for a
 * lane with scale 1 whose d exceeds floor(key_dim / 4) / 2.  Host only: fills
 * pairs[0..M-1] in host memory. */
int gdnx_gdn3_lane_rope_pairs(int M, int key_dim, int* pairs);

/* Prologue (gdn3/gdn3_upgrade.py:796-828, lane RoPE :378-401):
 *   b_gates = sigmoid(b_proj + 0.1 proj_a)        [B,T,H,M,key_dim]
 *   w_gates = sigmoid(w_proj + 0.1 proj_b)        [B,T,H,M,value_dim]
 *   decay   = min(mean_tau exp(-min(softplus(decay_proj), 5) rates[tau]), decay_clamp)   [B,T,H,M]
 *   q_rope, k_rope [B,T,H,M,key_dim]: lane m of q, k [B,T,H,key_dim] with
 *     x_i' = x_i c - x_{d+i} s,  x_{d+i}' = x_i' s + x_{d+i} c   (i < d_m)
 *   where the second half reads the updated first half (rounded to dtype),
 *   as the reference's in-place update does.
 * proj_a, proj_b [B,T,H]; decay_proj [B,T,H,M,4]; rates [4] float32;
 * rope_cos, rope_sin [M, T, key_dim/2] float32: lane m's angles at column
 * i < d_m (the values of _lane_rope_factors; other columns unread). */
int gdnx_gdn3_prologue_fwd(const void* q, const void* k, const void* b_proj, const void* proj_a,
                           const void* w_proj, const void* proj_b, const void* decay_proj,
                           const float* rates, const float* rope_cos, const float* rope_sin,
                           void* q_rope, void* k_rope, float* b_gates, float* w_gates, float* decay,
                           int B, int T, int H, int M, int key_dim, int value_dim, float decay_clamp,
                           int dtype, void* stream);

/* Prologue backward: from float32 gradients of the five outputs (forward
 * output layouts) to float32 gradients of the inputs: dq, dk [B,T,H,key_dim]
 * (summed over the lanes), d_b_proj, d_w_proj, d_decay_proj in their input
 * layouts, d_proj_a, d_proj_b [B,T,H].  Clamps pass the gradient where their
 * input is <= the bound (torch's convention). */
int gdnx_gdn3_prologue_bwd(const void* b_proj, const void* proj_a, const void* w_proj,
                           const void* proj_b, const void* decay_proj, const float* rates,
                           const float* rope_cos, const float* rope_sin, const float* d_q_rope,
                           const float* d_k_rope, const float* d_b_gates, const float* d_w_gates,
                           const float* d_decay, float* dq, float* dk, float* d_b_proj,
                           float* d_proj_a, float* d_w_proj, float* d_proj_b, float* d_decay_proj,
                           int B, int T, int H, int M, int key_dim, int value_dim, float decay_clamp,
                           int dtype, void* stream);

/* Epilogue (gdn3/gdn3_upgrade.py:842-851): y [B,T,H,M,value_dim] (the
 * recurrence output), router_logits [B,T,H,M] (dtype), norm [value_dim]
 * float32 ->
 *   out = u / max(|u|, 1e-6) * sqrt(value_dim) * norm,  u = sum_m softmax_m(logits) y_m
 * [B,T,H,value_dim] in dtype (the tensor _agg_proj receives). */
int gdnx_gdn3_epilogue_fwd(const void* y, const void* router_logits, const float* norm, void* out,
                           int B, int T, int H, int M, int value_dim, int dtype, void* stream);

/* Bytes of the epilogue backward's workspace (per-workgroup partial sums of
 * d_norm, reduced in a fixed order: the result is deterministic). */
long long gdnx_gdn3_epilogue_workspace_bytes(int B, int T, int H, int value_dim);

/* Epilogue backward: d_out [B,T,H,value_dim] (dtype) -> d_y [B,T,H,M,value_dim]
 * (dtype), d_router_logits [B,T,H,M] and d_norm [value_dim] (float32; d_norm
 * is written, not accumulated). */
int gdnx_gdn3_epilogue_bwd(const void* y, const void* router_logits, const float* norm,
                           const void* d_out, void* d_y, float* d_router_logits, float* d_norm,
                           void* workspace, int B, int T, int H, int M, int value_dim, int dtype,
                           void* stream);

/* ---- Rank-r block-Householder delta rule with the RLS T-factor: the scan of
 * KMD2LinearAttn._scan (gdn3/kmd2.py:166-214) and of the testbed mixer
 * (research/testbed_mqar.py:226-262, without its compaction).  Per chain
 * (b, h), state S [value_dim, key_dim] (value-major), per token, R slots:
 *   S <- S diag(a);  Kt = Bg * K;  S <- S - (S Kt^T)(eps I + Kt Kt^T)^-1 Kt
 *   S <- S + (Wg * V)^T K;
 *   (compact_P > 0, after the write of every compact_P-th token, the testbed's
 *    compaction research/testbed_mqar.py:245-260:  S <- s S_lr + (1-s) S, S_lr
 *    the best rank-compact_R approximation of S, s = slow_decay)
 *   y = sum_o mix_o S q_o  (mix = out_mix[h], or 1 when R_out = 1)
 * All tensors float32: q [B,T,H,R_out,key_dim]; K, Bg [B,T,H,R,key_dim];
 * V, Wg [B,T,H,R,value_dim]; a [B,T,H,key_dim]; out_mix [H,R_out];
 * states [B,H,value_dim,key_dim]; y [B,T,H,value_dim].  key_dim 32, 64 or 128;
 * value_dim a multiple of 16 up to 128; R, R_out 1..4 (callers zero-pad
 * other dims: zero key / value columns and a = 1 leave the scan unchanged).
 * Compaction: compact_P even, 1 <= compact_R <= min(key_dim, value_dim) <= 64,
 * key_dim * value_dim <= 4096; the truncation is exact (Jacobi eigensolver of
 * the smaller Gram of S, converged to 1e-12 of its mass). */

/* Bytes of the state checkpoints the backward needs (one state every few
 * tokens per chain, plus the final state). */
long long gdnx_rls_ckpt_bytes(int B, int T, int H, int R, int key_dim, int value_dim, int compact_P);

/* Forward.  state0 (initial state), state_out (final state) and ckpt (the
 * backward's checkpoints, gdnx_rls_ckpt_bytes) may be NULL. */
int gdnx_rls_fwd(const float* q, const float* K, const float* V, const float* Bg, const float* Wg,
                 const float* a, const float* out_mix, const float* state0, float* y, float* state_out,
                 float* ckpt, int B, int T, int H, int R, int R_out, int key_dim, int value_dim,
                 float eps, int compact_P, int compact_R, float slow_decay, void* stream);

/* Backward from dy [B,T,H,value_dim] (and d_state, the gradient of the final
 * state, or NULL) through the forward's checkpoints: gradients of every
 * input in its layout; d_out_mix_seq [B,H,R_out] holds each sequence's share
 * of out_mix's gradient (sum it over B); d_state0 (or NULL) the initial
 * state's.  Through a compaction the gradient is the testbed's: the truncation
 * carries none (it runs under no_grad), so the state's gradient is scaled by
 * 1 - slow_decay; with straight_through != 0 it passes unchanged (the
 * testbed's compact_ste).  Deterministic.  Without compaction and with a
 * workspace (gdnx_rls_bwd_workspace_bytes) the value rows are spread over
 * workgroups (16 rows each) and the column sums reduced by a second kernel;
 * with workspace NULL (or with compaction) one workgroup runs each chain. */
long long gdnx_rls_bwd_workspace_bytes(int B, int T, int H, int R, int key_dim, int value_dim);

int gdnx_rls_bwd(const float* q, const float* K, const float* V, const float* Bg, const float* Wg,
                 const float* a, const float* out_mix, const float* ckpt, const float* dy,
                 const float* d_state, float* dq, float* dK, float* dV, float* dBg, float* dWg,
                 float* da, float* d_out_mix_seq, float* d_state0, int B, int T, int H, int R,
                 int R_out, int key_dim, int value_dim, float eps, int compact_P, int compact_R,
                 float slow_decay, int straight_through, void* workspace, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GDNX_H */

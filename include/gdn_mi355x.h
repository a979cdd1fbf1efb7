/* gdn_mi355x.h: C ABI of the MI355X (gfx950) Gated DeltaNet forward + VJP engine.
 *
 * One delta-rule step per value head h (value head h reads key head h / (Hv/Hk)):
 *   A = S * decay;  r = v - A k;  delta = beta r;  S~ = A + delta (x) k;  y = S~ q;
 *   S_next = mask ? S~ : S            (y always reads the candidate S~)
 * with S the [Dv][Dk] state of one head.  This is the arithmetic of the reference's
 * tools/gdn_vjp.py:3-25 (_step_parts :238-256) and engine/include/gdn.h:27-38 (engine/src/gdn.c:63-108).
 *
 * Layouts (all row-major, contiguous):
 *   q, k    [B][T][Hk][Dk]          dtype in_dtype (GDN_F32 / GDN_BF16 / GDN_F16)
 *   v       [B][T][Hv][Dv]          dtype in_dtype
 *   g       [B][T][Hv]   (GDN_GATE_DECAY, GDN_GATE_LOG)   or [B][T][Hv][Dk] (GDN_GATE_DECAY_VEC, _LOG_VEC), fp32
 *   beta    [B][T][Hv]              fp32
 *   state   [B][Hv][Dv][Dk]         fp32 (initial state S0; NULL means zeros)
 *   mask    [B][T]                  uint8, nonzero keeps the candidate state; NULL means all ones
 *   y, dy   [B][T][Hv][Dv]          dtype out_dtype / dy_dtype
 * Every pointer is a device pointer owned by the caller; nothing is freed or retained.  Calls are
 * asynchronous on `stream` (a hipStream_t, NULL = default stream) and never synchronise the host,
 * except when the environment variable GDN_DEBUG_SYNC=1 asks for a synchronise after every launch.
 *
 * Return codes: 0 ok, negative on error; gdn_last_error() returns a message for the calling thread.
 * This follows the 0 / negative convention of the reference's C API (engine/include/qengine.h:13-14).
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum gdn_status {
    GDN_OK = 0,
    GDN_ERR_INVALID = -1,      /* bad shape, chunk, pointer or enum (reference: ValueError) */
    GDN_ERR_UNSUPPORTED = -2,  /* valid request the library does not implement (e.g. Dk > 256) */
    GDN_ERR_WORKSPACE = -3,    /* workspace smaller than gdn_bwd_workspace_bytes() */
    GDN_ERR_LAUNCH = -4        /* a HIP launch or runtime call failed */
};

enum gdn_dtype { GDN_F32 = 0, GDN_BF16 = 1, GDN_F16 = 2 };

enum gdn_gate {
    GDN_GATE_DECAY = 0,      /* g is the multiplicative decay, [B][T][Hv] (reference convention) */
    GDN_GATE_DECAY_VEC = 1,  /* g is a decay per key channel, [B][T][Hv][Dk] (tools/gdn_vjp.py:174-179) */
    GDN_GATE_LOG = 2,        /* g is the log decay, [B][T][Hv]; dg is returned w.r.t. the log decay */
    GDN_GATE_LOG_VEC = 3     /* g is a log decay per key channel, [B][T][Hv][Dk]; dg w.r.t. the log decay.  No
                              * counterpart in the reference (which takes per-channel gates as decays): the
                              * chunked form's backward is cheaper with it (dg from suffix sums, without the pass
                              * that forms d/d(decay) for GDN_GATE_DECAY_VEC) */
};

enum gdn_form {
    GDN_FORM_AUTO = 0,       /* the chunked form when eligible, else the recurrent form */
    GDN_FORM_RECURRENT = 1,  /* token-sequential recurrence, state rows resident in VGPRs; any shape */
    GDN_FORM_CHUNK = 2       /* chunked WY/UT form on MFMA (64-token tiles); Dk = Dv = 128, scalar gate; a mask runs
                                two chunked passes (see below) */
};

/* Library version, (major << 16) | minor. */
int gdn_version(void);

/* Message for the last non-zero status returned on the calling thread ("" if none). */
const char *gdn_last_error(void);

/* Benchmark support, no counterpart in the reference (which has no kernel-level timing): while enabled,
 * every launch is bracketed by two HIP events recorded on the launch's stream.  gdn_profile_collect waits
 * for the recorded events, writes up to max_entries distinct kernel names (name_len bytes each), their
 * summed milliseconds and launch counts, clears the records and returns the number of entries (< 0 on
 * error). */
int gdn_profile_enable(int on);
int gdn_profile_collect(int max_entries, char *names, int name_len, double *total_ms, int *counts);

/* Number of chunk snapshots the recurrent form keeps: ceil(T / chunk) - 1 states of [B][Hv][Dv][Dk] fp32, the
 * states at token chunk, 2*chunk, ... (the reference keeps the same boundaries, tools/gdn_vjp.py:205-235; the
 * first, S0, is the caller's input and the last is the returned final state). */
int64_t gdn_num_snapshots(int T, int chunk);

/* The form a call with these arguments runs in (GDN_FORM_RECURRENT or GDN_FORM_CHUNK), or < 0 when the
 * requested form cannot run them.  gdn_fwd, gdn_bwd and the size queries resolve the form the same way: GDN_FORM_AUTO
 * picks the chunked form for Dk = Dv = 128 with a scalar gate (with a mask: Hv <= 256) or with one gate per key
 * channel (GDN_GATE_DECAY_VEC or GDN_GATE_LOG_VEC: bf16 inputs, no mask); the recurrent form otherwise.  Decays
 * of any size, zeros included, hold the same bars on both forms (the chunked form takes decays below 2^-64 as
 * 2^-64). */
int gdn_select_form(int Hv, int Dk, int Dv, int has_mask, int gate_kind, int form, int in_dtype);

/* What `chunk` means.
 *   Recurrent form: the forward keeps the state every `chunk` tokens (gdn_num_snapshots) and the backward replays
 *   each chunk from its snapshot.
 *   Chunked form (WY/UT, 64-token MFMA tiles whatever `chunk` is):
 *     chunk <= 64  the forward keeps every 64-token tile the backward reads (fastest; the saved buffer grows with
 *                  T at about 3.2 KiB (bf16) / 4.2 KiB (fp32) per head-token);
 *     chunk > 64   checkpointing (tools/gdn_checkpoint.py:39-50): windows of W = chunk rounded up to a multiple of
 *                  64 tokens; the forward keeps only the ceil(T / W) - 1 fp32 states at the window boundaries, and
 *                  the backward rebuilds the tiles of one group of windows at a time from them.
 *   A forward-only call (saved = NULL) of the chunked form keeps nothing and runs group by group in the workspace.
 * Group-wise calls use the largest group of windows (or of 64-token chunks, forward-only) that fits the workspace
 * given, up to the size the *_workspace_bytes queries return; fewer groups is faster, one window (chunk) is the
 * minimum. */

/* Masks on the chunked form.  A masked step keeps the state but its output reads the candidate state.  The chunked
 * form runs the recurrence with decay 1 and beta 0 at masked tokens (the same states), once with q and once with k as
 * the query, and rewrites y at masked tokens as decay y' + beta (k . q) (v - decay z) from the two outputs; the
 * backward runs both passes' backwards and the rewrite's VJP.  Needs Hv <= 256; the saved buffer holds both passes
 * (checkpointing: pass 1's snapshots serve both) plus fp32 [B][T][Hv][Dv] copies of the two outputs. */

/* Size of the buffer gdn_fwd fills for gdn_bwd (the "saved" activations) for inputs of in_dtype. */
size_t gdn_saved_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind, int has_mask,
                       int form, int in_dtype);

/* Device workspace gdn_fwd uses during the call (released afterwards), with or without a saved buffer; 0 when the
 * call needs none (the recurrent form; the chunked form with chunk <= 64 and a saved buffer). */
size_t gdn_fwd_workspace_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind, int has_mask,
                               int form, int in_dtype, int with_saved);

/* Forward.  Replaces the forward of gated_delta_chunked (tools/gdn_vjp.py:503-528 via _forward :205-235)
 * and of gated_delta_ops_checkpointed (tools/gdn_checkpoint.py:53-95).
 * Writes y (out_dtype), state_T (fp32; may be NULL) and, when saved is not NULL, the gdn_saved_bytes()
 * buffer gdn_bwd reads.  saved = NULL is the forward-only path of frozen layers (tools/frozen_gdn.py:19-25,
 * mlx-lm gated_delta_kernel): nothing is kept.  workspace: gdn_fwd_workspace_bytes() bytes (256-byte aligned),
 * or NULL when that is 0. */
int gdn_fwd(const void *q, const void *k, const void *v, const float *g, const float *beta,
            const float *state0, const uint8_t *mask,
            void *y, float *state_T, void *saved, size_t saved_bytes, void *workspace, size_t workspace_bytes,
            int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk,
            int in_dtype, int out_dtype, int gate_kind, int form, void *stream);

/* gdn_fwd without a saved buffer (the forward-only call) that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Its group buffers live in a fixed 64 MiB device array, one per
 * GPU, held until the process ends; results equal gdn_fwd's.  The chunked form needs one 64-token group of all
 * B * Hv heads to fit (B * Hv up to about 300); larger calls return GDN_ERR_UNSUPPORTED.  Calls that overlap on
 * one GPU (other streams or threads) share the array and race; calls on one stream are ordered. */
int gdn_fwd_noalloc(const void *q, const void *k, const void *v, const float *g, const float *beta,
                    const float *state0, const uint8_t *mask, void *y, float *state_T, int B, int T, int Hk, int Hv,
                    int Dk, int Dv, int in_dtype, int out_dtype, int gate_kind, int form, void *stream);

/* One decode step: the recurrence over a single token of B sequences, replacing gdn_recurrent_step
 * (engine/include/gdn.h:27-38, engine/src/gdn.c:63-108) batched over sequences.
 *   q, k [B][Hk][Dk], v [B][Hv][Dv] (in_dtype); g, beta [B][Hv] (g as gate_kind: GDN_GATE_DECAY, GDN_GATE_LOG,
 *   or [B][Hv][Dk] for GDN_GATE_DECAY_VEC, GDN_GATE_LOG_VEC) fp32; y [B][Hv][Dv] (out_dtype);
 *   state_in, state_out [B][Hv][Dv][Dk] fp32: state_out may be state_in (updated in place, as gdn_recurrent_step
 *   does); state_in NULL means zeros.
 * Forward only; any Dk <= 256 and Dv. */
int gdn_decode_step(const void *q, const void *k, const void *v, const float *g, const float *beta,
                    const float *state_in, float *state_out, void *y, int B, int Hk, int Hv, int Dk, int Dv,
                    int in_dtype, int out_dtype, int gate_kind, void *stream);

/* Device workspace gdn_bwd needs, in bytes (256-byte aligned base expected). */
size_t gdn_bwd_workspace_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind,
                               int has_mask, int form, int in_dtype);

/* Backward (VJP).  Replaces _backward / _chunk_vjp / the Metal kernel gdn_chunk_backward
 * (tools/gdn_vjp.py:273-320, :341-423, :426-474) and the mx.checkpoint recompute of
 * tools/gdn_checkpoint.py:39-50.  Reads the saved buffer gdn_fwd wrote with the same arguments, recomputes
 * the states inside each chunk, and writes
 *   dq, dk [B][T][Hk][Dk] (grad_dtype; summed over the value heads of each key head, tools/gdn_vjp.py:266-270)
 *   dv     [B][T][Hv][Dv] (grad_dtype)
 *   dg     shaped like g, fp32 (w.r.t. the log decay for GDN_GATE_LOG and GDN_GATE_LOG_VEC)
 *   dbeta  [B][T][Hv] fp32
 *   dstate0 [B][Hv][Dv][Dk] fp32 (may be NULL)
 * dy has dy_dtype; dstate_T may be NULL (zero cotangent).  Results are deterministic (no atomics).
 * The chunked form needs 16-byte aligned q, k, v, dy, dq, dk and dv, and with bf16 inputs a bf16 or fp32 dy. */
int gdn_bwd(const void *q, const void *k, const void *v, const float *g, const float *beta,
            const float *state0, const uint8_t *mask, const void *saved, size_t saved_bytes,
            const void *dy, const float *dstate_T,
            void *dq, void *dk, void *dv, float *dg, float *dbeta, float *dstate0,
            void *workspace, size_t workspace_bytes,
            int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk,
            int in_dtype, int dy_dtype, int grad_dtype, int gate_kind, int form, void *stream);

/* ---------------------------------------------------------------------------------------------------------
 * Block ops around the recurrence: the steps of one GDN block (engine/src/gdn_layer.c:29-55) over a whole
 * sequence, each with its backward.  Tensors are contiguous; `tokens` = B*T.  Parameter gradients are reduced
 * deterministically (no atomics) through a caller workspace of the size the matching *_workspace_bytes call
 * returns.  Kernels use 8/16-byte vector loads when every tensor is 16-byte aligned and the row length allows,
 * and element loads otherwise; results do not depend on which path runs beyond fp32 rounding.
 * --------------------------------------------------------------------------------------------------------- */

/* Gates, replacing gdn_gates (engine/include/gdn.h:20-25) over all tokens:
 *   a, b [tokens][Hv] (in_dtype);  A_log, dt_bias [Hv] fp32;  g, beta [tokens][Hv] fp32 outputs
 *   log decay  l = -exp(A_log[h]) * softplus(a + dt_bias[h]),  softplus(t) = t > 20 ? t : log1p(exp(t))
 *   g = log_space ? l : exp(l)          (log_space = the log-decay convention of GDN_GATE_LOG)
 *   beta = s / (1 + exp(-b)),  s = 2 when allow_neg_eigval (mlx-lm gated_delta_update), else 1
 * Hv <= 256. */
int gdn_gates_fwd(const void *a, const void *b, const float *A_log, const float *dt_bias, float *g, float *beta,
                  int64_t tokens, int Hv, int in_dtype, int log_space, int allow_neg_eigval, void *stream);

size_t gdn_gates_bwd_workspace_bytes(int64_t tokens, int Hv);

/* Backward of gdn_gates_fwd.  g is the forward output; dg is the cotangent of g (w.r.t. the decay, or the log
 * decay when log_space); dbeta of beta.  Writes da, db [tokens][Hv] (grad_dtype) and dA_log, ddt_bias [Hv]
 * fp32 (summed over tokens). */
int gdn_gates_bwd(const void *a, const void *b, const float *A_log, const float *dt_bias, const float *g,
                  const float *dg, const float *dbeta, void *da, void *db, float *dA_log, float *ddt_bias,
                  void *workspace, size_t workspace_bytes, int64_t tokens, int Hv, int in_dtype, int grad_dtype,
                  int log_space, int allow_neg_eigval, void *stream);

/* Per-row L2 norm, replacing gdn_l2norm (engine/include/gdn.h:17-18; applied per head with scale
 * 1/sqrt(Dk) for q and 1 for k, engine/src/gdn_layer.c:35-39):
 *   y = scale * x / sqrt(sum x^2 + eps)  over rows of D elements;  x, y [rows][D] (dtype); y may equal x. */
int gdn_l2norm_fwd(const void *x, void *y, int64_t rows, int D, float eps, float scale, int dtype, void *stream);

/* dx = scale/n (dy - x (x.dy)/n^2), n = sqrt(sum x^2 + eps);  dx has dtype, dy has dy_dtype. */
int gdn_l2norm_bwd(const void *x, const void *dy, void *dx, int64_t rows, int D, float eps, float scale, int dtype,
                   int dy_dtype, void *stream);

/* Causal depthwise conv + SiLU over a whole sequence, replacing T calls of gdn_conv_step
 * (engine/include/gdn.h:7-15):
 *   x, out [B][T][C] (dtype);  w [C][K] fp32 (w[c*K + K-1] multiplies the current input);  2 <= K <= 8
 *   out[b,t,c] = silu( sum_j w[c*K + j] * x[b, t-(K-1)+j, c] ),  x before t = 0 taken from state_in
 *   state_in  [B][K-1][C] fp32, oldest input first, or NULL for zeros (a fresh state)
 *   state_out [B][K-1][C] fp32, the last K-1 inputs after the sequence, or NULL; must not alias state_in. */
int gdn_conv_silu_fwd(const void *x, const float *w, const float *state_in, void *out, float *state_out, int B,
                      int T, int C, int K, int dtype, void *stream);

size_t gdn_conv_silu_bwd_workspace_bytes(int B, int T, int C, int K);

/* Backward of gdn_conv_silu_fwd (no gradient w.r.t. state_in): dx [B][T][C] (dtype), dw [C][K] fp32. */
int gdn_conv_silu_bwd(const void *x, const float *w, const float *state_in, const void *dout, void *dx, float *dw,
                      void *workspace, size_t workspace_bytes, int B, int T, int C, int K, int dtype, int dout_dtype,
                      void *stream);

/* Conv + SiLU fused with the split into q, k, v and the per-head L2 norm of q and k: steps 2-4 of one block
 * (engine/src/gdn_layer.c:29-39, gdn_conv_step then gdn_l2norm per head) in one pass over the sequence.
 *   x [B][T][C], C = 2*Hk*Dk + Hv*Dv, channels [0, Hk*Dk) are q, [Hk*Dk, 2*Hk*Dk) k, the rest v;
 *   q, k [B][T][Hk][Dk] and v [B][T][Hv][Dv] (dtype) receive silu(conv(x)), q scaled by
 *   q_scale / sqrt(sum q_h^2 + eps) and k by 1 / sqrt(sum k_h^2 + eps) per head;
 *   w, state_in, state_out as gdn_conv_silu_fwd.
 * Needs K = 4, 16-byte aligned buffers, C % 4 == 0 and Dk / 8 (16-bit data; Dk / 4 for fp32) a power of two in
 * [4, 64]; other shapes return GDN_ERR_UNSUPPORTED (compose gdn_conv_silu_fwd and gdn_l2norm_fwd instead). */
int gdn_conv_qkv_fwd(const void *x, const float *w, const float *state_in, void *q, void *k, void *v,
                     float *state_out, int B, int T, int Hk, int Dk, int Hv, int Dv, int K, float q_scale, float eps,
                     int dtype, void *stream);

/* Backward of gdn_conv_qkv_fwd from the cotangents dq, dk, dv of its outputs (g_dtype): dx [B][T][C] (dtype) and
 * dw [C][K] fp32; workspace of gdn_conv_silu_bwd_workspace_bytes(B, T, C, K) bytes. */
int gdn_conv_qkv_bwd(const void *x, const float *w, const float *state_in, const void *dq, const void *dk,
                     const void *dv, void *dx, float *dw, void *workspace, size_t workspace_bytes, int B, int T,
                     int Hk, int Dk, int Hv, int Dv, int K, float q_scale, float eps, int dtype, int g_dtype,
                     void *stream);

/* Gated RMSNorm, replacing op_rmsnorm + op_silu_mul per value head (engine/include/ops.h:7-11,
 * engine/src/gdn_layer.c:47-55):
 *   out = y / sqrt(mean(y^2) + eps) * w * silu(z)   over rows of D;  y, out [rows][D] (dtype), z (z_dtype),
 *   w [D] fp32. */
int gdn_gated_rmsnorm_fwd(const void *y, const void *z, const float *w, void *out, int64_t rows, int D, float eps,
                          int dtype, int z_dtype, void *stream);

size_t gdn_gated_rmsnorm_bwd_workspace_bytes(int64_t rows, int D);

/* Backward: dy (dtype), dz (z_dtype), dw [D] fp32 (summed over rows); D <= 4096. */
int gdn_gated_rmsnorm_bwd(const void *y, const void *z, const float *w, const void *dout, void *dy, void *dz,
                          float *dw, void *workspace, size_t workspace_bytes, int64_t rows, int D, float eps,
                          int dtype, int z_dtype, int dout_dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif

/*
 * kda_hip.h -- C ABI of the gfx950 KDA (Kimi Delta Attention / gated delta
 * rule) chunkwise WY recurrence.
 *
 * Layouts (all contiguous, row-major):
 *   q, k, v, g, o, dq, dk, dv, dg, dout   [B, T, H, D]
 *   beta, dbeta                            [B, T, H]
 *   s0, s_final, ds_final, ds0             [B, H, D, D] fp32, reference
 *                                          orientation S[i_v][j_k] (o_t = S_t q_t)
 * dtype / g_dtype: 0 = fp32, 1 = bf16 (raw bfloat16 bits).  q, k, v, beta, o
 * and dq, dk, dv, dbeta use `dtype`; g and dg use `g_dtype` (or, with g_dtype
 * KDA_G_HEAD_F32, are fp32 [B, T, H]: one decay per head).  Arithmetic is
 * fp32 with an fp32 state; bf16 inputs use bf16 MFMA operands.
 * chunk is the reference's chunk_size: 8, 16, 32 or 64 (nope_gdn_mlx.py:676,
 * 4839-4856); the result does not depend on it (the reference's own
 * equivalence criterion, nope_gdn_mlx.py:4836-4914), and the kernels block at
 * 64 whatever its value.  D must be 32, 64, 96 or 128 (96 runs the D = 128
 * kernels with channels 96..127 zero; o, the states and the backward's dout
 * pass through zero-padded copies in the workspace).
 * stream is a hipStream_t (NULL = default stream).  Every call is stream
 * ordered and allocates nothing: the caller passes a device workspace of at
 * least kda_workspace_size() bytes (256-byte aligned).
 *
 * Return codes: 0 ok, KDA_E_* < 0 on error; kda_last_error() then describes
 * the failure (thread-local).  Argument checks happen before any device work.
 */
#ifndef KDA_HIP_H
#define KDA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_OK 0
#define KDA_E_INVALID (-1)      /* null pointer, negative size, misalignment */
#define KDA_E_UNSUPPORTED (-2)  /* chunk, D or dtype outside what the kernels support */
#define KDA_E_WORKSPACE (-3)    /* workspace smaller than kda_workspace_size() */
#define KDA_E_HIP (-4)          /* a HIP launch or runtime call failed */

#define KDA_DTYPE_F32 0
#define KDA_DTYPE_BF16 1
/* g_dtype only: g is fp32 [B, T, H], one decay per (b, t, h) shared by the
 * head's D channels (the scalar-alpha GDN, g = log alpha; the reference's
 * _gdn_step_fused, nope_gdn_mlx.py:641-650), and dg is fp32 [B, T, H], the
 * sum over the channels.  bf16 operands at D = 32 or 64 only. */
#define KDA_G_HEAD_F32 2

#define KDA_PASS_FWD 0
#define KDA_PASS_BWD 1
#define KDA_PASS_TRAIN 2   /* kda_fwd_train + kda_bwd_train share one workspace */

/* Workspace regions (see kda_workspace_offsets).  SEGX, SEGM and SEGS exist
 * only at bf16 D = 128 when the sequence is split into segments: per (b, h,
 * segment) the segment's state map and start state, for the forward (pass 0,
 * at least 8 segments or segments of 32 or more chunks) and for the
 * backward's state recompute and reverse carry (passes 1 and 2, at least 8
 * segments; in pass 2 among the backward's own regions).
 * PAD and PADB exist only at D = 96, which runs the D = 128 kernels with
 * channels 96..127 zero: the other regions are then those of D = 128; PAD
 * holds the padded s0 (and, for the forward passes, o and s_final), PADB the
 * backward's padded dout, ds_final and ds0.
 * Order: passes 0 and 1 lay the regions out in this order.  Pass 2 puts first
 * the regions kda_fwd_train writes and kda_bwd_train reads (the kept part,
 * kda_train_kept_size bytes: W .. EG and PAD) and after them those only the
 * backward uses (H, DH, VP, DVP, SEGX, SEGM, SEGS, PADB), so that the
 * backward's part can be a buffer of its own (kda_bwd_train_split). */
enum kda_ws_region {
    KDA_WS_W = 0, KDA_WS_U, KDA_WS_QP, KDA_WS_QPT, KDA_WS_KB, KDA_WS_KBT, KDA_WS_WT,
    KDA_WS_AQK, KDA_WS_AQKT, KDA_WS_AKK, KDA_WS_TII, KDA_WS_EG, KDA_WS_H, KDA_WS_DH,
    KDA_WS_VP, KDA_WS_DVP, KDA_WS_SEGX, KDA_WS_SEGM, KDA_WS_SEGS, KDA_WS_PAD, KDA_WS_PADB,
    KDA_WS_NREGIONS
};

/* ABI version of this header (bumped on any signature change). */
int kda_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* kda_last_error(void);

/* Bytes of workspace kda_fwd (pass 0), kda_bwd (pass 1) or the training pair
 * kda_fwd_train / kda_bwd_train (pass 2) needs; 0 on invalid arguments (see
 * kda_last_error). */
size_t kda_workspace_size(int pass, int B, int T, int H, int D, int chunk, int dtype);

/* Byte offsets of the workspace regions for a pass (-1 = unused), so tests can
 * inspect intermediates.  offsets must hold KDA_WS_NREGIONS entries. */
int kda_workspace_offsets(int pass, int B, int T, int H, int D, int chunk, int dtype,
                          int64_t* offsets);

/* Bytes at the start of the training pair's (pass 2) workspace that
 * kda_fwd_train writes and kda_bwd_train reads -- the per-chunk factors (and,
 * at D = 96, the padded s0) -- all a caller must keep between the two
 * calls; 0 on invalid arguments.  Where the training forward runs over
 * segments (bf16, D = 128 or 96; the plan of kda_fwd) the kept part ends with
 * that forward's segment temporaries, which kda_workspace_offsets does not
 * name and the backward does not read.  The rest of kda_workspace_size(2, ...) is
 * the backward's own scratch (the chunk-boundary states and their adjoints,
 * V' and dV'), which kda_bwd_train_split takes as a separate buffer.  No
 * counterpart in the reference, whose forward keeps U_traj and S_traj
 * (nope_gdn_mlx.py:2734-2745): it serves autograd callers that hold only what
 * the backward needs from the forward. */
size_t kda_train_kept_size(int B, int T, int H, int D, int chunk, int dtype);

/* Forward: o and (if s_final != NULL) the final state.  s0 == NULL means a zero
 * initial state.
 * Replaces GatedDeltaLayer._chunkwise_kda_forward (nope_gdn_mlx.py:2318-2456)
 * and the forward of _chunkwise_kda_vjp_path (nope_gdn_mlx.py:2829-2865), with
 * heads kept in place instead of folded; same result as _loop_compiled_kda
 * (nope_gdn_mlx.py:890-917). */
int kda_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
            const float* s0, void* o, float* s_final,
            int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
            void* workspace, size_t ws_bytes, void* stream);

/* Backward (VJP): gradients of <o, dout> + <s_final, ds_final> with respect to
 * q, k, v, g, beta and s0.  ds_final == NULL means zero; ds0 may be NULL.
 * Chunk-boundary states are recomputed; nothing is kept from kda_fwd.
 * Replaces the VJP of _get_chunkwise_kda_recurrence_fn (nope_gdn_mlx.py:2746-2808)
 * and _chunkwise_kda_backward (nope_gdn_mlx.py:2579-2720). */
int kda_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
            const float* s0, const void* dout, const float* ds_final,
            void* dq, void* dk, void* dv, void* dg, void* dbeta, float* ds0,
            int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
            void* workspace, size_t ws_bytes, void* stream);

/* kda_fwd without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The kernels of
 * kda_fwd run on a static device array of KDA_NOALLOC_MAX_WORKSPACE bytes that
 * the library holds on each GPU it runs on until the process ends; no call
 * allocates or frees anything.  Shapes whose kda_fwd workspace
 * (kda_workspace_size(KDA_PASS_FWD, ...)) exceeds that size are rejected with
 * KDA_E_WORKSPACE before any device work (128 MiB: config 1, B8 H12 T1568 D64
 * bf16, needs 98.9 MB).  Results are bit-identical to kda_fwd.  Every call on
 * one GPU shares that GPU's array, so calls that overlap on one GPU (on
 * different streams, or from several threads without ordering) race;
 * stream-ordered calls on one stream do not.
 * The array used is that of the stream's device (the current device for the
 * NULL stream); q, k, v, g, beta, o and the states must be device memory of
 * that device, or the call returns KDA_E_INVALID before any device work. */
#define KDA_NOALLOC_MAX_WORKSPACE ((size_t)128 << 20)
int kda_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                    const float* s0, void* o, float* s_final,
                    int B, int T, int H, int D, int chunk, int dtype, int g_dtype, void* stream);

/* Training pair.  kda_fwd_train computes what kda_fwd computes and also keeps,
 * in its (pass 2) workspace, every per-chunk factor the backward needs: W, U,
 * the decay-scaled Q / K operands and their transposes, A_qk and its transpose,
 * e^G (with fp32 inputs also A_kk and the inverted diagonal blocks of I + L).
 * No state is kept: kda_bwd_train recomputes the chunk-boundary states from
 * the factors and s0.  At D = 96 the pair's workspace also keeps the padded
 * s0 for the backward.
 * kda_fwd_train needs ws_bytes >= kda_train_kept_size (it writes nothing past
 * that); kda_bwd_train needs the whole pass-2 workspace, kda_workspace_size(2).
 * kda_bwd_train is kda_bwd without its prep: it requires the workspace that
 * kda_fwd_train filled for the same q, k, v, g, beta and s0 (and the same B,
 * T, H, D, dtype), unmodified in between, and returns the same gradients as
 * kda_bwd.
 * Replace the forward of _get_chunkwise_kda_recurrence_fn, which keeps U_traj
 * and S_traj for its VJP (nope_gdn_mlx.py:2734-2745), and that VJP
 * (nope_gdn_mlx.py:2746-2808) consuming them. */
int kda_fwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const float* s0, void* o, float* s_final,
                  int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                  void* workspace, size_t ws_bytes, void* stream);
int kda_bwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const float* s0, const void* dout, const float* ds_final,
                  void* dq, void* dk, void* dv, void* dg, void* dbeta, float* ds0,
                  int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                  void* workspace, size_t ws_bytes, void* stream);

/* kda_bwd_train with the backward's scratch in a buffer of its own: kept is
 * the workspace kda_fwd_train filled (kept_bytes >= kda_train_kept_size),
 * scratch any 256-byte aligned device buffer of scratch_bytes >=
 * kda_workspace_size(2, ...) - kda_train_kept_size(...) (its contents are
 * not read; NULL when that difference is 0).  Same gradients as kda_bwd_train,
 * bit for bit.  No counterpart in the reference (see kda_train_kept_size): for
 * autograd callers that keep only the forward's factors between the passes. */
int kda_bwd_train_split(const void* q, const void* k, const void* v, const void* g, const void* beta,
                        const float* s0, const void* dout, const float* ds_final,
                        void* dq, void* dk, void* dv, void* dg, void* dbeta, float* ds0,
                        int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                        const void* kept, size_t kept_bytes, void* scratch, size_t scratch_bytes,
                        void* stream);

/* Forward (pass KDA_PASS_FWD, workspace as kda_fwd) or training forward
 * (KDA_PASS_TRAIN, as kda_fwd_train) with the layer's output norm fused into
 * the store of o: besides o and the final state it writes
 *     y = o * rsqrt(mean_d o^2 + eps) * norm_w * sigmoid(z)
 * per head of D channels, y and z [B, T, *] with row strides ld_y and ld_z
 * (elements, multiples of 16 bytes; head h at column h*D), z and y in dtype,
 * norm_w fp32 [D].  o is still written: the norm's backward
 * (kda_layer_gated_rmsnorm_bwd) reads it.  Supported: bf16 with D = 64, fp32
 * with D in {32, 64} (KDA_E_UNSUPPORTED otherwise).
 * Replaces the recurrence call and the following RMSNormGated of
 * GatedDeltaLayer.__call__ (nope_gdn_mlx.py:823-885, RMSNormGated
 * nope_gdn_mlx.py:340-366): o_norm(o, gate) applied to the path's output. */
int kda_fwd_gated(int pass, const void* q, const void* k, const void* v, const void* g,
                  const void* beta, const float* s0, const void* z, int64_t ld_z,
                  const float* norm_w, float eps, void* o, void* y, int64_t ld_y, float* s_final,
                  int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                  void* workspace, size_t ws_bytes, void* stream);

/* y = M^-1 b for unit-triangular M (only the strict lower, or with upper != 0
 * the strict upper, part of M is read); M [BH, Cm, Cm], b and y [BH, Cm, N],
 * fp32, 1 <= Cm <= 64, N >= 1.
 * Replaces GatedDeltaLayer._metal_solve_triangular (nope_gdn_mlx.py:1160-1196)
 * and _metal_solve_triangular_upper (nope_gdn_mlx.py:1261-1286). */
int kda_solve_unit_triangular(const float* M, const float* b, float* y, int BH, int Cm, int N,
                              int upper, void* stream);

/* ---- GatedDeltaLayer ends around the recurrence ----
 * The layer turns its projections into the recurrence's inputs and its
 * output back into the residual stream (nope_gdn_mlx.py:796-885).  These
 * entry points replace the element-wise parts of that path; the projections
 * themselves stay plain GEMMs.  dtype (0 fp32, 1 bf16) is that of every
 * activation; g_dtype that of g and dg; parameters and their gradients are
 * fp32.  Row strides (ld_*) are in elements, multiples of 4; activation
 * pointers must be 8-byte (bf16) or 16-byte (fp32) aligned.  HD = H * D must
 * be a multiple of 4 and at most 2048.
 *
 * Producer (GatedDeltaLayer.__call__, nope_gdn_mlx.py:796-821, with
 * ShortCausalConv1d nope_gdn_mlx.py:369-431 and l2_normalize / softplus
 * nope_gdn_mlx.py:77-86), per row (b, t):
 *   q = l2norm(silu(conv4(xq))) * scale, k = l2norm(silu(conv4(xk))),
 *   v = silu(conv4(xv)), g = -exp(A_log[h]) * softplus(xf + dt_bias),
 *   beta = sigmoid(xb) * beta_mult (2 for allow_neg_eigval, else 1).
 * conv4 is the causal depthwise convolution of the 4 taps conv_w[i][c][0..3]
 * (tap 3 multiplies row t, tap 0 row t - 3) plus conv_b[i][c]; l2norm spans
 * the whole HD row (eps 1e-12), as the reference normalises before splitting
 * heads.
 *   xq, xk, xv  [B, T, HD] rows of ld_x; xf [B, T, HD] rows of ld_f;
 *   xb [B, T, H] rows of ld_b; conv_w [3][HD][4] (q, k, v);
 *   conv_b [3][HD] or NULL (no bias); dt_bias [HD]; A_log [H];
 *   q, k, v, g [B, T, H, D] contiguous; beta [B, T, H] contiguous.
 * For the scalar-alpha layer (channel_wise_decay=False) xf, dt_bias, A_log and
 * g are all NULL and no decay gate is formed. */
int kda_layer_producer_fwd(const void* xq, const void* xk, const void* xv, const void* xf, const void* xb,
                           int64_t ld_x, int64_t ld_f, int64_t ld_b,
                           const float* conv_w, const float* conv_b, const float* dt_bias, const float* A_log,
                           void* q, void* k, void* v, void* g, void* beta,
                           int B, int T, int H, int D, float scale, float beta_mult, int dtype, int g_dtype,
                           void* stream);
/* Adjoint of kda_layer_producer_fwd.  dq, dk, dv, dg [B, T, H, D] and dbeta
 * [B, T, H] contiguous in; dxq, dxk, dxv rows of ld_dx, dxf rows of ld_df,
 * dxb rows of ld_db out (they may be column slices of one fused buffer).
 * Parameter gradients are written, not accumulated: dconv_w [3][HD][4],
 * dconv_b [3][HD] (NULL iff conv_b is NULL), ddt_bias [HD], dA_log [H].
 * workspace: at least kda_layer_workspace_size(KDA_LAYER_PRODUCER, ...) bytes,
 * 16-byte aligned.  The gradients are deterministic.  Without a decay gate
 * (xf NULL) dg, dxf, ddt_bias and dA_log are NULL too. */
int kda_layer_producer_bwd(const void* xq, const void* xk, const void* xv, const void* xf, const void* xb,
                           int64_t ld_x, int64_t ld_f, int64_t ld_b,
                           const float* conv_w, const float* conv_b, const float* dt_bias, const float* A_log,
                           const void* dq, const void* dk, const void* dv, const void* dg, const void* dbeta,
                           void* dxq, void* dxk, void* dxv, void* dxf, void* dxb,
                           int64_t ld_dx, int64_t ld_df, int64_t ld_db,
                           float* dconv_w, float* dconv_b, float* ddt_bias, float* dA_log,
                           int B, int T, int H, int D, float scale, float beta_mult, int dtype, int g_dtype,
                           void* workspace, size_t ws_bytes, void* stream);

/* Gated RMSNorm (RMSNormGated, nope_gdn_mlx.py:340-366, applied per head at
 * nope_gdn_mlx.py:880-885): y = o * rsqrt(mean_d(o^2) + eps) * w * sigmoid(z)
 * over each head's D channels.  o [rows, H, D] contiguous; z rows of ld_z;
 * y rows of ld_y; w [D] fp32.  D must be a multiple of 4 in [4, 256] and
 * H * D at most 2048; a head takes D / 4 lanes rounded up to a power of two,
 * and H heads must fit 8 waves of 64 lanes (D = 96: H <= 16). */
int kda_layer_gated_rmsnorm_fwd(const void* o, const void* z, int64_t ld_z, const float* w,
                                void* y, int64_t ld_y, int rows, int H, int D, float eps, int dtype,
                                void* stream);
/* Adjoint: dy rows of ld_dy in; dout [rows, H, D] contiguous, dz rows of
 * ld_dz and dw [D] (written, not accumulated) out.  workspace: at least
 * kda_layer_workspace_size(KDA_LAYER_RMSNORM, ...) bytes with B = 1, T = rows. */
int kda_layer_gated_rmsnorm_bwd(const void* o, const void* z, int64_t ld_z, const float* w,
                                const void* dy, int64_t ld_dy, void* dout, void* dz, int64_t ld_dz, float* dw,
                                int rows, int H, int D, float eps, int dtype,
                                void* workspace, size_t ws_bytes, void* stream);

#define KDA_LAYER_PRODUCER 0
#define KDA_LAYER_RMSNORM 1
size_t kda_layer_workspace_size(int which, int B, int T, int H, int D);

/* ---- launch timing (instrumentation; no counterpart in the reference) ----
 * With profiling on, every kernel launch made by kda_fwd / kda_bwd (and each
 * kda_layer_* call) is bracketed by two HIP events recorded on the launch
 * stream.  Used by the benchmark to measure per-kernel durations live; the
 * kernels do the same work either way.  Kernel ids: 0 prep (forward),
 * 1 recurrence (forward), 2 prep (backward), 3 state recompute, 4 reverse
 * state recurrence, 5 local adjoints, 6 prep (training forward), 7 layer
 * producer (forward), 8 layer producer (backward, with its parameter-gradient
 * reduction), 9 gated RMSNorm (forward), 10 gated RMSNorm (backward, with its
 * reduction), 11-13 the segmented forward at D = 128 (bf16): 11 segment maps,
 * 12 segment start states, 13 the forward of every segment; 14 the backward's
 * state recompute and reverse carry in one launch (bf16 D = 128 without
 * segments: then ids 3 and 4 record nothing).
 * kda_profile_read must be called after the streams have completed. */
#define KDA_PROF_NKERNELS 15
int kda_profile_enable(int on);              /* 1: clear records and start; 0: stop */
const char* kda_profile_name(int id);
int kda_profile_read(int id, double* total_ms, int* launches);

#ifdef __cplusplus
}
#endif

#endif /* KDA_HIP_H */

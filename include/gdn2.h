/*
 * gdn2.h -- C ABI of the MI355X (gfx950) GDN-2 forward path and its chunked
 * backward.
 *
 * The entry points replace burn-gdn2's backend-gated kernel launchers:
 *
 *   gdn2_recurrent_step_f32  <- fused_step            src/kernel/fused_recurrent_cube.rs:108-172
 *   gdn2_chunk_fwd_f32       <- fused_chunk_forward   src/kernel/chunk_cube.rs:781-952
 *                               (and the tensor path chunk_wy_forward, src/forward.rs:44-278,
 *                                which is the only live chunk path in the reference)
 *   gdn2_chunk_fwd_states_f32   the same, with fused_chunk_forward's v_new and states
 *   gdn2_chunk_bwd_f32       <- fused_chunk_backward  src/kernel/chunk_adjoint_cube.rs:464-707
 *                               (gradients of the chunked forward; the reference's training
 *                                path otherwise takes them through autodiff)
 *   gdn2_decode_fused_f32    <- GatedDeltaNet2::forward at T == 1 between project() and
 *                               o_proj: short conv (src/short_conv.rs:22-65), gates
 *                               (src/module.rs:417-443), L2 norm (src/l2norm.rs:13-16),
 *                               the step, rms_norm_gate_per_head (src/module.rs:501-517)
 *   gdn2_short_conv_f32, gdn2_l2_normalize_f32, gdn2_rms_norm_gate_f32
 *                            <- short_conv_1d, l2_normalize(_4d), rms_norm_gate_per_head
 *                               (src/lib.rs:58-62)
 *   gdn2_hip_available       <- is_cuda / CudaBare TypeId gate
 *                               src/kernel/fused_recurrent_cube.rs:74-78
 *
 * Status GDN2_NOT_APPLICABLE plays the role of the reference's `None`: the
 * shapes or layout are outside what the kernels take, nothing was launched,
 * and the caller uses its own tensor path.  Every pointer is a device
 * pointer owned by the caller; no entry point allocates device memory except
 * where stated.  Launches are asynchronous on `stream` (NULL = the default
 * stream) and the calls are re-entrant across streams.
 *
 * Layout of strided operands: the last (channel) dimension is contiguous;
 * strides are in elements for (batch, head, time).  The reference's
 * contiguous [B, H, T, D] tensors have strides {H*T*D, T*D, D}; the
 * projection layout [B, T, H, D] has {T*H*D, D, H*D}.
 * Value head hv reads key head hv / (num_v_heads / num_heads).
 */
#ifndef GDN2_H_
#define GDN2_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define GDN2_API __attribute__((visibility("default")))
#else
#define GDN2_API
#endif

typedef enum gdn2_status {
    GDN2_OK = 0,
    GDN2_NOT_APPLICABLE = 1, /* outside the kernels' limits: fall back (reference `None`) */
    GDN2_EINVAL = 2,         /* invalid arguments (null pointer, inconsistent shapes) */
    GDN2_EHIP = 3,           /* HIP runtime error; see gdn2_last_error() */
} gdn2_status;

/* hipStream_t, passed opaquely so that this header needs no HIP include. */
typedef void *gdn2_stream_t;

/* Message of the last non-OK status returned on the calling thread. */
GDN2_API const char *gdn2_last_error(void);

/* 1 when a gfx950 device is current and usable, else 0.
 * Replaces the TypeId == CudaBare gate (fused_recurrent_cube.rs:76-78). */
GDN2_API int gdn2_hip_available(void);

/* ------------------------------------------------------------------------
 * One recurrent step for every (batch, value head)      -- fused_step
 * (src/kernel/fused_recurrent_cube.rs:108-172, math :14-57):
 *   S' = diag(exp g) S;  v_new = w*v - S'^T (b*k);  S'' = S' + k v_new^T;
 *   out = scale * S''^T q
 * q,k,g,b: [B, Hk, K] with stride_qk_b / stride_qk_h (last dim contiguous)
 * v,w:     [B, HV, V] with stride_vw_b / stride_vw_h
 * out:     [B, HV, V] with stride_o_b / stride_o_h
 * state_in / state_out: [B, HV, K, V] contiguous; may be the same buffer
 * (in-place update; the reference returns a new buffer).
 * Limits (else GDN2_NOT_APPLICABLE): K, V <= 1024, same as the reference.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_step_args {
    const float *q, *k, *g, *b;
    const float *v, *w;
    const float *state_in;
    float *state_out;
    float *out;
    int64_t batch, num_heads, num_v_heads, head_dim, head_v_dim;
    int64_t stride_qk_b, stride_qk_h;
    int64_t stride_vw_b, stride_vw_h;
    int64_t stride_o_b, stride_o_h;
    double scale;
} gdn2_step_args;

GDN2_API gdn2_status gdn2_recurrent_step_f32(const gdn2_step_args *args, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Per-token scan over T tokens in one launch       -- fused_recurrent_forward
 * (src/kernel/fused_recurrent.rs:11-55), the FusedRecurrent-mode path and
 * the rule for sequences of at most 64 tokens (src/module.rs:245-249).
 * q,k,g,b: [B, Hk, T, K] strided; v,w: [B, HV, T, V] strided;
 * out: [B, HV, T, V] strided; state_in/out: [B, HV, K, V] contiguous, may
 * alias.  S is read once and written once whatever T is.
 * Limits (else GDN2_NOT_APPLICABLE): K, V <= 1024.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_recurrent_args {
    const float *q, *k, *g, *b;
    const float *v, *w;
    const float *state_in;
    float *state_out;
    float *out;
    int64_t batch, num_heads, num_v_heads, seq_len, head_dim, head_v_dim;
    int64_t stride_qk_b, stride_qk_h, stride_qk_t;
    int64_t stride_vw_b, stride_vw_h, stride_vw_t;
    int64_t stride_o_b, stride_o_h, stride_o_t;
    double scale;
} gdn2_recurrent_args;

GDN2_API gdn2_status gdn2_recurrent_fwd_f32(const gdn2_recurrent_args *args, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Chunked forward over a whole sequence                  -- fused_chunk_forward
 * (src/kernel/chunk_cube.rs:781-952; semantics of src/forward.rs:44-278):
 * out[t] and the final state equal T steps of the recurrence above.
 * q,k,g,b: [B, Hk, T, K] strided;  v,w: [B, HV, T, V] strided
 * out:     [B, HV, T, V] strided (e.g. [B, T, HV, V] to skip a permute)
 * state:   [B, HV, K, V] contiguous, read as S0 and overwritten with S_T
 *          (in place, like the reference's chunk path).
 * T need not be a multiple of chunk_size.  The kernels always work on
 * 64-token chunks of four 16-row tiles; any chunk_size > 0 is accepted, since
 * the result does not depend on it beyond rounding, as in the reference.
 * workspace: device memory of at least gdn2_chunk_workspace_bytes(args)
 * bytes, 256-byte aligned.
 * Limits (else GDN2_NOT_APPLICABLE): (K, V) with K = 32 and V in {32, 64},
 * K = 64 and V in {64, 96, 128, 256}, K = 128 and V in {64, 128, 192, 256},
 * or K = 256 and V in {128, 256} (the reference takes K, V <= 256; these are
 * its own benchmark and test head shapes and expand_v 0.5, 1, 1.5, 2, 4);
 * q, k, b rows 16-byte aligned (strides multiples of 4 elements); token
 * strides at least the row length (stride_qk_t >= K, stride_vw_t >= V,
 * stride_o_t >= V) and 63 token strides plus a row under 2 GiB.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_chunk_args {
    const float *q, *k, *g, *b;
    const float *v, *w;
    float *state;
    float *out;
    int64_t batch, num_heads, num_v_heads, seq_len, head_dim, head_v_dim;
    int64_t stride_qk_b, stride_qk_h, stride_qk_t;
    int64_t stride_vw_b, stride_vw_h, stride_vw_t;
    int64_t stride_o_b, stride_o_h, stride_o_t;
    double scale;
    int64_t chunk_size;
    void *workspace;
    size_t workspace_bytes;
} gdn2_chunk_args;

GDN2_API size_t gdn2_chunk_workspace_bytes(const gdn2_chunk_args *args);
GDN2_API gdn2_status gdn2_chunk_fwd_f32(const gdn2_chunk_args *args, gdn2_stream_t stream);

/* The two phases of gdn2_chunk_fwd_f32, for phase-isolated timing; they
 * replace the reference's diagnostics intra_launch_raw / inter_launch_raw
 * (src/kernel/chunk_cube.rs:954-1137).  gdn2_chunk_intra_f32 (parallel over
 * all chunks) fills the workspace; gdn2_chunk_inter_f32 (sequential over
 * chunks) consumes it, writes out and updates state.  Called in this order
 * on one stream with the same args they equal gdn2_chunk_fwd_f32. */
GDN2_API gdn2_status gdn2_chunk_intra_f32(const gdn2_chunk_args *args, gdn2_stream_t stream);
GDN2_API gdn2_status gdn2_chunk_inter_f32(const gdn2_chunk_args *args, gdn2_stream_t stream);

/* The passes of gdn2_chunk_inter_f32 one at a time, for per-pass timing (the
 * same diagnostic role).  Few long sequences split each sequence into
 * gdn2_chunk_segments(args) segments so that the sequential walk spreads over
 * the compute units: pass 1 runs every segment but the last from a zero state
 * (its transition and offset), pass 2 chains the segments' entering states,
 * pass 3 re-runs every segment from its entering state and writes out and the
 * final state.  Where those segments are long (16 chunks and more), one more
 * segment is cut and segment 0, whose entering state is S0, is walked once
 * with the output during pass 1 (on a second stream the library forks from
 * and joins back to `stream`); passes 2 and 3 then cover the rest.  With one
 * segment, passes 1 and 2 launch nothing.  Called 1, 2, 3 in order on one
 * stream after gdn2_chunk_intra_f32 they equal gdn2_chunk_inter_f32.  Any
 * other pass is GDN2_EINVAL. */
GDN2_API int64_t gdn2_chunk_segments(const gdn2_chunk_args *args);
GDN2_API gdn2_status gdn2_chunk_inter_pass_f32(const gdn2_chunk_args *args, int pass, gdn2_stream_t stream);

/* The full return of fused_chunk_forward (src/kernel/chunk_cube.rs:781-952),
 * (out, state, v_new, states): gdn2_chunk_fwd_f32 plus, per chunk of
 * C = chunk_size tokens,
 *   v_new   [B*HV*NC, C, V] contiguous: row r of chunk n is the value the
 *           delta rule writes at token C n + r (the pseudo-values U - W S)
 *   states  [B*HV*NC, K, V] contiguous: the state entering chunk n
 * with chunk id (b * HV + hv) * NC + n, the reference's [nblk, C, V] /
 * [nblk, K, V].  C = 64: NC = ceil(T / 64), rows past T (a ragged last
 * chunk) are zero.  C < 64: C must divide T (the reference's C <= 64 and
 * T % C == 0, src/kernel/chunk_cube.rs:795-800), NC = T / C; the states at
 * boundaries inside a 64-token chunk are derived from the state entering it
 * by one or two more small kernels.  The workspace is
 * gdn2_chunk_workspace_bytes(args) as for gdn2_chunk_fwd_f32.  Limits: those
 * of gdn2_chunk_fwd_f32, and the chunk sizes above (else
 * GDN2_NOT_APPLICABLE). */
GDN2_API gdn2_status gdn2_chunk_fwd_states_f32(const gdn2_chunk_args *args, float *v_new, float *states,
                                               gdn2_stream_t stream);

/* gdn2_chunk_fwd_f32 without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The kernels and results are those of gdn2_chunk_fwd_f32;
 * the workspace is a static device array of gdn2_chunk_noalloc_scratch_bytes()
 * bytes (64 MiB) that each GPU holds until the process ends.  args->workspace
 * and args->workspace_bytes are ignored.  A call whose
 * gdn2_chunk_workspace_bytes(args) exceeds the array returns GDN2_EINVAL and
 * launches nothing (at K = V = 128 the array holds about 450 chunks of 64
 * tokens, counted over every (batch row, value head)).  All calls on one GPU
 * share its array: calls that overlap in time on one GPU (two streams or two
 * host threads) race and must be ordered by the caller.  The first call on a
 * device looks up that device's copy of the array (hipGetSymbolAddress),
 * which may load the code object: make that first call eagerly, before any
 * graph capture on that device. */
GDN2_API size_t gdn2_chunk_noalloc_scratch_bytes(void);
GDN2_API gdn2_status gdn2_chunk_fwd_noalloc_f32(const gdn2_chunk_args *args, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Standalone operators, the reference's public functions (src/lib.rs:58-62),
 * for a binding that calls them one by one (the layer fuses them into its
 * own kernels).  Contiguous f32 device arrays; every status as above.
 *
 * short_conv_1d (src/short_conv.rs:22-65): causal depthwise conv of 4 taps +
 * SiLU.  x [B, T, C], weight [C, 4], cache_in [B, 3, C] or NULL (Option::None:
 * the first token is repeated 3 times as padding), out [B, T, C],
 * cache_out [B, 3, C] = the last 3 rows of cat(cache or padding, x) along time.
 *   out[b, t, c] = silu(sum_{i<4} xpad[b, t + i, c] weight[c, i])
 * out must not overlap x (no in-place use), and cache_out must not overlap
 * x, out or cache_in.  T = 0 needs cache_in (cache_out = cache_in).
 *
 * l2_normalize / l2_normalize_4d (src/l2norm.rs:4-16): y = x / sqrt(sum x^2 +
 * eps) over each of `rows` rows of n values (any leading shape flattened);
 * y may be x.
 *
 * rms_norm_gate_per_head (src/module.rs:501-517):
 *   y = x / sqrt(mean x^2 + eps) * weight * silu(gate)
 * over each of `rows` rows of V values (x, gate [B, T, HV, V] flattened to
 * rows = B T HV), weight [V]; y may be x.
 * ---------------------------------------------------------------------- */
GDN2_API gdn2_status gdn2_short_conv_f32(const float *x, const float *weight, const float *cache_in, float *out,
                                         float *cache_out, int64_t B, int64_t T, int64_t C, gdn2_stream_t stream);
GDN2_API gdn2_status gdn2_l2_normalize_f32(const float *x, float *y, int64_t rows, int64_t n, double eps,
                                           gdn2_stream_t stream);
GDN2_API gdn2_status gdn2_rms_norm_gate_f32(const float *x, const float *gate, const float *weight, float *y,
                                            int64_t rows, int64_t V, double eps, gdn2_stream_t stream);

/* A streaming copy of n floats (dst, src 16-byte aligned, not overlapping)
 * over `workgroups` workgroups of 256 threads (0 = 8 per compute unit), each
 * looping over the array with 16-byte non-temporal loads and stores.  No
 * reference counterpart: the benchmark's measurement of the practical HBM
 * bandwidth (2 n x 4 bytes moved per call) beside the 8 TB/s peak. */
GDN2_API gdn2_status gdn2_stream_copy_f32(float *dst, const float *src, int64_t n, int64_t workgroups,
                                          gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Chunked backward                                     -- fused_chunk_backward
 * (src/kernel/chunk_adjoint_cube.rs:464-707; the reference's training path
 * otherwise differentiates chunk_wy_forward through autodiff): the gradients
 * of L = <d_out, out> + <d_state_out, S_T> for the forward of `fwd`.
 *   fwd          the forward's arguments: q, k, g, b, v, w, state = S0 (read
 *                only), strides, scale, chunk_size; out, workspace unused
 *   d_out        strided like out (fwd.stride_o_*), 16-byte aligned rows
 *   d_state_out  [B, HV, K, V] contiguous, or NULL (zero)
 *   dq, dk, dg, db  strided like q (fwd.stride_qk_*); with num_v_heads >
 *                num_heads the sum over the value heads of each key head
 *   dv, dw       strided like v (fwd.stride_vw_*)
 *   d_state0     [B, HV, K, V] contiguous
 * It recomputes the forward's per-chunk quantities (the reference's
 * FusedBackwardInputs) in its own workspace of
 * gdn2_chunk_bwd_workspace_bytes(args) bytes, 256-byte aligned.
 * Limits (else GDN2_NOT_APPLICABLE): those of gdn2_chunk_fwd_f32, the same
 * (K, V) pairs (other heads: gdn2_recurrent_bwd_f32).
 * ---------------------------------------------------------------------- */
typedef struct gdn2_chunk_bwd_args {
    gdn2_chunk_args fwd;
    const float *d_out;
    const float *d_state_out;
    float *dq, *dk, *dg, *db;
    float *dv, *dw;
    float *d_state0;
    void *workspace;
    size_t workspace_bytes;
} gdn2_chunk_bwd_args;

GDN2_API size_t gdn2_chunk_bwd_workspace_bytes(const gdn2_chunk_bwd_args *args);
GDN2_API gdn2_status gdn2_chunk_bwd_f32(const gdn2_chunk_bwd_args *args, gdn2_stream_t stream);

/* The training forward and the backward from its saved quantities, the
 * reference's pair fused_chunk_forward -> FusedBackwardInputs ->
 * fused_chunk_backward(fwd: &FusedBackwardInputs, ..)
 * (src/kernel/chunk_adjoint_cube.rs:426-520):
 *   gdn2_chunk_fwd_train_f32  the forward of args->fwd exactly as
 *       gdn2_chunk_fwd_f32 (out written, state updated in place to S_T), that
 *       also leaves in args->workspace (gdn2_chunk_bwd_workspace_bytes(args)
 *       bytes, 256-byte aligned) every per-chunk quantity the backward reads:
 *       the WY operands (W, U, Kd, e^{G_last}, A_qk, scale q e^G, (I + A_kk)^-1),
 *       the state entering every chunk and v_new.  The gradient pointers are
 *       not read.
 *   gdn2_chunk_bwd_saved_f32  gdn2_chunk_bwd_f32 on that workspace, untouched
 *       since, for the same q, k, g, b, v, w, shapes and strides: the forward's
 *       quantities are read instead of recomputed (args->fwd.state is not read).
 *       The gradients are bit-identical to gdn2_chunk_bwd_f32's.
 * Limits: those of gdn2_chunk_bwd_f32. */
GDN2_API gdn2_status gdn2_chunk_fwd_train_f32(const gdn2_chunk_bwd_args *args, gdn2_stream_t stream);
GDN2_API gdn2_status gdn2_chunk_bwd_saved_f32(const gdn2_chunk_bwd_args *args, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Backward of the per-token scan                 -- autodiff of the recurrence
 * (src/kernel/fused_recurrent.rs:27-52, differentiated by burn's autodiff in
 * the reference's training path, tests/autodiff.rs:153-206): the gradients
 * of L = <d_out, out> + <d_state_out, S_T> for the scan of `fwd`, for any
 * (K, V) whose working set fits one workgroup -- the shapes the chunked
 * backward does not take.
 *   fwd          the forward's arguments: q, k, g, b, v, w, state_in = S0
 *                (read only; NULL = zeros), strides, scale; state_out, out unused
 *   d_out        strided like out (fwd.stride_o_*)
 *   d_state_out  [B, HV, K, V] contiguous, or NULL (zero)
 *   dq, dk, dg, db  strided like q; with num_v_heads > num_heads the sum over
 *                the value heads of each key head
 *   dv, dw       strided like v
 *   d_state0     [B, HV, K, V] contiguous
 * workspace: gdn2_recurrent_bwd_workspace_bytes(args) bytes (the state every
 * 64 tokens, and the states of one 64-token segment, per key head).
 * Limits (else GDN2_NOT_APPLICABLE): 4 (2 K (V + 1) + 5 K + 3 V) bytes of LDS
 * at most 160 KB (e.g. K = V = 128).  One workgroup per (batch row, key
 * head), sequential over tokens: meant for small heads.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_recurrent_bwd_args {
    gdn2_recurrent_args fwd;
    const float *d_out;
    const float *d_state_out;
    float *dq, *dk, *dg, *db;
    float *dv, *dw;
    float *d_state0;
    void *workspace;
    size_t workspace_bytes;
} gdn2_recurrent_bwd_args;

GDN2_API size_t gdn2_recurrent_bwd_workspace_bytes(const gdn2_recurrent_bwd_args *args);
GDN2_API gdn2_status gdn2_recurrent_bwd_f32(const gdn2_recurrent_bwd_args *args, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused decode of one token for every batch row           -- forward at T=1
 * Inputs are the raw projections of one token (outputs of the Linear
 * layers, src/module.rs:400-402,417-418,442-443,474-475):
 *   q_raw, k_raw, f_raw, b_raw: [B, kd]   (f_raw = f_proj_1(f_proj_0(x)))
 *   v_raw, w_raw, gate:         [B, vd]   (gate = g_proj_1(g_proj_0(x)) + bias)
 * Conv caches [B, 3, kd|vd] hold the last 3 pre-conv rows (oldest first).
 * conv_*_in NULL means no prior state (src/short_conv.rs:42-54: the token
 * is replicated).  conv_*_out must not alias conv_*_in.
 * state [B, HV, K, V] is updated in place.
 * out [B, vd] = rms_norm_gate_per_head(o) (input of o_proj).
 * Limits (else GDN2_NOT_APPLICABLE): K <= 256, V <= 1024.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_layer_params {
    const float *q_conv_w, *k_conv_w, *v_conv_w; /* [kd,4],[kd,4],[vd,4]; unused without short conv */
    const float *a_log;                          /* [H] */
    const float *dt_bias;                        /* [kd] */
    const float *decay_factors;                  /* [H*K], NULL when min_decay is None */
    const float *o_norm_weight;                  /* [V] */
    double min_decay;
    double norm_eps;
    int32_t use_short_conv;
    int32_t allow_neg_eigval;
} gdn2_layer_params;

typedef struct gdn2_decode_args {
    const float *q_raw, *k_raw, *f_raw, *b_raw;
    const float *v_raw, *w_raw, *gate;
    const float *conv_q_in, *conv_k_in, *conv_v_in;
    float *conv_q_out, *conv_k_out, *conv_v_out;
    float *state;
    float *out;
    int64_t batch, num_heads, num_v_heads, head_dim, head_v_dim;
    double scale;
    const gdn2_layer_params *params;
} gdn2_decode_args;

GDN2_API gdn2_status gdn2_decode_fused_f32(const gdn2_decode_args *args, gdn2_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_H_ */

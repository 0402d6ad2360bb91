/*
 * gdn2_layer.h -- C ABI of the GDN-2 layer (config, parameters, state,
 * forward) built on the kernels of gdn2.h.
 *
 * It mirrors burn-gdn2's public surface:
 *
 *   gdn2_config, gdn2_config_default   <- Gdn2Config, Default      src/config.rs:23-58, :114-130
 *   gdn2_config_validate               <- Gdn2Config::validate     src/config.rs:71-111
 *   gdn2_config_dims                   <- shape algebra             src/module.rs:113-119
 *   gdn2_param_*, gdn2_layer_create    <- GatedDeltaNet2::new       src/module.rs:111-190
 *   gdn2_layer_project_f32             <- GatedDeltaNet2::project   src/module.rs:381-495
 *   gdn2_layer_forward_train_f32       <- forward_train             src/module.rs:326-375
 *   gdn2_layer_forward_f32             <- forward(.., update_state = true)
 *                                                                   src/module.rs:224-316
 *   gdn2_state_*                       <- Gdn2State / Option<Gdn2State>
 *                                                                   src/module.rs:30-63
 *   gdn2_state_serialize / _deserialize   Gdn2State interchange (safetensors)
 *
 * Status codes and gdn2_last_error() are those of gdn2.h.  Configuration
 * errors return GDN2_EINVAL with the reference's panic message.  The layer
 * owns its parameters and a workspace in device memory (allocated on the
 * device current at gdn2_layer_create; the workspace grows on the first
 * call at a larger batch x tokens).  x and out are caller-owned device
 * buffers [B, T, hidden_size], contiguous f32.  Calls are asynchronous on
 * `stream`; calls on one layer must not overlap (they share the workspace).
 */
#ifndef GDN2_LAYER_H_
#define GDN2_LAYER_H_

#include "gdn2.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gdn2_mode {
    GDN2_MODE_FUSED_RECURRENT = 0, /* Gdn2Mode::FusedRecurrent */
    GDN2_MODE_CHUNK = 1,           /* Gdn2Mode::Chunk */
} gdn2_mode;

/* How the key-side heads (q, k, g, b) reach the value heads under GVA
 * (num_v_heads > num_heads, rep = num_v_heads / num_heads).  Not a
 * Gdn2Config field: the reference has one layout, its tensor path's
 * unsqueeze/repeat/reshape (src/module.rs:456-468), which reads value head
 * h * rep + a at time t from key head h at time (a * T + t) / rep of the same
 * call, so that a T-token call differs from T one-token calls.
 * GDN2_GVA_HEAD_REPEAT (the default) gives value head hv key head hv / rep at
 * every time, so decode reproduces prefill; GDN2_GVA_REFERENCE reproduces the
 * reference's layout (the two coincide at T = 1). */
typedef enum gdn2_gva_layout {
    GDN2_GVA_HEAD_REPEAT = 0,
    GDN2_GVA_REFERENCE = 1,
} gdn2_gva_layout;

/* Gdn2Config (src/config.rs:23-58).  Option fields: num_v_heads = 0 is
 * None; has_min_decay = 0 is None.  gva_layout (gdn2_gva_layout) is this
 * library's own field, 0 in gdn2_config_default. */
typedef struct gdn2_config {
    int64_t hidden_size;
    int64_t num_heads;
    int64_t head_dim;
    float expand_v;
    int64_t num_v_heads;
    int32_t use_short_conv;
    int32_t allow_neg_eigval;
    double norm_eps;
    int32_t mode; /* gdn2_mode */
    int64_t chunk_size;
    int32_t has_min_decay;
    double min_decay;
    int32_t gva_layout;
} gdn2_config;

/* Gdn2Config::default() (src/config.rs:114-130). */
GDN2_API void gdn2_config_default(gdn2_config *cfg);

/* Gdn2Config::validate() (src/config.rs:71-111): GDN2_EINVAL with the
 * reference's panic message on the first failing check. */
GDN2_API gdn2_status gdn2_config_validate(const gdn2_config *cfg);

/* hv = num_v_heads or num_heads, head_v_dim = head_dim * expand_v,
 * kd = num_heads * head_dim, vd = hv * head_v_dim (src/module.rs:113-119).
 * Any output pointer may be NULL. */
GDN2_API gdn2_status gdn2_config_dims(const gdn2_config *cfg, int64_t *hv, int64_t *head_v_dim, int64_t *kd,
                                      int64_t *vd);

/* ------------------------------------------------------------------------
 * Parameters, by the reference's field names (src/module.rs:93-111):
 *   q_proj [D, kd]  k_proj [D, kd]  v_proj [D, vd]  f_proj_0 [D, V]
 *   f_proj_1 [V, kd]  b_proj [D, kd]  w_proj [D, vd]  g_proj_0 [D, V]
 *   g_proj_1 [V, vd]  g_proj_1_bias [vd]  a_log [H]  dt_bias [kd]
 *   o_norm_weight [V]  o_proj [vd, D]  q_conv_w [kd, 4]  k_conv_w [kd, 4]
 *   v_conv_w [vd, 4]  decay_factors [H, K] (present iff min_decay is set)
 * Linear weights are [in, out] (burn's layout: y = x W).  V = head_v_dim.
 * ---------------------------------------------------------------------- */
GDN2_API int gdn2_param_count(void);
GDN2_API const char *gdn2_param_name(int index); /* NULL outside [0, count) */

/* Number of elements of parameter `name` for `cfg` (0 when the parameter is
 * absent, i.e. decay_factors without min_decay; -1 for an unknown name);
 * rows/cols (nullable) receive its 2-D shape, cols = 1 for vectors. */
GDN2_API int64_t gdn2_param_shape(const gdn2_config *cfg, const char *name, int64_t *rows, int64_t *cols);

/* Host-side initial value of one parameter, drawn from the reference's
 * initialisers (src/module.rs:121-187): Xavier-uniform with gain 2^-2.5 for
 * the Linear weights, zero bias, U(-1/2, 1/2) conv weights, A_log ~
 * U(ln 1, ln 16), dt_bias = dt + ln(1 - e^-dt) with dt = max(e^U(ln 1e-3,
 * ln 0.1), 1e-4), ones for o_norm_weight, 2 for decay_factors.  The random
 * stream is a counter-based SplitMix64 of (seed, parameter index, element
 * index), so the values do not depend on the order of the calls.  burn's
 * own RNG stream is not reproduced (it cannot be without burn). */
GDN2_API gdn2_status gdn2_param_init(const gdn2_config *cfg, uint64_t seed, const char *name, float *host,
                                     int64_t numel);

/* ------------------------------------------------------------------------
 * The layer.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_layer gdn2_layer;
typedef struct gdn2_state gdn2_state;

/* GatedDeltaNet2::new (src/module.rs:111-190): validates cfg and
 * initialises every parameter with gdn2_param_init(cfg, seed, ...). */
GDN2_API gdn2_status gdn2_layer_create(const gdn2_config *cfg, uint64_t seed, gdn2_layer **out);
GDN2_API void gdn2_layer_destroy(gdn2_layer *layer);
GDN2_API const gdn2_config *gdn2_layer_config(const gdn2_layer *layer);

/* Copy one parameter from / to host memory (synchronous).  numel must equal
 * gdn2_param_shape(); an absent parameter is GDN2_EINVAL. */
GDN2_API gdn2_status gdn2_layer_set_param(gdn2_layer *layer, const char *name, const float *host, int64_t numel);
GDN2_API gdn2_status gdn2_layer_get_param(const gdn2_layer *layer, const char *name, float *host, int64_t numel);

/* forward_train (src/module.rs:326-375): x [B, T, D] -> out [B, T, D],
 * starting from S = 0 with no conv cache; the recurrence follows cfg->mode
 * (Chunk falls back to the per-token scan kernel outside the chunk kernels'
 * shapes: the same recurrence). */
GDN2_API gdn2_status gdn2_layer_forward_train_f32(gdn2_layer *layer, const float *x, int64_t batch, int64_t seq_len,
                                                  float *out, gdn2_stream_t stream);

/* forward(x, &mut state, update_state = true) (src/module.rs:224-316):
 * T <= 64 tokens use the per-token recurrence (T = 1: the fused decode
 * kernel), longer inputs cfg->mode.  An empty state (Option::None) starts
 * from S = 0 with the short conv padded by the first token and becomes
 * non-empty; the conv caches are replaced only with use_short_conv.
 * T = 0 is a no-op. */
GDN2_API gdn2_status gdn2_layer_forward_f32(gdn2_layer *layer, const float *x, int64_t batch, int64_t seq_len,
                                            gdn2_state *state, float *out, gdn2_stream_t stream);

/* project (src/module.rs:381-495): writes the recurrence's inputs q, k,
 * g, b, v, w [B, HV, T, V] and the gate signal [B, T, HV, V] (each
 * contiguous, caller-owned).  q, k, g, b are [B, H, T, K] under
 * GDN2_GVA_HEAD_REPEAT (the key heads, not repeated: value head hv reads key
 * head hv / rep) and [B, HV, T, K] under GDN2_GVA_REFERENCE (the reference's
 * repeated layout, what its project returns).  `state` (nullable, not
 * modified) supplies the conv caches when non-empty. */
GDN2_API gdn2_status gdn2_layer_project_f32(gdn2_layer *layer, const float *x, int64_t batch, int64_t seq_len,
                                            const gdn2_state *state, float *q, float *k, float *g, float *b,
                                            float *v, float *w, float *gate, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * Training.  The reference trains the layer through burn's autodiff
 * (tests/autodiff.rs:153-205: gradients of every parameter, through
 * forward_train in both modes and through token-by-token forward calls with
 * a state).  Here the backward is an explicit call that recomputes the
 * forward from x (or takes it from saved activations) and returns the same
 * gradients.
 * ---------------------------------------------------------------------- */
typedef struct gdn2_layer_grads gdn2_layer_grads;

/* One gradient buffer per parameter of `layer`, on its device, zeroed. */
GDN2_API gdn2_status gdn2_layer_grads_create(const gdn2_layer *layer, gdn2_layer_grads **out);
GDN2_API void gdn2_layer_grads_destroy(gdn2_layer_grads *grads);
/* Zero every gradient (stream-ordered fill kernels). */
GDN2_API gdn2_status gdn2_layer_grads_zero(gdn2_layer_grads *grads, gdn2_stream_t stream);
/* Synchronous copy of one parameter's gradient to host memory, in the
 * parameter's shape (gdn2_param_shape); an absent parameter is GDN2_EINVAL. */
GDN2_API gdn2_status gdn2_layer_grads_get(const gdn2_layer_grads *grads, const char *name, float *host,
                                          int64_t numel);

/* Activations kept from forward_train for the backward (what the forward
 * computes before the norm: the Linear outputs, the kernel operands and the
 * recurrence output; about 4 * B * T * (D_in + 8 kd + 4 vd) bytes with
 * D_in ~ 3 kd + 2 vd + 2 V), so that the backward need not recompute them.
 * For heads the chunked backward takes it also holds that backward's
 * workspace (gdn2_chunk_bwd_workspace_bytes), which the forward fills with
 * the recurrence's per-chunk quantities through gdn2_chunk_fwd_train_f32
 * wherever the recurrence runs the chunk kernels (mode chunk, or T > 64), and
 * the backward reads through gdn2_chunk_bwd_saved_f32 (about 5 GB more at
 * B = 8, T = 4096, 16 heads of 128).  One object per (batch, seq_len);
 * reusable. */
typedef struct gdn2_layer_saved gdn2_layer_saved;
GDN2_API gdn2_status gdn2_layer_saved_create(const gdn2_layer *layer, int64_t batch, int64_t seq_len,
                                             gdn2_layer_saved **out);
GDN2_API void gdn2_layer_saved_destroy(gdn2_layer_saved *saved);
/* gdn2_layer_forward_train_f32 that also fills `saved`. */
GDN2_API gdn2_status gdn2_layer_forward_train_saved_f32(gdn2_layer *layer, const float *x, int64_t batch,
                                                        int64_t seq_len, float *out, gdn2_layer_saved *saved,
                                                        gdn2_stream_t stream);

/* The gradients of L = <d_out, out> + <d_state, state after the call> for
 * gdn2_layer_forward_f32(x, state_in) -- and for forward_train when state_in
 * is NULL or empty (Option::None: S0 = 0, the first token pads the conv).
 *   x, d_out     [B, T, D]
 *   state_in     the state before the call (read only), NULL or empty = None
 *   saved        NULL: the forward is recomputed from x; else filled by
 *                gdn2_layer_forward_train_saved_f32 on this x (state_in must
 *                then be NULL or empty)
 *   d_state      NULL or empty = zero; else the gradient of the state after
 *                the call (recurrent and conv caches)
 *   dx           [B, T, D], or NULL
 *   d_state_in   NULL, or a state (not state_in, not d_state) that receives
 *                the gradient of the state before the call: recurrent = dS0
 *                (also for None, whose S0 is zero); conv caches = their
 *                gradient (zero for None with short conv; without short conv
 *                the caches pass through the call, and so does d_state's).
 *                It becomes non-empty.
 *   grads        accumulate = 0: overwritten; 1: added to (gradient
 *                accumulation, or a chain of calls run backwards, each with
 *                d_state = the d_state_in of the call after it)
 * The result does not depend on cfg->mode (both modes compute the same
 * recurrence).  The recurrence's adjoint is gdn2_chunk_bwd_f32 where it
 * applies (the (head_dim, head_v_dim) pairs of gdn2_chunk_fwd_f32), else
 * gdn2_recurrent_bwd_f32, whose limit is the only one here (else
 * GDN2_NOT_APPLICABLE). */
GDN2_API gdn2_status gdn2_layer_backward_f32(gdn2_layer *layer, const float *x, int64_t batch, int64_t seq_len,
                                             const gdn2_state *state_in, const gdn2_layer_saved *saved,
                                             const float *d_out,
                                             const gdn2_state *d_state, float *dx, gdn2_state *d_state_in,
                                             gdn2_layer_grads *grads, int accumulate, gdn2_stream_t stream);

/* ------------------------------------------------------------------------
 * State: Option<Gdn2State> (src/module.rs:30-63) for one layer and batch.
 * Tensors: 0 recurrent [B, HV, K, V], 1 conv_q [B, 3, kd], 2 conv_k
 * [B, 3, kd], 3 conv_v [B, 3, vd] (oldest cached token first).
 * ---------------------------------------------------------------------- */
enum { GDN2_STATE_RECURRENT = 0, GDN2_STATE_CONV_Q = 1, GDN2_STATE_CONV_K = 2, GDN2_STATE_CONV_V = 3 };

/* Allocates the state's device buffers; the state starts empty (None). */
GDN2_API gdn2_status gdn2_state_create(const gdn2_layer *layer, int64_t batch, gdn2_state **out);
GDN2_API void gdn2_state_destroy(gdn2_state *state);
/* Some(Gdn2State::zeros(..)) (src/module.rs:49-62); synchronous. */
GDN2_API gdn2_status gdn2_state_set_zeros(gdn2_state *state);
/* Back to None. */
GDN2_API void gdn2_state_clear(gdn2_state *state);
GDN2_API int gdn2_state_is_some(const gdn2_state *state);
GDN2_API int64_t gdn2_state_batch(const gdn2_state *state);
/* Element count of tensor `which`, and its current device buffer (the conv
 * caches alternate between two buffers, so the pointer changes after each
 * forward call). */
GDN2_API int64_t gdn2_state_numel(const gdn2_state *state, int which);
GDN2_API float *gdn2_state_tensor(gdn2_state *state, int which);
/* Synchronous host copies; a write makes the state non-empty (the tensors
 * not written keep their values, zeros for a fresh state). */
GDN2_API gdn2_status gdn2_state_read(const gdn2_state *state, int which, float *host, int64_t numel);
GDN2_API gdn2_status gdn2_state_write(gdn2_state *state, int which, const float *host, int64_t numel);

/* Gdn2State interchange.  The state as a safetensors byte stream: an 8-byte
 * little-endian header length, a JSON header padded with spaces to an 8-byte
 * boundary, then raw little-endian f32 data.  The tensors carry the
 * reference's field names (src/module.rs:30-40):
 *   "recurrent" [B, HV, K, V], "conv_q" and "conv_k" [B, 3, kd],
 *   "conv_v" [B, 3, vd].
 * __metadata__ holds {format: "gdn2_state", num_heads, num_v_heads,
 * head_dim, head_v_dim}.  Any safetensors reader can read it, for instance
 * the Rust safetensors crate that burn's recorders use; a state written by
 * one can be read here.
 * gdn2_state_serialize: with buf = NULL it only sets *len to the size;
 * otherwise cap must be at least that size.  An empty state (None) is
 * GDN2_EINVAL.
 * gdn2_state_deserialize: the four tensors must be present, F32, and of this
 * state's shapes (unknown tensors are GDN2_EINVAL; __metadata__ is not
 * checked).  The state becomes non-empty.
 * Both are synchronous host copies. */
GDN2_API gdn2_status gdn2_state_serialize(const gdn2_state *state, void *buf, size_t cap, size_t *len);
GDN2_API gdn2_status gdn2_state_deserialize(gdn2_state *state, const void *buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_LAYER_H_ */

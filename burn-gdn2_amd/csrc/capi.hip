// C ABI (include/gdn2.h): argument validation, limit checks that return
// GDN2_NOT_APPLICABLE (the reference's `None`), and dispatch to the kernels.
#include <cstring>
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

gdn2_status fail(gdn2_status st, const std::string &msg) {
    set_error(msg);
    return st;
}

}  // namespace gdn2

using namespace gdn2;

extern "C" const char *gdn2_last_error(void) { return g_last_error.c_str(); }

extern "C" int gdn2_hip_available(void) {
    int dev = 0, n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// fused_step (src/kernel/fused_recurrent_cube.rs:108-172): limits K, V <= 1024
// (:122-124); the reference's B*HV <= 65535 grid limit does not apply here.
extern "C" gdn2_status gdn2_recurrent_step_f32(const gdn2_step_args *a, gdn2_stream_t stream) {
    if (!a) return fail(GDN2_EINVAL, "gdn2_recurrent_step_f32: null args");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->state_in || !a->state_out || !a->out)
        return fail(GDN2_EINVAL, "gdn2_recurrent_step_f32: null tensor pointer");
    if (a->batch <= 0 || a->num_heads <= 0 || a->num_v_heads <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0)
        return fail(GDN2_EINVAL, "gdn2_recurrent_step_f32: dimensions must be positive");
    if (a->num_v_heads % a->num_heads != 0)
        return fail(GDN2_EINVAL, "gdn2_recurrent_step_f32: num_v_heads must be a multiple of num_heads");
    if (a->head_dim > 1024 || a->head_v_dim > 1024)
        return fail(GDN2_NOT_APPLICABLE, "gdn2_recurrent_step_f32: K or V above 1024");
    ScanParams p{};
    p.q = a->q; p.k = a->k; p.g = a->g; p.b = a->b; p.v = a->v; p.w = a->w;
    p.state_in = a->state_in; p.state_out = a->state_out; p.out = a->out;
    p.B = (int)a->batch; p.HV = (int)a->num_v_heads; p.rep = (int)(a->num_v_heads / a->num_heads);
    p.T = 1; p.K = (int)a->head_dim; p.V = (int)a->head_v_dim;
    p.sqb = a->stride_qk_b; p.sqh = a->stride_qk_h; p.sqt = 0;
    p.svb = a->stride_vw_b; p.svh = a->stride_vw_h; p.svt = 0;
    p.sob = a->stride_o_b; p.soh = a->stride_o_h; p.sot = 0;
    p.scale = (float)a->scale;
    GDN2_HIP_CHECK(launch_scan(p, (hipStream_t)stream));
    return GDN2_OK;
}

// Multi-token scan: the tensor path fused_recurrent_forward
// (src/kernel/fused_recurrent.rs:11-55) as one launch.
extern "C" gdn2_status gdn2_recurrent_fwd_f32(const gdn2_recurrent_args *a, gdn2_stream_t stream) {
    if (!a) return fail(GDN2_EINVAL, "gdn2_recurrent_fwd_f32: null args");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->state_in || !a->state_out || !a->out)
        return fail(GDN2_EINVAL, "gdn2_recurrent_fwd_f32: null tensor pointer");
    if (a->batch <= 0 || a->num_heads <= 0 || a->num_v_heads <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0 ||
        a->seq_len < 0)
        return fail(GDN2_EINVAL, "gdn2_recurrent_fwd_f32: invalid dimensions");
    if (a->num_v_heads % a->num_heads != 0)
        return fail(GDN2_EINVAL, "gdn2_recurrent_fwd_f32: num_v_heads must be a multiple of num_heads");
    if (a->head_dim > 1024 || a->head_v_dim > 1024)
        return fail(GDN2_NOT_APPLICABLE, "gdn2_recurrent_fwd_f32: K or V above 1024");
    ScanParams p{};
    p.q = a->q; p.k = a->k; p.g = a->g; p.b = a->b; p.v = a->v; p.w = a->w;
    p.state_in = a->state_in; p.state_out = a->state_out; p.out = a->out;
    p.B = (int)a->batch; p.HV = (int)a->num_v_heads; p.rep = (int)(a->num_v_heads / a->num_heads);
    p.T = (int)a->seq_len; p.K = (int)a->head_dim; p.V = (int)a->head_v_dim;
    p.sqb = a->stride_qk_b; p.sqh = a->stride_qk_h; p.sqt = a->stride_qk_t;
    p.svb = a->stride_vw_b; p.svh = a->stride_vw_h; p.svt = a->stride_vw_t;
    p.sob = a->stride_o_b; p.soh = a->stride_o_h; p.sot = a->stride_o_t;
    p.scale = (float)a->scale;
    GDN2_HIP_CHECK(launch_scan(p, (hipStream_t)stream));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_decode_fused_f32(const gdn2_decode_args *a, gdn2_stream_t stream) {
    if (!a || !a->params) return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: null args");
    const gdn2_layer_params *P = a->params;
    if (!a->q_raw || !a->k_raw || !a->f_raw || !a->b_raw || !a->v_raw || !a->w_raw || !a->gate || !a->state ||
        !a->out || !P->a_log || !P->dt_bias || !P->o_norm_weight)
        return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: null tensor pointer");
    if (P->use_short_conv &&
        (!P->q_conv_w || !P->k_conv_w || !P->v_conv_w || !a->conv_q_out || !a->conv_k_out || !a->conv_v_out))
        return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: short conv needs weights and output caches");
    if (P->use_short_conv && ((a->conv_q_in && a->conv_q_in == a->conv_q_out) ||
                              (a->conv_k_in && a->conv_k_in == a->conv_k_out) ||
                              (a->conv_v_in && a->conv_v_in == a->conv_v_out)))
        return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: conv cache output must not alias its input");
    if (a->batch <= 0 || a->num_heads <= 0 || a->num_v_heads <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0)
        return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: dimensions must be positive");
    if (a->num_v_heads % a->num_heads != 0)
        return fail(GDN2_EINVAL, "gdn2_decode_fused_f32: num_v_heads must be a multiple of num_heads");
    if (a->head_dim > 256 || a->head_v_dim > 1024)
        return fail(GDN2_NOT_APPLICABLE, "gdn2_decode_fused_f32: K above 256 or V above 1024");
    DecodeParams p{};
    p.q_raw = a->q_raw; p.k_raw = a->k_raw; p.f_raw = a->f_raw; p.b_raw = a->b_raw;
    p.v_raw = a->v_raw; p.w_raw = a->w_raw; p.gate = a->gate;
    p.conv_q_in = a->conv_q_in; p.conv_k_in = a->conv_k_in; p.conv_v_in = a->conv_v_in;
    p.conv_q_out = a->conv_q_out; p.conv_k_out = a->conv_k_out; p.conv_v_out = a->conv_v_out;
    p.q_conv_w = P->q_conv_w; p.k_conv_w = P->k_conv_w; p.v_conv_w = P->v_conv_w;
    p.a_log = P->a_log; p.dt_bias = P->dt_bias; p.decay_factors = P->decay_factors;
    p.o_norm_weight = P->o_norm_weight;
    p.state = a->state; p.out = a->out;
    const int64_t kd = a->num_heads * a->head_dim, vd = a->num_v_heads * a->head_v_dim;
    p.ld_q = p.ld_k = p.ld_f = p.ld_b = kd;
    p.ld_v = p.ld_w = p.ld_gate = p.ld_out = vd;
    p.B = (int)a->batch; p.H = (int)a->num_heads; p.HV = (int)a->num_v_heads;
    p.rep = (int)(a->num_v_heads / a->num_heads); p.K = (int)a->head_dim; p.V = (int)a->head_v_dim;
    p.use_short_conv = P->use_short_conv; p.allow_neg_eigval = P->allow_neg_eigval;
    p.min_decay = (float)P->min_decay; p.one_minus_min_decay = (float)(1.0 - P->min_decay);
    p.norm_eps = (float)P->norm_eps; p.scale = (float)a->scale;
    GDN2_HIP_CHECK(launch_decode(p, (hipStream_t)stream));
    return GDN2_OK;
}

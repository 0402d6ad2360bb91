// The GDN-2 layer on the device: Gdn2Config checks, parameter initialisation,
// GatedDeltaNet2::{project, forward, forward_train} and Gdn2State
// (src/config.rs, src/module.rs), driving rocBLAS for the Linear layers and
// the HIP kernels of this library for everything else.
//
// Data flow of one call over M = B * T tokens (all buffers row-major):
//   Y [M, ld_in] = x W_in            W_in = [q | k | b | v | w | f0 | g0] (one GEMM)
//   F [M, kd]    = Y[:, f0] W_f1     G [M, vd] = bias + Y[:, g0] W_g1
//   q, k, g, b [B, H, T, K], v, w [B, HV, T, V] = project epilogue (conv, SiLU, gates, L2 norm)
//   O [M, vd]    = recurrence (chunk or per-token scan) in the [B, T, HV, V] layout
//   O            = rms_norm_gate(O, G)  (in place)
//   out [M, D]   = O W_o
// At T = 1 with a state the fused decode kernel replaces the epilogue, the
// recurrence and the norm.
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "blas.hpp"
#include "common.hpp"
#include "gdn2_layer.h"
#include "kernels.hpp"

using namespace gdn2;

namespace {

// Parameter table: the reference's field order (src/module.rs:93-111).
const char *const kParamNames[] = {
    "q_proj", "k_proj", "v_proj", "f_proj_0", "f_proj_1", "b_proj", "w_proj", "g_proj_0", "g_proj_1",
    "g_proj_1_bias", "a_log", "dt_bias", "o_norm_weight", "o_proj", "q_conv_w", "k_conv_w", "v_conv_w",
    "decay_factors",
};
enum ParamId {
    P_Q, P_K, P_V, P_F0, P_F1, P_B, P_W, P_G0, P_G1, P_G1_BIAS, P_A_LOG, P_DT_BIAS, P_O_NORM, P_O, P_QCONV,
    P_KCONV, P_VCONV, P_DECAY, P_COUNT
};

struct Dims {
    int64_t D, H, K, HV, V, kd, vd;
    // key-side heads of the recurrence's q, k, g, b: H, or HV when they are
    // laid out as the reference's GVA repeat (GDN2_GVA_REFERENCE, HV > H)
    int64_t Hq, kq;
};

Dims dims_of(const gdn2_config &c) {
    Dims d;
    d.D = c.hidden_size;
    d.H = c.num_heads;
    d.K = c.head_dim;
    d.HV = c.num_v_heads > 0 ? c.num_v_heads : c.num_heads;
    d.V = (int64_t)((float)c.head_dim * c.expand_v);
    d.kd = d.H * d.K;
    d.vd = d.HV * d.V;
    d.Hq = (c.gva_layout == GDN2_GVA_REFERENCE && d.HV > d.H) ? d.HV : d.H;
    d.kq = d.Hq * d.K;
    return d;
}

int param_id(const char *name) {
    if (!name) return -1;
    for (int i = 0; i < P_COUNT; ++i)
        if (std::strcmp(name, kParamNames[i]) == 0) return i;
    return -1;
}

// Shape of a parameter (rows x cols); numel 0 when absent.
int64_t param_shape(const gdn2_config &c, int id, int64_t *rows, int64_t *cols) {
    const Dims d = dims_of(c);
    int64_t r = 0, k = 1;
    switch (id) {
        case P_Q: case P_K: case P_B: r = d.D; k = d.kd; break;
        case P_V: case P_W: r = d.D; k = d.vd; break;
        case P_F0: case P_G0: r = d.D; k = d.V; break;
        case P_F1: r = d.V; k = d.kd; break;
        case P_G1: r = d.V; k = d.vd; break;
        case P_G1_BIAS: r = d.vd; break;
        case P_A_LOG: r = d.H; break;
        case P_DT_BIAS: r = d.kd; break;
        case P_O_NORM: r = d.V; break;
        case P_O: r = d.vd; k = d.D; break;
        case P_QCONV: case P_KCONV: r = d.kd; k = 4; break;
        case P_VCONV: r = d.vd; k = 4; break;
        case P_DECAY:
            if (c.has_min_decay) { r = d.H; k = d.K; } else { r = 0; k = 0; }
            break;
        default: return -1;
    }
    if (rows) *rows = r;
    if (cols) *cols = k;
    return r * k;
}

// SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014).  Each (seed, parameter) pair gets its own
// mixed 64-bit key so that the streams of two parameters are not shifts of
// one another; element i is the (i + 1)-th output of the key's stream.
uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double uniform01(uint64_t seed, int id, uint64_t i) {
    const uint64_t key = mix64(seed ^ mix64(0xD1B54A32D192ED03ull * (uint64_t)(id + 1)));
    const uint64_t z = mix64(key + 0x9E3779B97F4A7C15ull * (i + 1));
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

void init_param(const gdn2_config &c, uint64_t seed, int id, float *out) {
    int64_t rows = 0, cols = 0;
    const int64_t n = param_shape(c, id, &rows, &cols);
    auto U = [&](int64_t i, double lo, double hi) { return lo + (hi - lo) * uniform01(seed, id, (uint64_t)i); };
    switch (id) {
        case P_Q: case P_K: case P_V: case P_F0: case P_F1: case P_B: case P_W: case P_G0: case P_G1: case P_O: {
            // Xavier uniform, gain 2^-2.5, fan_in = rows, fan_out = cols (src/module.rs:121-129)
            const double bound = std::pow(2.0, -2.5) * std::sqrt(6.0 / (double)(rows + cols));
            for (int64_t i = 0; i < n; ++i) out[i] = (float)U(i, -bound, bound);
            break;
        }
        case P_G1_BIAS:  // zero bias (src/module.rs:130-138)
            for (int64_t i = 0; i < n; ++i) out[i] = 0.0f;
            break;
        case P_A_LOG:  // U(ln 1, ln 16) (src/module.rs:151-155)
            for (int64_t i = 0; i < n; ++i) out[i] = (float)U(i, std::log(1.0), std::log(16.0));
            break;
        case P_DT_BIAS:  // inverse softplus of dt (src/module.rs:157-166)
            for (int64_t i = 0; i < n; ++i) {
                const double dt = std::fmax(std::exp(U(i, std::log(0.001), std::log(0.1))), 1e-4);
                out[i] = (float)(dt + std::log(-std::expm1(-dt)));
            }
            break;
        case P_O_NORM:
            for (int64_t i = 0; i < n; ++i) out[i] = 1.0f;
            break;
        case P_QCONV: case P_KCONV: case P_VCONV:  // U(-1/2, 1/2) (src/module.rs:142-149)
            for (int64_t i = 0; i < n; ++i) out[i] = (float)U(i, -0.5, 0.5);
            break;
        case P_DECAY:  // 2.0 iff min_decay (src/module.rs:185-187)
            for (int64_t i = 0; i < n; ++i) out[i] = 2.0f;
            break;
        default: break;
    }
}

std::string fmt_f(double v) {
    char buf[64];
    std::snprintf(buf, sizeof buf, "%g", v);
    return buf;
}

constexpr int kShortConvCache = 3;  // SHORT_CONV_CACHE (src/short_conv.rs:7)
constexpr int64_t kFusedRecurrentMaxSeq = 64;  // FUSED_RECURRENT_MAX_SEQ (src/module.rs:16)

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

struct gdn2_layer {
    gdn2_config cfg;
    Dims d;
    int device = 0;
    Gemm mm;  // the Linear layers' GEMMs
    // The input-side Linear weights share one [D, ld_in] matrix so that x is
    // read by a single GEMM; column offsets of each block:
    int64_t ld_in = 0, off_q = 0, off_k = 0, off_b = 0, off_v = 0, off_w = 0, off_f0 = 0, off_g0 = 0;
    float *w_in = nullptr;
    float *p[P_COUNT] = {};  // standalone parameters (null for those inside w_in)
    void *ws = nullptr;
    size_t ws_bytes = 0;
    void *bws = nullptr;  // backward workspace, grown on demand
    size_t bws_bytes = 0;

    int64_t col_offset(int id) const {
        switch (id) {
            case P_Q: return off_q;
            case P_K: return off_k;
            case P_B: return off_b;
            case P_V: return off_v;
            case P_W: return off_w;
            case P_F0: return off_f0;
            case P_G0: return off_g0;
            default: return -1;
        }
    }
};

struct gdn2_state {
    const gdn2_layer *layer = nullptr;
    int64_t batch = 0;
    bool some = false;
    float *S = nullptr;
    float *conv[2][3] = {};  // ping-pong buffers of the q, k, v caches
    int cur = 0;
};

namespace {

struct Work {
    float *Y, *F, *G, *q, *k, *g, *b, *v, *w, *O, *S0;
    // the recurrence's key-side operands: q, k, g, b themselves, or their
    // expansion to the reference's GVA layout [B, HV, T, K] (GDN2_GVA_REFERENCE)
    float *xq, *xk, *xg, *xb;
    void *chunk;
    size_t chunk_bytes;
};

// Points the recurrence's key-side operands at q, k, g, b (head repeat) or
// at the four expansion buffers that follow in `base` (reference layout),
// and returns the bytes those take.
size_t carve_expanded(const Dims &d, int64_t M, char *base, Work *wk) {
    if (d.Hq == d.H) {
        wk->xq = wk->q; wk->xk = wk->k; wk->xg = wk->g; wk->xb = wk->b;
        return 0;
    }
    const size_t n = align256(sizeof(float) * M * d.kq);
    float **dst[4] = {&wk->xq, &wk->xk, &wk->xg, &wk->xb};
    for (int i = 0; i < 4; ++i) *dst[i] = base ? reinterpret_cast<float *>(base + i * n) : nullptr;
    return 4 * n;
}

// The reference's GVA layout of q, k, g, b (nothing under head repeat).
gdn2_status expand_keys(const Dims &d, int64_t B, int64_t T, const Work &wk, hipStream_t s) {
    if (d.Hq == d.H) return GDN2_OK;
    GvaParams gp{};
    gp.src[0] = wk.q; gp.src[1] = wk.k; gp.src[2] = wk.g; gp.src[3] = wk.b;
    gp.dst[0] = wk.xq; gp.dst[1] = wk.xk; gp.dst[2] = wk.xg; gp.dst[3] = wk.xb;
    gp.B = B; gp.H = d.H; gp.T = T; gp.K = d.K; gp.rep = (int)(d.HV / d.H);
    GDN2_HIP_CHECK(launch_gva_expand(gp, s));
    return GDN2_OK;
}

gdn2_chunk_args chunk_args_for(const gdn2_layer &L, int64_t B, int64_t T, const Work &wk, float *S) {
    const Dims &d = L.d;
    gdn2_chunk_args a{};
    a.q = wk.xq; a.k = wk.xk; a.g = wk.xg; a.b = wk.xb; a.v = wk.v; a.w = wk.w;
    a.state = S; a.out = wk.O;
    a.batch = B; a.num_heads = d.Hq; a.num_v_heads = d.HV; a.seq_len = T; a.head_dim = d.K; a.head_v_dim = d.V;
    // q, k, g, b [B, Hq, T, K] and v, w [B, HV, T, V] (head-major, so that a
    // chunk's rows are one contiguous block); out [B, T, HV, V] for the norm
    a.stride_qk_b = d.Hq * T * d.K; a.stride_qk_h = T * d.K; a.stride_qk_t = d.K;
    a.stride_vw_b = d.HV * T * d.V; a.stride_vw_h = T * d.V; a.stride_vw_t = d.V;
    a.stride_o_b = T * d.vd; a.stride_o_h = d.V; a.stride_o_t = d.vd;
    a.scale = std::pow((double)d.K, -0.5);
    a.chunk_size = L.cfg.chunk_size;
    return a;
}

// Carve the workspace for M = B * T tokens, growing it when needed.
gdn2_status workspace(gdn2_layer &L, int64_t B, int64_t T, bool need_s0, Work *wk) {
    const Dims &d = L.d;
    const int64_t M = B * T;
    Work tmp{};
    gdn2_chunk_args ca = chunk_args_for(L, B, T, tmp, nullptr);
    const size_t chunk_bytes = gdn2_chunk_workspace_bytes(&ca);
    const size_t f = sizeof(float);
    size_t sz[11] = {f * M * L.ld_in, f * M * d.kd, f * M * d.vd, f * M * d.kd, f * M * d.kd, f * M * d.kd,
                     f * M * d.kd, f * M * d.vd, f * M * d.vd, f * M * d.vd,
                     need_s0 ? f * B * d.HV * d.K * d.V : 0};
    size_t total = 0;
    for (size_t s : sz) total += align256(s);
    total += carve_expanded(d, M, nullptr, wk);
    total += align256(chunk_bytes);
    if (total > L.ws_bytes) {
        if (L.ws) {
            GDN2_HIP_CHECK(hipDeviceSynchronize());
            GDN2_HIP_CHECK(hipFree(L.ws));
            L.ws = nullptr;
            L.ws_bytes = 0;
        }
        GDN2_HIP_CHECK(hipMalloc(&L.ws, total));
        L.ws_bytes = total;
    }
    char *base = static_cast<char *>(L.ws);
    float **dst[10] = {&wk->Y, &wk->F, &wk->G, &wk->q, &wk->k, &wk->g, &wk->b, &wk->v, &wk->w, &wk->O};
    for (int i = 0; i < 10; ++i) {
        *dst[i] = reinterpret_cast<float *>(base);
        base += align256(sz[i]);
    }
    wk->S0 = need_s0 ? reinterpret_cast<float *>(base) : nullptr;
    base += align256(sz[10]);
    base += carve_expanded(d, M, base, wk);
    wk->chunk = base;
    wk->chunk_bytes = chunk_bytes;
    return GDN2_OK;
}

// Linear layers of the input side: Y, F, G.
// G holds the g_proj_1 bias only with_bias; the kernels that read G otherwise
// add it themselves (one launch less per call).
gdn2_status input_gemms(gdn2_layer &L, const float *x, int64_t M, const Work &wk, hipStream_t s,
                        bool with_bias = false) {
    const Dims &d = L.d;
    gdn2_status st;
    if ((st = L.mm.run(false, false, M, L.ld_in, d.D, x, d.D, L.w_in, L.ld_in, wk.Y, L.ld_in, 0.0f, s)) != GDN2_OK)
        return st;
    if (lowrank_up_supported((int)d.V, M, wk.Y, L.ld_in, L.off_f0, L.off_g0)) { // a few rows (decode): one small launch for both
        LowRankParams lp{};
        lp.Y = wk.Y; lp.ldY = L.ld_in; lp.off_f0 = L.off_f0; lp.off_g0 = L.off_g0;
        lp.F1 = L.p[P_F1]; lp.G1 = L.p[P_G1]; lp.g_bias = with_bias ? L.p[P_G1_BIAS] : nullptr;
        lp.F = wk.F; lp.G = wk.G;
        lp.M = (int)M; lp.R = (int)d.V; lp.kd = (int)d.kd; lp.vd = (int)d.vd;
        GDN2_HIP_CHECK(launch_lowrank_up(lp, s));
        return GDN2_OK;
    }
    if ((st = L.mm.run(false, false, M, d.kd, d.V, wk.Y + L.off_f0, L.ld_in, L.p[P_F1], d.kd, wk.F, d.kd, 0.0f, s)) !=
        GDN2_OK)
        return st;
    if (with_bias) GDN2_HIP_CHECK(launch_fill_rows(wk.G, d.vd, L.p[P_G1_BIAS], M, d.vd, s));
    return L.mm.run(false, false, M, d.vd, d.V, wk.Y + L.off_g0, L.ld_in, L.p[P_G1], d.vd, wk.G, d.vd,
                    with_bias ? 1.0f : 0.0f, s);
}

gdn2_status project_epilogue(gdn2_layer &L, int64_t B, int64_t T, const float *const conv_in[3], const Work &wk,
                             hipStream_t s) {
    const Dims &d = L.d;
    ProjectParams p{};
    p.Y = wk.Y; p.ldY = L.ld_in;
    p.off_q = L.off_q; p.off_k = L.off_k; p.off_b = L.off_b; p.off_v = L.off_v; p.off_w = L.off_w;
    p.F = wk.F; p.ldF = d.kd;
    p.conv_q_in = conv_in ? conv_in[0] : nullptr;
    p.conv_k_in = conv_in ? conv_in[1] : nullptr;
    p.conv_v_in = conv_in ? conv_in[2] : nullptr;
    p.q_conv_w = L.p[P_QCONV]; p.k_conv_w = L.p[P_KCONV]; p.v_conv_w = L.p[P_VCONV];
    p.a_log = L.p[P_A_LOG]; p.dt_bias = L.p[P_DT_BIAS];
    p.decay_factors = L.cfg.has_min_decay ? L.p[P_DECAY] : nullptr;
    p.q = wk.q; p.k = wk.k; p.g = wk.g; p.b = wk.b; p.v = wk.v; p.w = wk.w;
    p.B = (int)B; p.T = (int)T; p.H = (int)d.H; p.K = (int)d.K; p.HV = (int)d.HV; p.V = (int)d.V;
    p.use_short_conv = L.cfg.use_short_conv; p.allow_neg_eigval = L.cfg.allow_neg_eigval;
    p.min_decay = (float)L.cfg.min_decay; p.one_minus_min_decay = (float)(1.0 - L.cfg.min_decay);
    GDN2_HIP_CHECK(launch_project(p, s));
    return expand_keys(d, B, T, wk, s);
}

// The scan's arguments for the same operands (state in place).
gdn2_recurrent_args recurrent_args_for(const gdn2_chunk_args &ca) {
    gdn2_recurrent_args ra{};
    ra.q = ca.q; ra.k = ca.k; ra.g = ca.g; ra.b = ca.b; ra.v = ca.v; ra.w = ca.w;
    ra.state_in = ca.state; ra.state_out = ca.state; ra.out = ca.out;
    ra.batch = ca.batch; ra.num_heads = ca.num_heads; ra.num_v_heads = ca.num_v_heads; ra.seq_len = ca.seq_len;
    ra.head_dim = ca.head_dim; ra.head_v_dim = ca.head_v_dim;
    ra.stride_qk_b = ca.stride_qk_b; ra.stride_qk_h = ca.stride_qk_h; ra.stride_qk_t = ca.stride_qk_t;
    ra.stride_vw_b = ca.stride_vw_b; ra.stride_vw_h = ca.stride_vw_h; ra.stride_vw_t = ca.stride_vw_t;
    ra.stride_o_b = ca.stride_o_b; ra.stride_o_h = ca.stride_o_h; ra.stride_o_t = ca.stride_o_t;
    ra.scale = ca.scale;
    return ra;
}

// The recurrence over the projected inputs into O; S is updated in place.
// FusedRecurrent mode is the reference's per-token scan (src/kernel/fused_recurrent.rs:11-55).
// Beyond the decode-sized limit (T > 64) it runs the chunk kernels instead: the same
// recurrence, parallel over chunks rather than sequential over every token (about 4x
// faster at a 2048-token prefill of 64 sequences).  Short inputs keep the scan.
gdn2_status recurrence(gdn2_layer &L, int64_t B, int64_t T, int mode, const Work &wk, float *S, hipStream_t s) {
    gdn2_chunk_args ca = chunk_args_for(L, B, T, wk, S);
    if (mode == GDN2_MODE_CHUNK || T > kFusedRecurrentMaxSeq) {
        ca.workspace = wk.chunk;
        ca.workspace_bytes = wk.chunk_bytes;
        const gdn2_status st = gdn2_chunk_fwd_f32(&ca, s);
        if (st != GDN2_NOT_APPLICABLE) return st;
    }
    gdn2_recurrent_args ra = recurrent_args_for(ca);
    return gdn2_recurrent_fwd_f32(&ra, s);
}

// Gated RMSNorm of wk.O into `normed` (wk.O itself when null), then out = normed W_o.
gdn2_status output_side(gdn2_layer &L, int64_t M, bool norm, const Work &wk, float *out, hipStream_t s,
                        float *normed = nullptr) {
    const Dims &d = L.d;
    float *y = normed ? normed : wk.O;
    if (norm)
        GDN2_HIP_CHECK(launch_rmsnorm_gate(y, d.vd, wk.O, d.vd, wk.G, d.vd, L.p[P_G1_BIAS], L.p[P_O_NORM], M, (int)d.HV,
                                           (int)d.V,
                                           (float)L.cfg.norm_eps, s));
    return L.mm.run(false, false, M, d.D, d.vd, y, d.vd, L.p[P_O], d.D, out, d.D, 0.0f, s);
}

gdn2_status check_layer_call(const gdn2_layer *L, const float *x, int64_t B, int64_t T, const void *out,
                             const char *who) {
    if (!L || !x || !out) return fail(GDN2_EINVAL, std::string(who) + ": null argument");
    if (B <= 0 || T < 0) return fail(GDN2_EINVAL, std::string(who) + ": batch must be > 0 and seq_len >= 0");
    if (B * T > INT32_MAX / 4) return fail(GDN2_EINVAL, std::string(who) + ": batch * seq_len too large");
    int dev = -1;
    GDN2_HIP_CHECK(hipGetDevice(&dev));
    if (dev != L->device)
        return fail(GDN2_EINVAL, std::string(who) + ": the layer lives on device " + std::to_string(L->device) +
                                     ", the current device is " + std::to_string(dev));
    return GDN2_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Config
// ---------------------------------------------------------------------------
extern "C" void gdn2_config_default(gdn2_config *c) {
    if (!c) return;
    std::memset(c, 0, sizeof *c);
    c->hidden_size = 2048;
    c->num_heads = 16;
    c->head_dim = 128;
    c->expand_v = 1.0f;
    c->num_v_heads = 0;
    c->use_short_conv = 1;
    c->allow_neg_eigval = 0;
    c->norm_eps = 1e-5;
    c->mode = GDN2_MODE_FUSED_RECURRENT;
    c->chunk_size = 64;
    c->has_min_decay = 0;
    c->min_decay = 0.0;
    c->gva_layout = GDN2_GVA_HEAD_REPEAT;
}

// Gdn2Config::validate (src/config.rs:71-111): same checks, same order, same messages.
extern "C" gdn2_status gdn2_config_validate(const gdn2_config *c) {
    if (!c) return fail(GDN2_EINVAL, "gdn2_config_validate: null config");
    const int64_t h = c->num_heads, hk = c->head_dim;
    if (c->hidden_size <= 0)
        return fail(GDN2_EINVAL, "hidden_size must be > 0, got " + std::to_string(c->hidden_size));
    if (h <= 0) return fail(GDN2_EINVAL, "num_heads must be > 0, got " + std::to_string(h));
    if (hk <= 0) return fail(GDN2_EINVAL, "head_dim must be > 0, got " + std::to_string(hk));
    const float prod = (float)hk * c->expand_v;
    if (!(c->expand_v > 0.0f && prod - std::trunc(prod) == 0.0f))
        return fail(GDN2_EINVAL, "expand_v=" + fmt_f(c->expand_v) +
                                     " must produce an integer head_v_dim when multiplied by head_dim=" +
                                     std::to_string(hk) + " (got " + fmt_f(prod) + ")");
    if (c->num_v_heads != 0) {
        const int64_t hv = c->num_v_heads;
        if (hv <= 0) return fail(GDN2_EINVAL, "num_v_heads must be > 0, got " + std::to_string(hv));
        if (hv < h)
            return fail(GDN2_EINVAL, "num_v_heads=" + std::to_string(hv) + " < num_heads=" + std::to_string(h) +
                                         " is not supported; use num_v_heads >= num_heads (GVA repeats key-side "
                                         "heads)");
        if (hv % h != 0)
            return fail(GDN2_EINVAL, "num_v_heads=" + std::to_string(hv) + " must be divisible by num_heads=" +
                                         std::to_string(h));
    }
    if (c->chunk_size <= 0) return fail(GDN2_EINVAL, "chunk_size must be > 0, got " + std::to_string(c->chunk_size));
    if (!(c->norm_eps > 0.0)) return fail(GDN2_EINVAL, "norm_eps must be > 0, got " + fmt_f(c->norm_eps));
    if (c->mode != GDN2_MODE_FUSED_RECURRENT && c->mode != GDN2_MODE_CHUNK)
        return fail(GDN2_EINVAL, "mode must be GDN2_MODE_FUSED_RECURRENT or GDN2_MODE_CHUNK");
    if (c->gva_layout != GDN2_GVA_HEAD_REPEAT && c->gva_layout != GDN2_GVA_REFERENCE)
        return fail(GDN2_EINVAL, "gva_layout must be GDN2_GVA_HEAD_REPEAT or GDN2_GVA_REFERENCE");
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_config_dims(const gdn2_config *c, int64_t *hv, int64_t *v_head, int64_t *kd,
                                        int64_t *vd) {
    if (!c) return fail(GDN2_EINVAL, "gdn2_config_dims: null config");
    const Dims d = dims_of(*c);
    if (hv) *hv = d.HV;
    if (v_head) *v_head = d.V;
    if (kd) *kd = d.kd;
    if (vd) *vd = d.vd;
    return GDN2_OK;
}

// ---------------------------------------------------------------------------
// Parameters
// ---------------------------------------------------------------------------
extern "C" int gdn2_param_count(void) { return P_COUNT; }

extern "C" const char *gdn2_param_name(int i) { return (i >= 0 && i < P_COUNT) ? kParamNames[i] : nullptr; }

extern "C" int64_t gdn2_param_shape(const gdn2_config *c, const char *name, int64_t *rows, int64_t *cols) {
    const int id = param_id(name);
    if (!c || id < 0) return -1;
    return param_shape(*c, id, rows, cols);
}

extern "C" gdn2_status gdn2_param_init(const gdn2_config *c, uint64_t seed, const char *name, float *host,
                                       int64_t numel) {
    const int id = param_id(name);
    if (!c || !host) return fail(GDN2_EINVAL, "gdn2_param_init: null argument");
    if (id < 0) return fail(GDN2_EINVAL, std::string("gdn2_param_init: unknown parameter ") + (name ? name : ""));
    const int64_t n = param_shape(*c, id, nullptr, nullptr);
    if (n != numel)
        return fail(GDN2_EINVAL, std::string("gdn2_param_init: ") + name + " has " + std::to_string(n) +
                                     " elements, got " + std::to_string(numel));
    init_param(*c, seed, id, host);
    return GDN2_OK;
}

// ---------------------------------------------------------------------------
// Layer
// ---------------------------------------------------------------------------
extern "C" void gdn2_layer_destroy(gdn2_layer *L) {
    if (!L) return;
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(L->device);
    (void)hipDeviceSynchronize();
    L->mm.destroy();
    (void)hipFree(L->w_in);
    for (float *p : L->p) (void)hipFree(p);
    (void)hipFree(L->ws);
    (void)hipFree(L->bws);
    if (prev >= 0) (void)hipSetDevice(prev);
    delete L;
}

extern "C" gdn2_status gdn2_layer_set_param(gdn2_layer *L, const char *name, const float *host, int64_t numel) {
    if (!L || !host) return fail(GDN2_EINVAL, "gdn2_layer_set_param: null argument");
    const int id = param_id(name);
    if (id < 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_set_param: unknown parameter ") + (name ? name : ""));
    int64_t rows = 0, cols = 0;
    const int64_t n = param_shape(L->cfg, id, &rows, &cols);
    if (n == 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_set_param: ") + name + " is absent in this config");
    if (n != numel)
        return fail(GDN2_EINVAL, std::string("gdn2_layer_set_param: ") + name + " has " + std::to_string(n) +
                                     " elements, got " + std::to_string(numel));
    const int64_t off = L->col_offset(id);
    if (off >= 0)
        GDN2_HIP_CHECK(hipMemcpy2D(L->w_in + off, sizeof(float) * L->ld_in, host, sizeof(float) * cols,
                                   sizeof(float) * cols, rows, hipMemcpyHostToDevice));
    else
        GDN2_HIP_CHECK(hipMemcpy(L->p[id], host, sizeof(float) * n, hipMemcpyHostToDevice));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_get_param(const gdn2_layer *L, const char *name, float *host, int64_t numel) {
    if (!L || !host) return fail(GDN2_EINVAL, "gdn2_layer_get_param: null argument");
    const int id = param_id(name);
    if (id < 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_get_param: unknown parameter ") + (name ? name : ""));
    int64_t rows = 0, cols = 0;
    const int64_t n = param_shape(L->cfg, id, &rows, &cols);
    if (n == 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_get_param: ") + name + " is absent in this config");
    if (n != numel)
        return fail(GDN2_EINVAL, std::string("gdn2_layer_get_param: ") + name + " has " + std::to_string(n) +
                                     " elements, got " + std::to_string(numel));
    const int64_t off = L->col_offset(id);
    if (off >= 0)
        GDN2_HIP_CHECK(hipMemcpy2D(host, sizeof(float) * cols, L->w_in + off, sizeof(float) * L->ld_in,
                                   sizeof(float) * cols, rows, hipMemcpyDeviceToHost));
    else
        GDN2_HIP_CHECK(hipMemcpy(host, L->p[id], sizeof(float) * n, hipMemcpyDeviceToHost));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_create(const gdn2_config *c, uint64_t seed, gdn2_layer **out) {
    if (!out) return fail(GDN2_EINVAL, "gdn2_layer_create: null output");
    *out = nullptr;
    gdn2_status st = gdn2_config_validate(c);
    if (st != GDN2_OK) return st;
    if (!gdn2_hip_available()) return fail(GDN2_EHIP, "gdn2_layer_create: no gfx950 device is current");
    const Dims d = dims_of(*c);
    if (d.kd > 8192) return fail(GDN2_NOT_APPLICABLE, "gdn2_layer_create: num_heads * head_dim above 8192");
    gdn2_layer *L = new gdn2_layer();
    L->cfg = *c;
    L->d = d;
    if (hipGetDevice(&L->device) != hipSuccess) {
        delete L;
        return fail(GDN2_EHIP, "gdn2_layer_create: hipGetDevice failed");
    }
    // W_in column blocks, each starting at a multiple of 4 columns (16-byte rows for the kernels)
    auto up4 = [](int64_t v) { return (v + 3) & ~(int64_t)3; };
    int64_t col = 0;
    L->off_q = col; col += up4(d.kd);
    L->off_k = col; col += up4(d.kd);
    L->off_b = col; col += up4(d.kd);
    L->off_v = col; col += up4(d.vd);
    L->off_w = col; col += up4(d.vd);
    L->off_f0 = col; col += up4(d.V);
    L->off_g0 = col; col += up4(d.V);
    L->ld_in = (col + 15) & ~(int64_t)15;
    auto cleanup = [&](gdn2_status s) {
        gdn2_layer_destroy(L);
        return s;
    };
    if ((st = L->mm.init()) != GDN2_OK) return cleanup(st);
    if (hipMalloc(&L->w_in, sizeof(float) * d.D * L->ld_in) != hipSuccess ||
        hipMemset(L->w_in, 0, sizeof(float) * d.D * L->ld_in) != hipSuccess)
        return cleanup(fail(GDN2_EHIP, "gdn2_layer_create: hipMalloc failed"));
    for (int id = 0; id < P_COUNT; ++id) {
        const int64_t n = param_shape(*c, id, nullptr, nullptr);
        if (n == 0) continue;
        if (L->col_offset(id) < 0 && hipMalloc(&L->p[id], sizeof(float) * n) != hipSuccess)
            return cleanup(fail(GDN2_EHIP, "gdn2_layer_create: hipMalloc failed"));
        float *host = new float[n];
        init_param(*c, seed, id, host);
        st = gdn2_layer_set_param(L, kParamNames[id], host, n);
        delete[] host;
        if (st != GDN2_OK) return cleanup(st);
    }
    *out = L;
    return GDN2_OK;
}

extern "C" const gdn2_config *gdn2_layer_config(const gdn2_layer *L) { return L ? &L->cfg : nullptr; }

extern "C" gdn2_status gdn2_layer_forward_train_f32(gdn2_layer *L, const float *x, int64_t B, int64_t T, float *out,
                                                    gdn2_stream_t stream) {
    gdn2_status st = check_layer_call(L, x, B, T, out, "gdn2_layer_forward_train_f32");
    if (st != GDN2_OK || T == 0) return st;
    hipStream_t s = (hipStream_t)stream;
    Work wk{};
    if ((st = workspace(*L, B, T, true, &wk)) != GDN2_OK) return st;
    const int64_t M = B * T;
    if ((st = input_gemms(*L, x, M, wk, s)) != GDN2_OK) return st;
    if ((st = project_epilogue(*L, B, T, nullptr, wk, s)) != GDN2_OK) return st;
    GDN2_HIP_CHECK(launch_fill_rows(wk.S0, 0, nullptr, 1, B * L->d.HV * L->d.K * L->d.V, s));
    if ((st = recurrence(*L, B, T, L->cfg.mode, wk, wk.S0, s)) != GDN2_OK) return st;
    return output_side(*L, M, true, wk, out, s);
}

extern "C" gdn2_status gdn2_layer_forward_f32(gdn2_layer *L, const float *x, int64_t B, int64_t T, gdn2_state *S,
                                              float *out, gdn2_stream_t stream) {
    gdn2_status st = check_layer_call(L, x, B, T, out, "gdn2_layer_forward_f32");
    if (st != GDN2_OK) return st;
    if (!S || S->layer != L) return fail(GDN2_EINVAL, "gdn2_layer_forward_f32: state missing or made for another layer");
    if (S->batch != B)
        return fail(GDN2_EINVAL, "gdn2_layer_forward_f32: state batch " + std::to_string(S->batch) +
                                     " != input batch " + std::to_string(B));
    if (T == 0) return GDN2_OK;
    hipStream_t s = (hipStream_t)stream;
    const Dims &d = L->d;
    const bool sc = L->cfg.use_short_conv != 0;
    Work wk{};
    if ((st = workspace(*L, B, T, false, &wk)) != GDN2_OK) return st;
    const int64_t M = B * T;
    // Option::None: S = 0; Gdn2State::zeros caches when the conv does not replace them
    if (!S->some) {
        GDN2_HIP_CHECK(launch_fill_rows(S->S, 0, nullptr, 1, B * d.HV * d.K * d.V, s));
        if (!sc)
            for (int i = 0; i < 3; ++i)
                GDN2_HIP_CHECK(launch_fill_rows(S->conv[S->cur][i], 0, nullptr, 1, B * 3 * (i < 2 ? d.kd : d.vd), s));
    }
    const float *conv_in[3] = {S->conv[S->cur][0], S->conv[S->cur][1], S->conv[S->cur][2]};
    float *const *conv_out = S->conv[1 - S->cur];
    const bool has_cache = S->some;
    if ((st = input_gemms(*L, x, M, wk, s)) != GDN2_OK) return st;
    if (T == 1 && d.K <= 256 && d.V <= 1024) {
        gdn2_layer_params lp{};
        lp.q_conv_w = L->p[P_QCONV]; lp.k_conv_w = L->p[P_KCONV]; lp.v_conv_w = L->p[P_VCONV];
        lp.a_log = L->p[P_A_LOG]; lp.dt_bias = L->p[P_DT_BIAS];
        lp.decay_factors = L->cfg.has_min_decay ? L->p[P_DECAY] : nullptr;
        lp.o_norm_weight = L->p[P_O_NORM];
        lp.min_decay = L->cfg.min_decay; lp.norm_eps = L->cfg.norm_eps;
        lp.use_short_conv = L->cfg.use_short_conv; lp.allow_neg_eigval = L->cfg.allow_neg_eigval;
        DecodeParams p{};
        p.q_raw = wk.Y + L->off_q; p.k_raw = wk.Y + L->off_k; p.b_raw = wk.Y + L->off_b;
        p.v_raw = wk.Y + L->off_v; p.w_raw = wk.Y + L->off_w; p.f_raw = wk.F; p.gate = wk.G;
        p.gate_bias = L->p[P_G1_BIAS];
        p.ld_q = p.ld_k = p.ld_b = p.ld_v = p.ld_w = L->ld_in;
        p.ld_f = d.kd; p.ld_gate = d.vd; p.ld_out = d.vd;
        p.conv_q_in = has_cache ? conv_in[0] : nullptr;
        p.conv_k_in = has_cache ? conv_in[1] : nullptr;
        p.conv_v_in = has_cache ? conv_in[2] : nullptr;
        p.conv_q_out = conv_out[0]; p.conv_k_out = conv_out[1]; p.conv_v_out = conv_out[2];
        p.q_conv_w = lp.q_conv_w; p.k_conv_w = lp.k_conv_w; p.v_conv_w = lp.v_conv_w;
        p.a_log = lp.a_log; p.dt_bias = lp.dt_bias; p.decay_factors = lp.decay_factors;
        p.o_norm_weight = lp.o_norm_weight;
        p.state = S->S; p.out = wk.O;
        p.B = (int)B; p.H = (int)d.H; p.HV = (int)d.HV; p.rep = (int)(d.HV / d.H); p.K = (int)d.K; p.V = (int)d.V;
        p.use_short_conv = lp.use_short_conv; p.allow_neg_eigval = lp.allow_neg_eigval;
        p.min_decay = (float)lp.min_decay; p.one_minus_min_decay = (float)(1.0 - lp.min_decay);
        p.norm_eps = (float)lp.norm_eps; p.scale = (float)std::pow((double)d.K, -0.5);
        GDN2_HIP_CHECK(launch_decode(p, s));
        if ((st = output_side(*L, M, false, wk, out, s)) != GDN2_OK) return st;
    } else {
        if ((st = project_epilogue(*L, B, T, has_cache ? conv_in : nullptr, wk, s)) != GDN2_OK) return st;
        if (sc) {
            ConvCacheParams cp{};
            cp.Y = wk.Y; cp.ldY = L->ld_in; cp.off_q = L->off_q; cp.off_k = L->off_k; cp.off_v = L->off_v;
            cp.in_q = has_cache ? conv_in[0] : nullptr;
            cp.in_k = has_cache ? conv_in[1] : nullptr;
            cp.in_v = has_cache ? conv_in[2] : nullptr;
            cp.out_q = conv_out[0]; cp.out_k = conv_out[1]; cp.out_v = conv_out[2];
            cp.B = (int)B; cp.T = (int)T; cp.kd = (int)d.kd; cp.vd = (int)d.vd;
            GDN2_HIP_CHECK(launch_conv_cache(cp, s));
        }
        const int mode = T <= kFusedRecurrentMaxSeq ? GDN2_MODE_FUSED_RECURRENT : L->cfg.mode;
        if ((st = recurrence(*L, B, T, mode, wk, S->S, s)) != GDN2_OK) return st;
        if ((st = output_side(*L, M, true, wk, out, s)) != GDN2_OK) return st;
    }
    if (sc) S->cur = 1 - S->cur;
    S->some = true;
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_project_f32(gdn2_layer *L, const float *x, int64_t B, int64_t T,
                                              const gdn2_state *S, float *q, float *k, float *g, float *b, float *v,
                                              float *w, float *gate, gdn2_stream_t stream) {
    gdn2_status st = check_layer_call(L, x, B, T, q, "gdn2_layer_project_f32");
    if (st != GDN2_OK) return st;
    if (!k || !g || !b || !v || !w || !gate) return fail(GDN2_EINVAL, "gdn2_layer_project_f32: null output");
    if (S && (S->layer != L || S->batch != B))
        return fail(GDN2_EINVAL, "gdn2_layer_project_f32: state made for another layer or batch");
    if (T == 0) return GDN2_OK;
    hipStream_t s = (hipStream_t)stream;
    const Dims &d = L->d;
    Work wk{};
    if ((st = workspace(*L, B, T, false, &wk)) != GDN2_OK) return st;
    const int64_t M = B * T;
    if ((st = input_gemms(*L, x, M, wk, s, true)) != GDN2_OK) return st;  // gate out with its bias
    const float *conv_in[3] = {};
    const bool has_cache = S && S->some;
    if (has_cache)
        for (int i = 0; i < 3; ++i) conv_in[i] = S->conv[S->cur][i];
    if ((st = project_epilogue(*L, B, T, has_cache ? conv_in : nullptr, wk, s)) != GDN2_OK) return st;
    // q, k, g, b as the recurrence takes them: [B, H, T, K], or [B, HV, T, K]
    // in the reference's GVA layout (which is what its project returns)
    const size_t nk = sizeof(float) * M * d.kq, nv = sizeof(float) * M * d.vd;
    GDN2_HIP_CHECK(hipMemcpyAsync(q, wk.xq, nk, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(k, wk.xk, nk, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(g, wk.xg, nk, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(b, wk.xb, nk, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(v, wk.v, nv, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(w, wk.w, nv, hipMemcpyDeviceToDevice, s));
    GDN2_HIP_CHECK(hipMemcpyAsync(gate, wk.G, nv, hipMemcpyDeviceToDevice, s));
    return GDN2_OK;
}

// ---------------------------------------------------------------------------
// State
// ---------------------------------------------------------------------------
namespace {
int64_t state_numel(const gdn2_state *S, int which) {
    if (!S || !S->layer) return -1;
    const Dims &d = S->layer->d;
    switch (which) {
        case GDN2_STATE_RECURRENT: return S->batch * d.HV * d.K * d.V;
        case GDN2_STATE_CONV_Q: case GDN2_STATE_CONV_K: return S->batch * kShortConvCache * d.kd;
        case GDN2_STATE_CONV_V: return S->batch * kShortConvCache * d.vd;
        default: return -1;
    }
}

float *state_ptr(const gdn2_state *S, int which) {
    if (which == GDN2_STATE_RECURRENT) return S->S;
    return S->conv[S->cur][which - 1];
}
}  // namespace

extern "C" void gdn2_state_destroy(gdn2_state *S) {
    if (!S) return;
    (void)hipDeviceSynchronize();
    (void)hipFree(S->S);
    for (auto &buf : S->conv)
        for (float *p : buf) (void)hipFree(p);
    delete S;
}

extern "C" gdn2_status gdn2_state_create(const gdn2_layer *L, int64_t batch, gdn2_state **out) {
    if (!L || !out) return fail(GDN2_EINVAL, "gdn2_state_create: null argument");
    if (batch <= 0) return fail(GDN2_EINVAL, "gdn2_state_create: batch must be > 0");
    *out = nullptr;
    gdn2_state *S = new gdn2_state();
    S->layer = L;
    S->batch = batch;
    bool ok = hipMalloc(&S->S, sizeof(float) * state_numel(S, GDN2_STATE_RECURRENT)) == hipSuccess;
    for (int j = 0; j < 2 && ok; ++j)
        for (int i = 0; i < 3 && ok; ++i) {
            const size_t n = sizeof(float) * state_numel(S, i + 1);
            ok = hipMalloc(&S->conv[j][i], n) == hipSuccess && hipMemset(S->conv[j][i], 0, n) == hipSuccess;
        }
    if (!ok || hipMemset(S->S, 0, sizeof(float) * state_numel(S, GDN2_STATE_RECURRENT)) != hipSuccess) {
        gdn2_state_destroy(S);
        return fail(GDN2_EHIP, "gdn2_state_create: device allocation failed");
    }
    *out = S;
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_state_set_zeros(gdn2_state *S) {
    if (!S) return fail(GDN2_EINVAL, "gdn2_state_set_zeros: null state");
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    GDN2_HIP_CHECK(hipMemset(S->S, 0, sizeof(float) * state_numel(S, GDN2_STATE_RECURRENT)));
    for (int i = 0; i < 3; ++i)
        GDN2_HIP_CHECK(hipMemset(S->conv[S->cur][i], 0, sizeof(float) * state_numel(S, i + 1)));
    S->some = true;
    return GDN2_OK;
}

extern "C" void gdn2_state_clear(gdn2_state *S) {
    if (S) S->some = false;
}

extern "C" int gdn2_state_is_some(const gdn2_state *S) { return S && S->some ? 1 : 0; }

extern "C" int64_t gdn2_state_batch(const gdn2_state *S) { return S ? S->batch : -1; }

extern "C" int64_t gdn2_state_numel(const gdn2_state *S, int which) { return state_numel(S, which); }

extern "C" float *gdn2_state_tensor(gdn2_state *S, int which) {
    if (state_numel(S, which) < 0) return nullptr;
    return state_ptr(S, which);
}

extern "C" gdn2_status gdn2_state_read(const gdn2_state *S, int which, float *host, int64_t numel) {
    const int64_t n = state_numel(S, which);
    if (n < 0 || !host) return fail(GDN2_EINVAL, "gdn2_state_read: bad state, tensor index or buffer");
    if (n != numel) return fail(GDN2_EINVAL, "gdn2_state_read: expected " + std::to_string(n) + " elements");
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    GDN2_HIP_CHECK(hipMemcpy(host, state_ptr(S, which), sizeof(float) * n, hipMemcpyDeviceToHost));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_state_write(gdn2_state *S, int which, const float *host, int64_t numel) {
    const int64_t n = state_numel(S, which);
    if (n < 0 || !host) return fail(GDN2_EINVAL, "gdn2_state_write: bad state, tensor index or buffer");
    if (n != numel) return fail(GDN2_EINVAL, "gdn2_state_write: expected " + std::to_string(n) + " elements");
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    if (!S->some) {
        GDN2_HIP_CHECK(hipMemset(S->S, 0, sizeof(float) * state_numel(S, GDN2_STATE_RECURRENT)));
        for (int i = 0; i < 3; ++i)
            GDN2_HIP_CHECK(hipMemset(S->conv[S->cur][i], 0, sizeof(float) * state_numel(S, i + 1)));
    }
    GDN2_HIP_CHECK(hipMemcpy(state_ptr(S, which), host, sizeof(float) * n, hipMemcpyHostToDevice));
    S->some = true;
    return GDN2_OK;
}

// ---------------------------------------------------------------------------
// State interchange: safetensors (8-byte little-endian header length, JSON
// header padded with spaces to an 8-byte boundary, raw little-endian data).
// Tensor names are the reference's Gdn2State fields (src/module.rs:30-40).
// ---------------------------------------------------------------------------
namespace {

const char *const kStateNames[4] = {"recurrent", "conv_q", "conv_k", "conv_v"};

std::vector<int64_t> state_shape(const gdn2_state *S, int which) {
    const Dims &d = S->layer->d;
    if (which == GDN2_STATE_RECURRENT) return {S->batch, d.HV, d.K, d.V};
    return {S->batch, kShortConvCache, which == GDN2_STATE_CONV_V ? d.vd : d.kd};
}

// A minimal JSON reader for safetensors headers: objects, arrays, strings and
// non-negative integers.  Values are kept as raw text spans; objects map keys
// to spans.
struct Json {
    const char *p, *end;
    bool ok = true;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) { ++p; return true; }
        return false;
    }
    std::string str() {
        ws();
        std::string s;
        if (p >= end || *p != '"') { ok = false; return s; }
        for (++p; p < end && *p != '"'; ++p) {
            if (*p == '\\') { // escapes: keep the escaped character
                if (++p >= end) break;
            }
            s.push_back(*p);
        }
        if (p >= end) { ok = false; return s; }
        ++p;
        return s;
    }
    int64_t integer() {
        ws();
        int64_t v = 0;
        if (p >= end || *p < '0' || *p > '9') { ok = false; return 0; }
        for (; p < end && *p >= '0' && *p <= '9'; ++p) {
            if (v > (int64_t(1) << 58)) { ok = false; return 0; }
            v = v * 10 + (*p - '0');
        }
        return v;
    }
    // skips any value (used for unknown metadata entries); nesting deeper
    // than kMaxDepth is rejected rather than recursed into
    static constexpr int kMaxDepth = 64;
    void skip(int depth = 0) {
        ws();
        if (p >= end || depth > kMaxDepth) { ok = false; return; }
        if (*p == '"') { str(); return; }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            ++p;
            if (eat(close)) return;
            do {
                if (open == '{') { str(); if (!eat(':')) { ok = false; return; } }
                skip(depth + 1);
                if (!ok) return;
            } while (eat(','));
            if (!eat(close)) ok = false;
            return;
        }
        while (p < end && *p != ',' && *p != '}' && *p != ']') ++p; // number / literal
    }
};

struct TensorEntry {
    std::string dtype;
    std::vector<int64_t> shape;
    int64_t begin = -1, end = -1;
};

}  // namespace

// Gdn2State interchange (the reference keeps the state as four tensors,
// src/module.rs:30-40): serialised as safetensors with those names.
extern "C" gdn2_status gdn2_state_serialize(const gdn2_state *S, void *buf, size_t cap, size_t *len) {
    if (!S || !len) return fail(GDN2_EINVAL, "gdn2_state_serialize: null argument");
    if (!S->some) return fail(GDN2_EINVAL, "gdn2_state_serialize: the state is empty (None)");
    const Dims &d = S->layer->d;
    std::string h = "{\"__metadata__\":{\"format\":\"gdn2_state\",\"num_heads\":\"" + std::to_string(d.H) +
                    "\",\"num_v_heads\":\"" + std::to_string(d.HV) + "\",\"head_dim\":\"" + std::to_string(d.K) +
                    "\",\"head_v_dim\":\"" + std::to_string(d.V) + "\"}";
    int64_t off = 0;
    for (int w = 0; w < 4; ++w) {
        const std::vector<int64_t> sh = state_shape(S, w);
        const int64_t bytes = 4 * state_numel(S, w);
        h += ",\"" + std::string(kStateNames[w]) + "\":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t i = 0; i < sh.size(); ++i) h += (i ? "," : "") + std::to_string(sh[i]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + bytes) + "]}";
        off += bytes;
    }
    h += "}";
    while ((8 + h.size()) % 8) h.push_back(' ');
    const size_t total = 8 + h.size() + (size_t)off;
    *len = total;
    if (!buf) return GDN2_OK;
    if (cap < total) return fail(GDN2_EINVAL, "gdn2_state_serialize: buffer too small (" + std::to_string(total) +
                                                  " bytes needed)");
    unsigned char *b = static_cast<unsigned char *>(buf);
    const uint64_t hn = h.size();
    for (int i = 0; i < 8; ++i) b[i] = (unsigned char)(hn >> (8 * i));
    std::memcpy(b + 8, h.data(), h.size());
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    unsigned char *data = b + 8 + h.size();
    for (int w = 0; w < 4; ++w) { // f32 is little-endian on the host and the device
        const size_t bytes = 4 * (size_t)state_numel(S, w);
        GDN2_HIP_CHECK(hipMemcpy(data, state_ptr(S, w), bytes, hipMemcpyDeviceToHost));
        data += bytes;
    }
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_state_deserialize(gdn2_state *S, const void *buf, size_t len) {
    const std::string who = "gdn2_state_deserialize: ";
    if (!S || !buf) return fail(GDN2_EINVAL, who + "null argument");
    const unsigned char *b = static_cast<const unsigned char *>(buf);
    if (len < 8) return fail(GDN2_EINVAL, who + "truncated header");
    uint64_t hn = 0;
    for (int i = 0; i < 8; ++i) hn |= (uint64_t)b[i] << (8 * i);
    if (hn > len - 8) return fail(GDN2_EINVAL, who + "header length beyond the buffer");
    const size_t data_len = len - 8 - (size_t)hn;
    Json js{reinterpret_cast<const char *>(b + 8), reinterpret_cast<const char *>(b + 8 + hn)};
    TensorEntry ent[4];
    bool seen[4] = {false, false, false, false};
    if (!js.eat('{')) return fail(GDN2_EINVAL, who + "header is not a JSON object");
    if (!js.eat('}')) {
        do {
            const std::string key = js.str();
            if (!js.ok || !js.eat(':')) return fail(GDN2_EINVAL, who + "malformed header");
            int w = -1;
            for (int i = 0; i < 4; ++i)
                if (key == kStateNames[i]) w = i;
            if (key == "__metadata__") {
                js.skip();
            } else if (w < 0) {
                return fail(GDN2_EINVAL, who + "unexpected tensor '" + key + "'");
            } else {
                if (seen[w]) return fail(GDN2_EINVAL, who + "tensor '" + key + "' twice");
                seen[w] = true;
                if (!js.eat('{')) return fail(GDN2_EINVAL, who + "malformed entry for '" + key + "'");
                do {
                    const std::string f = js.str();
                    if (!js.ok || !js.eat(':')) return fail(GDN2_EINVAL, who + "malformed entry for '" + key + "'");
                    if (f == "dtype") {
                        ent[w].dtype = js.str();
                    } else if (f == "shape" || f == "data_offsets") {
                        std::vector<int64_t> v;
                        if (!js.eat('[')) return fail(GDN2_EINVAL, who + "malformed " + f);
                        if (!js.eat(']')) {
                            do v.push_back(js.integer());
                            while (js.ok && js.eat(','));
                            if (!js.eat(']')) return fail(GDN2_EINVAL, who + "malformed " + f);
                        }
                        if (f == "shape") {
                            ent[w].shape = v;
                        } else if (v.size() == 2) {
                            ent[w].begin = v[0];
                            ent[w].end = v[1];
                        }
                    } else {
                        js.skip();
                    }
                    if (!js.ok) return fail(GDN2_EINVAL, who + "malformed entry for '" + key + "'");
                } while (js.eat(','));
                if (!js.eat('}')) return fail(GDN2_EINVAL, who + "malformed entry for '" + key + "'");
            }
            if (!js.ok) return fail(GDN2_EINVAL, who + "malformed header");
        } while (js.eat(','));
        if (!js.eat('}')) return fail(GDN2_EINVAL, who + "malformed header");
    }
    for (int w = 0; w < 4; ++w) {
        const std::string nm = kStateNames[w];
        if (!seen[w]) return fail(GDN2_EINVAL, who + "tensor '" + nm + "' missing");
        if (ent[w].dtype != "F32") return fail(GDN2_EINVAL, who + "'" + nm + "' is " + ent[w].dtype + ", not F32");
        if (ent[w].shape != state_shape(S, w)) return fail(GDN2_EINVAL, who + "'" + nm + "' has the wrong shape");
        if (ent[w].begin < 0 || ent[w].end - ent[w].begin != 4 * state_numel(S, w) || (size_t)ent[w].end > data_len)
            return fail(GDN2_EINVAL, who + "'" + nm + "' has bad data offsets");
    }
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    const unsigned char *data = b + 8 + hn;
    for (int w = 0; w < 4; ++w)
        GDN2_HIP_CHECK(hipMemcpy(state_ptr(S, w), data + ent[w].begin, 4 * (size_t)state_numel(S, w),
                                 hipMemcpyHostToDevice));
    S->some = true;
    return GDN2_OK;
}

// ---------------------------------------------------------------------------
// Backward: the gradients burn's autodiff takes through forward /
// forward_train (tests/autodiff.rs:153-205), with the chunked recurrence
// adjoint of gdn2_chunk_bwd_f32 in the middle.  Everything is recomputed from
// x; nothing is kept from the forward call.
//
//   dy [M, vd]       = d_out W_o^T                      dW_o   (+)= y^T d_out
//   dO, dG           = rms_norm_gate adjoint            d o_norm_weight (+)= column sums
//   dq .. dw         = gdn2_chunk_bwd_f32(dO, d_state)  dS0
//   dY [M, ld_in]    = projection epilogue + short-conv adjoints (q|k|b|v|w columns)
//   dY[:, f0] = dF W_f1^T, dY[:, g0] = dG W_g1^T        dW_f1, dW_g1, bias, dt_bias, A_log, decay
//   dW_in (+)= x^T dY,  dx = dY W_in^T
// ---------------------------------------------------------------------------
struct gdn2_layer_grads {
    const gdn2_layer *layer = nullptr;
    float *g_in = nullptr;   // [D, ld_in]: gradient of W_in, same column blocks
    float *p[P_COUNT] = {};  // gradients of the standalone parameters
};

// What forward_train computes before the norm, kept for the backward instead
// of recomputing it: Y, F, G, the kernel operands q .. w and the recurrence
// output O (pre-norm); for heads the chunked backward takes, also the
// recurrence's per-chunk quantities (the chunked backward's workspace as
// gdn2_chunk_fwd_train_f32 leaves it, the reference's FusedBackwardInputs).
struct gdn2_layer_saved {
    const gdn2_layer *layer = nullptr;
    int64_t batch = 0, seq_len = 0;
    bool filled = false;
    void *buf = nullptr;
    Work fw{};
    void *chunk = nullptr;    // the chunked backward's workspace (inside buf), or null
    size_t chunk_bytes = 0;
    bool chunk_filled = false; // the last forward_train_saved ran the training forward into it
};

namespace {

constexpr int kColParts = 256;  // row split of the column sums
constexpr int kConvTBlock = 64; // tokens per thread in the short-conv adjoint

struct BwdWork {
    Work fw;                      // the forward's buffers (Y, F, G, q .. w, O) and the chunk workspace
    float *S0, *Sf;               // state entering the call; the forward's working copy
    float *y, *dy, *dO, *dG;      // [M, vd]
    float *dq, *dk, *dg, *db;     // [B, H, T, K]
    float *dxq, *dxk, *dxg, *dxb; // the recurrence's: dq .. db, or [B, HV, T, K] in the reference's GVA layout
    float *dv, *dw;               // [B, HV, T, V]
    float *dY;                    // [M, ld_in]
    float *DU;                    // [M, 2 kd + vd], short conv only
    float *dF, *PA, *PD;          // [M, kd]; PD with min_decay only
    float *dS0;                   // dS0 when the caller takes none
    float *wpart;                 // conv weight partials, short conv only
    float *part;                  // column-sum partials
};

gdn2_status bwd_workspace(gdn2_layer &L, int64_t B, int64_t T, bool recompute, BwdWork *bw) {
    const Dims &d = L.d;
    const int64_t M = B * T;
    const bool sc = L.cfg.use_short_conv != 0, md = L.cfg.has_min_decay != 0;
    const int64_t ctot = 2 * d.kd + d.vd, nblk = (T + kConvTBlock - 1) / kConvTBlock;
    Work tmp{};
    gdn2_chunk_args ca = chunk_args_for(L, B, T, tmp, nullptr);
    gdn2_chunk_bwd_args ba{};
    ba.fwd = ca;
    gdn2_recurrent_bwd_args ra{};
    ra.fwd = recurrent_args_for(ca);
    const size_t chunk_bytes = std::max({gdn2_chunk_workspace_bytes(&ca), gdn2_chunk_bwd_workspace_bytes(&ba),
                                         chunk_bwd_supported((int)d.K, (int)d.V) ? size_t(0)
                                                                             : gdn2_recurrent_bwd_workspace_bytes(&ra)});
    const size_t f = sizeof(float), nS = f * B * d.HV * d.K * d.V;
    const size_t nk = f * M * d.kd, nv = f * M * d.vd, nY = f * M * L.ld_in;
    const size_t rk = recompute ? nk : 0, rv = recompute ? nv : 0;  // the forward's buffers, when recomputed
    const size_t nx = d.Hq == d.H ? 0 : f * M * d.kq;               // the reference's GVA layout
    const int64_t part_cols = std::max<int64_t>(std::max(d.kd, d.vd), 4 * ctot);
    struct Slot {
        float **ptr;
        size_t bytes;
    } slots[] = {
        {&bw->fw.Y, recompute ? nY : 0}, {&bw->fw.F, rk}, {&bw->fw.G, rv}, {&bw->fw.q, rk}, {&bw->fw.k, rk},
        {&bw->fw.g, rk}, {&bw->fw.b, rk}, {&bw->fw.v, rv}, {&bw->fw.w, rv}, {&bw->fw.O, rv},
        {&bw->S0, nS}, {&bw->Sf, recompute ? nS : 0}, {&bw->dS0, nS},
        {&bw->y, nv}, {&bw->dy, nv}, {&bw->dO, nv}, {&bw->dG, nv},
        {&bw->dq, nk}, {&bw->dk, nk}, {&bw->dg, nk}, {&bw->db, nk}, {&bw->dv, nv}, {&bw->dw, nv},
        {&bw->dxq, nx}, {&bw->dxk, nx}, {&bw->dxg, nx}, {&bw->dxb, nx},
        {&bw->fw.xq, recompute ? nx : 0}, {&bw->fw.xk, recompute ? nx : 0}, {&bw->fw.xg, recompute ? nx : 0},
        {&bw->fw.xb, recompute ? nx : 0},
        {&bw->dY, nY}, {&bw->DU, sc ? f * M * ctot : 0}, {&bw->dF, nk}, {&bw->PA, nk}, {&bw->PD, md ? nk : 0},
        {&bw->wpart, sc ? f * B * nblk * 4 * ctot : 0}, {&bw->part, f * kColParts * part_cols},
    };
    size_t total = align256(chunk_bytes);
    for (const Slot &sl : slots) total += align256(sl.bytes);
    if (total > L.bws_bytes) {
        if (L.bws) {
            GDN2_HIP_CHECK(hipDeviceSynchronize());
            GDN2_HIP_CHECK(hipFree(L.bws));
            L.bws = nullptr;
            L.bws_bytes = 0;
        }
        GDN2_HIP_CHECK(hipMalloc(&L.bws, total));
        L.bws_bytes = total;
    }
    char *base = static_cast<char *>(L.bws);
    bw->fw.chunk = base;
    bw->fw.chunk_bytes = chunk_bytes;
    base += align256(chunk_bytes);
    for (const Slot &sl : slots) {
        *sl.ptr = sl.bytes ? reinterpret_cast<float *>(base) : nullptr;
        base += align256(sl.bytes);
    }
    bw->fw.S0 = nullptr;
    if (d.Hq == d.H) { // head repeat: the recurrence works on q .. b themselves
        bw->dxq = bw->dq; bw->dxk = bw->dk; bw->dxg = bw->dg; bw->dxb = bw->db;
        bw->fw.xq = bw->fw.q; bw->fw.xk = bw->fw.k; bw->fw.xg = bw->fw.g; bw->fw.xb = bw->fw.b;
    }
    return GDN2_OK;
}

gdn2_status check_state_arg(const gdn2_layer *L, const gdn2_state *S, int64_t B, const char *what) {
    if (S && (S->layer != L || S->batch != B))
        return fail(GDN2_EINVAL, std::string("gdn2_layer_backward_f32: ") + what + " made for another layer or batch");
    return GDN2_OK;
}

}  // namespace

extern "C" void gdn2_layer_saved_destroy(gdn2_layer_saved *A) {
    if (!A) return;
    (void)hipDeviceSynchronize();
    (void)hipFree(A->buf);
    delete A;
}

extern "C" gdn2_status gdn2_layer_saved_create(const gdn2_layer *L, int64_t B, int64_t T, gdn2_layer_saved **out) {
    if (!L || !out) return fail(GDN2_EINVAL, "gdn2_layer_saved_create: null argument");
    *out = nullptr;
    if (B <= 0 || T < 0 || B * T > INT32_MAX / 4)
        return fail(GDN2_EINVAL, "gdn2_layer_saved_create: batch must be > 0, seq_len >= 0, batch * seq_len bounded");
    const Dims &d = L->d;
    const size_t M = (size_t)(B * T), f = sizeof(float);
    size_t cbytes = 0;
    if (T > 0 && chunk_bwd_supported((int)d.K, (int)d.V)) {
        Work tmp{};
        gdn2_chunk_bwd_args ba{};
        ba.fwd = chunk_args_for(*L, B, T, tmp, nullptr);
        cbytes = gdn2_chunk_bwd_workspace_bytes(&ba);
    }
    const size_t sz[11] = {f * M * L->ld_in, f * M * d.kd, f * M * d.vd, f * M * d.kd, f * M * d.kd, f * M * d.kd,
                           f * M * d.kd,     f * M * d.vd, f * M * d.vd, f * M * d.vd, cbytes};
    size_t total = 0;
    for (size_t v : sz) total += align256(v);
    Work probe{};
    total += carve_expanded(d, (int64_t)M, nullptr, &probe);
    gdn2_layer_saved *A = new gdn2_layer_saved();
    A->layer = L;
    A->batch = B;
    A->seq_len = T;
    if (total && hipMalloc(&A->buf, total) != hipSuccess) {
        delete A;
        return fail(GDN2_EHIP, "gdn2_layer_saved_create: device allocation failed");
    }
    char *base = static_cast<char *>(A->buf);
    float **dst[10] = {&A->fw.Y, &A->fw.F, &A->fw.G, &A->fw.q, &A->fw.k, &A->fw.g, &A->fw.b, &A->fw.v, &A->fw.w, &A->fw.O};
    for (int i = 0; i < 10; ++i) {
        *dst[i] = reinterpret_cast<float *>(base);
        base += align256(sz[i]);
    }
    A->chunk = cbytes ? base : nullptr;
    A->chunk_bytes = cbytes;
    base += align256(cbytes);
    carve_expanded(d, (int64_t)M, base, &A->fw);
    *out = A;
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_forward_train_saved_f32(gdn2_layer *L, const float *x, int64_t B, int64_t T,
                                                          float *out, gdn2_layer_saved *A, gdn2_stream_t stream) {
    gdn2_status st = check_layer_call(L, x, B, T, out, "gdn2_layer_forward_train_saved_f32");
    if (st != GDN2_OK) return st;
    if (!A || A->layer != L || A->batch != B || A->seq_len != T)
        return fail(GDN2_EINVAL, "gdn2_layer_forward_train_saved_f32: saved missing or made for another layer or shape");
    A->filled = false;
    A->chunk_filled = false;
    if (T == 0) {
        A->filled = true;
        return GDN2_OK;
    }
    hipStream_t s = (hipStream_t)stream;
    Work wk{};
    if ((st = workspace(*L, B, T, true, &wk)) != GDN2_OK) return st;
    Work sv = A->fw;
    sv.chunk = wk.chunk;
    sv.chunk_bytes = wk.chunk_bytes;
    sv.S0 = wk.S0;
    const int64_t M = B * T;
    if ((st = input_gemms(*L, x, M, sv, s)) != GDN2_OK) return st;
    if ((st = project_epilogue(*L, B, T, nullptr, sv, s)) != GDN2_OK) return st;
    GDN2_HIP_CHECK(launch_fill_rows(wk.S0, 0, nullptr, 1, B * L->d.HV * L->d.K * L->d.V, s));
    st = GDN2_NOT_APPLICABLE;
    // where the recurrence runs the chunk kernels, the training forward keeps
    // their per-chunk quantities for the backward
    if (A->chunk && (L->cfg.mode == GDN2_MODE_CHUNK || T > kFusedRecurrentMaxSeq)) {
        gdn2_chunk_bwd_args ba{};
        ba.fwd = chunk_args_for(*L, B, T, sv, wk.S0);
        ba.workspace = A->chunk;
        ba.workspace_bytes = A->chunk_bytes;
        st = gdn2_chunk_fwd_train_f32(&ba, s);
        if (st != GDN2_OK && st != GDN2_NOT_APPLICABLE) return st;
        A->chunk_filled = st == GDN2_OK;
    }
    if (st == GDN2_NOT_APPLICABLE && (st = recurrence(*L, B, T, L->cfg.mode, sv, wk.S0, s)) != GDN2_OK) return st;
    if ((st = output_side(*L, M, true, sv, out, s, wk.O)) != GDN2_OK) return st;  // O stays pre-norm
    A->filled = true;
    return GDN2_OK;
}

extern "C" void gdn2_layer_grads_destroy(gdn2_layer_grads *G) {
    if (!G) return;
    (void)hipDeviceSynchronize();
    (void)hipFree(G->g_in);
    for (float *p : G->p) (void)hipFree(p);
    delete G;
}

extern "C" gdn2_status gdn2_layer_grads_create(const gdn2_layer *L, gdn2_layer_grads **out) {
    if (!L || !out) return fail(GDN2_EINVAL, "gdn2_layer_grads_create: null argument");
    *out = nullptr;
    gdn2_layer_grads *G = new gdn2_layer_grads();
    G->layer = L;
    const size_t nin = sizeof(float) * L->d.D * L->ld_in;
    bool ok = hipMalloc(&G->g_in, nin) == hipSuccess && hipMemset(G->g_in, 0, nin) == hipSuccess;
    for (int id = 0; id < P_COUNT && ok; ++id) {
        const int64_t n = param_shape(L->cfg, id, nullptr, nullptr);
        if (n == 0 || L->col_offset(id) >= 0) continue;
        ok = hipMalloc(&G->p[id], sizeof(float) * n) == hipSuccess &&
             hipMemset(G->p[id], 0, sizeof(float) * n) == hipSuccess;
    }
    if (!ok) {
        gdn2_layer_grads_destroy(G);
        return fail(GDN2_EHIP, "gdn2_layer_grads_create: device allocation failed");
    }
    *out = G;
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_grads_zero(gdn2_layer_grads *G, gdn2_stream_t stream) {
    if (!G) return fail(GDN2_EINVAL, "gdn2_layer_grads_zero: null grads");
    hipStream_t s = (hipStream_t)stream;
    GDN2_HIP_CHECK(launch_fill_rows(G->g_in, 0, nullptr, 1, G->layer->d.D * G->layer->ld_in, s));
    for (int id = 0; id < P_COUNT; ++id)
        if (G->p[id])
            GDN2_HIP_CHECK(launch_fill_rows(G->p[id], 0, nullptr, 1, param_shape(G->layer->cfg, id, nullptr, nullptr), s));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_grads_get(const gdn2_layer_grads *G, const char *name, float *host, int64_t numel) {
    if (!G || !host) return fail(GDN2_EINVAL, "gdn2_layer_grads_get: null argument");
    const gdn2_layer *L = G->layer;
    const int id = param_id(name);
    if (id < 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_grads_get: unknown parameter ") + (name ? name : ""));
    int64_t rows = 0, cols = 0;
    const int64_t n = param_shape(L->cfg, id, &rows, &cols);
    if (n == 0) return fail(GDN2_EINVAL, std::string("gdn2_layer_grads_get: ") + name + " is absent in this config");
    if (n != numel)
        return fail(GDN2_EINVAL, std::string("gdn2_layer_grads_get: ") + name + " has " + std::to_string(n) +
                                     " elements, got " + std::to_string(numel));
    GDN2_HIP_CHECK(hipDeviceSynchronize());
    const int64_t off = L->col_offset(id);
    if (off >= 0)
        GDN2_HIP_CHECK(hipMemcpy2D(host, sizeof(float) * cols, G->g_in + off, sizeof(float) * L->ld_in,
                                   sizeof(float) * cols, rows, hipMemcpyDeviceToHost));
    else
        GDN2_HIP_CHECK(hipMemcpy(host, G->p[id], sizeof(float) * n, hipMemcpyDeviceToHost));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_layer_backward_f32(gdn2_layer *L, const float *x, int64_t B, int64_t T,
                                               const gdn2_state *state_in, const gdn2_layer_saved *saved,
                                               const float *d_out,
                                               const gdn2_state *d_state, float *dx, gdn2_state *d_state_in,
                                               gdn2_layer_grads *G, int accumulate, gdn2_stream_t stream) {
    const char *who = "gdn2_layer_backward_f32";
    gdn2_status st = check_layer_call(L, x, B, T, d_out, who);
    if (st != GDN2_OK) return st;
    if (!G || G->layer != L) return fail(GDN2_EINVAL, "gdn2_layer_backward_f32: grads missing or made for another layer");
    if ((st = check_state_arg(L, state_in, B, "state_in")) != GDN2_OK) return st;
    if ((st = check_state_arg(L, d_state, B, "d_state")) != GDN2_OK) return st;
    if ((st = check_state_arg(L, d_state_in, B, "d_state_in")) != GDN2_OK) return st;
    if (d_state_in && (d_state_in == state_in || d_state_in == d_state))
        return fail(GDN2_EINVAL, "gdn2_layer_backward_f32: d_state_in must be a state of its own");
    if (saved && (saved->layer != L || saved->batch != B || saved->seq_len != T || !saved->filled))
        return fail(GDN2_EINVAL, "gdn2_layer_backward_f32: saved made for another layer or shape, or never filled");
    if (saved && state_in && state_in->some)
        return fail(GDN2_EINVAL, "gdn2_layer_backward_f32: saved activations come from forward_train (no state_in)");
    const Dims &d = L->d;
    // the recurrence's adjoint: the chunked kernels where they apply, else the
    // scan's (which returns GDN2_NOT_APPLICABLE for heads beyond its LDS)
    const bool use_chunk = chunk_bwd_supported((int)d.K, (int)d.V);
    hipStream_t s = (hipStream_t)stream;
    const bool sc = L->cfg.use_short_conv != 0, md = L->cfg.has_min_decay != 0;
    const bool has_state = state_in && state_in->some, has_ds = d_state && d_state->some;
    const float beta = accumulate ? 1.0f : 0.0f;
    const int64_t M = B * T, nS = B * d.HV * d.K * d.V;
    const int64_t ncache[3] = {B * 3 * d.kd, B * 3 * d.kd, B * 3 * d.vd};

    // gradient of the caches on entry when they do not enter the conv: a pass-through
    // without short conv (the forward leaves them unchanged), zero otherwise
    auto pass_caches = [&](bool through) -> gdn2_status {
        for (int i = 0; i < 3; ++i) {
            float *dst = d_state_in->conv[d_state_in->cur][i];
            if (through && has_ds)
                GDN2_HIP_CHECK(hipMemcpyAsync(dst, d_state->conv[d_state->cur][i], sizeof(float) * ncache[i],
                                              hipMemcpyDeviceToDevice, s));
            else
                GDN2_HIP_CHECK(launch_fill_rows(dst, 0, nullptr, 1, ncache[i], s));
        }
        return GDN2_OK;
    };

    if (T == 0) {  // forward is a no-op: the state's gradient passes through
        if (!accumulate && (st = gdn2_layer_grads_zero(G, stream)) != GDN2_OK) return st;
        if (d_state_in) {
            if (has_ds)
                GDN2_HIP_CHECK(hipMemcpyAsync(d_state_in->S, d_state->S, sizeof(float) * nS, hipMemcpyDeviceToDevice, s));
            else
                GDN2_HIP_CHECK(launch_fill_rows(d_state_in->S, 0, nullptr, 1, nS, s));
            if ((st = pass_caches(true)) != GDN2_OK) return st;
            d_state_in->some = true;
        }
        return GDN2_OK;
    }

    BwdWork bw{};
    if ((st = bwd_workspace(*L, B, T, saved == nullptr, &bw)) != GDN2_OK) return st;
    if (saved) {  // the forward's buffers come from forward_train_saved
        void *chunk = bw.fw.chunk;
        const size_t chunk_bytes = bw.fw.chunk_bytes;
        bw.fw = saved->fw;
        bw.fw.chunk = chunk;
        bw.fw.chunk_bytes = chunk_bytes;
    }
    const Work &fw = bw.fw;
    const float *conv_in[3] = {};
    if (has_state)
        for (int i = 0; i < 3; ++i) conv_in[i] = state_in->conv[state_in->cur][i];
    if (has_state)
        GDN2_HIP_CHECK(hipMemcpyAsync(bw.S0, state_in->S, sizeof(float) * nS, hipMemcpyDeviceToDevice, s));
    else
        GDN2_HIP_CHECK(launch_fill_rows(bw.S0, 0, nullptr, 1, nS, s));

    if (!saved) {  // forward recomputation up to the recurrence output O
        if ((st = input_gemms(*L, x, M, fw, s)) != GDN2_OK) return st;
        if ((st = project_epilogue(*L, B, T, has_state ? conv_in : nullptr, fw, s)) != GDN2_OK) return st;
        GDN2_HIP_CHECK(hipMemcpyAsync(bw.Sf, bw.S0, sizeof(float) * nS, hipMemcpyDeviceToDevice, s));
        if ((st = recurrence(*L, B, T, use_chunk ? GDN2_MODE_CHUNK : GDN2_MODE_FUSED_RECURRENT, fw, bw.Sf, s)) !=
            GDN2_OK)
            return st;
    }

    // o_proj and the gated RMSNorm
    if ((st = L->mm.run(false, true, M, d.vd, d.D, d_out, d.D, L->p[P_O], d.D, bw.dy, d.vd, 0.0f, s)) != GDN2_OK)
        return st;
    NormBwdParams np{};
    np.O = fw.O; np.G = fw.G; np.weight = L->p[P_O_NORM]; np.gate_bias = L->p[P_G1_BIAS]; np.HV = (int)d.HV;
    np.dy = bw.dy; np.y = bw.y; np.dO = bw.dO; np.dG = bw.dG;
    np.rows = M * d.HV; np.V = (int)d.V; np.eps = (float)L->cfg.norm_eps;
    GDN2_HIP_CHECK(launch_rmsnorm_gate_bwd(np, s));
    if ((st = L->mm.run(true, false, d.vd, d.D, M, bw.y, d.vd, d_out, d.D, G->p[P_O], d.D, beta, s)) != GDN2_OK)
        return st;
    GDN2_HIP_CHECK(launch_colsum(bw.dy, M, d.vd, d.vd, 1, (int)d.HV, G->p[P_O_NORM], accumulate, bw.part, kColParts, s));

    // the recurrence
    if (use_chunk) {
        gdn2_chunk_bwd_args ba{};
        ba.fwd = chunk_args_for(*L, B, T, fw, bw.S0);
        ba.d_out = bw.dO;
        ba.d_state_out = has_ds ? d_state->S : nullptr;
        ba.dq = bw.dxq; ba.dk = bw.dxk; ba.dg = bw.dxg; ba.db = bw.dxb; ba.dv = bw.dv; ba.dw = bw.dw;
        ba.d_state0 = d_state_in ? d_state_in->S : bw.dS0;
        if (saved && saved->chunk_filled) { // the forward's per-chunk quantities are kept
            ba.workspace = saved->chunk;
            ba.workspace_bytes = saved->chunk_bytes;
            if ((st = gdn2_chunk_bwd_saved_f32(&ba, s)) != GDN2_OK) return st;
        } else {
            ba.workspace = fw.chunk;
            ba.workspace_bytes = fw.chunk_bytes;
            if ((st = gdn2_chunk_bwd_f32(&ba, s)) != GDN2_OK) return st;
        }
    } else {
        gdn2_recurrent_bwd_args ra{};
        ra.fwd = recurrent_args_for(chunk_args_for(*L, B, T, fw, bw.S0));
        ra.d_out = bw.dO;
        ra.d_state_out = has_ds ? d_state->S : nullptr;
        ra.dq = bw.dxq; ra.dk = bw.dxk; ra.dg = bw.dxg; ra.db = bw.dxb; ra.dv = bw.dv; ra.dw = bw.dw;
        ra.d_state0 = d_state_in ? d_state_in->S : bw.dS0;
        ra.workspace = fw.chunk;
        ra.workspace_bytes = fw.chunk_bytes;
        if ((st = gdn2_recurrent_bwd_f32(&ra, s)) != GDN2_OK) return st;
    }
    if (d.Hq != d.H) { // the reference's GVA layout back to the key heads
        GvaParams gp{};
        gp.src[0] = bw.dxq; gp.src[1] = bw.dxk; gp.src[2] = bw.dxg; gp.src[3] = bw.dxb;
        gp.dst[0] = bw.dq; gp.dst[1] = bw.dk; gp.dst[2] = bw.dg; gp.dst[3] = bw.db;
        gp.B = B; gp.H = d.H; gp.T = T; gp.K = d.K; gp.rep = (int)(d.HV / d.H);
        GDN2_HIP_CHECK(launch_gva_fold(gp, s));
    }

    // projection epilogue and short conv
    ProjectBwdParams pp{};
    pp.Y = fw.Y; pp.ldY = L->ld_in;
    pp.off_q = L->off_q; pp.off_k = L->off_k; pp.off_b = L->off_b; pp.off_v = L->off_v; pp.off_w = L->off_w;
    pp.F = fw.F; pp.ldF = d.kd;
    pp.conv_q_in = conv_in[0]; pp.conv_k_in = conv_in[1]; pp.conv_v_in = conv_in[2];
    pp.q_conv_w = L->p[P_QCONV]; pp.k_conv_w = L->p[P_KCONV]; pp.v_conv_w = L->p[P_VCONV];
    pp.a_log = L->p[P_A_LOG]; pp.dt_bias = L->p[P_DT_BIAS]; pp.decay_factors = md ? L->p[P_DECAY] : nullptr;
    pp.dq = bw.dq; pp.dk = bw.dk; pp.dg = bw.dg; pp.db = bw.db; pp.dv = bw.dv; pp.dw = bw.dw;
    pp.dY = bw.dY; pp.DU = sc ? bw.DU : nullptr; pp.dF = bw.dF; pp.PA = bw.PA; pp.PD = md ? bw.PD : nullptr;
    pp.B = (int)B; pp.T = (int)T; pp.H = (int)d.H; pp.K = (int)d.K; pp.HV = (int)d.HV; pp.V = (int)d.V;
    pp.use_short_conv = L->cfg.use_short_conv; pp.allow_neg_eigval = L->cfg.allow_neg_eigval;
    pp.min_decay = (float)L->cfg.min_decay; pp.one_minus_min_decay = (float)(1.0 - L->cfg.min_decay);
    GDN2_HIP_CHECK(launch_project_bwd(pp, s));
    if (sc) {
        ConvBwdParams cp{};
        cp.Y = fw.Y; cp.ldY = L->ld_in; cp.off_q = L->off_q; cp.off_k = L->off_k; cp.off_v = L->off_v;
        cp.DU = bw.DU;
        cp.cache_q = conv_in[0]; cp.cache_k = conv_in[1]; cp.cache_v = conv_in[2];
        if (has_ds) {
            cp.d_out_q = d_state->conv[d_state->cur][0];
            cp.d_out_k = d_state->conv[d_state->cur][1];
            cp.d_out_v = d_state->conv[d_state->cur][2];
        }
        cp.q_conv_w = L->p[P_QCONV]; cp.k_conv_w = L->p[P_KCONV]; cp.v_conv_w = L->p[P_VCONV];
        cp.dY = bw.dY;
        if (d_state_in && has_state) {
            cp.d_in_q = d_state_in->conv[d_state_in->cur][0];
            cp.d_in_k = d_state_in->conv[d_state_in->cur][1];
            cp.d_in_v = d_state_in->conv[d_state_in->cur][2];
        }
        cp.wpart = bw.wpart;
        cp.B = (int)B; cp.T = (int)T; cp.kd = (int)d.kd; cp.vd = (int)d.vd; cp.tblock = kConvTBlock;
        GDN2_HIP_CHECK(launch_conv_bwd(cp, s));
        const int64_t parts = B * conv_bwd_blocks((int)T, kConvTBlock), ld = 4 * (2 * d.kd + d.vd);
        GDN2_HIP_CHECK(launch_colsum(bw.wpart, parts, 4 * d.kd, ld, 1, 1, G->p[P_QCONV], accumulate, bw.part, kColParts, s));
        GDN2_HIP_CHECK(launch_colsum(bw.wpart + 4 * d.kd, parts, 4 * d.kd, ld, 1, 1, G->p[P_KCONV], accumulate, bw.part,
                                     kColParts, s));
        GDN2_HIP_CHECK(launch_colsum(bw.wpart + 8 * d.kd, parts, 4 * d.vd, ld, 1, 1, G->p[P_VCONV], accumulate, bw.part,
                                     kColParts, s));
        if (d_state_in && !has_state && (st = pass_caches(false)) != GDN2_OK) return st;
    } else {
        if (!accumulate)
            for (int id : {P_QCONV, P_KCONV, P_VCONV})
                GDN2_HIP_CHECK(launch_fill_rows(G->p[id], 0, nullptr, 1, param_shape(L->cfg, id, nullptr, nullptr), s));
        if (d_state_in && (st = pass_caches(has_state)) != GDN2_OK) return st;
    }
    // columns of dY between the blocks stay zero, so that dW_in's padding does too
    const int64_t blocks[7][2] = {{L->off_q, d.kd}, {L->off_k, d.kd}, {L->off_b, d.kd}, {L->off_v, d.vd},
                                  {L->off_w, d.vd}, {L->off_f0, d.V}, {L->off_g0, d.V}};
    for (int i = 0; i < 7; ++i) {
        const int64_t end = blocks[i][0] + blocks[i][1], next = i < 6 ? blocks[i + 1][0] : L->ld_in;
        if (next > end) GDN2_HIP_CHECK(launch_fill_rows(bw.dY + end, L->ld_in, nullptr, M, next - end, s));
    }

    // gates: f_proj_1, g_proj_1 (+ bias), dt_bias, A_log, decay_factors
    const float *Yf0 = fw.Y + L->off_f0, *Yg0 = fw.Y + L->off_g0;
    if ((st = L->mm.run(false, true, M, d.V, d.kd, bw.dF, d.kd, L->p[P_F1], d.kd, bw.dY + L->off_f0, L->ld_in,
                     0.0f, s)) != GDN2_OK)
        return st;
    if ((st = L->mm.run(true, false, d.V, d.kd, M, Yf0, L->ld_in, bw.dF, d.kd, G->p[P_F1], d.kd, beta, s)) != GDN2_OK)
        return st;
    if ((st = L->mm.run(false, true, M, d.V, d.vd, bw.dG, d.vd, L->p[P_G1], d.vd, bw.dY + L->off_g0, L->ld_in,
                     0.0f, s)) != GDN2_OK)
        return st;
    if ((st = L->mm.run(true, false, d.V, d.vd, M, Yg0, L->ld_in, bw.dG, d.vd, G->p[P_G1], d.vd, beta, s)) != GDN2_OK)
        return st;
    GDN2_HIP_CHECK(launch_colsum(bw.dG, M, d.vd, d.vd, 1, 1, G->p[P_G1_BIAS], accumulate, bw.part, kColParts, s));
    GDN2_HIP_CHECK(launch_colsum(bw.dF, M, d.kd, d.kd, 1, 1, G->p[P_DT_BIAS], accumulate, bw.part, kColParts, s));
    GDN2_HIP_CHECK(launch_colsum(bw.PA, M, d.kd, d.kd, (int)d.K, 1, G->p[P_A_LOG], accumulate, bw.part, kColParts, s));
    if (md) GDN2_HIP_CHECK(launch_colsum(bw.PD, M, d.kd, d.kd, 1, 1, G->p[P_DECAY], accumulate, bw.part, kColParts, s));

    // the input Linear layers
    if ((st = L->mm.run(true, false, d.D, L->ld_in, M, x, d.D, bw.dY, L->ld_in, G->g_in, L->ld_in, beta, s)) !=
        GDN2_OK)
        return st;
    if (dx && (st = L->mm.run(false, true, M, d.D, L->ld_in, bw.dY, L->ld_in, L->w_in, L->ld_in, dx, d.D,
                           0.0f, s)) != GDN2_OK)
        return st;
    if (d_state_in) d_state_in->some = true;
    return GDN2_OK;
}

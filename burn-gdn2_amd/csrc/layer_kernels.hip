// Layer kernels around the recurrence: the projection epilogue (short conv,
// SiLU, gates, L2 norm; written head-major [B, H, T, D], as the reference's
// project() returns them, so that each chunk of a head is one contiguous
// block), the conv-cache update, the gated RMSNorm and a row fill for Linear
// biases.
#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {
namespace {

__device__ __forceinline__ float sigmoid_(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_(float x) { return x / (1.0f + __expf(-x)); }
// burn's softplus(x, beta = 1) = ln(1 + e^x); above 20 the f32 value is x.
__device__ __forceinline__ float softplus_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Causal depthwise conv with four taps at token t of one sequence
// (src/short_conv.rs:22-65): y = sum_i xpad[t + i] * w[c, i] with
// xpad = cat(cache, x); without a cache the first token is replicated.
// `x` points at the sequence's token 0 in column c (row stride ldx).
__device__ __forceinline__ float conv4(const float *x, int64_t ldx, int t, const float *cache, int64_t n_ch,
                                       const float *w) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tp = t + i - 3;
        float xv;
        if (tp >= 0)
            xv = x[(int64_t)tp * ldx];
        else if (cache)
            xv = cache[(int64_t)(3 + tp) * n_ch];
        else
            xv = x[0];
        acc += xv * w[i];
    }
    return acc;
}

// One workgroup per token m = b * T + t.
__global__ __launch_bounds__(256) void project_kernel(ProjectParams p) {
    extern __shared__ float sm[];
    const int kd = p.H * p.K, vd = p.HV * p.V;
    float *s_q = sm, *s_k = sm + kd;
    const int64_t m = blockIdx.x;
    const int bi = (int)(m / p.T), t = (int)(m % p.T);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)bi * p.T;
    const float *Y = p.Y + m * p.ldY;
    const float *Y0 = p.Y + m0 * p.ldY;
    const bool sc = p.use_short_conv != 0;

    // q, k: conv (or plain) + SiLU into LDS
    for (int c = tid; c < kd; c += 256) {
        float aq, ak;
        if (sc) {
            const int64_t cb = (int64_t)bi * 3 * kd + c;
            aq = conv4(Y0 + p.off_q + c, p.ldY, t, p.conv_q_in ? p.conv_q_in + cb : nullptr, kd, p.q_conv_w + 4 * c);
            ak = conv4(Y0 + p.off_k + c, p.ldY, t, p.conv_k_in ? p.conv_k_in + cb : nullptr, kd, p.k_conv_w + 4 * c);
        } else {
            aq = Y[p.off_q + c];
            ak = Y[p.off_k + c];
        }
        s_q[c] = silu_(aq);
        s_k[c] = silu_(ak);
    }
    // g, b (src/module.rs:417-443, :470-472)
    for (int c = tid; c < kd; c += 256) {
        float gv = -expf(p.a_log[c / p.K]) * softplus_(p.F[m * p.ldF + c] + p.dt_bias[c]);
        if (p.decay_factors) gv = logf(sigmoid_(p.decay_factors[c]) * p.one_minus_min_decay * expf(gv) + p.min_decay);
        float bv = sigmoid_(Y[p.off_b + c]);
        if (p.allow_neg_eigval) bv *= 2.0f;
        const int64_t o = ((int64_t)bi * p.H + c / p.K) * p.T * p.K + (int64_t)t * p.K + c % p.K;
        p.g[o] = gv;
        p.b[o] = bv;
    }
    // v = SiLU(conv(v_raw)), w = sigmoid(w_raw)
    for (int c = tid; c < vd; c += 256) {
        float av;
        if (sc) {
            const int64_t cb = (int64_t)bi * 3 * vd + c;
            av = conv4(Y0 + p.off_v + c, p.ldY, t, p.conv_v_in ? p.conv_v_in + cb : nullptr, vd, p.v_conv_w + 4 * c);
        } else {
            av = Y[p.off_v + c];
        }
        const int64_t o = ((int64_t)bi * p.HV + c / p.V) * p.T * p.V + (int64_t)t * p.V + c % p.V;
        p.v[o] = silu_(av);
        p.w[o] = sigmoid_(Y[p.off_w + c]);
    }
    __syncthreads();
    // L2 norm per head over K channels (src/l2norm.rs:13-16): one wave per head.
    for (int h = wave; h < p.H; h += 4) {
        float sq = 0.f, sk = 0.f;
        for (int i = lane; i < p.K; i += 64) {
            const float a = s_q[h * p.K + i], b = s_k[h * p.K + i];
            sq += a * a;
            sk += b * b;
        }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        const float nq = sqrtf(sq + 1e-6f), nk = sqrtf(sk + 1e-6f);
        const int64_t o = ((int64_t)bi * p.H + h) * p.T * p.K + (int64_t)t * p.K;
        for (int i = lane; i < p.K; i += 64) {
            p.q[o + i] = s_q[h * p.K + i] / nq;
            p.k[o + i] = s_k[h * p.K + i] / nk;
        }
    }
}

// New conv caches: xpad[T .. T + 3) = the last three pre-conv tokens.
__global__ __launch_bounds__(256) void conv_cache_kernel(ConvCacheParams p) {
    const int64_t nq = (int64_t)p.B * 3 * p.kd, nv = (int64_t)p.B * 3 * p.vd;
    const int64_t total = 2 * nq + nv;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t idx = i;
        const float *in;
        float *out;
        int64_t n, off;
        if (idx < nq) {
            in = p.in_q; out = p.out_q; n = p.kd; off = p.off_q;
        } else if (idx < 2 * nq) {
            idx -= nq; in = p.in_k; out = p.out_k; n = p.kd; off = p.off_k;
        } else {
            idx -= 2 * nq; in = p.in_v; out = p.out_v; n = p.vd; off = p.off_v;
        }
        const int64_t c = idx % n, j = (idx / n) % 3, bi = idx / (3 * n);
        const int64_t tp = p.T + j - 3;
        float val;
        if (tp >= 0)
            val = p.Y[(bi * p.T + tp) * p.ldY + off + c];
        else if (in)
            val = in[(bi * 3 + p.T + j) * n + c];
        else
            val = p.Y[(bi * p.T) * p.ldY + off + c];
        out[(bi * 3 + j) * n + c] = val;
    }
}

// rms_norm_gate_per_head (src/module.rs:501-517): one wave per (token, value head).
__global__ __launch_bounds__(256) void rmsnorm_gate_kernel(float *out, int64_t ld_out, const float *x, int64_t ld_x,
                                                           const float *gate, int64_t ld_gate, const float *weight,
                                                           int64_t rows, int HV, int V, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t m = row / HV;
    const int hv = (int)(row % HV);
    const float *xr = x + m * ld_x + (int64_t)hv * V;
    const float *gr = gate + m * ld_gate + (int64_t)hv * V;
    float *orow = out + m * ld_out + (int64_t)hv * V;
    float ss = 0.f;
    for (int i = lane; i < V; i += 64) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)V + eps);
    for (int i = lane; i < V; i += 64) orow[i] = xr[i] / rms * weight[i] * silu_(gr[i]);
}

__global__ __launch_bounds__(256) void fill_rows_kernel(float *y, int64_t ld, const float *row, int64_t M, int64_t N) {
    const int64_t total = M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / N, c = i % N;
        y[r * ld + c] = row ? row[c] : 0.0f;
    }
}

int grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (int)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

}  // namespace

size_t project_lds_bytes(int kd) { return sizeof(float) * 2 * (size_t)kd; }

hipError_t launch_project(const ProjectParams &p, hipStream_t s) {
    const int64_t M = (int64_t)p.B * p.T;
    if (M == 0) return hipSuccess;
    hipLaunchKernelGGL(project_kernel, dim3((unsigned)M), dim3(256), project_lds_bytes(p.H * p.K), s, p);
    return hipGetLastError();
}

hipError_t launch_conv_cache(const ConvCacheParams &p, hipStream_t s) {
    const int64_t total = (int64_t)p.B * 3 * (2 * p.kd + p.vd);
    hipLaunchKernelGGL(conv_cache_kernel, dim3(grid_for(total)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_gate(float *out, int64_t ld_out, const float *x, int64_t ld_x, const float *gate,
                               int64_t ld_gate, const float *weight, int64_t M, int HV, int V, float eps,
                               hipStream_t s) {
    const int64_t rows = M * HV;
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_gate_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, out, ld_out, x, ld_x,
                       gate, ld_gate, weight, rows, HV, V, eps);
    return hipGetLastError();
}

hipError_t launch_fill_rows(float *y, int64_t ld, const float *row, int64_t M, int64_t N, hipStream_t s) {
    if (M * N == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_rows_kernel, dim3(grid_for(M * N)), dim3(256), 0, s, y, ld, row, M, N);
    return hipGetLastError();
}

}  // namespace gdn2

// The reference's standalone public operators (src/lib.rs:58-62) as C-ABI
// entry points, for a binding that calls them one by one rather than through
// the fused layer kernels:
//   gdn2_short_conv_f32      short_conv_1d           src/short_conv.rs:22-65
//   gdn2_l2_normalize_f32    l2_normalize(_4d)       src/l2norm.rs:4-16
//   gdn2_rms_norm_gate_f32   rms_norm_gate_per_head  src/module.rs:501-517
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace {

using gdn2::fail;

constexpr int kConvTaps = 4;  // SHORT_CONV_KERNEL (src/short_conv.rs:5)
constexpr int kConvCache = 3; // SHORT_CONV_CACHE (src/short_conv.rs:7)
constexpr int kConvTile = 64; // tokens per thread

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// Padded input row i of sequence b: rows 0..2 are the cache (or token 0
// repeated), row 3 + t is token t.
__device__ __forceinline__ float xpad(const float *x, const float *cache, int64_t b, int64_t i, int64_t T,
                                      int64_t C, int64_t c) {
    if (i >= kConvCache) return x[(b * T + (i - kConvCache)) * C + c];
    return cache ? cache[(b * kConvCache + i) * C + c] : x[b * T * C + c];
}

// Thread = (sequence b, channel c, 64 tokens): a sliding window of the four
// taps over the padded input, each input read once; the tile's first thread
// of each sequence also writes the new cache (the last three padded rows).
__global__ __launch_bounds__(256) void short_conv_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                         const float *__restrict__ cache_in, float *__restrict__ out,
                                                         float *__restrict__ cache_out, int64_t T, int64_t C) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = blockIdx.y, t0 = (int64_t)blockIdx.z * kConvTile;
    if (c >= C) return;
    const float w0 = w[c * kConvTaps], w1 = w[c * kConvTaps + 1], w2 = w[c * kConvTaps + 2],
                w3 = w[c * kConvTaps + 3];
    // window: padded rows t0 .. t0 + 2, then one more per token
    float a = xpad(x, cache_in, b, t0, T, C, c), bb = xpad(x, cache_in, b, t0 + 1, T, C, c),
          cc = xpad(x, cache_in, b, t0 + 2, T, C, c);
    const int64_t t1 = t0 + kConvTile < T ? t0 + kConvTile : T;
    for (int64_t t = t0; t < t1; ++t) {
        const float d = x[(b * T + t) * C + c]; // padded row t + 3
        out[(b * T + t) * C + c] = silu_f(a * w0 + bb * w1 + cc * w2 + d * w3);
        a = bb;
        bb = cc;
        cc = d;
    }
    if (blockIdx.z == 0)
        for (int j = 0; j < kConvCache; ++j)
            cache_out[(b * kConvCache + j) * C + c] = xpad(x, cache_in, b, T + j, T, C, c);
}

// One wave per row of n values: y = x / sqrt(sum x^2 + eps).  Each lane
// writes only the elements it read, so y may be x.
__global__ __launch_bounds__(256) void l2_normalize_kernel(const float *x, float *y,
                                                           int64_t rows, int64_t n, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * n;
    float ss = 0.f;
    for (int64_t i = lane; i < n; i += 64) ss += xr[i] * xr[i];
    ss = gdn2::wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss + eps);
    for (int64_t i = lane; i < n; i += 64) y[row * n + i] = xr[i] * inv;
}

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const char *pa = static_cast<const char *>(a), *pb = static_cast<const char *>(b);
    return pa < pb + nb && pb < pa + na;
}

}  // namespace

extern "C" gdn2_status gdn2_short_conv_f32(const float *x, const float *weight, const float *cache_in, float *out,
                                           float *cache_out, int64_t B, int64_t T, int64_t C, gdn2_stream_t stream) {
    const std::string who = "gdn2_short_conv_f32: ";
    if (B < 0 || T < 0 || C < 0) return fail(GDN2_EINVAL, who + "negative dimension");
    if (B == 0 || C == 0) return GDN2_OK;
    if (!weight || !cache_out || (T > 0 && (!x || !out))) return fail(GDN2_EINVAL, who + "null pointer");
    if (T == 0 && !cache_in)
        return fail(GDN2_EINVAL, who + "no tokens and no cache: nothing to pad from");
    const size_t nc = sizeof(float) * (size_t)B * kConvCache * C;
    if ((cache_in && overlaps(cache_in, nc, cache_out, nc)) || overlaps(x, sizeof(float) * B * T * C, cache_out, nc) ||
        overlaps(out, sizeof(float) * B * T * C, cache_out, nc))
        return fail(GDN2_EINVAL, who + "cache_out must not overlap x, out or cache_in");
    // Each tile reads the three rows before it and the cache reads the last
    // three rows of x, while other tiles write their outputs: out must not
    // overlap x (no in-place use).
    if (T > 0 && overlaps(x, sizeof(float) * B * T * C, out, sizeof(float) * B * T * C))
        return fail(GDN2_EINVAL, who + "out must not overlap x");
    if (B > 65535 || (T + kConvTile - 1) / kConvTile > 65535) return fail(GDN2_NOT_APPLICABLE, who + "grid limits");
    const int64_t tiles = T > 0 ? (T + kConvTile - 1) / kConvTile : 1;
    hipLaunchKernelGGL(short_conv_kernel, dim3((unsigned)((C + 255) / 256), (unsigned)B, (unsigned)tiles), dim3(256),
                       0, (hipStream_t)stream, x, weight, cache_in, out, cache_out, T, C);
    GDN2_HIP_CHECK(hipGetLastError());
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_l2_normalize_f32(const float *x, float *y, int64_t rows, int64_t n, double eps,
                                             gdn2_stream_t stream) {
    if (rows < 0 || n < 0) return fail(GDN2_EINVAL, "gdn2_l2_normalize_f32: negative dimension");
    if (rows == 0 || n == 0) return GDN2_OK;
    if (!x || !y) return fail(GDN2_EINVAL, "gdn2_l2_normalize_f32: null pointer");
    hipLaunchKernelGGL(l2_normalize_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x, y,
                       rows, n, (float)eps);
    GDN2_HIP_CHECK(hipGetLastError());
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_rms_norm_gate_f32(const float *x, const float *gate, const float *weight, float *y,
                                              int64_t rows, int64_t V, double eps, gdn2_stream_t stream) {
    if (rows < 0 || V < 0) return fail(GDN2_EINVAL, "gdn2_rms_norm_gate_f32: negative dimension");
    if (rows == 0 || V == 0) return GDN2_OK;
    if (!x || !gate || !weight || !y) return fail(GDN2_EINVAL, "gdn2_rms_norm_gate_f32: null pointer");
    if (V > (int64_t(1) << 30)) return fail(GDN2_NOT_APPLICABLE, "gdn2_rms_norm_gate_f32: rows too long");
    GDN2_HIP_CHECK(gdn2::launch_rmsnorm_gate(y, V, x, V, gate, V, nullptr, weight, rows, 1, (int)V, (float)eps,
                                             (hipStream_t)stream));
    return GDN2_OK;
}

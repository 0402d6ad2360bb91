// gdn2_stream_copy_f32: a streaming device-to-device copy, the measurement
// helper behind the practical HBM roof that the benchmark reports beside the
// 8 TB/s peak.  No reference counterpart.
//
// Each thread moves kUnroll float4 per grid-stride step: all loads of a step
// are issued before its stores, with non-temporal hints (every byte is used
// once), so a wave keeps kUnroll 16-byte requests per lane in flight.  The
// grid is a fixed number of workgroups per compute unit, looping over the
// array, so that the work does not depend on the launch shape.
#include <string>

#include "common.hpp"

namespace {

using gdn2::floatx4;
constexpr int kUnroll = 4;
constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void stream_copy_kernel(floatx4 *__restrict__ dst,
                                                               const floatx4 *__restrict__ src, int64_t n4) {
    const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
    for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < n4; base += step) {
        floatx4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + (int64_t)u * kThreads;
            if (i < n4) v[u] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + (int64_t)u * kThreads;
            if (i < n4) __builtin_nontemporal_store(v[u], dst + i);
        }
    }
}

__global__ __launch_bounds__(kThreads) void tail_copy_kernel(float *__restrict__ dst, const float *__restrict__ src,
                                                             int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

}  // namespace

extern "C" gdn2_status gdn2_stream_copy_f32(float *dst, const float *src, int64_t n, int64_t workgroups,
                                            gdn2_stream_t stream) {
    const char *who = "gdn2_stream_copy_f32";
    if (n < 0 || workgroups < 0) return gdn2::fail(GDN2_EINVAL, std::string(who) + ": negative size");
    if (n == 0) return GDN2_OK;
    if (!dst || !src) return gdn2::fail(GDN2_EINVAL, std::string(who) + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u)
        return gdn2::fail(GDN2_EINVAL, std::string(who) + ": dst and src must be 16-byte aligned");
    if (workgroups > (int64_t(1) << 20)) return gdn2::fail(GDN2_EINVAL, std::string(who) + ": too many workgroups");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n4 = n / 4, rest = n - 4 * n4;
    if (n4 > 0) {
        int64_t wg = workgroups ? workgroups : 256 * 8; // 8 per compute unit of an MI355X
        const int64_t need = (n4 + kThreads * kUnroll - 1) / (kThreads * kUnroll);
        if (wg > need) wg = need;
        hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)wg), dim3(kThreads), 0, s,
                           reinterpret_cast<floatx4 *>(dst), reinterpret_cast<const floatx4 *>(src), n4);
        GDN2_HIP_CHECK(hipGetLastError());
    }
    if (rest > 0) {
        hipLaunchKernelGGL(tail_copy_kernel, dim3(1), dim3(kThreads), 0, s, dst + 4 * n4, src + 4 * n4, rest);
        GDN2_HIP_CHECK(hipGetLastError());
    }
    return GDN2_OK;
}

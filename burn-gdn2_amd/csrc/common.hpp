// Shared device/host helpers for the gfx950 GDN-2 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "gdn2.h"

namespace gdn2 {

// Error reporting for the C ABI (thread-local message, see gdn2_last_error).
void set_error(const std::string &msg);
gdn2_status fail(gdn2_status st, const std::string &msg);

#define GDN2_HIP_CHECK(expr)                                                        \
    do {                                                                            \
        hipError_t e_ = (expr);                                                     \
        if (e_ != hipSuccess)                                                       \
            return ::gdn2::fail(GDN2_EHIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// MFMA 16x16x4 f32 (v_mfma_f32_16x16x4_f32).  Lane l of the wave supplies
//   A[i = l % 16][kk = l / 16]     (16 x 4)
//   B[kk = l / 16][j = l % 16]     (4 x 16)
// and holds D[i = 4 * (l / 16) + r][j = l % 16], r = 0..3, of the 16 x 16
// result.  The contraction index kk is only a label: any bijection between
// (lane group, step) and the reduced dimension works as long as A and B use
// the same one.  The kernels use "k = 4 * group + step" inside a 16-wide
// block, which makes an accumulator tile directly usable as the B operand of
// the next product (its rows become the contraction index) and lets the A
// operand come from one 16-byte load per lane per four steps.
// ---------------------------------------------------------------------------
__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

}  // namespace gdn2

// gdn2_chunk_fwd_noalloc_f32: the chunked forward for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// It runs exactly the kernels of gdn2_chunk_fwd_f32.  Their workspace (the
// per-chunk W, U, scale q exp(G), Kd^T, A_qk, exp(G_last) and, for few long
// sequences, the segment summaries) comes from `scratch`, a file-scope device
// array of kScratchBytes that every GPU the library runs on holds until the
// process ends, instead of a caller-provided buffer.
//
// In host code `scratch` names a host-side stand-in, not device memory: the
// device address of each GPU's copy comes from hipGetSymbolAddress, looked up
// once per device (with that device current) on the first call there, and
// only that address is handed to the kernels.
//
// Every word the kernels read from the workspace is written earlier in the
// same call, so nothing needs clearing between calls.  All calls on one GPU
// share its array: calls that overlap in time on one GPU (two streams, two
// host threads) race on it, and must be ordered by the caller.
#include <mutex>
#include <string>

#include "common.hpp"

namespace {
constexpr size_t kScratchBytes = size_t(64) << 20; // 64 MiB per GPU
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices]; // device address of `scratch` per device, null until looked up

gdn2_status scratch_address(const char *who, void **out) {
    int dev = -1;
    GDN2_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return gdn2::fail(GDN2_EINVAL, std::string(who) + ": device index " + std::to_string(dev) + " beyond " +
                                           std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return gdn2::fail(GDN2_EHIP, std::string(who) + ": hipGetSymbolAddress(scratch): " +
                                             (e != hipSuccess ? hipGetErrorString(e) : "null address"));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GDN2_OK;
}

}  // namespace

extern "C" size_t gdn2_chunk_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" gdn2_status gdn2_chunk_fwd_noalloc_f32(const gdn2_chunk_args *a, gdn2_stream_t stream) {
    const char *who = "gdn2_chunk_fwd_noalloc_f32";
    if (!a) return gdn2::fail(GDN2_EINVAL, std::string(who) + ": null args");
    const size_t need = gdn2_chunk_workspace_bytes(a); // 0 for no tokens or invalid shapes (checked below)
    if (need > kScratchBytes)
        return gdn2::fail(GDN2_EINVAL, std::string(who) + ": the call needs " + std::to_string(need) +
                                           " bytes of workspace; the static scratch holds " +
                                           std::to_string(kScratchBytes) +
                                           " (use gdn2_chunk_fwd_f32 with a caller workspace)");
    void *ptr = nullptr;
    const gdn2_status st = scratch_address(who, &ptr);
    if (st != GDN2_OK) return st;
    gdn2_chunk_args c = *a;
    c.workspace = ptr;
    c.workspace_bytes = kScratchBytes;
    return gdn2_chunk_fwd_f32(&c, stream);
}

// Chunked forward: entry points (kernels follow).
#include "common.hpp"
#include "kernels.hpp"

using namespace gdn2;

extern "C" size_t gdn2_chunk_workspace_bytes(const gdn2_chunk_args *a) { return 0; }

extern "C" gdn2_status gdn2_chunk_fwd_f32(const gdn2_chunk_args *a, gdn2_stream_t stream) {
    return fail(GDN2_NOT_APPLICABLE, "gdn2_chunk_fwd_f32: chunk kernels not built yet");
}

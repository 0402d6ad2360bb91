// Device helpers shared by the chunked forward (chunk.hip) and backward
// (chunk_bwd.hip) kernels: chunk geometry, MFMA fragment helpers, the
// range-checked row loads and the XCD-aware workgroup mapping.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {

constexpr int C = kChunk;   // chunk length of the kernels
constexpr int NT = C / 16;  // 16-row tiles per chunk

// Waves per workgroup of the sequential kernels (each wave owns 16 value
// columns): four when V and K are multiples of 64, else two (V = 32, 96 and
// K = 32, whose segment transitions P have 32 columns).
constexpr int inter_nwv(int K, int V) { return (V % 64 == 0 && K % 64 == 0) ? 4 : 2; }

// Rows [0, valid) of a row-strided f32 matrix (row stride rs, rowlen
// elements used per row) as a buffer resource.  The hardware's range check
// returns 0 for every load past the last valid row, which is the zero padding
// of a ragged last chunk (src/forward.rs:94-99), so a load needs neither a
// clamp nor a mask, and its offset is a 32-bit element index.  Requires
// rs >= rowlen and ((valid - 1) rs + rowlen) * 4 < 2^31 (checked on the host).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float *base, int rs, int valid, int rowlen) {
    const int bytes = ((valid - 1) * rs + rowlen) * 4;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ float bld1(__amdgpu_buffer_rsrc_t r, int idx) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, idx * 4, 0, 0));
}

// A store through a rows_rsrc resource: dropped past its last valid row.
__device__ __forceinline__ void bst1(__amdgpu_buffer_rsrc_t r, int idx, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, idx * 4, 0, 0);
}

__device__ __forceinline__ floatx4 bld4(__amdgpu_buffer_rsrc_t r, int idx) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, idx * 4, 0, 0));
}
// 16 bytes through a rows_rsrc resource (idx a multiple of 4 within a row):
// dropped past its last valid row.
__device__ __forceinline__ void bst4(__amdgpu_buffer_rsrc_t r, int idx, floatx4 v) {
    typedef int intx4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(intx4, v), r, idx * 4, 0, 0);
}

__device__ __forceinline__ floatx4 mfma4(float4 a, floatx4 b, floatx4 c) {
    c = mfma16(a.x, b[0], c);
    c = mfma16(a.y, b[1], c);
    c = mfma16(a.z, b[2], c);
    c = mfma16(a.w, b[3], c);
    return c;
}

// D = X^T for an accumulator tile X, i.e. the A-operand layout of X
// (lane (g, r) gets X[r][4g..4g+3]): the accumulator is a valid A operand
// of X^T under the k = 4g + step labelling, multiplied by the identity.
// Exact in f32 (products with 1 and 0).
__device__ __forceinline__ floatx4 transpose16(floatx4 x, int lr, int lg) {
    floatx4 d = floatx4{0.f, 0.f, 0.f, 0.f};
    d = mfma16(x[0], lr == 4 * lg + 0 ? 1.f : 0.f, d);
    d = mfma16(x[1], lr == 4 * lg + 1 ? 1.f : 0.f, d);
    d = mfma16(x[2], lr == 4 * lg + 2 ? 1.f : 0.f, d);
    d = mfma16(x[3], lr == 4 * lg + 3 ? 1.f : 0.f, d);
    return d;
}

__device__ __forceinline__ floatx4 mfma4n(float4 a, floatx4 b, floatx4 c) {
    c = mfma16(-a.x, b[0], c);
    c = mfma16(-a.y, b[1], c);
    c = mfma16(-a.z, b[2], c);
    c = mfma16(-a.w, b[3], c);
    return c;
}

// Streaming store: the workspace is read back by chunk-inter much later, so
// keeping it out of L2 leaves room for the chunk's inputs, which chunk-intra
// reads more than once.
__device__ __forceinline__ void st_stream(floatx4 *dst, floatx4 v) { __builtin_nontemporal_store(v, dst); }

// Pins a loaded value in a register where it is loaded: the compiler would
// otherwise sink a load used only under a lane condition into a divergent
// branch with its own wait, serialising the loads of an unrolled loop.
__device__ __forceinline__ float pin(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ float2 pin(float2 x) {
    asm volatile("" : "+v"(x.x), "+v"(x.y));
    return x;
}

__device__ __forceinline__ floatx4 exp2v(floatx4 x) {
    return floatx4{fast_exp2(x[0]), fast_exp2(x[1]), fast_exp2(x[2]), fast_exp2(x[3])};
}

// The two steps of a 4 x 4 transpose among the four lanes of a quad, whose
// lane i holds row i (elements 0 .. 3): afterwards lane i holds column i.
// Step 1, partner i ^ 2 (dpp quad_perm [2, 3, 0, 1]): the lower two lanes
// trade elements 2, 3 for the partner's 0, 1.  Step 2, partner i ^ 1
// (quad_perm [1, 0, 3, 2]): the even lanes trade elements 1, 3 for the
// partner's 0, 2.  Every lane of the wave must be active.
template <int CTRL> __device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ void quad_swap_halves(floatx4 &x, bool upper) { // upper = i & 2
    const float r0 = quad_perm<0x4E>(upper ? x[0] : x[2]), r1 = quad_perm<0x4E>(upper ? x[1] : x[3]);
    if (upper) {
        x[0] = r0;
        x[1] = r1;
    } else {
        x[2] = r0;
        x[3] = r1;
    }
}
__device__ __forceinline__ void quad_swap_pairs(floatx4 &x, bool odd) { // odd = i & 1
    const float r0 = quad_perm<0xB1>(odd ? x[0] : x[1]), r1 = quad_perm<0xB1>(odd ? x[2] : x[3]);
    if (odd) {
        x[0] = r0;
        x[2] = r1;
    } else {
        x[1] = r0;
        x[3] = r1;
    }
}

// Direct global -> LDS copy of one float4 per lane (global_load_lds_dwordx4):
// lane l of the calling wave writes wave_base[l]; wave_base is wave-uniform.
// The copy counts in vmcnt: wait with vm_wait0() before the barrier that
// publishes it.
__device__ __forceinline__ void lds_copy4(const floatx4 *src, floatx4 *wave_base) {
    __builtin_amdgcn_global_load_lds(static_cast<const void *>(src),
                                     (__attribute__((address_space(3))) void *)(wave_base), 16, 0, 0);
}
// The same copy through a buffer resource (buffer_load_dwordx4 ... lds): the
// range check zero-fills the lanes whose 16 bytes at byte offset `off` lie
// past the resource, e.g. the rows past T of a rows_rsrc.
__device__ __forceinline__ void lds_copy4_rsrc(__amdgpu_buffer_rsrc_t r, int off, floatx4 *wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(wave_base), 16, off, 0, 0, 0);
}
// Pulls the 128-byte line holding `line` toward this XCD's L2: a 4-byte copy
// into the calling lane's word of wave_slot (64 floats per wave, never read).
// It counts in vmcnt like lds_copy4, so a wait that must not cover it leaves
// it among the most recent operations (vm_wait<N>).
__device__ __forceinline__ void l2_touch(const void *line, float *wave_slot) {
    __builtin_amdgcn_global_load_lds(line, (__attribute__((address_space(3))) void *)(wave_slot), 4, 0, 0);
}
// s_waitcnt vmcnt(N): every vector memory operation of the wave but the N
// most recent has completed (they complete in issue order); expcnt and
// lgkmcnt are not waited on.
template <int N> __device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
__device__ __forceinline__ void vm_wait0() { vm_wait<0>(); }
// Workgroup barrier that leaves vmcnt alone (__syncthreads' fence would wait
// for every copy and touch in flight): lgkmcnt(0) completes this wave's LDS
// accesses, and the asm's memory clobber keeps the compiler from moving
// memory accesses across it.  The caller's vm_wait<N>() decides which
// global -> LDS copies have landed.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0); vmcnt(63) and expcnt(7) are no-ops
    asm volatile("s_barrier" ::: "memory");
}

// Sequences are spread over the 8 XCDs (workgroup i runs on XCD i % 8) so
// that the V-slices of one sequence, which read the same W, M and Kd^T,
// land on the same XCD and share its L2.  Identity when the sequence count
// is not a multiple of 8.
__device__ __forceinline__ void inter_block(int blk, int nseq, int nvs, int *bh, int *vs) {
    if (nseq % 8 == 0) {
        const int x = blk % 8, j = blk / 8;
        *bh = x + 8 * (j / nvs);
        *vs = j % nvs;
    } else {
        *bh = blk / nvs;
        *vs = blk % nvs;
    }
}

// Host side of the chunked forward, shared with the backward (chunk.hip).
gdn2_status chunk_setup(const gdn2_chunk_args *a, const char *who, bool need_out, ChunkParams *p);
size_t chunk_fwd_ws_bytes(const gdn2_chunk_args *a);
// Segments per sequence of the sequential kernels (1 = unsegmented).
int chunk_segments(int64_t seqs, int64_t K, int64_t V, int64_t NC);
void chunk_bind_ws(const gdn2_chunk_args *a, char *ws, ChunkParams *p);

}  // namespace gdn2

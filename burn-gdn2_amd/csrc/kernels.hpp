// Kernel parameter blocks and launchers (internal to libgdn2_amd).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gdn2 {

// Per-token scan over T tokens (T = 1 is the decode step).
struct ScanParams {
    const float *q, *k, *g, *b; // [B, Hk, T, K] strided
    const float *v, *w;         // [B, HV, T, V] strided
    const float *state_in;      // [B, HV, K, V]
    float *state_out;           // [B, HV, K, V] (may equal state_in)
    float *out;                 // [B, HV, T, V] strided
    int B, HV, rep, T, K, V;
    int64_t sqb, sqh, sqt;
    int64_t svb, svh, svt;
    int64_t sob, soh, sot;
    float scale;
};

// Fused single-token decode.
struct DecodeParams {
    const float *q_raw, *k_raw, *f_raw, *b_raw; // [B, kd]
    const float *v_raw, *w_raw, *gate;          // [B, vd]
    const float *gate_bias;                     // [vd] added to gate, or null (gate includes it)
    const float *conv_q_in, *conv_k_in, *conv_v_in;
    float *conv_q_out, *conv_k_out, *conv_v_out;
    const float *q_conv_w, *k_conv_w, *v_conv_w;
    const float *a_log, *dt_bias, *decay_factors, *o_norm_weight;
    float *state; // [B, HV, K, V] in place
    float *out;   // [B, vd]
    // row strides (elements between batch rows) of the raw inputs and out
    int64_t ld_q, ld_k, ld_f, ld_b, ld_v, ld_w, ld_gate, ld_out;
    int B, H, HV, rep, K, V;
    int use_short_conv, allow_neg_eigval;
    float min_decay, one_minus_min_decay, norm_eps, scale;
};

// Chunked forward (two kernels: chunk-intra, then chunk-inter).
struct ChunkParams {
    const float *q, *k, *g, *b; // [B, Hk, T, K] strided
    const float *v, *w;         // [B, HV, T, V] strided
    float *state;               // [B, HV, K, V] in/out
    float *out;                 // [B, HV, T, V] strided
    int B, HV, rep, T, K, V, NC; // NC = number of chunks per sequence
    int64_t sqb, sqh, sqt;
    int64_t svb, svh, svt;
    int64_t sob, soh, sot;
    float scale;
    // workspace, per chunk (chunk id = (b * HV + hv) * NC + n), in MFMA
    // fragment order: 16x16 tiles of 64 lanes x float4 (see chunk.hip)
    float *ws_w;   // C*K   W = (I + A_kk)^-1 (b*k*gamma), A-operand tiles (row tile, col tile)
    float *ws_qg;  // C*K   scale * (q * gamma), same order
    float *ws_u;   // C*V   U = (I + A_kk)^-1 (w*v), accumulator tiles (col tile, row tile)
    float *ws_aqk; // C*C   A_qk (scale included, zero above the diagonal), A-operand tiles (row tile, col tile);
                   //       the tiles above the diagonal are left unwritten
    float *ws_kdt; // K*C   (k * exp(G_last - G))^T, A-operand tiles (key tile, time tile)
    float *ws_gam; // K     exp(G_last)
    // Segmented recurrence for few long sequences (NSEG > 1): the chunks of a
    // sequence are split into NSEG runs of SEGL chunks.  Per (b, hv):
    float *ws_pseg; // NSEG x K*K      transition of each segment (row-major; the last
                    //                 one only in the training forward)
    float *ws_qseg; // NSEG x K*V      state entering each segment (slot j + 1 first
                    //                 holds segment j's state from S = 0)
    int NSEG, SEGL;
    // Inference output split (SLOT0 = 1): segment 0 has SEG0 chunks and is
    // walked with the output from S0 beside pass 1, segment j >= 1 starts at
    // chunk SEG0 + (j - 1) SEGL and its slots are j - 1; pass 1 covers
    // segments 1 .. NSEG - 2.  Uniform runs: SEG0 = SLOT0 = 0.  NSLOT is the
    // slots per (b, hv) of ws_pseg / ws_qseg (the uniform run's NSEG).
    int SEG0, NSLOT, SLOT0;
    // Training forward (null in inference): the operands of the backward.
    float *ws_wt;   // C*K  W^T as A-operand tiles (key tile, time tile)
    float *ws_qgt;  // C*K  (scale q exp(G))^T, same order
    float *ws_kd;   // C*K  Kd as A-operand tiles (time tile, key tile)
    float *ws_aqkt; // C*C  A_qk^T as A-operand tiles (column tile, row tile)
    float *ws_akk;  // C*C  (I + A_kk)^-1, accumulator-layout tiles (row tile, column tile)
    float *ws_sn;   // K*V  state entering each chunk (row-major; for the backward, 16 x 16
                    //      accumulator fragments in (value tile, key tile) order)
    float *ws_vn;   // C*V  v_new of each chunk (row-major; for the backward, fragments in
                    //      (value tile, time tile) order)
    // Layout of ws_sn / ws_vn for a caller chunk size st_cc < 64 with T a
    // multiple of it (0: the 64-token chunk layout above).  st_chunks = T /
    // st_cc slots per (b, hv), slot j holding the state after st_cc j tokens;
    // v_new is written as token rows [B * HV, T, V] (rows < T only).  The
    // state entering 64-token chunk n goes to slot j0(n) = ceil(64 n / st_cc),
    // the first caller chunk that starts inside it (none when j0(n) >=
    // st_chunks); chunk_states_kernel derives the other slots from it.
    int st_cc, st_chunks;
    // Training forward with the output (the backward's saved inputs): the
    // training chunk-intra also writes scale q exp(G) and A_qk for the output.
    int fwd_out;
};

// Projection epilogue: raw Linear outputs -> kernel inputs, one token per
// workgroup.  Y rows hold the fused input projection [q | k | b | v | w | ..]
// at the given column offsets; F = f_proj_1 output.
struct ProjectParams {
    const float *Y;
    int64_t ldY, off_q, off_k, off_b, off_v, off_w;
    const float *F;
    int64_t ldF;
    const float *conv_q_in, *conv_k_in, *conv_v_in; // [B, 3, kd|vd]; null: pad with token 0
    const float *q_conv_w, *k_conv_w, *v_conv_w;
    const float *a_log, *dt_bias, *decay_factors; // decay_factors null without min_decay
    float *q, *k, *g, *b; // [B, H, T, K]
    float *v, *w;         // [B, HV, T, V]
    int B, T, H, K, HV, V;
    int use_short_conv, allow_neg_eigval;
    float min_decay, one_minus_min_decay;
};

// New conv caches [B, 3, kd|vd] from the raw projections (and the old caches).
struct ConvCacheParams {
    const float *Y;
    int64_t ldY, off_q, off_k, off_v;
    const float *in_q, *in_k, *in_v; // null: pad with token 0
    float *out_q, *out_k, *out_v;
    int B, T, kd, vd;
};

// Adjoint of the gated RMSNorm over rows of V values (rows = M * HV, each
// row contiguous).  y = O / rms * weight * silu(G) is recomputed on the way.
struct NormBwdParams {
    const float *O, *G, *weight;
    const float *gate_bias; // [HV * V] added to G (row r is value head r % HV), or null
    float *dy;     // in: gradient of y; out: dy * (O / rms) * silu(G) (weight-gradient terms)
    float *y;      // out: y (input of o_proj)
    float *dO, *dG;
    int64_t rows;
    int V, HV;
    float eps;
};

// Adjoint of the projection epilogue for one token per workgroup: recomputes
// the conv / SiLU pre-activations and the gates from Y and F, and maps the
// gradients of q, k, g, b [B, H, T, K] and v, w [B, HV, T, V] back to the
// Linear outputs.
struct ProjectBwdParams {
    const float *Y;
    int64_t ldY, off_q, off_k, off_b, off_v, off_w;
    const float *F;
    int64_t ldF;
    const float *conv_q_in, *conv_k_in, *conv_v_in; // null: pad with token 0
    const float *q_conv_w, *k_conv_w, *v_conv_w;
    const float *a_log, *dt_bias, *decay_factors;
    const float *dq, *dk, *dg, *db, *dv, *dw;
    float *dY;     // [M, ldY]: b and w columns; q, k, v columns without short conv
    float *DU;     // [M, 2 kd + vd]: gradient of the conv outputs (pre-SiLU), with short conv
    float *dF;     // [M, kd]: gradient of f_proj_1's output
    float *PA;     // [M, kd]: A_log gradient terms (dg_pre * g_pre)
    float *PD;     // [M, kd]: decay_factors gradient terms, null without min_decay
    int B, T, H, K, HV, V;
    int use_short_conv, allow_neg_eigval;
    float min_decay, one_minus_min_decay;
};

// Adjoint of the four-tap causal conv: columns of DU (q | k | v channels)
// back to the raw Linear outputs, the conv caches and the conv weights.
struct ConvBwdParams {
    const float *Y;
    int64_t ldY, off_q, off_k, off_v;
    const float *DU;
    const float *cache_q, *cache_k, *cache_v;        // caches on entry, null: pad with token 0
    const float *d_out_q, *d_out_k, *d_out_v;        // gradients of the caches after the call, or null
    const float *q_conv_w, *k_conv_w, *v_conv_w;
    float *dY;
    float *d_in_q, *d_in_k, *d_in_v;                 // gradients of the caches on entry, or null
    float *wpart;  // [B * nblk, (2 kd + vd) * 4] per-block conv weight gradients
    int B, T, kd, vd, tblock;
};

constexpr int kChunk = 64; // chunk length of the kernels (four 16-row tiles)

size_t project_lds_bytes(int kd);
hipError_t launch_project(const ProjectParams &p, hipStream_t s);
hipError_t launch_conv_cache(const ConvCacheParams &p, hipStream_t s);
// gate_bias [HV * V] (nullable) is added to the gate before its SiLU.
hipError_t launch_rmsnorm_gate(float *out, int64_t ld_out, const float *x, int64_t ld_x, const float *gate,
                               int64_t ld_gate, const float *gate_bias, const float *weight, int64_t M, int HV, int V,
                               float eps, hipStream_t s);
hipError_t launch_fill_rows(float *y, int64_t ld, const float *row, int64_t M, int64_t N, hipStream_t s);

// The reference's GVA layout of the key-side operands (src/module.rs:456-468:
// unsqueeze at 3, repeat rep times, reshape to [B, H rep, T, K]): value head
// h rep + a at time t reads key head h at time (a T + t) / rep.  Four tensors
// (q, k, g, b) at once.
struct GvaParams {
    const float *src[4];
    float *dst[4];
    int64_t B, H, T, K;
    int rep;
};
// dst [B, H rep, T, K] <- src [B, H, T, K] in that layout
hipError_t launch_gva_expand(const GvaParams &p, hipStream_t s);
// the adjoint: dst [B, H, T, K] = sum over the rep places each element went to in src [B, H rep, T, K]
hipError_t launch_gva_fold(const GvaParams &p, hipStream_t s);
// Reads buf[0, n) (16-byte aligned) to push other data out of the caches; writes
// nothing but, in theory, sink[0].
hipError_t launch_cache_sweep(const float *buf, int64_t n, float *sink, hipStream_t s);

// f_proj_1 and g_proj_1 for at most kLowRankMaxM rows and rank R in {64, 128,
// 256} (lowrank_up_kernel), Y 16-byte aligned with ldY and the offsets
// multiples of 4.
constexpr int kLowRankMaxM = 256;
struct LowRankParams {
    const float *Y;           // rows of the input GEMM's output, row stride ldY
    int64_t ldY, off_f0, off_g0;
    const float *F1, *G1;     // [R, kd], [R, vd] row-major
    const float *g_bias;      // [vd] or null
    float *F, *G;             // [M, kd], [M, vd] row-major
    int M, R, kd, vd;
};
bool lowrank_up_supported(int R, int64_t M, const float *Y, int64_t ldY, int64_t off_f0, int64_t off_g0);
hipError_t launch_lowrank_up(const LowRankParams &p, hipStream_t s);
hipError_t launch_rmsnorm_gate_bwd(const NormBwdParams &p, hipStream_t s);
hipError_t launch_project_bwd(const ProjectBwdParams &p, hipStream_t s);
int conv_bwd_blocks(int T, int tblock);
hipError_t launch_conv_bwd(const ConvBwdParams &p, hipStream_t s);
// out[j] (+)= sum over rows r, f < fold and i < group of
// A[r, f * (N / fold) + j * group + i], j < N / (group * fold); deterministic
// (fixed split of the rows into `parts`; part holds parts * N floats).
hipError_t launch_colsum(const float *A, int64_t rows, int64_t N, int64_t lda, int group, int fold, float *out,
                         bool accumulate, float *part, int parts, hipStream_t s);

hipError_t launch_scan(const ScanParams &p, hipStream_t s);
hipError_t launch_decode(const DecodeParams &p, hipStream_t s);
bool chunk_supported(int K, int V);     // the chunked forward's instances
bool chunk_bwd_supported(int K, int V); // the chunked backward's
// phases: bit 0 intra (with the training outputs when ws_akk is set), bit 1
// inter with the output, bit 2 inter writing ws_sn / ws_vn in the backward's
// layouts (with bit 1: the output and the final state as well; without: neither).
hipError_t launch_chunk(const ChunkParams &p, hipStream_t s, int phases);

}  // namespace gdn2

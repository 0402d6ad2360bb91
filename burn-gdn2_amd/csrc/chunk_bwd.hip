// Chunked GDN-2 backward on gfx950: the gradients of
//   L = <d_out, out> + <d_state_out, S_T>
// with respect to q, k, g, b, v, w and S0 -- the seven outputs of the
// reference's fused_chunk_backward (src/kernel/chunk_adjoint_cube.rs:464-707);
// its training path otherwise differentiates chunk_wy_forward
// (src/forward.rs:44-278) through autodiff.
//
// Per chunk, with S the state entering it, dS' = dL/d(state leaving it), dO
// the chunk's rows of d_out and the forward's quantities of chunk.hip
// (W, U, A_qk, A_kk, Kd, QG = scale q e^G, Rk = b k e^G, Ai = (I + A_kk)^-1):
//   dv_new = A_qk^T dO + Kd dS'                                  (reverse, sequential)
//   dS     = e^{G_last} dS' + QG^T dO - W^T dv_new               (reverse, sequential)
//   dQG = dO S^T,  dW = -dv_new S^T,  dKd = v_new dS'^T,  dgam = rowsum(dS' * S)
//   dA_qk = tril(dO v_new^T),  dRk = Ai^T dW,  dRv = Ai^T dv_new
//   dA_kk = strict_tril(-(dRk W^T + Ai^T dv_new U^T)),  dw = dRv * v,  dv = dRv * w
// and the decay-weighted terms of A_qk, A_kk, QG, Rk, Kd and e^{G_last} give
// dq, dk, db and dG; dg is the reverse cumulative sum of dG over the chunk.
//
// Kernels (in launch order):
//   chunk_intra_kernel<K, V, true>       the forward operands plus W^T, QG^T, Kd, A_qk^T, (I + A_kk)^-1
//   chunk_inter_kernel<K, kInterStates>  the state entering every chunk and v_new
//   bwd_inter_kernel   the reverse recurrence (one workgroup per (b, hv, 64 columns))
//   bwd_vprod_kernel   dQG, dKd, dA_qk, dgam, then dRk, dRv -> dv, dw and dA_kk, per chunk
//   bwd_decay_kernel   dq, dk, db, dg, per chunk
//   bwd_gva_kernel     key-side gradients summed over the value heads of a key head
#include "chunk_common.hpp"

namespace gdn2 {
namespace {

struct BwdParams {
    ChunkParams f;                    // forward shapes, strides, operands and workspace
    const float *d_out;               // strided like out (f.sob, f.soh, f.sot)
    const float *d_state_out;         // [B, HV, K, V] or null (zero)
    float *dq, *dk, *dg, *db;         // strided like q (f.sqb, f.sqh, f.sqt)
    float *dv, *dw;                   // strided like v (f.svb, f.svh, f.svt)
    float *d_state0;                  // [B, HV, K, V]
    // per chunk (chunk id = (b * HV + hv) * NC + n).  "Row-major",
    // "fragments": 16 x 16 tiles (row tile, column tile) in row-major tile
    // order, each 64 lanes x float4 in accumulator layout (lane (g, c) holds
    // rows 4 g .. 4 g + 3 of column c), so that every access is one 16-byte
    // load, or "column fragments": the same tiles in (column tile, row tile)
    // order, so that each 16-column slice of an R x V matrix is one block.
    float *ws_dsn;                    // K*V  dL/d(state leaving the chunk), column fragments
    float *ws_dvn;                    // C*V  dL/dv_new, column fragments
    float *ws_dqg, *ws_dkd;           // C*K  dL/dQG, dL/dKd, fragments
    float *ws_daqk;                   // C*C  dL/dA_qk, fragments (the lower block triangle only)
    float *ws_dgam;                   // K    dL/d e^{G_last}
    float *ws_drk;                    // C*K  dL/dRk, fragments
    float *ws_dakk;                   // C*C  dL/dA_kk, fragments (the lower block triangle only)
    float *ws_kgrad;                  // rep > 1: 4 x (C*K per chunk): dq, dk, dg, db per value head
    // segmented reverse recurrence (NSEG > 1), per (b, hv):
    float *ws_rseg;                   // NSEG x K*V  the gradient leaving each segment (slot j - 1
                                      //             first holds R_j of segment j)
};

__device__ __forceinline__ floatx4 mfma4x(floatx4 a, floatx4 b, floatx4 c) {
    c = mfma16(a[0], b[0], c);
    c = mfma16(a[1], b[1], c);
    c = mfma16(a[2], b[2], c);
    c = mfma16(a[3], b[3], c);
    return c;
}

// ---------------------------------------------------------------------------
// Reverse recurrence.  One workgroup per (b, hv, 16 NW value columns), wave w
// owns 16 columns; dS' stays in MFMA accumulators (key rows x 16 columns).
// NW = 4, or 2 where V is not a multiple of 64 (V = 32, 96) and for K = 32,
// as in the forward's chunk-inter.
// Per chunk n, last to first:
//   1: dv_new = A_qk^T dO + Kd dS'         (reads sAT, sKd)
//      dS' and dv_new go to the workspace for the per-chunk kernels
//   2: dS' <- e^{G_last} dS' + QG^T dO - W^T dv_new   (reads sQT, sWT)
// The operands are A-operand fragments written by the training forward, so
// every product has the shape of the forward's chunk-inter products.  As
// there, each LDS buffer is refilled by direct copies while the other phase
// runs, behind fence-free barriers that wait only for those copies.
//
// Segmented form (NSEG > 1), the mirror of the forward's: over a segment the
// map from the gradient leaving it to the gradient entering it is affine,
//   dS_in = P^T dS_out + R,
// with P the segment's forward transition (from the training forward's
// segment pass) and R the segment run from dS' = 0.  Pass 1 (kRevLocal)
// computes R of every segment but the first, bwd_chain_kernel chains the
// segments from the last, and pass 3 (kRevOut) re-runs every segment from
// its gradient with the stores; the first segment writes dS0.
// ---------------------------------------------------------------------------
constexpr int kRevOut = 0, kRevLocal = 1;

template <int K, int MODE, int NW>
__global__ __launch_bounds__(64 * NW, 1) void bwd_inter_kernel(BwdParams bp, int seg0, int nseg_launch) {
    const ChunkParams &p = bp.f;
    constexpr bool LOCAL = MODE == kRevLocal;
    constexpr int NTH = 64 * NW, NKT = K / 16;
    constexpr int OPF4 = NKT * NT * 64, PFO = OPF4 / NTH;
    constexpr int AF4 = NT * NT * 64, APF = AF4 / NTH;
    static_assert(OPF4 % NTH == 0 && AF4 % NTH == 0, "K");
    // K = 256: Kd and W^T take 64 KiB of LDS each, so (scale q e^G)^T, whose
    // product QG^T dO feeds only dS (not the dS -> dv_new chain), is read from
    // L2 into registers in phase 2 instead of through a third LDS buffer.
    constexpr bool QLDS = K <= 128;
    __shared__ floatx4 sKd[OPF4], sAT[AF4], sQT[QLDS ? OPF4 : 1], sWT[OPF4];
    __shared__ float sPf[256]; // destination of the L2 touches, never read
    // e^{G_last} of the chunk, copied with the Q^T / W^T operands and read
    // in phase 2: one copy for the workgroup instead of every wave's loads
    __shared__ floatx4 sGam[K / 4];
    // K = 128: the chunk's d_out rows of the workgroup's 16 NW columns,
    // double-buffered, copied with Kd and A_qk^T (16-byte copies, a quarter of
    // the vector memory instructions of per-lane row loads), in the LDS left
    // beside its one workgroup per CU.  K = 256 has none left, and at K <= 64
    // they would cost a second workgroup per CU: those load them into registers.
    constexpr bool DOLDS = K == 128;
    constexpr int VSW = 16 * NW, DOF4 = C * VSW / 4, DOPF = DOF4 / NTH;
    static_assert(DOF4 % NTH == 0, "d_out block");
    __shared__ floatx4 sDO[DOLDS ? 2 : 1][DOLDS ? DOF4 : 1];

    const int V = p.V, nvv = V / (16 * NW);
    int sq, vs;
    inter_block(blockIdx.x, p.B * p.HV * nseg_launch, nvv, &sq, &vs);
    const int bh = sq / nseg_launch, seg = seg0 + sq % nseg_launch;
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int col = 16 * (vs * NW + wave) + lr;
    const int n0 = seg * p.SEGL, n1 = min(p.NC, n0 + p.SEGL);

    // the gradient leaving the segment: d_state_out (one segment), the chained
    // gradient (pass 3) or 0 (pass 1)
    floatx4 dS[NKT];
    const float *din = nullptr;
    if (!LOCAL) din = p.NSEG == 1 ? bp.d_state_out : bp.ws_rseg + ((size_t)bh * p.NSEG + seg) * K * V;
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * kb + 4 * lg + i;
            dS[kb][i] = LOCAL ? 0.f : (din ? din[(p.NSEG == 1 ? (size_t)bh * K * V : 0) + (size_t)row * V + col] : 0.f);
        }

    const floatx4 *__restrict__ KD4 = reinterpret_cast<const floatx4 *>(p.ws_kd);
    const floatx4 *__restrict__ AT4 = reinterpret_cast<const floatx4 *>(p.ws_aqkt);
    const floatx4 *__restrict__ QT4 = reinterpret_cast<const floatx4 *>(p.ws_qgt);
    const floatx4 *__restrict__ WT4 = reinterpret_cast<const floatx4 *>(p.ws_wt);
    const floatx4 *__restrict__ G4 = reinterpret_cast<const floatx4 *>(p.ws_gam);
    const size_t cid0 = (size_t)bh * p.NC;
    const int wv = 64 * wave;

    // The operands go from global memory straight into LDS (lds_copy4: thread
    // tid's float4 i lands at index i * NTH + tid).  Each is also pulled
    // toward L2 ahead of its copy (l2_touch, one 128-byte line per thread):
    // Kd, A_qk^T of chunk n - 2 and QT, WT of chunk n - 1, both issued after
    // the copies that follow chunk n's second barrier, so that they land during
    // its phase 2; outside the segment the chunk is clamped to it.
    float *pf_slot = &sPf[wv];
    constexpr int LOP = OPF4 / 8, LA = AF4 / 8; // 128-byte lines per operand block
    auto clamp_c = [&](int n) { return cid0 + (size_t)max(n0, min(n1 - 1, n)); };
    auto touch_ka = [&](size_t c) {
        l2_touch(reinterpret_cast<const char *>(KD4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
        l2_touch(reinterpret_cast<const char *>(AT4 + c * AF4) + 128 * (tid % LA), pf_slot);
    };
    auto touch_qw = [&](size_t c) {
        l2_touch(reinterpret_cast<const char *>(QT4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
        l2_touch(reinterpret_cast<const char *>(WT4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
    };
    auto copy_ka = [&](size_t c) {
#pragma unroll
        for (int i = 0; i < PFO; ++i) lds_copy4(&KD4[c * OPF4 + i * NTH + tid], &sKd[i * NTH + wv]);
#pragma unroll
        for (int i = 0; i < APF; ++i) { // this wave's tile (st, rt) of the copy: A_qk^T needs rt >= st only
            const int f = i * NW + wave;
            if (f % NT >= f / NT) lds_copy4(&AT4[c * AF4 + i * NTH + tid], &sAT[i * NTH + wv]);
        }
    };
    // chunk n's rows of d_out through a buffer resource over its valid rows
    // (rows past T read 0).  Registers: row 4 lg of each 16-row tile, the rest
    // of the row offset wave-uniform.  LDS: the block [C][VSW] row-major in
    // buffer n & 1, thread tid's float4 i at index i * NTH + tid.
    const float *dob = bp.d_out + (int64_t)bi * p.sob + (int64_t)hv * p.soh;
    const int ro = (int)p.sot, dol = 4 * lg * ro + col;
    auto load_dO = [&](floatx4 *dO, int n) {
        const __amdgpu_buffer_rsrc_t R = rows_rsrc(dob + (int64_t)n * C * p.sot, ro, min(C, p.T - n * C), V);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) dO[mt][i] = bld1(R, dol + (16 * mt + i) * ro);
    };
    const int col0 = 16 * vs * NW; // the workgroup's first column
    auto copy_dO = [&](int n) {
        const __amdgpu_buffer_rsrc_t R = rows_rsrc(dob + (int64_t)n * C * p.sot, ro, min(C, p.T - n * C), V);
#pragma unroll
        for (int i = 0; i < DOPF; ++i) {
            const int f = i * NTH + tid, row = f / (VSW / 4), c4 = f % (VSW / 4);
            lds_copy4_rsrc(R, 4 * (row * ro + col0 + 4 * c4), &sDO[n & 1][i * NTH + wv]);
        }
    };
    auto read_dO = [&](floatx4 *dO, int n) { // this lane's B-fragment values from the block
        const float *blk = reinterpret_cast<const float *>(sDO[n & 1]);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) dO[mt][i] = blk[(16 * mt + 4 * lg + i) * VSW + 16 * wave + lr];
    };

    floatx4 dO[NT]; // rows of d_out of the current chunk, loaded a phase ahead
    if (n1 > n0) {
        copy_ka(cid0 + n1 - 1);
        if constexpr (DOLDS)
            copy_dO(n1 - 1);
        else
            load_dO(dO, n1 - 1);
        __builtin_amdgcn_sched_barrier(0);
        touch_qw(cid0 + n1 - 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    // dS and the first copies have landed: nothing from before the loop is
    // left in flight for the compiler's own vmcnt waits inside it
    vm_wait0();

    for (int n = n1 - 1; n >= n0; --n) {
        const size_t cid = cid0 + n;
        vm_wait<2>();  // this wave's copies of Kd, A_qk^T (n) and its dO rows have landed (not the last 2 touches)
        lds_barrier(); // sKd, sAT hold chunk n; every wave is done with sQT, sWT (n+1)
        if constexpr (DOLDS) read_dO(dO, n); // used from the end of phase 1 on
#pragma unroll
        for (int i = 0; i < PFO; ++i) {
            if (QLDS) lds_copy4(&QT4[cid * OPF4 + i * NTH + tid], &sQT[i * NTH + wv]);
            lds_copy4(&WT4[cid * OPF4 + i * NTH + tid], &sWT[i * NTH + wv]);
        }
        if (!LOCAL) { // dL/d(state leaving chunk n)
            float *Dsn = bp.ws_dsn + cid * K * V;
#pragma unroll
            for (int kb = 0; kb < NKT; ++kb)
                reinterpret_cast<floatx4 *>(Dsn)[((col >> 4) * NKT + kb) * 64 + lane] = dS[kb];
        }
        if (wave == 0 && lane < K / 4) lds_copy4(&G4[cid * (K / 4) + lane], sGam);

        // 1: dv_new = Kd dS' + A_qk^T dO (A_qk^T is upper block-triangular).
        // Each k-step's Kd fragments are requested after the first quarter of
        // the previous step's products, the A_qk^T tiles during the last step.
        floatx4 dvn[NT];
#pragma unroll
        for (int st = 0; st < NT; ++st) dvn[st] = floatx4{0.f, 0.f, 0.f, 0.f};
        {
            floatx4 ka[2][NT], at[NT][NT]; // at[st][rt], rt >= st
            auto load_k = [&](int kb, int bf) {
#pragma unroll
                for (int st = 0; st < NT; ++st) ka[bf][st] = sKd[(st * NKT + kb) * 64 + lane];
            };
            load_k(0, 0);
#pragma unroll
            for (int kb = 0; kb < NKT; ++kb) {
                const int cb = kb & 1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int st = 0; st < NT; ++st) dvn[st] = mfma16(ka[cb][st][j], dS[kb][j], dvn[st]);
                    if (j == 0) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (kb + 1 < NKT)
                            load_k(kb + 1, cb ^ 1);
                        else
#pragma unroll
                            for (int st = 0; st < NT; ++st)
#pragma unroll
                                for (int rt = st; rt < NT; ++rt) at[st][rt] = sAT[(st * NT + rt) * 64 + lane];
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                    for (int st = 0; st <= rt; ++st) dvn[st] = mfma16(at[st][rt][j], dO[rt][j], dvn[st]);
        }
        vm_wait0();    // this wave's copies of QT, WT (n) and its e^{G_last} have landed
        lds_barrier(); // phase 1 done everywhere (sKd, sAT free); sQT, sWT (n) visible

        // Kd, A_qk^T and the dO rows of chunk n - 1; dv_new to the workspace
        floatx4 dO_next[NT];
        __builtin_amdgcn_sched_barrier(0);
        if (n > n0) {
            copy_ka(cid - 1);
            if constexpr (DOLDS)
                copy_dO(n - 1); // into the other buffer: every wave read this one after the last barrier
            else
                load_dO(dO_next, n - 1);
        }
        if (!LOCAL) {
            float *Dvn = bp.ws_dvn + cid * C * V;
#pragma unroll
            for (int st = 0; st < NT; ++st)
                reinterpret_cast<floatx4 *>(Dvn)[((col >> 4) * NT + st) * 64 + lane] = dvn[st];
        }
        // the touches last, after this barrier's copies: issued before the
        // barrier they would occupy the memory pipeline's outstanding line
        // requests (64 lines per touch instruction, from HBM) while the copies
        // above queue behind them
        __builtin_amdgcn_sched_barrier(0);
        touch_qw(clamp_c(n - 1));
        touch_ka(clamp_c(n - 2));
        __builtin_amdgcn_sched_barrier(0);

        // 2: dS' <- e^{G_last} dS' + QG^T dO - W^T dv_new
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            const floatx4 gam = sGam[4 * kb + lg]; // rows 16 kb + 4 lg .. + 3 of dS'
            dS[kb][0] *= gam[0];
            dS[kb][1] *= gam[1];
            dS[kb][2] *= gam[2];
            dS[kb][3] *= gam[3];
        }
        // each time tile's QG^T and W^T fragments are requested after the first
        // quarter of the previous tile's products.  -W^T dv_new = W^T (-dv_new):
        // the MFMA takes no sign on an f32 operand, so the 16 values of -dv_new are
        // formed once rather than the 128 of -W^T
        {
            floatx4 ndv[NT];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) ndv[tt] = -dvn[tt];
            floatx4 qa[2][NKT], wa[2][NKT];
            auto load_qw = [&](int tt, int bf) {
#pragma unroll
                for (int kb = 0; kb < NKT; ++kb) {
                    qa[bf][kb] = QLDS ? sQT[(kb * NT + tt) * 64 + lane] : QT4[cid * OPF4 + (kb * NT + tt) * 64 + lane];
                    wa[bf][kb] = sWT[(kb * NT + tt) * 64 + lane];
                }
            };
            load_qw(0, 0);
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const int cb = tt & 1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int kb = 0; kb < NKT; ++kb) {
                        dS[kb] = mfma16(qa[cb][kb][j], dO[tt][j], dS[kb]);
                        dS[kb] = mfma16(wa[cb][kb][j], ndv[tt][j], dS[kb]);
                    }
                    if (j == 0) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (tt + 1 < NT) load_qw(tt + 1, cb ^ 1);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (!DOLDS && n > n0) {
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) dO[mt] = dO_next[mt];
        }
    }
    vm_wait0(); // the last touches have landed in sPf
    // the gradient entering the segment: dS0 (first segment) or R_j (pass 1)
    float *out = nullptr;
    if (!LOCAL) {
        if (seg == 0) out = bp.d_state0 + (size_t)bh * K * V;
    } else {
        out = bp.ws_rseg + ((size_t)bh * p.NSEG + seg - 1) * K * V;
    }
    if (out) {
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) out[(size_t)(16 * kb + 4 * lg + i) * V + col] = dS[kb][i];
    }
}

// Pass 2 of the segmented reverse recurrence.  ws_rseg holds NSEG slots of
// K x V per (b, hv): slot NSEG-1 <- d_state_out (or 0), then slot j - 1 (R_j
// from pass 1) <- P_j^T slot j + R_j for j = NSEG-1 .. 1: the gradient leaving
// every segment.  Same MFMA layout as the forward's chunk_chain_kernel, with
// P_j^T's A fragments gathered from the forward's row-major P_j.
template <int K, int NW>
__global__ __launch_bounds__(64 * NW, 1) void bwd_chain_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int NKT = K / 16;
    const int V = p.V, nvv = V / (16 * NW);
    int bh, vs;
    inter_block(blockIdx.x, p.B * p.HV, nvv, &bh, &vs);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int col = 16 * (vs * NW + wave) + lr;
    float *slot0 = bp.ws_rseg + (size_t)bh * p.NSEG * K * V;
    float *last = slot0 + (size_t)(p.NSEG - 1) * K * V;
    floatx4 S[NKT];
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t o = (size_t)(16 * kb + 4 * lg + i) * V + col;
            S[kb][i] = bp.d_state_out ? bp.d_state_out[(size_t)bh * K * V + o] : 0.f;
            last[o] = S[kb][i];
        }
    for (int j = p.NSEG - 1; j >= 1; --j) {
        const float *P = p.ws_pseg + ((size_t)bh * p.NSEG + j) * K * K; // P_j, row-major
        float *Q = slot0 + (size_t)(j - 1) * K * V;
        floatx4 N[NKT];
#pragma unroll
        for (int it = 0; it < NKT; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i) N[it][i] = Q[(size_t)(16 * it + 4 * lg + i) * V + col];
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            floatx4 pa[NKT];
#pragma unroll
            for (int it = 0; it < NKT; ++it) // P_j^T[16 it + lr][16 kb + 4 lg + st] = P_j[16 kb + 4 lg + st][16 it + lr]
#pragma unroll
                for (int st = 0; st < 4; ++st) pa[it][st] = P[(size_t)(16 * kb + 4 * lg + st) * K + 16 * it + lr];
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int it = 0; it < NKT; ++it) N[it] = mfma16(pa[it][st], S[kb][st], N[it]);
        }
#pragma unroll
        for (int it = 0; it < NKT; ++it) {
            S[it] = N[it];
#pragma unroll
            for (int i = 0; i < 4; ++i) Q[(size_t)(16 * it + 4 * lg + i) * V + col] = N[it][i];
        }
    }
}

// ---------------------------------------------------------------------------
// Per-chunk products over the value dimension, then the solve adjoint (MFMA,
// four waves, one workgroup per chunk):
//   dQG = dO S^T, dW = -dv_new S^T, dKd = v_new dS'^T       (C x K)
//   dA_qk = tril(dO v_new^T), dUU = strict_tril(dv_new U^T)  (C x C)
//   dgam = rowsum(dS' * S)
// and, with Ai = (I + A_kk)^-1 from the training forward (accumulator-layout
// tiles, i.e. the A fragments of Ai^T):
//   [dRk | dRv] = Ai^T [dW | dv_new]   (dv = dRv * w, dw = dRv * v)
//   dA_kk = strict_tril(-(dRk W^T + Ai^T dUU))
// Value loop: wave w owns the 16 rows of time tile w of every product; its A
// fragments (rows of dO, dv_new, v_new) come straight from memory, and its
// accumulators stay in registers over the V loop.  The B operands (16 columns
// of S, dS', v_new and U per step) are read once per workgroup into a
// double-buffered LDS slice; the slice loads of step vb+1 are issued before
// step vb's products.
// dW and dUU never leave the compute unit: after the loop they take the
// staging buffers' place in LDS (dW row-major, dUU as fragments).  Wave w then
// owns column tiles w, w + 4, ... of [dRk | dRv]: it reads a dW column tile
// whole before writing dRk over it, as rows for dA_kk's A fragments, and
// reads dv_new's column tiles from memory.  Last,
// wave w computes dA_kk tiles w, w + 4, ... (W's stored A fragments are the B
// fragments of W^T).
// ---------------------------------------------------------------------------
template <int K, int V>
struct VprodSmem {
    static constexpr int SP = 20;     // padded row of a 16-column slice
    static constexpr int KP = K + 4;  // padded row of dW / dRk
    // value loop: S, dS' slices [2][K][SP]; v_new, dv_new and U slices [2][C][SP]
    static constexpr size_t oS = 0, oD = oS + 4 * 2 * K * SP, oV = oD + 4 * 2 * K * SP, oDV = oV + 4 * 2 * C * SP;
    static constexpr size_t oU = oDV + 4 * 2 * C * SP, stage = oU + 4 * 2 * C * SP;
    // solve: dW, then dRk [C][KP]; dUU fragments [NT * NT * 64]; per wave a
    // [C][SP] tile of v, w, dv or dw rows (the transpose between 16-byte rows
    // and accumulator fragments)
    static constexpr size_t oR = 0, oUU = oR + 4 * C * KP, oX = oUU + 16 * NT * NT * 64;
    static constexpr size_t solve = oX + 4 * 4 * C * SP;
    static constexpr size_t bytes = stage > solve ? stage : solve;
    static_assert(oU % 16 == 0 && oUU % 16 == 0 && oX % 16 == 0, "float4 alignment");
};

template <int K, int V>
__global__ __launch_bounds__(256, K >= 256 ? 1 : 2) void bwd_vprod_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    using SM = VprodSmem<K, V>;
    constexpr int NKT = K / 16, NVB = V / 16, NVT = V / 16, NCT = NKT + NVT;
    constexpr int SP = SM::SP, KP = SM::KP;
    // float4 per thread of an S (and dS') slice and of a v_new slice; at K = 32
    // an S slice is 128 float4, taken by threads 0 .. 127
    constexpr int SF4 = (K * 4 + 255) / 256, VF4 = C * 4 / 256;
    constexpr bool SPART = K * 4 < 256;
    constexpr int NLT = NT * (NT + 1) / 2;              // lower tiles
    __shared__ __attribute__((aligned(16))) char smem[SM::bytes];
    float(*sS)[K][SP] = reinterpret_cast<float(*)[K][SP]>(smem + SM::oS);
    float(*sD)[K][SP] = reinterpret_cast<float(*)[K][SP]>(smem + SM::oD);
    float(*sV)[C][SP] = reinterpret_cast<float(*)[C][SP]>(smem + SM::oV);
    float(*sDV)[C][SP] = reinterpret_cast<float(*)[C][SP]>(smem + SM::oDV);
    float(*sU)[C][SP] = reinterpret_cast<float(*)[C][SP]>(smem + SM::oU);
    float(*sR)[KP] = reinterpret_cast<float(*)[KP]>(smem + SM::oR);
    floatx4 *sUU = reinterpret_cast<floatx4 *>(smem + SM::oUU);
    const int cid = blockIdx.x, bh = cid / p.NC, n = cid % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int cv = min(C, p.T - n * C);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // = the time tile of the value loop
    const int lr = lane & 15, lg = lane >> 4;

    const float *dO = bp.d_out + (int64_t)bi * p.sob + (int64_t)hv * p.soh + (int64_t)(n * C) * p.sot;
    const int ro = (int)p.sot;
    const __amdgpu_buffer_rsrc_t RdO = rows_rsrc(dO, ro, cv, V);
    // S, dS', v_new, dv_new and U of the chunk as accumulator fragments in
    // (value tile, row tile) order: slice vb is one contiguous block, and
    // thread tid's float4 i of it is lane tid % 64 of row tile 4 i + tid / 64
    const floatx4 *Sn = reinterpret_cast<const floatx4 *>(p.ws_sn + (size_t)cid * K * V);
    const floatx4 *dSn = reinterpret_cast<const floatx4 *>(bp.ws_dsn + (size_t)cid * K * V);
    const floatx4 *vn = reinterpret_cast<const floatx4 *>(p.ws_vn + (size_t)cid * C * V);
    const floatx4 *dvn = reinterpret_cast<const floatx4 *>(bp.ws_dvn + (size_t)cid * C * V);
    const floatx4 *Uf = reinterpret_cast<const floatx4 *>(p.ws_u + (size_t)cid * C * V);
    const int arow = 16 * wave + lr;

    floatx4 aQ[NKT], aW[NKT], aK[NKT], aA[NT], aU[NT];
#pragma unroll
    for (int t = 0; t < NKT; ++t) aQ[t] = aW[t] = aK[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) aA[t] = aU[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    // this thread's fragment lane: rows 4 g .. 4 g + 3 (of its row tiles) of column c
    const int g4 = 4 * ((tid >> 4) & 3), fc = tid & 15;
    floatx4 gam[SF4]; // dS' * S partial sums of those rows, over this thread's columns
#pragma unroll
    for (int i = 0; i < SF4; ++i) gam[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    floatx4 ls[SF4], ld_[SF4], lv[VF4], ldv[VF4], lu;
    auto load_slice = [&](int vb) {
#pragma unroll
        for (int i = 0; i < SF4; ++i)
            if (!SPART || tid < K * 4) {
                ls[i] = Sn[vb * K * 4 + i * 256 + tid];
                ld_[i] = dSn[vb * K * 4 + i * 256 + tid];
            }
#pragma unroll
        for (int i = 0; i < VF4; ++i) {
            lv[i] = vn[vb * C * 4 + i * 256 + tid];
            ldv[i] = dvn[vb * C * 4 + i * 256 + tid];
        }
        lu = Uf[vb * NT * 64 + tid]; // tiles (vb, 0 .. NT-1): NT * 64 float4 = 256
    };
    // the fragments go to LDS as row-major slices (row, 16 columns)
    auto store_slice = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SF4; ++i)
            if (!SPART || tid < K * 4) {
                const int r0 = 16 * (4 * i + (tid >> 6)) + g4;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sS[buf][r0 + j][fc] = ls[i][j];
                    sD[buf][r0 + j][fc] = ld_[i][j];
                }
                gam[i] += ls[i] * ld_[i];
            }
#pragma unroll
        for (int i = 0; i < VF4; ++i) {
            const int r0 = 16 * (4 * i + (tid >> 6)) + g4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sV[buf][r0 + j][fc] = lv[i][j];
                sDV[buf][r0 + j][fc] = ldv[i][j];
            }
        }
        const int ur = 16 * (tid >> 6) + g4;
#pragma unroll
        for (int j = 0; j < 4; ++j) sU[buf][ur + j][fc] = lu[j];
    };
    static_assert(NT * 64 == 256, "one U fragment per thread");

    load_slice(0);
    store_slice(0);
    __syncthreads();
#pragma unroll 1
    for (int vb = 0; vb < NVB; ++vb) {
        const int buf = vb & 1;
        if (vb + 1 < NVB) load_slice(vb + 1);
        const int c0 = 16 * vb + 4 * lg;
        const floatx4 fO = bld4(RdO, arow * ro + c0);
        const floatx4 fD = *reinterpret_cast<const floatx4 *>(&sDV[buf][arow][4 * lg]);
        const floatx4 fV = *reinterpret_cast<const floatx4 *>(&sV[buf][arow][4 * lg]);
#pragma unroll
        for (int t = 0; t < NKT; ++t) {
            const floatx4 bS = *reinterpret_cast<const floatx4 *>(&sS[buf][16 * t + lr][4 * lg]);
            const floatx4 bD = *reinterpret_cast<const floatx4 *>(&sD[buf][16 * t + lr][4 * lg]);
            aQ[t] = mfma4x(fO, bS, aQ[t]);
            aW[t] = mfma4x(fD, bS, aW[t]);
            aK[t] = mfma4x(fV, bD, aK[t]);
        }
#pragma unroll
        for (int st = 0; st < NT; ++st) {
            if (st <= wave) {
                const floatx4 bV = *reinterpret_cast<const floatx4 *>(&sV[buf][16 * st + lr][4 * lg]);
                const floatx4 bU = *reinterpret_cast<const floatx4 *>(&sU[buf][16 * st + lr][4 * lg]);
                aA[st] = mfma4x(fO, bV, aA[st]);
                aU[st] = mfma4x(fD, bU, aU[st]);
            }
        }
        if (vb + 1 < NVB) {
            store_slice(buf ^ 1);
            __syncthreads();
        }
    }
    // dQG, dKd, dA_qk (fragments; tiles (wave, st <= wave) only, the decay kernel
    // reads no other) and dgam go to the decay kernel
    floatx4 *oQ = reinterpret_cast<floatx4 *>(bp.ws_dqg) + (size_t)cid * (C * K / 4);
    floatx4 *oK = reinterpret_cast<floatx4 *>(bp.ws_dkd) + (size_t)cid * (C * K / 4);
    floatx4 *oA = reinterpret_cast<floatx4 *>(bp.ws_daqk) + (size_t)cid * (C * C / 4);
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
        oQ[(wave * NKT + t) * 64 + lane] = aQ[t];
        oK[(wave * NKT + t) * 64 + lane] = aK[t];
    }
#pragma unroll
    for (int st = 0; st < NT; ++st)
        if (st <= wave) { // wave-uniform
            floatx4 a = aA[st];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = 16 * st + lr <= 16 * wave + 4 * lg + i ? a[i] : 0.f;
            oA[(wave * NT + st) * 64 + lane] = a;
        }
    // dgam: a row's 16 columns of every slice were staged by the 16 lanes 16 g .. 16 g + 15
#pragma unroll
    for (int i = 0; i < SF4; ++i) {
        floatx4 g = gam[i];
#pragma unroll
        for (int m = 1; m < 16; m <<= 1)
#pragma unroll
            for (int j = 0; j < 4; ++j) g[j] += __shfl_xor(g[j], m, 64);
        if (fc == 0 && (!SPART || tid < K * 4))
#pragma unroll
            for (int j = 0; j < 4; ++j) bp.ws_dgam[(size_t)cid * K + 16 * (4 * i + (tid >> 6)) + g4 + j] = g[j];
    }
    __syncthreads(); // every wave is done with the last slice: the staging buffers are free
    // dW = -(dv_new S^T) rows of time tile `wave` (lane (lg, lr): rows 4 lg + i of column lr)
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sR[16 * wave + 4 * lg + i][16 * t + lr] = -aW[t][i];
    // dUU tiles (wave, st), zero on and above the diagonal
#pragma unroll
    for (int st = 0; st < NT; ++st) {
        floatx4 u = aU[st];
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = 16 * st + lr < 16 * wave + 4 * lg + i ? u[i] : 0.f;
        sUU[(wave * NT + st) * 64 + lane] = u;
    }
    __syncthreads();

    // [dRk | dRv] = Ai^T [dW | dv_new].  Ai^T A fragments (rt, st), st >= rt: Ai's tile (st, rt)
    const floatx4 *Aif = reinterpret_cast<const floatx4 *>(p.ws_akk) + (size_t)cid * (C * C / 4);
    floatx4 ai[NLT];
#pragma unroll
    for (int rt = 0, f = 0; rt < NT; ++rt)
#pragma unroll
        for (int st = rt; st < NT; ++st, ++f) ai[f] = Aif[(st * NT + rt) * 64 + lane];
    auto aiT = [&](int rt, int st) -> floatx4 { // index of (rt, st) in the list above
        return ai[rt * NT - rt * (rt - 1) / 2 + (st - rt)];
    };
    floatx4 *drk = reinterpret_cast<floatx4 *>(bp.ws_drk) + (size_t)cid * (C * K / 4);
    const int64_t vo = (int64_t)bi * p.svb + (int64_t)hv * p.svh + (int64_t)(n * C) * p.svt;
    const int rv = (int)p.svt;
    const __amdgpu_buffer_rsrc_t Rv = rows_rsrc(p.v + vo, rv, cv, V), Rw = rows_rsrc(p.w + vo, rv, cv, V);
    const __amdgpu_buffer_rsrc_t Rdv = rows_rsrc(bp.dv + vo, rv, cv, V), Rdw = rows_rsrc(bp.dw + vo, rv, cv, V);
    // this wave's [C][SP] tile: v, w, dv, dw move as 16-byte row pieces (lane
    // l: row 16 m + l / 4, columns 4 (l % 4) .. + 3 of the 16-column tile) and
    // are read or written there in accumulator layout (rows 4 lg + i, column
    // lr): 8 loads and 8 stores per value column tile where per-element
    // accesses took 64
    float(*sX)[SP] = reinterpret_cast<float(*)[SP]>(smem + SM::oX) + wave * C;
    const int xr = lane >> 2, xc = 4 * (lane & 3);
#pragma unroll 1
    for (int ct = wave; ct < NCT; ct += 4) {
        const bool kcol = ct < NKT;
        const int vc = ct - NKT;
        floatx4 xb[NT]; // B fragments X[16 st + 4 g + j][column lr]
        float vv[NT][4], ww[NT][4];
        if (kcol) {
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
                for (int j = 0; j < 4; ++j) xb[st][j] = sR[16 * st + 4 * lg + j][16 * ct + lr];
        } else {
#pragma unroll
            for (int st = 0; st < NT; ++st) xb[st] = dvn[(vc * NT + st) * 64 + lane];
            floatx4 v4[NT], w4[NT];
#pragma unroll
            for (int m = 0; m < NT; ++m) {
                const int o = (16 * m + xr) * rv + 16 * vc + xc;
                v4[m] = bld4(Rv, o);
                w4[m] = bld4(Rw, o);
            }
#pragma unroll
            for (int m = 0; m < NT; ++m) *reinterpret_cast<floatx4 *>(&sX[16 * m + xr][xc]) = v4[m];
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) vv[rt][i] = sX[16 * rt + 4 * lg + i][lr];
#pragma unroll
            for (int m = 0; m < NT; ++m) *reinterpret_cast<floatx4 *>(&sX[16 * m + xr][xc]) = w4[m];
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) ww[rt][i] = sX[16 * rt + 4 * lg + i][lr];
        }
        floatx4 dr[NT]; // dRv tiles of a value column tile
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = rt; st < NT; ++st) acc = mfma4x(aiT(rt, st), xb[st], acc);
            if (kcol) {
                // this lane read these four elements of dW above (rows 16 st + 4 lg + j, column lr)
                drk[(rt * NKT + ct) * 64 + lane] = acc;
#pragma unroll
                for (int i = 0; i < 4; ++i) sR[16 * rt + 4 * lg + i][16 * ct + lr] = acc[i];
            } else {
                dr[rt] = acc;
            }
        }
        if (!kcol) { // dv = dRv * w, then dw = dRv * v, out as 16-byte row pieces
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) sX[16 * rt + 4 * lg + i][lr] = dr[rt][i] * ww[rt][i];
#pragma unroll
            for (int m = 0; m < NT; ++m)
                bst4(Rdv, (16 * m + xr) * rv + 16 * vc + xc, *reinterpret_cast<const floatx4 *>(&sX[16 * m + xr][xc]));
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) sX[16 * rt + 4 * lg + i][lr] = dr[rt][i] * vv[rt][i];
#pragma unroll
            for (int m = 0; m < NT; ++m)
                bst4(Rdw, (16 * m + xr) * rv + 16 * vc + xc, *reinterpret_cast<const floatx4 *>(&sX[16 * m + xr][xc]));
        }
    }
    __syncthreads(); // sR holds dRk

    // dA_kk tiles (rt, st), st <= rt (the decay kernel reads no other): the
    // j-th of the ten, j = rt (rt + 1) / 2 + st, goes to wave j % 4 (three or
    // two tiles each); -(dRk W^T + Ai^T dUU), zero on and above the diagonal,
    // as fragments
    const floatx4 *Wf = reinterpret_cast<const floatx4 *>(p.ws_w) + (size_t)cid * (C * K / 4);
    floatx4 *dakk = reinterpret_cast<floatx4 *>(bp.ws_dakk) + (size_t)cid * (C * C / 4);
#pragma unroll 1
    for (int j = wave; j < NLT; j += 4) {
        int rt = 0;
        while ((rt + 1) * (rt + 2) / 2 <= j) ++rt;
        const int st = j - rt * (rt + 1) / 2;
        floatx4 wb[NKT], ub[NT], ab[NT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) wb[kt] = Wf[(st * NKT + kt) * 64 + lane];
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            ub[mt] = mt >= rt ? sUU[(mt * NT + st) * 64 + lane] : floatx4{0.f, 0.f, 0.f, 0.f};
            ab[mt] = mt >= rt ? Aif[(mt * NT + rt) * 64 + lane] : floatx4{0.f, 0.f, 0.f, 0.f}; // Ai^T (rt, mt)
        }
        floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) // A: dRk rows 16 rt + lr; B: W^T = W's A fragment (st, kt)
            acc = mfma4x(*reinterpret_cast<const floatx4 *>(&sR[16 * rt + lr][16 * kt + 4 * lg]), wb[kt], acc);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
            if (mt >= rt) acc = mfma4x(ab[mt], ub[mt], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = 16 * st + lr < 16 * rt + 4 * lg + i ? -acc[i] : 0.f;
        dakk[(rt * NT + st) * 64 + lane] = acc;
    }
}

// ---------------------------------------------------------------------------
// Per-chunk decay-weighted terms and the elementwise chain.  One workgroup
// of K/16 waves per chunk; wave w owns key channels 16 w .. 16 w + 15 for all
// 64 rows.  With G = cumsum g (log2 units) and E_rs = exp(G_r - G_s), r >= s:
//   rq_r  = sum_{s<=r} dA_qk[r][s] k_s E_rs        rkb_r = sum_{s<r} dA_kk[r][s] k_s E_rs
//   ck_s  = sum_{r>=s} (scale dA_qk[r][s] q_r + dA_kk[r][s] b_r k_r) E_rs
// as MFMA products over the time tiles, with the forward's split around the
// row tile's reference Gb_p (G at the end of tile p-1):
//   E_rs = exp(G_r - Gb_p) exp(Gb_p - G_s),
// both factors <= 1 off the diagonal block; on it the second is bounded by
// the tile's decay span. Channels whose span lies in (96, 192] move Gb_p to
// the middle of the tile's range, and channels above 192 take the exact
// pairwise terms instead.  Then, per (row r, channel c):
//   dq = scale (e^G dQG + rq),  dkb = e^G dRk + rkb,  db = dkb k
//   dk = e^{G_last - G} dKd + ck + dkb b
//   dG = scale q e^G dQG + b k e^G dRk - k e^{G_last - G} dKd + scale q rq + b k rkb - k ck
//        (+ sum_s k_s e^{G_last - G_s} dKd_s + e^{G_last} dgam at the last row)
//   dg_t = sum_{r >= t} dG_r.
// Lane (g, n) holds channel 16 w + n at rows 16 t + 4 g + j of every tile t:
// the rows of its B fragments, accumulator rows and elementwise terms.
// ---------------------------------------------------------------------------
template <int K, int V>
__global__ __launch_bounds__(K * 4, K >= 256 ? 4 : K / 32) void bwd_decay_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int NTH = K * 4, NSEG = NTH / K, RPS = C / NSEG; // cumsum: NSEG row segments per channel
    constexpr int KP = K + 4, CP = C + 4;
    // sG: per row the cumulative sum of g from its tile's first row (nats),
    // then dG; G (log2 units) = (sG + sOff) * log2 e, sOff the sum of the
    // tiles before (the tiles are the scan's segments: NSEG == NT)
    __shared__ __attribute__((aligned(16))) float sG[C][KP];
    __shared__ __attribute__((aligned(16))) float sDA[C][CP], sDK[C][CP];
    __shared__ float sTot[NSEG][K], sOff[NSEG][K];
    static_assert(NSEG == NT && RPS == 16, "one scan segment per row tile");
    const int cid = blockIdx.x, bh = cid / p.NC, n = cid % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int cv = min(C, p.T - n * C);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const float scale = p.scale;
    const int ch = 16 * wave + lr; // this lane's channel

    const int64_t ko = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + (int64_t)(n * C) * p.sqt;
    const int rq_ = (int)p.sqt;
    const __amdgpu_buffer_rsrc_t Rq = rows_rsrc(p.q + ko, rq_, cv, K), Rk = rows_rsrc(p.k + ko, rq_, cv, K);
    const __amdgpu_buffer_rsrc_t Rg = rows_rsrc(p.g + ko, rq_, cv, K), Rb = rows_rsrc(p.b + ko, rq_, cv, K);

    // this lane's k at rows 16 t + 4 lg + j (q and b are loaded where used)
    float kv[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) kv[t][j] = bld1(Rk, (16 * t + 4 * lg + j) * rq_ + ch);
    // G = cumsum_t g per channel, in log2 units; dA_qk, dA_kk to LDS
    {
        const int c = tid % K, seg = tid / K;
        float vals[RPS];
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < RPS; ++i) vals[i] = bld1(Rg, (seg * RPS + i) * rq_ + c);
#pragma unroll
        for (int i = 0; i < RPS; ++i) {
            acc += vals[i];
            sG[seg * RPS + i][c] = acc;
        }
        sTot[seg][c] = acc;
        // dA_qk, dA_kk: the fragments of the lower block triangle (tile (rt, st),
        // lane (g, c): rows 16 rt + 4 g .. + 3 of column 16 st + c), the only
        // tiles read below, into row-major LDS
        const floatx4 *da = reinterpret_cast<const floatx4 *>(bp.ws_daqk + (size_t)cid * C * C);
        const floatx4 *dk = reinterpret_cast<const floatx4 *>(bp.ws_dakk + (size_t)cid * C * C);
        for (int f = tid; f < C * C / 4; f += NTH) {
            const int tile = f >> 6, rt = tile / NT, st = tile % NT; // wave-uniform (NTH % 64 == 0)
            if (st > rt) continue;
            const int l = f & 63, r0 = 16 * rt + 4 * (l >> 4), c = 16 * st + (l & 15);
            const floatx4 a = da[f], b = dk[f];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sDA[r0 + i][c] = a[i];
                sDK[r0 + i][c] = b[i];
            }
        }
        __syncthreads();
        float off = 0.f;
        for (int s2 = 0; s2 < seg; ++s2) off += sTot[s2][c];
        sOff[seg][c] = off;
        __syncthreads();
    }
    // G at row r of this lane's channel, log2 units
    auto Gat = [&](int r) { return (sG[r][ch] + sOff[r / 16][ch]) * kLog2e; };
    // Gb_t: G at the end of tile t-1, or, for a span in (96, 192], the middle
    // of tile t's range, (Gb_t + G_end) / 2, as in the forward: the diagonal
    // factors then lie in [2^-96, 2^96] and the off-diagonal column factors
    // stay <= 1 (one that underflows drops a term below 2^-30 of its operands)
    float gb[NT];
    bool msk[NT]; // diagonal block of tile t beyond 192: exact pairwise terms
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float b0 = t ? Gat(16 * t - 1) : 0.f, ge = Gat(16 * t + 15);
        const float span = b0 - ge;
        msk[t] = span > 192.f;
        gb[t] = (span > 96.f && span <= 192.f) ? 0.5f * (b0 + ge) : b0;
    }

    float *oq, *okk, *og, *ob;
    int64_t ot, obase;
    if (p.rep == 1) {
        oq = bp.dq; okk = bp.dk; og = bp.dg; ob = bp.db;
        ot = p.sqt;
        obase = ko;
    } else {
        const size_t plane = (size_t)p.B * p.HV * p.NC * C * K;
        oq = bp.ws_kgrad; okk = oq + plane; og = okk + plane; ob = og + plane;
        ot = K;
        obase = (int64_t)cid * C * K;
    }
    // The four gradients go through buffer resources over the chunk's valid
    // rows: the hardware drops the stores past the last one, and the offsets
    // are 32-bit (a chunk's rows span less than 2 GiB, checked on the host).
    const int ot_ = (int)ot;
    const __amdgpu_buffer_rsrc_t Oq = rows_rsrc(oq + obase, ot_, cv, K), Ok = rows_rsrc(okk + obase, ot_, cv, K);
    const __amdgpu_buffer_rsrc_t Og = rows_rsrc(og + obase, ot_, cv, K), Ob = rows_rsrc(ob + obase, ot_, cv, K);
    // dQG, dKd, dRk tiles (t, wave): lane (lg, lr) holds rows 16 t + 4 lg + i of channel ch
    const floatx4 *dqg = reinterpret_cast<const floatx4 *>(bp.ws_dqg) + (size_t)cid * (C * K / 4);
    const floatx4 *dkd = reinterpret_cast<const floatx4 *>(bp.ws_dkd) + (size_t)cid * (C * K / 4);
    const floatx4 *drk = reinterpret_cast<const floatx4 *>(bp.ws_drk) + (size_t)cid * (C * K / 4);
    constexpr int NKT = K / 16;
    float kt_sum = 0.f;

    // Tiles from the last to the first.  Step t forms the column operands of
    // row tile t (scale q and b k, decay-weighted, rows 16 t + 4 lg + j) once
    // and adds their products to the column sums of every column tile <= t;
    // column tile t then has all its terms (they come from row tiles >= t), so
    // the step finishes it with the row sums of row tile t and tile t's
    // elementwise terms.  Those overwrite tile t's rows of sG with dG: only
    // this wave reads this channel's sG, later steps read tiles < t only, the
    // pairwise terms of tile t's diagonal block read it earlier in the step,
    // and each elementwise row reads its own tile-local sum before writing.
    floatx4 ckt[NT]; // column sums of column tiles 0 .. t
#pragma unroll
    for (int t = 0; t < NT; ++t) ckt[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = NT - 1; t >= 0; --t) {
        float gt[4]; // G at this lane's rows of tile t
#pragma unroll
        for (int j = 0; j < 4; ++j) gt[j] = Gat(16 * t + 4 * lg + j);
        floatx4 bq, bb; // column operands of row tile t
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float e = fast_exp2(gt[j] - gb[t]);
            const int o = (16 * t + 4 * lg + j) * rq_ + ch;
            bq[j] = scale * bld1(Rq, o) * e;
            bb[j] = bld1(Rb, o) * kv[t][j] * e;
        }
        floatx4 rq, rkb;
        {
            floatx4 aq = floatx4{0.f, 0.f, 0.f, 0.f}, ab = aq;
#pragma unroll
            for (int ct = 0; ct <= t; ++ct) {
                // e^{Gb_t - G_s} at rows s = 16 ct + 4 lg + j: the weight of k_s in row tile t's
                // row sums and of row tile t's products in column tile ct's sums
                floatx4 wd, kt, a1, a2;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    wd[j] = (ct == t && msk[t]) ? 0.f : fast_exp2(gb[t] - Gat(16 * ct + 4 * lg + j));
                    kt[j] = kv[ct][j] * wd[j];
                    a1[j] = sDA[16 * t + 4 * lg + j][16 * ct + lr];
                    a2[j] = sDK[16 * t + 4 * lg + j][16 * ct + lr];
                }
                aq = mfma4x(*reinterpret_cast<const floatx4 *>(&sDA[16 * t + lr][16 * ct + 4 * lg]), kt, aq);
                ab = mfma4x(*reinterpret_cast<const floatx4 *>(&sDK[16 * t + lr][16 * ct + 4 * lg]), kt, ab);
                floatx4 tmp = mfma4x(a1, bq, floatx4{0.f, 0.f, 0.f, 0.f});
                tmp = mfma4x(a2, bb, tmp);
#pragma unroll
                for (int i = 0; i < 4; ++i) ckt[ct][i] += tmp[i] * wd[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = fast_exp2(gt[i] - gb[t]);
                rq[i] = aq[i] * e;
                rkb[i] = ab[i] * e;
            }
            if (__ballot(msk[t])) {
                // Exact diagonal-block terms, wave-uniform so that lanes can
                // exchange operands: each E_rs of the lane's rows r = 16 t + 4 lg + i
                // and the tile's rows s <= r is formed once and feeds the row
                // sum of r and the lane's part of the column sum of s; k_s
                // comes from lane (s / 4, n), G_s from LDS.  Lanes of channels
                // at or below 192 (their diagonal block is in the products)
                // take E = 0: every lane of a column shares its channel.
                const bool on = msk[t];
                float sq[4], sbk[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int o = (16 * t + 4 * lg + i) * rq_ + ch;
                    sq[i] = scale * bld1(Rq, o);
                    sbk[i] = bld1(Rb, o) * kv[t][i];
                }
#pragma unroll 1
                for (int sg = 0; sg < 4; ++sg) // rows s = 16 t + 4 sg + u
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int s = 4 * sg + u;
                        const float gs = Gat(16 * t + s);
                        const float ks = __shfl(kv[t][u], 16 * sg + lr, 64);
                        float cs = 0.f;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = 16 * t + 4 * lg + i;
                            const float e = on && s <= 4 * lg + i ? fast_exp2(gt[i] - gs) : 0.f;
                            const float da = sDA[r][16 * t + s], dk = sDK[r][16 * t + s];
                            const float ke = ks * e;
                            rq[i] += da * ke;
                            rkb[i] += dk * ke;
                            cs += (sq[i] * da + sbk[i] * dk) * e;
                        }
                        // the column sum of s over the four lanes (lg, n), kept at lane (sg, n)
                        cs += __shfl_xor(cs, 16, 64);
                        cs += __shfl_xor(cs, 32, 64);
                        if (lg == sg) ckt[t][u] += cs;
                    }
            }
        }
        const floatx4 ck = ckt[t];
        const floatx4 fqg = dqg[(t * NKT + wave) * 64 + lane], fkd = dkd[(t * NKT + wave) * 64 + lane];
        const floatx4 frk = drk[(t * NKT + wave) * 64 + lane];
        // e^{G_last - G_r} from the sum of g after row r: the rest of tile t
        // (its total less row r's tile-local sum) and the tiles after it, added
        // at that sum's own magnitude, where gl - G_r would subtract two sums
        // from the chunk's start rounded at theirs
        const float tot = sTot[t][ch];
        float later = 0.f;
#pragma unroll
        for (int u = t + 1; u < NT; ++u) later += sTot[u][ch];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 16 * t + 4 * lg + i;
            const float eG = fast_exp2(gt[i]), eKd = fast_exp2((tot - sG[r][ch] + later) * kLog2e);
            const float vqg = fqg[i], vkd = fkd[i], vrk = frk[i];
            const int o = r * rq_ + ch;
            const float qr = bld1(Rq, o), kr = kv[t][i], br = bld1(Rb, o);
            const float dkb = eG * vrk + rkb[i];
            const float kd = kr * eKd;
            const int oo = r * ot_ + ch;
            bst1(Oq, oo, scale * (eG * vqg + rq[i]));
            bst1(Ok, oo, eKd * vkd + ck[i] + dkb * br);
            bst1(Ob, oo, dkb * kr);
            kt_sum += vkd * kd;
            const float dG = scale * qr * (eG * vqg + rq[i]) + br * kr * dkb - vkd * kd - kr * ck[i];
            sG[r][ch] = dG;
        }
    }
    kt_sum += __shfl_xor(kt_sum, 16, 64);
    kt_sum += __shfl_xor(kt_sum, 32, 64);
    // dg = the dG_last terms + the reverse cumulative sum of dG over the
    // chunk's rows.  Lane (lg, n) sums rows 16 lg .. 16 lg + 15 of channel ch
    // from the last up and adds the totals of the blocks after its own.
    float part[16], tot = 0.f;
#pragma unroll
    for (int m = 15; m >= 0; --m) {
        tot += sG[16 * lg + m][ch];
        part[m] = tot;
    }
    // G_last from the last tile's total (its last row's tile-local sum; that
    // row of sG holds dG by now)
    const float gl = (sTot[NT - 1][ch] + sOff[NT - 1][ch]) * kLog2e;
    float after = kt_sum + bp.ws_dgam[(size_t)cid * K + ch] * fast_exp2(gl);
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        const float tj = __shfl(tot, 16 * j + lr, 64);
        after += j > lg ? tj : 0.f;
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) bst1(Og, (16 * lg + m) * ot_ + ch, after + part[m]);
}

// Key-side gradients of a key head: the sum over its rep value heads.
__global__ __launch_bounds__(256) void bwd_gva_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    const int H = p.HV / p.rep, K = p.K;
    const int64_t total = (int64_t)p.B * H * p.T * K;
    const size_t plane = (size_t)p.B * p.HV * p.NC * C * K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int c = (int)(i % K);
        const int t = (int)((i / K) % p.T);
        const int hk = (int)((i / ((int64_t)K * p.T)) % H);
        const int bi = (int)(i / ((int64_t)K * p.T * H));
        const int n = t / C, r = t % C;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        for (int hv = hk * p.rep; hv < (hk + 1) * p.rep; ++hv) {
            const size_t o = (((size_t)bi * p.HV + hv) * p.NC + n) * C * K + (size_t)r * K + c;
#pragma unroll
            for (int w = 0; w < 4; ++w) s[w] += bp.ws_kgrad[w * plane + o];
        }
        const int64_t o = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + (int64_t)t * p.sqt + c;
        bp.dq[o] = s[0];
        bp.dk[o] = s[1];
        bp.dg[o] = s[2];
        bp.db[o] = s[3];
    }
}

template <int K, int V>
hipError_t launch_bwd_t(const BwdParams &bp, hipStream_t s) {
    const ChunkParams &p = bp.f;
    constexpr int NW = inter_nwv(K, V), VSW = 16 * NW; // waves and value columns per reverse-recurrence workgroup
    static_assert(V % VSW == 0, "V");
    const int seqs = p.B * p.HV, nch = seqs * p.NC;
    hipError_t e;
    if (p.NSEG > 1) {
        hipLaunchKernelGGL((bwd_inter_kernel<K, kRevLocal, NW>), dim3(seqs * (p.NSEG - 1) * (V / VSW)), dim3(64 * NW),
                           0, s, bp, 1, p.NSEG - 1);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL((bwd_chain_kernel<K, NW>), dim3(seqs * (V / VSW)), dim3(64 * NW), 0, s, bp);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    hipLaunchKernelGGL((bwd_inter_kernel<K, kRevOut, NW>), dim3(seqs * p.NSEG * (V / VSW)), dim3(64 * NW), 0, s, bp,
                       0, p.NSEG);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_vprod_kernel<K, V>), dim3(nch), dim3(256), 0, s, bp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_decay_kernel<K, V>), dim3(nch), dim3(K * 4), 0, s, bp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (p.rep > 1) {
        const int64_t total = (int64_t)p.B * (p.HV / p.rep) * p.T * p.K;
        const int64_t g = (total + 255) / 256;
        hipLaunchKernelGGL(bwd_gva_kernel, dim3((unsigned)(g < 8192 ? g : 8192)), dim3(256), 0, s, bp);
        e = hipGetLastError();
    }
    return e;
}

hipError_t launch_bwd(const BwdParams &bp, hipStream_t s) {
    const int K = bp.f.K, V = bp.f.V;
    if (K == 128 && V == 128) return launch_bwd_t<128, 128>(bp, s);
    if (K == 128 && V == 256) return launch_bwd_t<128, 256>(bp, s);
    if (K == 128 && V == 64) return launch_bwd_t<128, 64>(bp, s);
    if (K == 64 && V == 64) return launch_bwd_t<64, 64>(bp, s);
    if (K == 64 && V == 128) return launch_bwd_t<64, 128>(bp, s);
    if (K == 64 && V == 256) return launch_bwd_t<64, 256>(bp, s);
    if (K == 256 && V == 256) return launch_bwd_t<256, 256>(bp, s);
    if (K == 256 && V == 128) return launch_bwd_t<256, 128>(bp, s);
    if (K == 128 && V == 192) return launch_bwd_t<128, 192>(bp, s);
    if (K == 64 && V == 96) return launch_bwd_t<64, 96>(bp, s);
    if (K == 32 && V == 32) return launch_bwd_t<32, 32>(bp, s);
    if (K == 32 && V == 64) return launch_bwd_t<32, 64>(bp, s);
    return hipErrorInvalidValue;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The backward's workspace after the forward's: the training operands of the
// forward, then the backward's per-chunk arrays.
struct BwdLayout {
    size_t fwd, wt, qgt, kd, aqkt, akk, sn, vn, dsn, dvn, dqg, rseg, dkd, daqk, dgam, drk, dakk, kgrad, total;
};

BwdLayout bwd_layout(const gdn2_chunk_args *a) {
    BwdLayout L;
    const size_t nch = (size_t)a->batch * a->num_v_heads * ((a->seq_len + kChunk - 1) / kChunk);
    const size_t K = a->head_dim, V = a->head_v_dim, Cs = kChunk, f = sizeof(float);
    size_t off = align256(chunk_fwd_ws_bytes(a));
    L.fwd = 0;
    auto take = [&](size_t elems) { const size_t o = off; off = align256(off + f * nch * elems); return o; };
    L.wt = take(Cs * K);
    L.qgt = take(Cs * K);
    L.kd = take(Cs * K);
    L.aqkt = take(Cs * Cs);
    L.akk = take(Cs * Cs);
    L.sn = take(K * V);
    L.vn = take(Cs * V);
    L.dsn = take(K * V);
    L.dvn = take(Cs * V);
    L.dqg = take(Cs * K);
    L.dkd = take(Cs * K);
    L.daqk = take(Cs * Cs);
    L.dgam = take(K);
    L.drk = take(Cs * K);
    L.dakk = take(Cs * Cs);
    L.kgrad = take(a->num_v_heads != a->num_heads ? 4 * Cs * K : 0);
    { // segment buffers of the reverse recurrence, per sequence (not per chunk)
        const size_t seqs = (size_t)a->batch * a->num_v_heads, NC = (a->seq_len + kChunk - 1) / kChunk;
        const size_t nseg = (size_t)chunk_segments(seqs, K, V, NC);
        const size_t ns = nseg > 1 ? seqs * nseg : 0;
        L.rseg = off; off = align256(off + f * ns * K * V);
    }
    L.total = off;
    return L;
}

bool aligned16b(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace gdn2

using namespace gdn2;

extern "C" size_t gdn2_chunk_bwd_workspace_bytes(const gdn2_chunk_bwd_args *a) {
    if (!a || a->fwd.batch <= 0 || a->fwd.num_v_heads <= 0 || a->fwd.seq_len <= 0 || a->fwd.head_dim <= 0 ||
        a->fwd.head_v_dim <= 0)
        return 0;
    return bwd_layout(&a->fwd).total;
}

namespace {

// The three entry points below share this: checks, the workspace binding, and
// by `what` the launches -- 1 the training forward (output, final state and the
// backward's inputs), 2 the backward from those inputs, 3 both forward
// quantities (recomputed, without the output) and the backward.
gdn2_status chunk_bwd_call(const gdn2_chunk_bwd_args *a, gdn2_stream_t stream, int what, const char *who) {
    const std::string w = std::string(who) + ": ";
    if (!a) return fail(GDN2_EINVAL, w + "null args");
    BwdParams bp{};
    if (!chunk_bwd_supported((int)a->fwd.head_dim, (int)a->fwd.head_v_dim))
        return fail(GDN2_NOT_APPLICABLE, w + "(K, V) outside the chunked backward's instances");
    gdn2_status st = chunk_setup(&a->fwd, who, what == 1, &bp.f);
    if (st != GDN2_OK) return st;
    const gdn2_chunk_args &f = a->fwd;
    if (what != 1) {
        if (!a->d_out || !a->dq || !a->dk || !a->dg || !a->db || !a->dv || !a->dw || !a->d_state0)
            return fail(GDN2_EINVAL, w + "null gradient pointer");
        if (!aligned16b(a->d_out) || (f.stride_o_b % 4) || (f.stride_o_h % 4) || (f.stride_o_t % 4) ||
            f.stride_o_t < f.head_v_dim || ((kChunk - 1) * f.stride_o_t + f.head_v_dim) * 4 >= (int64_t(1) << 31))
            return fail(GDN2_NOT_APPLICABLE, w + "d_out needs 16-byte aligned rows within the row loads' range");
    }
    hipStream_t s = (hipStream_t)stream;
    const size_t sbytes = sizeof(float) * (size_t)f.batch * f.num_v_heads * f.head_dim * f.head_v_dim;
    if (f.seq_len == 0) { // no tokens: dS0 = d_state_out (or 0), by the fill kernel (a copy when a row is given)
        if (what != 1)
            GDN2_HIP_CHECK(launch_fill_rows(a->d_state0, 0, a->d_state_out, 1, (int64_t)(sbytes / sizeof(float)), s));
        return GDN2_OK;
    }
    const BwdLayout L = bwd_layout(&f);
    if (!a->workspace || a->workspace_bytes < L.total || (reinterpret_cast<uintptr_t>(a->workspace) & 255u))
        return fail(GDN2_EINVAL, w + "workspace missing, too small or not 256-byte aligned");
    char *ws = static_cast<char *>(a->workspace);
    chunk_bind_ws(&f, ws, &bp.f);
    ChunkParams &p = bp.f;
    p.ws_wt = reinterpret_cast<float *>(ws + L.wt);
    p.ws_qgt = reinterpret_cast<float *>(ws + L.qgt);
    p.ws_kd = reinterpret_cast<float *>(ws + L.kd);
    p.ws_aqkt = reinterpret_cast<float *>(ws + L.aqkt);
    p.ws_akk = reinterpret_cast<float *>(ws + L.akk);
    p.ws_sn = reinterpret_cast<float *>(ws + L.sn);
    p.ws_vn = reinterpret_cast<float *>(ws + L.vn);
    bp.d_out = a->d_out;
    bp.d_state_out = a->d_state_out;
    bp.dq = a->dq; bp.dk = a->dk; bp.dg = a->dg; bp.db = a->db; bp.dv = a->dv; bp.dw = a->dw;
    bp.d_state0 = a->d_state0;
    bp.ws_dsn = reinterpret_cast<float *>(ws + L.dsn);
    bp.ws_dvn = reinterpret_cast<float *>(ws + L.dvn);
    bp.ws_dqg = reinterpret_cast<float *>(ws + L.dqg);
    bp.ws_dkd = reinterpret_cast<float *>(ws + L.dkd);
    bp.ws_daqk = reinterpret_cast<float *>(ws + L.daqk);
    bp.ws_dgam = reinterpret_cast<float *>(ws + L.dgam);
    bp.ws_drk = reinterpret_cast<float *>(ws + L.drk);
    bp.ws_dakk = reinterpret_cast<float *>(ws + L.dakk);
    bp.ws_kgrad = p.rep > 1 ? reinterpret_cast<float *>(ws + L.kgrad) : nullptr;
    bp.ws_rseg = reinterpret_cast<float *>(ws + L.rseg);
    if (what == 1) { // the forward with its output, keeping the backward's inputs
        p.fwd_out = 1;
        GDN2_HIP_CHECK(launch_chunk(p, s, 1 | 2 | 4));
        return GDN2_OK;
    }
    // forward: per-chunk operands (training outputs), then the state entering every chunk
    if (what == 3) GDN2_HIP_CHECK(launch_chunk(p, s, 1 | 4));
    GDN2_HIP_CHECK(launch_bwd(bp, s));
    return GDN2_OK;
}

}  // namespace

// fused_chunk_backward (src/kernel/chunk_adjoint_cube.rs:464-707), recomputing
// the forward's per-chunk quantities.
extern "C" gdn2_status gdn2_chunk_bwd_f32(const gdn2_chunk_bwd_args *a, gdn2_stream_t stream) {
    return chunk_bwd_call(a, stream, 3, "gdn2_chunk_bwd_f32");
}

// The training forward: gdn2_chunk_fwd_f32's output and final state, and in
// the backward's workspace the quantities the reference exports as
// FusedBackwardInputs (src/kernel/chunk_adjoint_cube.rs:426-447).
extern "C" gdn2_status gdn2_chunk_fwd_train_f32(const gdn2_chunk_bwd_args *a, gdn2_stream_t stream) {
    return chunk_bwd_call(a, stream, 1, "gdn2_chunk_fwd_train_f32");
}

// fused_chunk_backward from the training forward's saved quantities
// (fused_chunk_backward(fwd: &FusedBackwardInputs, ..),
// src/kernel/chunk_adjoint_cube.rs:464-520).
extern "C" gdn2_status gdn2_chunk_bwd_saved_f32(const gdn2_chunk_bwd_args *a, gdn2_stream_t stream) {
    return chunk_bwd_call(a, stream, 2, "gdn2_chunk_bwd_saved_f32");
}

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
//   chunk_intra_kernel<K, V, true>       the forward operands plus W^T, QG^T, Kd, A_qk^T, A_kk
//   chunk_inter_kernel<K, kInterStates>  the state entering every chunk and v_new
//   bwd_inter_kernel   the reverse recurrence (one workgroup per (b, hv, 64 columns))
//   bwd_gemm_kernel    dQG, dW, dKd, dA_qk, dv_new U^T (MFMA) and dgam, per chunk
//   bwd_solve_kernel   Ai, dRk, dRv -> dv, dw; dA_kk, per chunk
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
    // per chunk (chunk id = (b * HV + hv) * NC + n), row-major
    float *ws_dsn;                    // K*V  dL/d(state leaving the chunk)
    float *ws_dvn;                    // C*V  dL/dv_new
    float *ws_dqg, *ws_dwm, *ws_dkd;  // C*K  dL/dQG, dL/dW, dL/dKd
    float *ws_daqk, *ws_duu;          // C*C  dL/dA_qk (lower), dv_new U^T (strictly lower)
    float *ws_dgam;                   // K    dL/d e^{G_last}
    float *ws_drk;                    // C*K  dL/dRk
    float *ws_dakk;                   // C*C  dL/dA_kk (strictly lower)
    float *ws_kgrad;                  // rep > 1: 4 x (C*K per chunk): dq, dk, dg, db per value head
};

__device__ __forceinline__ floatx4 mfma4x(floatx4 a, floatx4 b, floatx4 c) {
    c = mfma16(a[0], b[0], c);
    c = mfma16(a[1], b[1], c);
    c = mfma16(a[2], b[2], c);
    c = mfma16(a[3], b[3], c);
    return c;
}

// ---------------------------------------------------------------------------
// Reverse recurrence.  One workgroup per (b, hv, 64 value columns), wave w
// owns 16 columns; dS' stays in MFMA accumulators (key rows x 16 columns).
// Per chunk n = NC-1 .. 0:
//   1: dv_new = A_qk^T dO + Kd dS'         (reads sAT, sKd)
//      dS' and dv_new go to the workspace for the per-chunk kernels
//   2: dS' <- e^{G_last} dS' + QG^T dO - W^T dv_new   (reads sQT, sWT, sGam)
// The operands are A-operand fragments written by the training forward, so
// every product has the shape of the forward's chunk-inter products.  As
// there, each LDS buffer is refilled while the other phase runs.
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(256, 1) void bwd_inter_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int NKT = K / 16;
    constexpr int OPF4 = NKT * NT * 64, PFO = OPF4 / 256;
    constexpr int AF4 = NT * NT * 64, APF = AF4 / 256;
    __shared__ floatx4 sKd[OPF4], sAT[AF4], sQT[OPF4], sWT[OPF4];
    __shared__ floatx4 sGam[K / 4];

    const int V = p.V, nvv = V / 64;
    int bh, vs;
    inter_block(blockIdx.x, p.B * p.HV, nvv, &bh, &vs);
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int col = 16 * (vs * 4 + wave) + lr;

    floatx4 dS[NKT];
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dS[kb][i] = bp.d_state_out ? bp.d_state_out[(size_t)bh * K * V + (size_t)(16 * kb + 4 * lg + i) * V + col]
                                       : 0.f;

    const floatx4 *__restrict__ KD4 = reinterpret_cast<const floatx4 *>(p.ws_kd);
    const floatx4 *__restrict__ AT4 = reinterpret_cast<const floatx4 *>(p.ws_aqkt);
    const floatx4 *__restrict__ QT4 = reinterpret_cast<const floatx4 *>(p.ws_qgt);
    const floatx4 *__restrict__ WT4 = reinterpret_cast<const floatx4 *>(p.ws_wt);
    const floatx4 *__restrict__ G4 = reinterpret_cast<const floatx4 *>(p.ws_gam);
    const size_t cid0 = (size_t)bh * p.NC;

    if (p.NC > 0) {
        const size_t cl = cid0 + p.NC - 1;
#pragma unroll
        for (int i = 0; i < PFO; ++i) sKd[i * 256 + tid] = KD4[cl * OPF4 + i * 256 + tid];
#pragma unroll
        for (int i = 0; i < APF; ++i) sAT[i * 256 + tid] = AT4[cl * AF4 + i * 256 + tid];
    }
    // row 4 lg of each 16-row tile of d_out; the rest of the row offset is wave-uniform
    const float *dob = bp.d_out + (int64_t)bi * p.sob + (int64_t)hv * p.soh + col + (int64_t)(4 * lg) * p.sot;

    for (int n = p.NC - 1; n >= 0; --n) {
        const size_t cid = cid0 + n;
        __syncthreads(); // sKd, sAT hold chunk n; every wave is done with sQT, sWT (n+1)
        floatx4 qpre[PFO], wpre[PFO], g_cur = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < PFO; ++i) {
            qpre[i] = QT4[cid * OPF4 + i * 256 + tid];
            wpre[i] = WT4[cid * OPF4 + i * 256 + tid];
        }
        if (tid < K / 4) g_cur = G4[cid * (K / 4) + tid];
        const int cv = min(C, p.T - n * C);
        floatx4 dO[NT];
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dO[mt][i] = (16 * mt + 4 * lg + i < cv) ? dob[(int64_t)(n * C + 16 * mt + i) * p.sot] : 0.f;

        // 1: dv_new = Kd dS' + A_qk^T dO (A_qk^T is upper block-triangular)
        floatx4 dvn[NT];
#pragma unroll
        for (int st = 0; st < NT; ++st) dvn[st] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            floatx4 ka[NT];
#pragma unroll
            for (int st = 0; st < NT; ++st) ka[st] = sKd[(st * NKT + kb) * 64 + lane];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int st = 0; st < NT; ++st) dvn[st] = mfma16(ka[st][j], dS[kb][j], dvn[st]);
        }
#pragma unroll
        for (int st = 0; st < NT; ++st)
#pragma unroll
            for (int rt = st; rt < NT; ++rt) dvn[st] = mfma4x(sAT[(st * NT + rt) * 64 + lane], dO[rt], dvn[st]);

        {
            float *Dsn = bp.ws_dsn + cid * K * V;
#pragma unroll
            for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) Dsn[(size_t)(16 * kb + 4 * lg + i) * V + col] = dS[kb][i];
            float *Dvn = bp.ws_dvn + cid * C * V;
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
                for (int i = 0; i < 4; ++i) Dvn[(size_t)(16 * st + 4 * lg + i) * V + col] = dvn[st][i];
        }
#pragma unroll
        for (int i = 0; i < PFO; ++i) {
            sQT[i * 256 + tid] = qpre[i];
            sWT[i * 256 + tid] = wpre[i];
        }
        if (tid < K / 4) sGam[tid] = g_cur;
        __syncthreads(); // phase 1 done everywhere (sKd, sAT free); sQT, sWT, sGam (n) visible

        // Kd, A_qk^T of chunk n-1 (the first chunk re-fetches itself)
        const size_t cpv = cid - (n > 0 ? 1 : 0);
        floatx4 kpre[PFO], apre[APF];
#pragma unroll
        for (int i = 0; i < PFO; ++i) kpre[i] = KD4[cpv * OPF4 + i * 256 + tid];
#pragma unroll
        for (int i = 0; i < APF; ++i) apre[i] = AT4[cpv * AF4 + i * 256 + tid];

        // 2: dS' <- e^{G_last} dS' + QG^T dO - W^T dv_new
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            const floatx4 gm = sGam[4 * kb + lg];
            dS[kb][0] *= gm[0];
            dS[kb][1] *= gm[1];
            dS[kb][2] *= gm[2];
            dS[kb][3] *= gm[3];
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            floatx4 qa[NKT], wa[NKT];
#pragma unroll
            for (int kb = 0; kb < NKT; ++kb) {
                qa[kb] = sQT[(kb * NT + tt) * 64 + lane];
                wa[kb] = sWT[(kb * NT + tt) * 64 + lane];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int kb = 0; kb < NKT; ++kb) {
                    dS[kb] = mfma16(qa[kb][j], dO[tt][j], dS[kb]);
                    dS[kb] = mfma16(-wa[kb][j], dvn[tt][j], dS[kb]);
                }
        }
#pragma unroll
        for (int i = 0; i < PFO; ++i) sKd[i * 256 + tid] = kpre[i];
#pragma unroll
        for (int i = 0; i < APF; ++i) sAT[i * 256 + tid] = apre[i];
    }
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) bp.d_state0[(size_t)bh * K * V + (size_t)(16 * kb + 4 * lg + i) * V + col] = dS[kb][i];
}

// ---------------------------------------------------------------------------
// Per-chunk products over the value dimension (MFMA, four waves):
//   dQG = dO S^T, dW = -dv_new S^T, dKd = v_new dS'^T       (C x K)
//   dA_qk = tril(dO v_new^T), dUU = strict_tril(dv_new U^T)  (C x C)
// and dgam = rowsum(dS' * S).  A tile (rt, ct) of X Y^T takes rows 16 rt + r
// of X and 16 ct + r of Y as A and B fragments (16-byte loads along V).
// ---------------------------------------------------------------------------
template <int K, int V>
__global__ __launch_bounds__(256) void bwd_gemm_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int NKT = K / 16, NVB = V / 16;
    constexpr int NJ1 = 3 * NT * NKT, NJ = NJ1 + 2 * NT * NT;
    const int cid = blockIdx.x, bh = cid / p.NC, n = cid % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int cv = min(C, p.T - n * C);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;

    const float *dO = bp.d_out + (int64_t)bi * p.sob + (int64_t)hv * p.soh + (int64_t)(n * C) * p.sot;
    const int ro = (int)p.sot;
    const __amdgpu_buffer_rsrc_t RdO = rows_rsrc(dO, ro, cv, V);
    const float *Sn = p.ws_sn + (size_t)cid * K * V, *dSn = bp.ws_dsn + (size_t)cid * K * V;
    const float *vn = p.ws_vn + (size_t)cid * C * V, *dvn = bp.ws_dvn + (size_t)cid * C * V;
    const float *Uf = p.ws_u + (size_t)cid * C * V; // accumulator fragments (column tile, row tile)

    for (int j = wave; j < NJ; j += 4) {
        int mat, rt, ct;
        if (j < NJ1) {
            mat = j / (NT * NKT);
            rt = (j % (NT * NKT)) / NKT;
            ct = j % NKT;
        } else {
            const int jj = j - NJ1;
            mat = 3 + jj / (NT * NT);
            rt = (jj % (NT * NT)) / NT;
            ct = jj % NT;
        }
        floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
        if (mat < 3 || ct <= rt) {
            const int arow = 16 * rt + lr, brow = 16 * ct + lr;
#pragma unroll
            for (int vb = 0; vb < NVB; ++vb) {
                const int c0 = 16 * vb + 4 * lg;
                floatx4 a, b;
                if (mat == 0 || mat == 3)
                    a = bld4(RdO, arow * ro + c0);
                else if (mat == 1 || mat == 4)
                    a = *reinterpret_cast<const floatx4 *>(dvn + arow * V + c0);
                else
                    a = *reinterpret_cast<const floatx4 *>(vn + arow * V + c0);
                if (mat <= 1)
                    b = *reinterpret_cast<const floatx4 *>(Sn + brow * V + c0);
                else if (mat == 2)
                    b = *reinterpret_cast<const floatx4 *>(dSn + brow * V + c0);
                else if (mat == 3)
                    b = *reinterpret_cast<const floatx4 *>(vn + brow * V + c0);
                else // U[brow][c0 + i]: tile (vb, ct), lane (lr / 4, 4 lg + i), component lr % 4
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        b[i] = Uf[((vb * NT + ct) * 64 + (lr >> 2) * 16 + 4 * lg + i) * 4 + (lr & 3)];
                acc = mfma4x(a, b, acc);
            }
        }
        float *dst;
        int ld = K;
        if (mat == 0) dst = bp.ws_dqg + (size_t)cid * C * K;
        else if (mat == 1) dst = bp.ws_dwm + (size_t)cid * C * K;
        else if (mat == 2) dst = bp.ws_dkd + (size_t)cid * C * K;
        else if (mat == 3) { dst = bp.ws_daqk + (size_t)cid * C * C; ld = C; }
        else { dst = bp.ws_duu + (size_t)cid * C * C; ld = C; }
        const int s = 16 * ct + lr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 16 * rt + 4 * lg + i;
            float val = mat == 1 ? -acc[i] : acc[i];
            if (mat == 3 && s > r) val = 0.f;
            if (mat == 4 && s >= r) val = 0.f;
            dst[r * ld + s] = val;
        }
    }

    // dgam[c] = sum_v dS'[c][v] S[c][v]: 256 / K threads per row
    constexpr int TPR = 256 / K;
    {
        const int c = tid / TPR, part = tid % TPR;
        float acc = 0.f;
        for (int v = part; v < V; v += TPR) acc += dSn[(size_t)c * V + v] * Sn[(size_t)c * V + v];
#pragma unroll
        for (int off = 1; off < TPR; off <<= 1) acc += __shfl_xor(acc, off, 64);
        if (part == 0) bp.ws_dgam[(size_t)cid * K + c] = acc;
    }
}

// ---------------------------------------------------------------------------
// Per-chunk solve adjoint (four waves):
//   Ai = (I + A_kk)^-1 by column-wise forward substitution (thread j: column j)
//   dRk = Ai^T dW;  dRv = Ai^T dv_new -> dv = dRv * w, dw = dRv * v
//   dA_kk = strict_tril(-(dRk W^T + Ai^T dUU))
// ---------------------------------------------------------------------------
template <int K, int V>
__global__ __launch_bounds__(256) void bwd_solve_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int NKT = K / 16;
    constexpr int TW = (K > V ? K : V) + 1;
    __shared__ float sM[C][C + 1];  // A_kk, then dv_new U^T
    __shared__ float sAi[C][C + 1]; // (I + A_kk)^-1
    __shared__ float sR[C][K + 1];  // dRk
    __shared__ float sT[C][TW];     // dW, then dv_new, then W
    const int cid = blockIdx.x, bh = cid / p.NC, n = cid % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int cv = min(C, p.T - n * C);
    const int tid = threadIdx.x;

    {
        const float *Akk = p.ws_akk + (size_t)cid * C * C;
        for (int idx = tid; idx < C * C; idx += 256) sM[idx / C][idx % C] = Akk[idx];
        const float *dWm = bp.ws_dwm + (size_t)cid * C * K;
        for (int idx = tid; idx < C * K; idx += 256) sT[idx / K][idx % K] = dWm[idx];
    }
    __syncthreads();
    if (tid < C) { // column j of Ai: x_i = [i == j] - sum_{j <= m < i} A_kk[i][m] x_m
        const int j = tid;
        for (int i = 0; i < C; ++i) {
            float x = i == j ? 1.f : 0.f;
            for (int m = j; m < i; ++m) x -= sM[i][m] * sAi[m][j];
            sAi[i][j] = i < j ? 0.f : x;
        }
    }
    __syncthreads();
    {
        float *drk = bp.ws_drk + (size_t)cid * C * K;
        for (int idx = tid; idx < C * K; idx += 256) {
            const int r = idx / K, c = idx % K;
            float acc = 0.f;
            for (int s = r; s < C; ++s) acc += sAi[s][r] * sT[s][c];
            sR[r][c] = acc;
            drk[idx] = acc;
        }
    }
    __syncthreads();
    {
        const float *dvn = bp.ws_dvn + (size_t)cid * C * V;
        for (int idx = tid; idx < C * V; idx += 256) sT[idx / V][idx % V] = dvn[idx];
    }
    __syncthreads();
    {
        const int64_t vo = (int64_t)bi * p.svb + (int64_t)hv * p.svh + (int64_t)(n * C) * p.svt;
        for (int idx = tid; idx < C * V; idx += 256) {
            const int r = idx / V, j = idx % V;
            if (r >= cv) continue;
            float acc = 0.f;
            for (int s = r; s < C; ++s) acc += sAi[s][r] * sT[s][j];
            const int64_t o = vo + (int64_t)r * p.svt + j;
            bp.dv[o] = acc * p.w[o];
            bp.dw[o] = acc * p.v[o];
        }
    }
    __syncthreads();
    {
        const float *Wf = p.ws_w + (size_t)cid * C * K; // A-operand fragments (row tile, key tile)
        for (int idx = tid; idx < C * K; idx += 256) {
            const int s = idx / K, c = idx % K;
            sT[s][c] = Wf[((s >> 4) * NKT + (c >> 4)) * 256 + (((c & 15) >> 2) * 16 + (s & 15)) * 4 + (c & 3)];
        }
        const float *duu = bp.ws_duu + (size_t)cid * C * C;
        for (int idx = tid; idx < C * C; idx += 256) sM[idx / C][idx % C] = duu[idx];
    }
    __syncthreads();
    {
        float *dakk = bp.ws_dakk + (size_t)cid * C * C;
        for (int idx = tid; idx < C * C; idx += 256) {
            const int r = idx / C, s = idx % C;
            float val = 0.f;
            if (s < r) {
                float a = 0.f, b = 0.f;
                for (int c = 0; c < K; ++c) a += sR[r][c] * sT[s][c];
                for (int m = r; m < C; ++m) b += sAi[m][r] * sM[m][s];
                val = -(a + b);
            }
            dakk[idx] = val;
        }
    }
}

// ---------------------------------------------------------------------------
// Per-chunk decay-weighted terms and the elementwise chain (four waves), in
// blocks of 32 key channels staged in LDS with G = cumsum g (log2 units).
// For channel c and row r (E_rs = exp(G_r - G_s) <= 1 for s <= r):
//   rq_r  = sum_{s<=r} dA_qk[r][s] k_s E_rs      (dq from A_qk, before scale)
//   rkb_r = sum_{s<r}  dA_kk[r][s] k_s E_rs      (d(b k) from A_kk)
//   ck_r  = sum_{t>=r} (scale dA_qk[t][r] q_t + [t>r] dA_kk[t][r] b_t k_t) E_tr
//   dq  = scale (e^G dQG + rq)
//   dkb = e^G dRk + rkb,  db = dkb k
//   dk  = e^{G_last - G} dKd + ck + dkb b
//   dG  = dQG QG + dRk Rk - dKd Kd + scale q rq + b k rkb - k ck
//         (+ sum_s dKd_s Kd_s + dgam e^{G_last} at the last row)
//   dg_t = sum_{r>=t} dG_r
// ---------------------------------------------------------------------------
template <int K, int V>
__global__ __launch_bounds__(256) void bwd_decay_kernel(BwdParams bp) {
    const ChunkParams &p = bp.f;
    constexpr int CB = 32, RPT = C * CB / 256; // channels per block, rows per thread
    __shared__ float sDA[C][C + 1], sDK[C][C + 1];
    __shared__ float sG[C][CB + 1], sQ[C][CB + 1], sKk[C][CB + 1], sB[C][CB + 1];
    __shared__ float sDG[C][CB + 1], sKT[C][CB + 1];
    const int cid = blockIdx.x, bh = cid / p.NC, n = cid % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int cv = min(C, p.T - n * C);
    const int tid = threadIdx.x;
    const float scale = p.scale;

    {
        const float *daqk = bp.ws_daqk + (size_t)cid * C * C, *dakk = bp.ws_dakk + (size_t)cid * C * C;
        for (int idx = tid; idx < C * C; idx += 256) {
            sDA[idx / C][idx % C] = daqk[idx];
            sDK[idx / C][idx % C] = dakk[idx];
        }
    }
    const int64_t ko = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + (int64_t)(n * C) * p.sqt;
    const int rq_ = (int)p.sqt;
    const __amdgpu_buffer_rsrc_t Rq = rows_rsrc(p.q + ko, rq_, cv, K), Rk = rows_rsrc(p.k + ko, rq_, cv, K);
    const __amdgpu_buffer_rsrc_t Rg = rows_rsrc(p.g + ko, rq_, cv, K), Rb = rows_rsrc(p.b + ko, rq_, cv, K);
    // outputs: the caller's tensors (one value head per key head) or per value head for the GVA sum
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
    const float *dqg = bp.ws_dqg + (size_t)cid * C * K, *dkd = bp.ws_dkd + (size_t)cid * C * K;
    const float *drk = bp.ws_drk + (size_t)cid * C * K, *dgam = bp.ws_dgam + (size_t)cid * K;

    const int c = tid % CB, r0 = tid / CB; // rows r0 + 8 j
    for (int cb = 0; cb < K; cb += CB) {
        __syncthreads(); // the previous block's LDS is consumed
        for (int idx = tid; idx < C * CB; idx += 256) {
            const int r = idx / CB, cc = idx % CB, o = r * rq_ + cb + cc;
            sQ[r][cc] = bld1(Rq, o);
            sKk[r][cc] = bld1(Rk, o);
            sB[r][cc] = bld1(Rb, o);
            sG[r][cc] = bld1(Rg, o);
        }
        __syncthreads();
        if (tid < CB) {
            float acc = 0.f;
            for (int r = 0; r < C; ++r) {
                acc += sG[r][tid];
                sG[r][tid] = acc * kLog2e;
            }
        }
        __syncthreads();
        const float gl = sG[C - 1][c];
#pragma unroll 1
        for (int jr = 0; jr < RPT; ++jr) {
            const int r = r0 + 8 * jr;
            const float Gr = sG[r][c], qr = sQ[r][c], kr = sKk[r][c], br = sB[r][c];
            float rq = 0.f, rkb = 0.f, ck = 0.f;
            for (int s = 0; s <= r; ++s) {
                const float ke = sKk[s][c] * fast_exp2(Gr - sG[s][c]);
                rq += sDA[r][s] * ke;
                rkb += sDK[r][s] * ke; // dA_kk is zero on the diagonal
            }
            for (int t = r; t < C; ++t) {
                const float e = fast_exp2(sG[t][c] - Gr);
                ck += (scale * sDA[t][r] * sQ[t][c] + sDK[t][r] * sB[t][c] * sKk[t][c]) * e;
            }
            const int ch = cb + c;
            const float eG = fast_exp2(Gr), eKd = fast_exp2(gl - Gr);
            const float vqg = dqg[r * K + ch], vkd = dkd[r * K + ch], vrk = drk[r * K + ch];
            const float dkb = eG * vrk + rkb;
            const float dq = scale * (eG * vqg + rq);
            const float dk = eKd * vkd + ck + dkb * br;
            const float db = dkb * kr;
            const float kd = kr * eKd;
            sDG[r][c] = vqg * scale * qr * eG + vrk * br * kr * eG - vkd * kd + scale * qr * rq + br * kr * rkb - kr * ck;
            sKT[r][c] = vkd * kd;
            if (r < cv) {
                oq[obase + r * ot + ch] = dq;
                okk[obase + r * ot + ch] = dk;
                ob[obase + r * ot + ch] = db;
            }
        }
        __syncthreads();
        if (tid < CB) { // dG_last, then dg = reverse cumulative sum of dG
            float run = dgam[cb + tid] * fast_exp2(sG[C - 1][tid]);
            for (int r = 0; r < C; ++r) run += sKT[r][tid];
            for (int r = C - 1; r >= 0; --r) {
                run += sDG[r][tid];
                if (r < cv) og[obase + r * ot + cb + tid] = run;
            }
        }
    }
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
    const int seqs = p.B * p.HV, nch = seqs * p.NC;
    hipLaunchKernelGGL((bwd_inter_kernel<K>), dim3(seqs * (V / 64)), dim3(256), 0, s, bp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_gemm_kernel<K, V>), dim3(nch), dim3(256), 0, s, bp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_solve_kernel<K, V>), dim3(nch), dim3(256), 0, s, bp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_decay_kernel<K, V>), dim3(nch), dim3(256), 0, s, bp);
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
    return hipErrorInvalidValue;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The backward's workspace after the forward's: the training operands of the
// forward, then the backward's per-chunk arrays.
struct BwdLayout {
    size_t fwd, wt, qgt, kd, aqkt, akk, sn, vn, dsn, dvn, dqg, dwm, dkd, daqk, duu, dgam, drk, dakk, kgrad, total;
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
    L.dwm = take(Cs * K);
    L.dkd = take(Cs * K);
    L.daqk = take(Cs * Cs);
    L.duu = take(Cs * Cs);
    L.dgam = take(K);
    L.drk = take(Cs * K);
    L.dakk = take(Cs * Cs);
    L.kgrad = take(a->num_v_heads != a->num_heads ? 4 * Cs * K : 0);
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

// fused_chunk_backward (src/kernel/chunk_adjoint_cube.rs:464-707).
extern "C" gdn2_status gdn2_chunk_bwd_f32(const gdn2_chunk_bwd_args *a, gdn2_stream_t stream) {
    if (!a) return fail(GDN2_EINVAL, "gdn2_chunk_bwd_f32: null args");
    BwdParams bp{};
    gdn2_status st = chunk_setup(&a->fwd, "gdn2_chunk_bwd_f32", false, &bp.f);
    if (st != GDN2_OK) return st;
    if (!a->d_out || !a->dq || !a->dk || !a->dg || !a->db || !a->dv || !a->dw || !a->d_state0)
        return fail(GDN2_EINVAL, "gdn2_chunk_bwd_f32: null gradient pointer");
    const gdn2_chunk_args &f = a->fwd;
    if (!aligned16b(a->d_out) || (f.stride_o_b % 4) || (f.stride_o_h % 4) || (f.stride_o_t % 4) ||
        f.stride_o_t < f.head_v_dim || ((kChunk - 1) * f.stride_o_t + f.head_v_dim) * 4 >= (int64_t(1) << 31))
        return fail(GDN2_NOT_APPLICABLE, "gdn2_chunk_bwd_f32: d_out needs 16-byte aligned rows within the row loads' range");
    hipStream_t s = (hipStream_t)stream;
    const size_t sbytes = sizeof(float) * (size_t)f.batch * f.num_v_heads * f.head_dim * f.head_v_dim;
    if (f.seq_len == 0) { // no tokens: dS0 = d_state_out
        if (a->d_state_out)
            GDN2_HIP_CHECK(hipMemcpyAsync(a->d_state0, a->d_state_out, sbytes, hipMemcpyDeviceToDevice, s));
        else
            GDN2_HIP_CHECK(hipMemsetAsync(a->d_state0, 0, sbytes, s));
        return GDN2_OK;
    }
    const BwdLayout L = bwd_layout(&f);
    if (!a->workspace || a->workspace_bytes < L.total || (reinterpret_cast<uintptr_t>(a->workspace) & 255u))
        return fail(GDN2_EINVAL, "gdn2_chunk_bwd_f32: workspace missing, too small or not 256-byte aligned");
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
    bp.ws_dwm = reinterpret_cast<float *>(ws + L.dwm);
    bp.ws_dkd = reinterpret_cast<float *>(ws + L.dkd);
    bp.ws_daqk = reinterpret_cast<float *>(ws + L.daqk);
    bp.ws_duu = reinterpret_cast<float *>(ws + L.duu);
    bp.ws_dgam = reinterpret_cast<float *>(ws + L.dgam);
    bp.ws_drk = reinterpret_cast<float *>(ws + L.drk);
    bp.ws_dakk = reinterpret_cast<float *>(ws + L.dakk);
    bp.ws_kgrad = p.rep > 1 ? reinterpret_cast<float *>(ws + L.kgrad) : nullptr;
    // forward: per-chunk operands (training outputs), then the state entering every chunk
    GDN2_HIP_CHECK(launch_chunk(p, s, 1 | 4));
    GDN2_HIP_CHECK(launch_bwd(bp, s));
    return GDN2_OK;
}

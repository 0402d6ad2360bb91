// Chunked GDN-2 forward on gfx950.
//
// Semantics: src/forward.rs:44-278 (chunk_wy_forward).  Per chunk of C = 64
// tokens with G = cumsum_t g (per key channel, from the chunk start):
//   A_qk[r,s] = scale sum_c q_r k_s exp(G_r - G_s)   (s <= r)
//   A_kk[r,s] =       sum_c b_r k_r k_s exp(G_r - G_s) (s <  r)
//   W = (I + A_kk)^-1 (b k exp(G)),  U = (I + A_kk)^-1 (w v)
//   v_new = U - W S,  out = A_qk v_new + scale (q exp(G)) S
//   S <- exp(G_last) S + (k exp(G_last - G))^T v_new
// chunk-intra writes W, U, Kd^T = (k exp(G_last - G))^T, exp(G_last), A_qk
// and scale (q exp(G)); chunk-inter runs the recurrence and the output
// out = A_qk v_new + scale (q exp(G)) S of each chunk (src/forward.rs:264-274).
//
// Numerical scheme (every exponent fed to exp2 is <= 0 except where noted):
//  * A_qk / A_kk off-diagonal 16x16 blocks (row tile p > column tile q):
//    exp(G_r - G_s) = exp(G_r - Gb_p) * exp(Gb_p - G_s), Gb_p = G at the
//    last row of tile p-1; both factors <= 1.  One MFMA product per block.
//  * diagonal blocks: the same split, whose column factor exp(Gb_p - G_s)
//    is >= 1 but bounded by exp(span) with span = Gb_p - G at the tile end.
//    Channels with span <= 96 (log2 units) keep that MFMA product. Channels
//    with 96 < span <= 192 move the reference (for their whole row tile) to
//    the middle of the tile's range, Gb_p - span / 2, so that both diagonal
//    factors lie in [2^-96, 2^96] (the bounds of the split above): still one
//    MFMA product, whose discarded upper triangle may overflow.  Channels
//    above 192 (e.g. |g| ~ 30 per token) are zeroed in that product.  Where
//    both 8-token halves of the tile span at most 192 they are formed from
//    half-block products (each half's own mid reference for its diagonal
//    8x8 blocks, G at row 7 for rows 8-15 x columns 0-7); otherwise they are
//    added exactly with pairwise exp2(G_r - G_s), r >= s.
//  * WY solve per 16-row tile (src/forward.rs:192-261): the 16x16 diagonal
//    blocks of I + A_kk are inverted by forward substitution and the tiles
//    are eliminated in order, never as one 64x64 solve.
//
// MFMA mapping (v_mfma_f32_16x16x4_f32, see common.hpp): an accumulator tile
// holds rows 4*(lane/16)+i, column lane%16; with the contraction label
// k = 4*(lane/16) + step inside a 16-wide block it is directly the B operand
// of the next product.  The solve, A_qk [W|U] and, in the inter kernel, the
// state S and v_new therefore never leave registers.
#include "chunk_common.hpp"

#include <mutex>

namespace gdn2 {

namespace {

static_assert(NT == 4, "the diagonal-block inverse maps 4 tiles x 16 columns onto one wave");
constexpr float kSafeSpan = 96.0f;      // log2 units: reference at the tile start
constexpr float kSafeSpanMid = 192.0f;  // reference in the middle of the tile's range

// ---------------------------------------------------------------------------
// chunk-intra: one workgroup (8 waves) per (b, hv, chunk).
// Every global load of a phase is issued before that phase's arithmetic
// (g and k at the start, q / b rows before the score tiles, the right-hand
// sides of row tile p+1 while tile p is solved, k for Kd^T in one batch), so
// that a workgroup pays a handful of memory round trips instead of one per
// loop iteration.
// ---------------------------------------------------------------------------
// TRAIN adds the backward's operands (ws_wt, ws_qgt, ws_kd, ws_aqkt, and
// (I + A_kk)^-1 in ws_akk).
// K = 256 needs 141 KiB of LDS: one workgroup per CU, two waves per SIMD,
// and up to 256 VGPRs per wave.
template <int K, int V, bool TRAIN>
__global__ __launch_bounds__(512, K > 128 ? 2 : 4) void chunk_intra_kernel(ChunkParams p) {
    constexpr int NW = 8; // waves per workgroup; two workgroups per CU = four waves per SIMD (K <= 128)
    constexpr int KP = K + 4, CP = C + 4;
    constexpr int NKT = K / 16, NVT = V / 16, NTOT = NKT + NVT;
    static_assert(NKT % 2 == 0 && (NKT <= NW || NKT % NW == 0), "K in {32, 64, 96, 128, 256}");
    constexpr int NTW = (NTOT + NW - 1) / NW; // column tiles per wave in the solve (nt = wave + NW u)
    constexpr int NKW = (NKT + NW - 1) / NW;  // key-column tiles per wave (nt = wave + NW u, u < NKW)
    constexpr int NKH = NKT / 2;              // 16-channel blocks per wave in the score products
    constexpr int NSEG = 512 / K, RPS = C / NSEG;
    static_assert(512 % K == 0 && C % NSEG == 0, "K");
    constexpr int KF4 = C * K / 4 / 512; // float4 of the chunk's k per lane
    constexpr int RSZ = (C * KP > 2 * C * CP) ? C * KP : 2 * C * CP;

    // Region A: G (phases 1-2), then b k exp(G) (staging for the solve).
    __shared__ __attribute__((aligned(16))) float sG[C][KP];
    // Region B: k (phases 1-2), then A_qk | A_kk (phases 3-4).
    __shared__ __attribute__((aligned(16))) float sR[RSZ];
    __shared__ __attribute__((aligned(16))) float sAinv[NT][16][20];
    __shared__ float sTot[NSEG][K];
    __shared__ uint32_t sMask[NT][K / 32]; // diagonal-tile channels with span > kSafeSpanMid
    __shared__ uint32_t sPair[NT][K / 32]; // those of them with a half-tile span > kSafeSpanMid
    __shared__ float sRef[NT][K];          // the score products' reference G per row tile
    float(*sK)[KP] = reinterpret_cast<float(*)[KP]>(sR);
    float(*sBKG)[KP] = sG;
    float(*sAqk)[CP] = reinterpret_cast<float(*)[CP]>(sR);
    float(*sAkk)[CP] = reinterpret_cast<float(*)[CP]>(sR + C * CP);

    const int ci = blockIdx.x;
    const int bh = ci / p.NC, n = ci % p.NC;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int t0 = n * C;
    const int cv = min(C, p.T - t0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (scalar)
    const int lr = lane & 15, lg = lane >> 4;
    const int64_t sqt = p.sqt, svt = p.svt;

    const int64_t kofs = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + (int64_t)t0 * sqt;
    const int64_t vofs = (int64_t)bi * p.svb + (int64_t)hv * p.svh + (int64_t)t0 * svt;
    const float *qc = p.q + kofs, *kc = p.k + kofs, *gc = p.g + kofs, *bc = p.b + kofs;
    const float *vc = p.v + vofs, *wc = p.w + vofs;
    const size_t cid = (size_t)ci;
    // Row loads go through range-checked buffer resources (rows >= cv read 0)
    // with 32-bit offsets: row * stride + column, the row part split into a
    // per-lane term computed once and a wave-uniform term.
    const int rq = (int)sqt, rv = (int)svt;
    const __amdgpu_buffer_rsrc_t Rq = rows_rsrc(qc, rq, cv, K), Rk = rows_rsrc(kc, rq, cv, K);
    const __amdgpu_buffer_rsrc_t Rg = rows_rsrc(gc, rq, cv, K), Rb = rows_rsrc(bc, rq, cv, K);
    const __amdgpu_buffer_rsrc_t Rv = rows_rsrc(vc, rv, cv, V), Rw = rows_rsrc(wc, rv, cv, V);
    const int lr_q = lr * rq;      // row lr of a tile, q/k/g/b
    const int lg_q = 4 * lg * rq;  // row 4 lg of a tile, q/k/g/b
    const int lg_v = 4 * lg * rv;  // row 4 lg of a tile, v/w

    // Wave roles of the score products (phase 2): A_qk (mat 0) or A_kk (mat 1),
    // row tiles {half, NT-1-half}, channel half kh.  Their row operands (q or
    // b rows, araw) are requested in phase 1, right after its own loads, so
    // that they arrive while phase 1 computes instead of after its barriers.
    const int mat = wave >> 2, half = (wave >> 1) & 1, kh = wave & 1;
    const int m0 = kh * NKH;
    floatx4 araw[2][NKH];

    // 1. k -> sK; G = cumsum_t g per channel -> sG in log2 units.  Rows past
    //    the end of a ragged last chunk are zero (src/forward.rs:94-99).
    {
        floatx4 kreg[KF4];
#pragma unroll
        for (int i = 0; i < KF4; ++i) // 512 % (K / 4) == 0: row = i 512 / (K / 4) + tid / (K / 4)
            kreg[i] = bld4(Rk, (tid / (K / 4)) * rq + 4 * (tid % (K / 4)) + i * (512 / (K / 4)) * rq);
        const int c = tid % K, seg = K >= 64 ? wave * 64 / K : tid / K; // tid / K (wave-uniform for K >= 64)
        float vals[RPS];
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < RPS; ++i) vals[i] = bld1(Rg, c + (seg * RPS + i) * rq);
#pragma unroll
        for (int pi = 0; pi < 2; ++pi) {
            const int row = 16 * (pi ? (NT - 1 - half) : half) + lr;
#pragma unroll
            for (int m = 0; m < NKH; ++m)
                araw[pi][m] = bld4(mat == 0 ? Rq : Rb, lr_q + (row - lr) * rq + 16 * (m0 + m) + 4 * lg);
        }
        __builtin_amdgcn_sched_barrier(0); // the waits below leave araw in flight
#pragma unroll
        for (int i = 0; i < RPS; ++i) {
            acc += vals[i];
            vals[i] = acc;
        }
        sTot[seg][c] = acc;
        if (tid < NT * (K / 32)) (&sMask[0][0])[tid] = (&sPair[0][0])[tid] = 0u;
#pragma unroll
        for (int i = 0; i < KF4; ++i) {
            const int f = i * 512 + tid, row = f / (K / 4), c4 = f % (K / 4);
            *reinterpret_cast<floatx4 *>(&sK[row][4 * c4]) = kreg[i];
        }
        __syncthreads();
        float off = 0.f, later = 0.f;
        for (int s2 = 0; s2 < seg; ++s2) off += sTot[s2][c];
        for (int s2 = seg + 1; s2 < NSEG; ++s2) later += sTot[s2][c];
#pragma unroll
        for (int i = 0; i < RPS; ++i) sG[seg * RPS + i][c] = (vals[i] + off) * kLog2e;
        // Kd = k exp(G_last - G), this thread's rows of channel c, with the
        // exponent summed from the chunk's end: the segment's own later rows
        // (acc - vals[i]) plus the later segments' totals.  Formed as the
        // difference of the two cumulative sums (the reference's form,
        // src/forward.rs:271-274) it carries their rounding at |G| up to 64 |g|:
        // at strong decay (|G| near 2900 in log2 units, f32 spacing 2.4e-4) that
        // is ~1e-4 relative in every factor, the last tokens' (the largest)
        // included.  Kd^T as A-operand fragments (kb, tt): lane (g, r) holds
        // Kd[16 tt + 4 g + j][16 kb + r], four rows per 16-byte store.  The
        // training variant's Kd, fragments (tt, kb) with lane (g, r) holding
        // Kd[16 tt + r][16 kb + 4 g + j], takes a 4 x 4 transpose among the
        // four lanes of consecutive channels (two quad exchanges) first, then
        // one 16-byte store per row.
        {
            static_assert(RPS % 4 == 0, "four rows per store");
            floatx4 *Kf = reinterpret_cast<floatx4 *>(p.ws_kdt) + cid * (C * K / 4);
            floatx4 *Kdf = reinterpret_cast<floatx4 *>(p.ws_kd) + cid * (C * K / 4);
            const int kb = c / 16, r = c % 16, qi = lane & 3; // c % 4 == lane % 4
#pragma unroll
            for (int q4 = 0; q4 < RPS / 4; ++q4) {
                const int t0 = seg * RPS + 4 * q4; // rows t0 .. t0 + 3: one tile, one lane group
                floatx4 val;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 4 * q4 + j;
                    val[j] = sK[t0 + j][c] * fast_exp2((acc - vals[i] + later) * kLog2e);
                }
                st_stream(Kf + (kb * NT + t0 / 16) * 64 + 16 * ((t0 % 16) / 4) + r, val);
                if (TRAIN) {
                    // lane qi of the quad holds rows t0 .. t0 + 3 of channel c;
                    // afterwards row t0 + qi of channels c - qi .. c - qi + 3
                    floatx4 x = val;
                    quad_swap_halves(x, (qi & 2) != 0);
                    quad_swap_pairs(x, (qi & 1) != 0);
                    const int t = t0 + qi;
                    st_stream(Kdf + ((t / 16) * NKT + kb) * 64 + 16 * ((c % 16) / 4) + t % 16, x);
                }
            }
        }
        __syncthreads();
    }
    if (tid < K) p.ws_gam[cid * K + tid] = fast_exp2(sG[C - 1][tid]); // exp(G_last)

    // The score products' reference per (row tile, channel): Gb = G at the end
    // of the previous tile (0 for the first); for a mid-range span the middle
    // of the tile's range, (Gb + G_end) / 2, for the whole row tile. Its
    // diagonal factors then lie in [2^-96, 2^96]; in the off-diagonal blocks
    // the row factor is at most 2^96 and the column factor at most 1, and a
    // column factor that underflows drops a term below 2^-30 |row operand k|.
    // Spans above kSafeSpanMid leave the diagonal block's MFMA product (sMask):
    // if both 8-token halves span at most kSafeSpanMid, the block is formed from
    // three half-block products (below); else from exact pairwise terms (sPair).
    for (int idx = tid; idx < NT * K; idx += 512) {
        const int pt = idx / K, c = idx % K;
        const float gb = pt ? sG[16 * pt - 1][c] : 0.f, g7 = sG[16 * pt + 7][c], ge = sG[16 * pt + 15][c];
        const float span = gb - ge;
        if (span > kSafeSpanMid) {
            atomicOr(&sMask[pt][c >> 5], 1u << (c & 31));
            if (gb - g7 > kSafeSpanMid || g7 - ge > kSafeSpanMid) atomicOr(&sPair[pt][c >> 5], 1u << (c & 31));
        }
        sRef[pt][c] = (span > kSafeSpan && span <= kSafeSpanMid) ? 0.5f * (gb + ge) : gb;
    }
    __syncthreads();

    // 2. A_qk (waves 0-3) and A_kk (waves 4-7).  Wave (mat, h, kh) takes the
    //    row tiles {h, NT-1-h}, so that all waves do the same number of
    //    blocks, over the channel half kh; the two halves are summed through
    //    LDS below.  The row operands, with exp(G) applied, are kept for the
    //    solve: q exp(G) (A_qk waves) and b k exp(G) (A_kk waves).
    // The solve's value-column right-hand sides w, v of row tile pt, for the
    // column tiles nt = wave + NW u past the key columns (slot sl of r1 / r2).
    // With one value-column tile per wave every row tile gets its own slot
    // (all requested at once); with more, two slots rotate.
    constexpr bool ALLV = NTW - NKW <= 1;
    constexpr int NSL = ALLV ? NT : 2;
    floatx4 r1[NSL][NTW], r2[NSL][NTW];
    auto load_vw = [&](int pt, int sl) {
#pragma unroll
        for (int u = 0; u < NTW; ++u) {
            const int nt = wave + NW * u;
            if (nt < NTOT && nt >= NKT) {
                const int c = 16 * (nt - NKT) + lr;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * pt + 4 * lg + i;
                    r1[sl][u][i] = bld1(Rw, lg_v + (t - 4 * lg) * rv + c);
                    r2[sl][u][i] = bld1(Rv, lg_v + (t - 4 * lg) * rv + c);
                }
            }
        }
    };
    floatx4 stR[NKW][NT]; // the solve's key-column right-hand sides (staged below)
    floatx4 *QGf = reinterpret_cast<floatx4 *>(p.ws_qg) + cid * (C * K / 4);
    {
        floatx4 acc[2][NT];
#pragma unroll
        for (int pi = 0; pi < 2; ++pi) {
            const int pt = pi ? (NT - 1 - half) : half;
            const int row = 16 * pt + lr;
#pragma unroll
            for (int q = 0; q < NT; ++q) acc[pi][q] = floatx4{0.f, 0.f, 0.f, 0.f};
            // Diagonal block, channels split into 8-token halves: rows and columns
            // 0-7 and 8-15 each with the middle of their half's range as reference
            // (one product, whose cross-half terms are discarded), rows 8-15 x
            // columns 0-7 with G at row 7 (both factors <= 1).  A lane's row and
            // column are the same token, 16 pt + lr.  These terms start the
            // diagonal block's accumulator; the products below leave the
            // channels out.
            {
                floatx4 dsp = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int m = 0; m < NKH; ++m) {
                    const int wix = (16 * (m0 + m)) >> 5, wsh = (16 * (m0 + m)) & 31;
                    const uint32_t w16s = ((__builtin_amdgcn_readfirstlane(sMask[pt][wix]) &
                                            ~__builtin_amdgcn_readfirstlane(sPair[pt][wix])) >> wsh) & 0xffffu;
                    if (w16s == 0u) continue; // wave-uniform
                    const int c0 = 16 * (m0 + m) + 4 * lg;
                    const uint32_t sl = ((sMask[pt][c0 >> 5] & ~sPair[pt][c0 >> 5]) >> (c0 & 31)) & 0xfu;
                    floatx4 aac = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (((w16s >> j) & 0x1111u) == 0u) continue; // none of channels 16 (m0 + m) + 4 g + j
                        const int c = c0 + j;
                        const float gr = sG[row][c], kr = sK[row][c], g7 = sG[16 * pt + 7][c];
                        const float ref = lr < 8 ? 0.5f * (sRef[pt][c] + g7) : 0.5f * (g7 + sG[16 * pt + 15][c]);
                        const float raw = mat == 1 ? araw[pi][m][j] * kr : araw[pi][m][j];
                        const bool sp = (sl >> j) & 1u;
                        const float a1 = sp ? raw * fast_exp2(gr - ref) : 0.f;
                        const float b1 = sp ? kr * fast_exp2(ref - gr) : 0.f;
                        const float a2 = (sp && lr >= 8) ? raw * fast_exp2(gr - g7) : 0.f;
                        const float b2 = (sp && lr < 8) ? kr * fast_exp2(g7 - gr) : 0.f;
                        aac = mfma16(a1, b1, aac);
                        dsp = mfma16(a2, b2, dsp); // exactly zero outside rows 8-15 x columns 0-7
                    }
                    if ((lg < 2) == (lr < 8)) dsp += aac; // rows 4 lg + i and column lr in one half
                }
#pragma unroll
                for (int q = 0; q < NT; ++q)
                    if (q == pt) acc[pi][q] = dsp;
            }
#pragma unroll
            for (int m = 0; m < NKH; ++m) {
                const int c0 = 16 * (m0 + m) + 4 * lg;
                const floatx4 gr = *reinterpret_cast<const floatx4 *>(&sG[row][c0]);
                const floatx4 gb = *reinterpret_cast<const floatx4 *>(&sRef[pt][c0]);
                const floatx4 kr = *reinterpret_cast<const floatx4 *>(&sK[row][c0]);
                floatx4 a = araw[pi][m] * (mat == 1 ? kr : floatx4{1.f, 1.f, 1.f, 1.f});
                a *= exp2v(gr - gb);
                // scale q exp(G_r): the sequential kernel's A operand, fragment (pt, m0 + m)
                if (mat == 0) {
                    const floatx4 qg = a * exp2v(gb) * p.scale;
                    // (the backward takes QG^T only; its training forward, fwd_out, both)
                    if (!TRAIN || p.fwd_out) st_stream(QGf + (pt * NKT + m0 + m) * 64 + lane, qg);
                    if (TRAIN) // (q exp(G))^T fragment (m0 + m, pt)
                        st_stream(reinterpret_cast<floatx4 *>(p.ws_qgt) + cid * (C * K / 4) +
                                      ((m0 + m) * NT + pt) * 64 + lane,
                                  transpose16(qg, lr, lg));
                }
                const uint32_t mw = sMask[pt][c0 >> 5] >> (c0 & 31);
#pragma unroll
                for (int q = 0; q < NT; ++q) {
                    if (q <= pt && (pi == 1 || q < NT / 2)) { // pi = 0: row tile h < NT/2
                        const int srow = 16 * q + lr;
                        const floatx4 gs = *reinterpret_cast<const floatx4 *>(&sG[srow][c0]);
                        floatx4 bv = *reinterpret_cast<const floatx4 *>(&sK[srow][c0]) * exp2v(gb - gs);
                        const bool diag = q == pt;
                        bv[0] = (diag && (mw & 1u)) ? 0.f : bv[0];
                        bv[1] = (diag && (mw & 2u)) ? 0.f : bv[1];
                        bv[2] = (diag && (mw & 4u)) ? 0.f : bv[2];
                        bv[3] = (diag && (mw & 8u)) ? 0.f : bv[3];
                        acc[pi][q] = mfma16(a[0], bv[0], acc[pi][q]);
                        acc[pi][q] = mfma16(a[1], bv[1], acc[pi][q]);
                        acc[pi][q] = mfma16(a[2], bv[2], acc[pi][q]);
                        acc[pi][q] = mfma16(a[3], bv[3], acc[pi][q]);
                    }
                }
            }
        }
        // Diagonal blocks, channels (of this half) outside the mid-tile reference's
        // span: half-block products where both halves allow it, else exact
        // pairwise terms.  The row operand q or b of channel c and row 16 pt + r
        // is already in this wave's registers: component c % 4 of
        // araw[pi][c / 16 - m0] in lane 16 ((c % 16) / 4) + r.  It is gathered
        // across lanes (ds_bpermute) rather than read again from memory, which
        // costs one round trip per masked channel.  The channels are visited in
        // register order (block m, then the four lane groups cg, each holding
        // channels 16 (m0 + m) + 4 cg + j in component j), so that the registers
        // are known at compile time; the terms are summed in dacc and added to
        // the diagonal block's accumulator once.  (A vector element goes
        // through a scalar before __builtin_bit_cast: the cast of a vector
        // element lvalue reads the vector's first element.)  The training variant, whose
        // registers are fuller, reads the row operand from memory (keeping araw
        // live here would spill 72 bytes per lane); its arithmetic and order are
        // the same, so that both variants give bit-identical scores.
        {
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int pt = pi ? (NT - 1 - half) : half;
                // pairwise mask words of one channel half (K = 32: the half's 16 bits of word 0)
                constexpr int NWD = K >= 64 ? K / 64 : 1;
                uint32_t pwh[NWD];
                uint32_t anyw = 0u;
#pragma unroll
                for (int x = 0; x < NWD; ++x) {
                    uint32_t wp = __builtin_amdgcn_readfirstlane(sPair[pt][K >= 64 ? kh * NWD + x : 0]);
                    if (K < 64) wp = (wp >> (16 * kh)) & 0xffffu;
                    pwh[x] = wp;
                    anyw |= wp;
                }
                if (anyw == 0u) continue; // wave-uniform
                floatx4 dacc = floatx4{0.f, 0.f, 0.f, 0.f};
                const int srow = 16 * pt + lr;
                // the row conditions of the lower triangle: r >= s (A_qk), r > s (A_kk)
                bool rowok[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) rowok[i] = mat == 0 ? (4 * lg + i >= lr) : (4 * lg + i > lr);
                // two channels c0, c0 + 1 (c0 = 16 (m0 + m) + 4 cg + 2 jh) per step when
                // both are masked (their G and k in 8-byte LDS reads), else the one
                // that is; their row operands are components 2 jh, 2 jh + 1 of
                // araw[pi][m] in lane group cg
#pragma unroll
                for (int m = 0; m < NKH; ++m) {
                    const uint32_t w16 = (pwh[(16 * m) >> 5] >> ((16 * m) & 31)) & 0xffffu;
                    if (w16 == 0u) continue; // wave-uniform
                    for (int cg = 0; cg < 4; ++cg) {
#pragma unroll
                        for (int jh = 0; jh < 2; ++jh) { // channel pairs c0 + 2 jh + {0, 1}
                            const uint32_t bits = (w16 >> (4 * cg + 2 * jh)) & 0x3u;
                            if (bits == 0u) continue; // wave-uniform
                            const int c0 = 16 * (m0 + m) + 4 * cg + 2 * jh;
                            // All of a step's loads are issued first and pinned (the
                            // compiler would otherwise sink a load used only in a
                            // lane-selected term into a divergent branch with its
                            // own wait), then the terms are formed.
                            if (bits != 0x3u) { // one channel of the pair (wave-uniform): it alone
                                const int jj = bits >> 1, c = c0 + jj;
                                const float gs1 = sG[srow][c], ks1 = sK[srow][c];
                                float o = 0.f;
                                if constexpr (!TRAIN) o = jj ? araw[pi][m][2 * jh + 1] : araw[pi][m][2 * jh];
                                float x[4], kx[4], gx[4];
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    const int r = 4 * lg + i;
                                    const int rrow = 16 * pt + r;
                                    if constexpr (TRAIN)
                                        x[i] = bld1(mat == 0 ? Rq : Rb, lg_q + (16 * pt + i) * rq + c);
                                    else
                                        x[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                             4 * (16 * cg + r), __builtin_bit_cast(int, o)));
                                    kx[i] = sK[rrow][c];
                                    gx[i] = sG[rrow][c];
                                }
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    kx[i] = pin(kx[i]);
                                    gx[i] = pin(gx[i]);
                                }
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    const float xi = mat == 1 ? x[i] * kx[i] : x[i];
                                    const float d = rowok[i] ? gx[i] - gs1 : -__builtin_inff();
                                    dacc[i] += xi * ks1 * fast_exp2(d);
                                }
                                continue;
                            }
                            const float2 gs = *reinterpret_cast<const float2 *>(&sG[srow][c0]);
                            const float2 ks = *reinterpret_cast<const float2 *>(&sK[srow][c0]);
                            float o0 = 0.f, o1 = 0.f;
                            if constexpr (!TRAIN) {
                                o0 = araw[pi][m][2 * jh]; // scalars (see above)
                                o1 = araw[pi][m][2 * jh + 1];
                            }
                            float x0[4], x1[4];
                            float2 gr[4], kr[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int r = 4 * lg + i;
                                const int rrow = 16 * pt + r;
                                if constexpr (TRAIN) { // row rrow of q or b, channels c0, c0 + 1
                                    x0[i] = bld1(mat == 0 ? Rq : Rb, lg_q + (16 * pt + i) * rq + c0);
                                    x1[i] = bld1(mat == 0 ? Rq : Rb, lg_q + (16 * pt + i) * rq + c0 + 1);
                                } else {
                                    x0[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                          4 * (16 * cg + r), __builtin_bit_cast(int, o0)));
                                    x1[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                          4 * (16 * cg + r), __builtin_bit_cast(int, o1)));
                                }
                                gr[i] = *reinterpret_cast<const float2 *>(&sG[rrow][c0]);
                                kr[i] = *reinterpret_cast<const float2 *>(&sK[rrow][c0]);
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                gr[i] = pin(gr[i]);
                                kr[i] = pin(kr[i]);
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const float xa = mat == 1 ? x0[i] * kr[i].x : x0[i];
                                const float xb = mat == 1 ? x1[i] * kr[i].y : x1[i];
                                // branch-free: exp2(-inf) = 0 outside the triangle
                                const float d0 = rowok[i] ? gr[i].x - gs.x : -__builtin_inff();
                                const float d1 = rowok[i] ? gr[i].y - gs.y : -__builtin_inff();
                                dacc[i] += xa * ks.x * fast_exp2(d0) + xb * ks.y * fast_exp2(d1);
                            }
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < NT; ++q)
                    if (q == pt) acc[pi][q] += dacc;
            }
        }
        // Row tile 0's value-column right-hand sides: requested now, so that
        // they arrive during the reductions and the diagonal inverses.
        load_vw(0, 0);
        // The solve's right-hand sides b k exp(G_r) (A_kk waves), from the b
        // rows still held in araw since the score products (128 VGPRs, no
        // spill): a second read from global memory missed L2 about half the
        // time.  The training variant, whose extra stores already spill a
        // little, reads them again instead.
        floatx4 stg[2][NKH];
        if (mat == 1) {
            floatx4 ar2[2][NKH];
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int row = 16 * (pi ? (NT - 1 - half) : half) + lr;
#pragma unroll
                for (int m = 0; m < NKH; ++m)
                    ar2[pi][m] = TRAIN ? bld4(Rb, lr_q + (row - lr) * rq + 16 * (m0 + m) + 4 * lg) : araw[pi][m];
            }
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int row = 16 * (pi ? (NT - 1 - half) : half) + lr;
#pragma unroll
                for (int m = 0; m < NKH; ++m) {
                    const int c0 = 16 * (m0 + m) + 4 * lg;
                    const floatx4 gr = *reinterpret_cast<const floatx4 *>(&sG[row][c0]);
                    const floatx4 kr = *reinterpret_cast<const floatx4 *>(&sK[row][c0]);
                    stg[pi][m] = ar2[pi][m] * kr * exp2v(gr);
                }
            }
        }
        __syncthreads(); // sK and sG are dead
        // region A <- the right-hand sides; region B <- channel half 1's partial sums
        if (mat == 1) {
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int row = 16 * (pi ? (NT - 1 - half) : half) + lr;
#pragma unroll
                for (int m = 0; m < NKH; ++m)
                    *reinterpret_cast<floatx4 *>(&sBKG[row][16 * (m0 + m) + 4 * lg]) = stg[pi][m];
            }
        }
        if (kh == 1) {
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int pt = pi ? (NT - 1 - half) : half;
#pragma unroll
                for (int q = 0; q < NT; ++q)
                    if (q <= pt && (pi == 1 || q < NT / 2))
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float *dst = mat == 0 ? &sAqk[16 * pt + 4 * lg + i][16 * q + lr]
                                                  : &sAkk[16 * pt + 4 * lg + i][16 * q + lr];
                            *dst = acc[pi][q][i];
                        }
            }
        }
        __syncthreads();
        // The solve's owner of key column tile nt = wave + NW u reads its
        // columns in accumulator layout (rows 4 g + i, column r of each 16 x 16
        // tile); channel half 0 completes the score matrices.
#pragma unroll
        for (int u = 0; u < NKW; ++u) {
            if (wave + NW * u < NKT) {
                const int col = 16 * (wave + NW * u) + lr;
#pragma unroll
                for (int tp = 0; tp < NT; ++tp)
#pragma unroll
                    for (int i = 0; i < 4; ++i) stR[u][tp][i] = sBKG[16 * tp + 4 * lg + i][col];
            }
        }
        if (kh == 0) {
#pragma unroll
            for (int pi = 0; pi < 2; ++pi) {
                const int pt = pi ? (NT - 1 - half) : half;
#pragma unroll
                for (int q = 0; q < NT; ++q) {
                    if (q <= pt && (pi == 1 || q < NT / 2)) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = 4 * lg + i;
                            if (mat == 0) {
                                float *dst = &sAqk[16 * pt + r][16 * q + lr];
                                float val = (acc[pi][q][i] + *dst) * p.scale;
                                if (q == pt && r < lr) val = 0.f;
                                *dst = val;
                            } else {
                                float *dst = &sAkk[16 * pt + r][16 * q + lr];
                                float val = acc[pi][q][i] + *dst;
                                if (q == pt && r <= lr) val = 0.f;
                                *dst = val;
                            }
                        }
                    }
                }
            }
        }
    }
    __syncthreads();

    // A_qk -> the sequential kernel as A-operand fragments (mt, qt), the lower
    // block triangle qt <= mt only: chunk-inter reads no other tile (the
    // backward takes A_qk^T only; its training forward, fwd_out, both).
    {
        floatx4 *Af = reinterpret_cast<floatx4 *>(p.ws_aqk) + cid * (C * C / 4);
        if (!TRAIN || p.fwd_out) {
#pragma unroll
            for (int j = 0; j < NT * NT / NW; ++j) {
                const int f = wave + NW * j, mt = f / NT, qt = f % NT;
                if (qt > mt) continue; // wave-uniform
                st_stream(Af + f * 64 + lane,
                          *reinterpret_cast<const floatx4 *>(&sAqk[16 * mt + lr][16 * qt + 4 * lg]));
            }
        }
        if (TRAIN) {
            // A_qk^T fragments (st, rt): lane (g, r) holds A_qk[16 rt + 4 g + j][16 st + r]
            floatx4 *ATf = reinterpret_cast<floatx4 *>(p.ws_aqkt) + cid * (C * C / 4);
#pragma unroll
            for (int j = 0; j < NT * NT / NW; ++j) {
                const int f = wave + NW * j, st = f / NT, rt = f % NT;
                floatx4 val = floatx4{0.f, 0.f, 0.f, 0.f};
                if (rt >= st)
#pragma unroll
                    for (int i = 0; i < 4; ++i) val[i] = sAqk[16 * rt + 4 * lg + i][16 * st + lr];
                st_stream(ATf + f * 64 + lane, val);
            }
        }
    }

    // 3. (I + A_kk_pp)^-1 for the four diagonal 16x16 blocks: lane = (tile, column).
    if (wave == 0) {
        const int pt = lane >> 4, j = lane & 15;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = (i == j) ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) s -= sAkk[16 * pt + i][16 * pt + m] * x[m];
            x[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sAinv[pt][i][j] = x[i];
    }
    __syncthreads();

    // 4. Blocked solve of (I + A_kk) [W | U] = [b k exp(G) | w v]; wave w owns
    //    column tiles w, w + 8, ... of [W | U]
    //    (key columns first, whose right-hand sides were staged above; the
    //    value columns' w, v rows of tile 0 were requested after the score
    //    products, those of the other tiles are requested here at once, or
    //    one tile ahead when a wave owns several value-column tiles).
    //    Outputs go to the workspace in MFMA fragment order (one
    //    1 KB block of 64 lanes x float4 per 16x16 tile) so that every store
    //    here and every load in chunk-inter is a contiguous 16-byte access per
    //    lane:
    //      W : A-operand fragments (lane (g, r) holds rows r, cols 4g..4g+3)
    //      U : accumulator fragments (lane (g, c) holds rows 4g..4g+3, col c)
    floatx4 *Wf = reinterpret_cast<floatx4 *>(p.ws_w) + cid * (C * K / 4);
    floatx4 *Uf = reinterpret_cast<floatx4 *>(p.ws_u) + cid * (C * V / 4);
    floatx4 X[NTW][NT];
    if constexpr (ALLV) {
#pragma unroll
        for (int pt = 1; pt < NT; ++pt) load_vw(pt, pt); // the other row tiles' value columns, all at once
    }
#pragma unroll
    for (int pt = 1; pt <= NT; ++pt) {
        if (!ALLV && pt < NT) load_vw(pt, pt & 1); // row tile pt's value columns, consumed at iteration pt + 1
        const int tp = pt - 1, sl = ALLV ? tp : tp & 1; // the row tile solved in this iteration
#pragma unroll
        for (int u = 0; u < NTW; ++u) {
            const int nt = wave + NW * u;
            const bool kcol = nt < NKT; // then u < NKW
            if (nt >= NTOT) continue;
            floatx4 R = kcol ? stR[u < NKW ? u : 0][tp] : r1[sl][u] * r2[sl][u];
#pragma unroll
            for (int q = 0; q < NT; ++q)
                if (q < tp) R = mfma4n(*reinterpret_cast<const float4 *>(&sAkk[16 * tp + lr][16 * q + 4 * lg]), X[u][q], R);
            floatx4 Xp = mfma4(*reinterpret_cast<const float4 *>(&sAinv[tp][lr][4 * lg]), R,
                               floatx4{0.f, 0.f, 0.f, 0.f});
            X[u][tp] = Xp;
            if (kcol) {
                st_stream(Wf + (tp * NKT + nt) * 64 + lane, transpose16(Xp, lr, lg));
                if (TRAIN) // W^T fragment (nt, tp): the accumulator layout of W's tile
                    st_stream(reinterpret_cast<floatx4 *>(p.ws_wt) + cid * (C * K / 4) + (nt * NT + tp) * 64 + lane,
                              Xp);
            } else
                st_stream(Uf + ((nt - NKT) * NT + tp) * 64 + lane, Xp);
        }
    }
    if (TRAIN && wave < NT) {
        // Ai = (I + A_kk)^-1 for the backward: the same blocked solve with the
        // identity's column tile `wave` as right-hand side; tile (tp, it) stored in
        // accumulator layout (lane (g, c) holds Ai[16 tp + 4 g + i][16 it + c]).
        const int it = wave;
        floatx4 *Aif = reinterpret_cast<floatx4 *>(p.ws_akk) + cid * (C * C / 4);
        floatx4 Xi[NT];
#pragma unroll
        for (int tp = 0; tp < NT; ++tp) {
            floatx4 R;
#pragma unroll
            for (int i = 0; i < 4; ++i) R[i] = (tp == it && 4 * lg + i == lr) ? 1.f : 0.f;
#pragma unroll
            for (int q = 0; q < NT; ++q)
                if (q < tp) R = mfma4n(*reinterpret_cast<const float4 *>(&sAkk[16 * tp + lr][16 * q + 4 * lg]), Xi[q], R);
            Xi[tp] = tp < it ? floatx4{0.f, 0.f, 0.f, 0.f}
                             : mfma4(*reinterpret_cast<const float4 *>(&sAinv[tp][lr][4 * lg]), R,
                                     floatx4{0.f, 0.f, 0.f, 0.f});
            st_stream(Aif + (tp * NT + it) * 64 + lane, Xi[tp]);
        }
    }
}

// ---------------------------------------------------------------------------
// chunk-inter: one workgroup per (b, hv, 64 value columns); wave w owns 16
// columns.  S[:, cols] stays in MFMA accumulators for the whole sequence.
// Per chunk n:
//   A: X1 = W S, X2 = scale (q exp(G)) S      (reads sW, sQ)
//   B: v_new = U - X1
//   C: S = exp(G_last) S + Kd^T v_new         (reads sKd)
//   D: out = X2 + A_qk v_new                  (reads sA; independent of C)
// D(n) runs at the top of iteration n + 1, before the wait for chunk n + 1's
// copies, whose latency its MFMAs cover.
// LDS holds one chunk of W, q exp(G) (2 C K floats), Kd^T (K C) and A_qk
// (C C).  Each buffer is refilled while another phase runs: Kd^T(n) and
// A_qk(n) are fetched during A(n) and stored after it; W, q exp(G)(n+1) are
// fetched during B-D(n) and stored after them.  HBM latency is therefore off
// the sequential path without a second copy of the buffers.
//
// Segmented form (NSEG > 1, few long sequences).  Over one segment the
// recurrence is affine in its entering state:
//   S_out = P S_in + Q,  P = prod_n (diag(exp(G_last)) - Kd^T W)  (K x K),
// and Q is the segment run from S_in = 0.  P is the same recurrence run on
// the K columns of an identity with U = 0.  So:
//   pass 1 (OUT = false): every segment but the last, from S = 0 on the V
//     value columns and from S = I, U = 0 on K extra columns; no output;
//     the results go to ws_qseg / ws_pseg (the training forward also runs the
//     last segment, for its P only);
//   pass 2 (chunk_chain_kernel): S_in(j + 1) = P_j S_in(j) + Q_j, in order;
//   pass 3 (OUT = true): every segment from its S_in, with the output; the
//     last segment writes the final state.
// With NSEG = 1 pass 3 alone is the plain sequential kernel.
//
// MODE: kInterOut (pass 3), kInterLocal (pass 1), kInterStates (pass 3 for
// the backward: no output and no final state; instead the state entering
// every chunk (ws_sn) and every chunk's v_new (ws_vn), both as accumulator
// fragments in (value tile, row tile) order, so that each 16-column slice is
// one contiguous block), kInterOutStates (pass 3 with both, the reference's
// fused_chunk_forward tuple) or kInterOutTrain (pass 3 with the output and
// the final state, and the per-chunk states and v_new in the backward's
// fragment layout: the training forward whose quantities the backward keeps).
// ---------------------------------------------------------------------------
constexpr int kInterOut = 0, kInterLocal = 1, kInterStates = 2, kInterOutStates = 3, kInterOutTrain = 4;

// NWV waves per workgroup (NWV = 4: 64 value columns; NWV = 2: 32, for value
// dimensions that are not a multiple of 64 and for K = 32; NWV = 8: 128, pass 1
// at K = 128).
// Chunks [*n0, *n1) of segment seg (uniform runs of SEGL, or the inference
// split's first segment of SEG0 then runs of SEGL), and the slot of segment
// j's entering state in ws_qseg (its transition's in ws_pseg), per (b, hv).
__device__ __forceinline__ void seg_range(const ChunkParams &p, int seg, int *n0, int *n1) {
    const int a = p.SLOT0 ? (seg == 0 ? 0 : p.SEG0 + (seg - 1) * p.SEGL) : seg * p.SEGL;
    *n0 = a;
    *n1 = min(p.NC, p.SLOT0 && seg == 0 ? p.SEG0 : a + p.SEGL);
}
__device__ __forceinline__ size_t seg_slot(const ChunkParams &p, int bh, int j) {
    return (size_t)bh * p.NSLOT + (j - p.SLOT0);
}

template <int K, int MODE, int NWV>
__global__ __launch_bounds__(64 * NWV, 1) void chunk_inter_kernel(ChunkParams p, int nseg_launch, int seg_base) {
    constexpr bool OUT = MODE == kInterOut || MODE == kInterOutStates || MODE == kInterOutTrain;
    constexpr bool LOCAL = MODE == kInterLocal;
    constexpr bool STATES = MODE == kInterStates || MODE == kInterOutStates || MODE == kInterOutTrain;
    constexpr bool FRAG = MODE == kInterStates || MODE == kInterOutTrain; // the backward's layouts
    constexpr int NTH = 64 * NWV;  // threads per workgroup
    constexpr int VSW = 16 * NWV;  // value columns per workgroup
    constexpr int NKT = K / 16;
    constexpr int FR = NKT * NT;   // 16x16 fragments per operand per chunk
    constexpr int OPF4 = FR * 64;  // float4 per operand per chunk
    constexpr int PFO = OPF4 / NTH; // float4 per lane per operand
    static_assert(OPF4 % NTH == 0 && K % VSW == 0, "K");
    constexpr int AF4 = NT * NT * 64; // float4 of A_qk per chunk
    constexpr int APF = AF4 / NTH;
    __shared__ floatx4 sW[OPF4], sKd[OPF4];
    // K = 256: W and Kd^T take 64 KiB each, so scale q exp(G), which feeds only
    // the output (off the sequential chain), is read from L2 into registers in
    // phase A instead of through a third LDS buffer (145 KiB in all).
    constexpr bool QLDS = OUT && K <= 128;
    __shared__ floatx4 sQ[QLDS ? OPF4 : 1], sA[OUT ? AF4 : 1];
    __shared__ float sPf[NTH]; // destination of the L2 touches, never read
    // exp(G_last) of the chunk, copied with Kd^T: read just before phase C, so
    // that it holds no registers through phases A and D
    __shared__ floatx4 sGam[K / 4];

    const int V = p.V;
    const int nvv = V / VSW;                    // value slices
    const int nvs = LOCAL ? nvv + K / VSW : nvv; // pass 1 adds the slices of P
    int sq, vs;
    inter_block(blockIdx.x, p.B * p.HV * nseg_launch, nvs, &sq, &vs);
    const int bh = sq / nseg_launch, seg = seg_base + sq % nseg_launch;
    const int bi = bh / p.HV, hv = bh % p.HV;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform (scalar)
    const int lr = lane & 15, lg = lane >> 4;
    const bool pcol = LOCAL && vs >= nvv;          // a slice of P (wave-uniform)
    const int vt = (pcol ? vs - nvv : vs) * NWV + wave; // this wave's 16-column tile
    const int col = 16 * vt + lr;
    int n0, n1;
    seg_range(p, seg, &n0, &n1);

    // entering state: S0 (one segment, or the split's segment 0), the chained
    // state (pass 3; in uniform runs slot 0 is a copy of S0, so that no
    // workgroup reads the state that the last segment overwrites), 0 (pass 1
    // value columns) or the identity (pass 1, P columns)
    const float *Sin = nullptr;
    if (!LOCAL)
        Sin = p.NSEG == 1 || (p.SLOT0 && seg == 0) ? p.state + (size_t)bh * K * V
                                                   : p.ws_qseg + seg_slot(p, bh, seg) * K * V;
    floatx4 S[NKT];
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * kb + 4 * lg + i;
            S[kb][i] = !LOCAL ? Sin[(size_t)row * V + col] : (pcol && row == col ? 1.f : 0.f);
        }

    const floatx4 *__restrict__ W4 = reinterpret_cast<const floatx4 *>(p.ws_w);
    const floatx4 *__restrict__ Q4 = reinterpret_cast<const floatx4 *>(p.ws_qg);
    const floatx4 *__restrict__ K4 = reinterpret_cast<const floatx4 *>(p.ws_kdt);
    const floatx4 *__restrict__ U4 = reinterpret_cast<const floatx4 *>(p.ws_u);
    const floatx4 *__restrict__ A4 = reinterpret_cast<const floatx4 *>(p.ws_aqk);
    const floatx4 *__restrict__ G4 = reinterpret_cast<const floatx4 *>(p.ws_gam);
    const size_t cid0 = (size_t)bh * p.NC;
    const size_t uvf4 = (size_t)C * V / 4;

    // the operands go from global memory straight into LDS (lds_copy4):
    // thread tid's float4 i lands at index i * NTH + tid, as a wave's 64 lanes.
    // (The buffer-resource form of these copies, buffer_load_dwordx4 ... lds
    // with 32-bit offsets, needs fewer registers but measured 1.8 % slower.)
    const int wv = 64 * wave;
    // Each chunk's operands are also pulled toward L2 one phase before their
    // LDS copy (l2_touch, one 128-byte line per thread): W, q exp(G) of chunk
    // n + 1 during A(n), Kd^T, A_qk, U of chunk n + 1 during B-D(n).  Every
    // wave issues the same count (2, then 3) last before the vmcnt waits, which
    // leave them in flight; past the last chunk the current one is touched.
    float *pf_slot = &sPf[wv];
    constexpr int LOP = OPF4 / 8, LA = AF4 / 8, LU = NWV * NT * 64 / 8; // lines per operand block
    const int vsu = pcol ? 0 : vs; // the P slices of pass 1 read no U
    auto touch_wq = [&](size_t c) { // 2 per wave
        l2_touch(reinterpret_cast<const char *>(W4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
        l2_touch(reinterpret_cast<const char *>((OUT ? Q4 : K4) + c * OPF4) + 128 * (tid % LOP), pf_slot);
    };
    auto touch_kau = [&](size_t c) { // 3 per wave
        l2_touch(reinterpret_cast<const char *>(K4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
        if (OUT)
            l2_touch(reinterpret_cast<const char *>(A4 + c * AF4) + 128 * (tid % LA), pf_slot);
        else
            l2_touch(reinterpret_cast<const char *>(W4 + c * OPF4) + 128 * (tid % LOP), pf_slot);
        l2_touch(reinterpret_cast<const char *>(U4 + c * uvf4 + (size_t)vsu * NWV * NT * 64) + 128 * (tid % LU), pf_slot);
    };
    if (n1 > n0) {
#pragma unroll
        for (int i = 0; i < PFO; ++i) {
            lds_copy4(&W4[(cid0 + n0) * OPF4 + i * NTH + tid], &sW[i * NTH + wv]);
            if (QLDS) lds_copy4(&Q4[(cid0 + n0) * OPF4 + i * NTH + tid], &sQ[i * NTH + wv]);
        }
        __builtin_amdgcn_sched_barrier(0);
        touch_kau(cid0 + n0);
        __builtin_amdgcn_sched_barrier(0);
    }
    // S and the first copies have landed: nothing from before the loop is
    // left in flight for the compiler's own vmcnt waits inside it
    vm_wait0();

    // chunk nn's output rows from X2 through a buffer resource over its valid
    // rows: rows past T fall outside its range and the hardware drops those
    // stores, and each store's offset is a per-lane term (row 4 lg of each
    // 16-row tile, column col) plus a wave-uniform row term, both 32-bit, in
    // place of 64-bit row addresses.  Needs sot >= V and 63 sot + V < 2^29
    // (checked on the host).
    float *obh = p.out + (int64_t)bi * p.sob + (int64_t)hv * p.soh;
    const int sot = (int)p.sot, olane = 4 * (4 * lg * sot + col);
    auto store_out = [&](const floatx4 *o, int nn) {
        const __amdgpu_buffer_rsrc_t R = rows_rsrc(obh + (int64_t)nn * C * p.sot, sot, min(C, p.T - nn * C), V);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float val = o[mt][i]; // through a scalar: a bit_cast of the element lvalue reads element 0
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, val), R, olane, 4 * (16 * mt + i) * sot, 0);
            }
    };
    floatx4 X1[NT], X2[NT]; // chunk n's v_new and output, both read again in iteration n + 1
    // D: out = X2 + A_qk v_new (A_qk is lower block-triangular; the chains of
    // the four time tiles interleave).  D(n) runs at the top of iteration
    // n + 1, where its MFMAs cover this wave's wait for the next copies.  Its
    // A_qk tiles are read from sA during the last time tile of C(n), so that
    // D waits on no LDS read.
    floatx4 aq[NT][NT]; // A_qk tiles (mt, qt), mt >= qt
    auto load_aq = [&]() {
#pragma unroll
        for (int qt = 0; qt < NT; ++qt)
#pragma unroll
            for (int mt = qt; mt < NT; ++mt) aq[mt][qt] = sA[(mt * NT + qt) * 64 + lane];
    };
    auto phase_d = [&]() {
#pragma unroll
        for (int qt = 0; qt < NT; ++qt)
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int mt = qt; mt < NT; ++mt) X2[mt] = mfma16(aq[mt][qt][st], X1[qt][st], X2[mt]);
    };
    for (int n = n0; n < n1; ++n) {
        const size_t cid = cid0 + n;
        const size_t cnext = n + 1 < n1 ? cid + 1 : cid;
        if (OUT && n > n0) phase_d(); // D(n - 1)
        vm_wait<3>();  // this wave's copies of chunk n's W, q exp(G) have landed (not the 3 touches after them)
        lds_barrier(); // sW, sQ hold chunk n; every wave is done with sKd, sA (n-1)
#pragma unroll
        for (int i = 0; i < PFO; ++i) lds_copy4(&K4[cid * OPF4 + i * NTH + tid], &sKd[i * NTH + wv]);
        if (OUT) {
            // A_qk is lower block-triangular: copy i of wave w brings tile
            // f = NWV i + w = (f / NT, f % NT), copied only on or below the
            // diagonal (10 of the 16 tiles)
#pragma unroll
            for (int i = 0; i < APF; ++i) {
                const int f = NWV * i + wave;
                if (f % NT <= f / NT) lds_copy4(&A4[cid * AF4 + i * NTH + tid], &sA[i * NTH + wv]);
            }
            if (n > n0) store_out(X2, n - 1);
        }
        if (wave == 0 && lane < K / 4) lds_copy4(&G4[cid * (K / 4) + lane], sGam);
        floatx4 u_cur[NT];
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
            u_cur[mt] = pcol ? floatx4{0.f, 0.f, 0.f, 0.f} : U4[cid * uvf4 + (size_t)(vt * NT + mt) * 64 + lane];
        if (STATES) { // the state entering chunk n
            size_t slot = cid;
            bool keep = true;
            if (p.st_cc) { // the first caller chunk starting inside chunk n (wave-uniform)
                const int j0 = (n * C + p.st_cc - 1) / p.st_cc;
                keep = j0 < p.st_chunks;
                slot = (size_t)bh * p.st_chunks + j0;
            }
            float *Sn = p.ws_sn + slot * K * V;
            if (keep) {
                // row-major: 32-bit offsets in a buffer resource over the slot
                const __amdgpu_buffer_rsrc_t R = __builtin_amdgcn_make_buffer_rsrc(Sn, (short)0, K * V * 4, 0x00020000);
#pragma unroll
                for (int kb = 0; kb < NKT; ++kb)
                    if (FRAG) // the backward's fragment layout: tile (value tile, key tile)
                        reinterpret_cast<floatx4 *>(Sn)[(vt * NKT + kb) * 64 + lane] = S[kb];
                    else
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float val = S[kb][i]; // (through a scalar, see store_out)
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, val), R, 4 * (4 * lg * V + col),
                                                                  4 * (16 * kb + i) * V, 0);
                        }
            }
        }
        // keep these loads here, a whole phase ahead of their use and of the
        // vmcnt wait before the next barrier, and the touches last
        __builtin_amdgcn_sched_barrier(0);
        touch_wq(cnext);
        __builtin_amdgcn_sched_barrier(0);

        // A: X1 = W S, X2 = scale (q exp(G)) S
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) X1[mt] = X2[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        floatx4 wa[2][NT], ma[2][NT];
        auto load_a = [&](int kb, int bf) {
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) {
                wa[bf][mt] = sW[(mt * NKT + kb) * 64 + lane];
                if (OUT)
                    ma[bf][mt] = QLDS ? sQ[(mt * NKT + kb) * 64 + lane] : Q4[cid * OPF4 + (mt * NKT + kb) * 64 + lane];
            }
        };
        load_a(0, 0);
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            const int cb = kb & 1;
            // eight (pass 1: four) independent accumulator chains per k-step;
            // the next step's operands are requested after the first quarter
#pragma unroll
            for (int st = 0; st < 4; ++st) {
#pragma unroll
                for (int mt = 0; mt < NT; ++mt) {
                    X1[mt] = mfma16(wa[cb][mt][st], S[kb][st], X1[mt]);
                    if (OUT) X2[mt] = mfma16(ma[cb][mt][st], S[kb][st], X2[mt]);
                }
                if (st == 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (kb + 1 < NKT) load_a(kb + 1, cb ^ 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        vm_wait<2>();  // this wave's copies of chunk n's Kd, A_qk, exp(G_last) and its U have landed (not the 2 touches)
        lds_barrier(); // A done everywhere (sW, sQ free); sKd(n), sA(n) visible
        // exp(G_last) and phase C's first Kd^T tile, requested before the
        // copies below so that their latency is spent on the copies' issue
        floatx4 gk[NKT], ka[2][NKT];
        auto load_c = [&](int tt, int bf) {
#pragma unroll
            for (int kb = 0; kb < NKT; ++kb) ka[bf][kb] = sKd[(kb * NT + tt) * 64 + lane];
        };
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) gk[kb] = sGam[4 * kb + lg]; // rows 16 kb + 4 lg .. + 3
        load_c(0, 0);
        __builtin_amdgcn_sched_barrier(0);

        // B: v_new = U - X1 (kept in X1)
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) X1[mt] = u_cur[mt] - X1[mt];
        if (STATES) {
            // row-major rows through a buffer resource over the chunk's rows:
            // token rows [B * HV, T, V] (the resource ends at row T, so rows past T
            // of a ragged last chunk are dropped) or the chunk's [C, V] block
            if (p.st_cc || !FRAG) {
                float *Vn = p.st_cc ? p.ws_vn + ((size_t)bh * p.T + (size_t)n * C) * V : p.ws_vn + cid * C * V;
                const __amdgpu_buffer_rsrc_t R = rows_rsrc(Vn, V, p.st_cc ? min(C, p.T - n * C) : C, V);
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float val = X1[mt][i]; // (through a scalar, see store_out)
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, val), R, 4 * (4 * lg * V + col),
                                                              4 * (16 * mt + i) * V, 0);
                    }
            } else { // tile (value tile, time tile)
                float *Vn = p.ws_vn + cid * C * V;
#pragma unroll
                for (int mt = 0; mt < NT; ++mt) reinterpret_cast<floatx4 *>(Vn)[(vt * NT + mt) * 64 + lane] = X1[mt];
            }
        }

        // W, q exp(G) of chunk n+1, then the touches of its Kd^T, A_qk, U
        __builtin_amdgcn_sched_barrier(0);
        if (n + 1 < n1) {
#pragma unroll
            for (int i = 0; i < PFO; ++i) {
                lds_copy4(&W4[(cid + 1) * OPF4 + i * NTH + tid], &sW[i * NTH + wv]);
                if (QLDS) lds_copy4(&Q4[(cid + 1) * OPF4 + i * NTH + tid], &sQ[i * NTH + wv]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        touch_kau(cnext);
        __builtin_amdgcn_sched_barrier(0);

        // C: S = exp(G_last) S + Kd^T v_new
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            S[kb][0] *= gk[kb][0];
            S[kb][1] *= gk[kb][1];
            S[kb][2] *= gk[kb][2];
            S[kb][3] *= gk[kb][3];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            const int cb = tt & 1;
            // NKT independent accumulator chains per k-step; the next time
            // tile's operands are requested after the first quarter
#pragma unroll
            for (int st = 0; st < 4; ++st) {
#pragma unroll
                for (int kb = 0; kb < NKT; ++kb) S[kb] = mfma16(ka[cb][kb][st], X1[tt][st], S[kb]);
                if (st == 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (tt + 1 < NT) load_c(tt + 1, cb ^ 1);
                    else if (OUT) load_aq(); // for D(n), at the top of iteration n + 1
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    vm_wait0(); // the last touches have landed in sPf
    if (OUT && n1 > n0) {
        phase_d();
        store_out(X2, n1 - 1);
    }

    // leaving state: the final state (last segment), the state entering
    // segment 1 (the split's segment 0), Q_j or P_j (pass 1)
    float *Sout = nullptr;
    int ld = V;
    if (OUT) {
        if (seg == p.NSEG - 1)
            Sout = p.state + (size_t)bh * K * V;
        else if (MODE == kInterOut && p.SLOT0 && seg == 0)
            Sout = p.ws_qseg + seg_slot(p, bh, 1) * K * V;
    } else if (LOCAL && pcol) {
        Sout = p.ws_pseg + seg_slot(p, bh, seg) * K * K;
        ld = K;
    } else if (LOCAL && seg + 1 < p.NSEG) { // (the last segment runs for its P only: training)
        Sout = p.ws_qseg + seg_slot(p, bh, seg + 1) * K * V;
    }
    if (Sout) {
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) Sout[(size_t)(16 * kb + 4 * lg + i) * ld + col] = S[kb][i];
    }
}

// Pass 2 of the segmented form.  Per (b, hv), the slot of segment j + 1
// (Q_j from pass 1) <- S_in(j + 1) = P_j S_in(j) + Q_j for j = j0 .. NSEG - 2:
// in uniform runs j0 = 0 and slot 0 <- S0 first; in the split j0 = 1 and
// S_in(1) is already in its slot (segment 0's walk left it there).  One
// workgroup per (b, hv, 64 value columns); S in MFMA accumulators, P_j read
// as A-operand fragments (lane (g, r): row r of a 16-row tile, columns 4g ..
// 4g + 3) from L2.
template <int K, int NWV>
__global__ __launch_bounds__(64 * NWV, 1) void chunk_chain_kernel(ChunkParams p) {
    constexpr int NKT = K / 16;
    const int V = p.V, nvv = V / (16 * NWV);
    int bh, vs;
    inter_block(blockIdx.x, p.B * p.HV, nvv, &bh, &vs);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int col = 16 * (vs * NWV + wave) + lr;

    const int j0 = p.SLOT0;
    const float *S0 = j0 ? p.ws_qseg + seg_slot(p, bh, 1) * K * V : p.state + (size_t)bh * K * V;
    float *slot0 = p.ws_qseg + seg_slot(p, bh, j0) * K * V; // the slot of segment j0
    floatx4 S[NKT];
#pragma unroll
    for (int kb = 0; kb < NKT; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t o = (size_t)(16 * kb + 4 * lg + i) * V + col;
            S[kb][i] = S0[o];
            if (!j0) slot0[o] = S[kb][i];
        }
    // Every operand is requested one step ahead of its products: the next
    // k-block of P_j (two register buffers), the first k-block of P_{j+1} during
    // the last one of P_j, and Q_{j+1} during the products of step j, so that
    // a step waits on no memory round trip but its own first one.
    const int nsteps = p.NSEG - 1 - j0; // step i chains segment j0 + i
    auto P_of = [&](int i) { return p.ws_pseg + seg_slot(p, bh, j0 + i) * K * K; };
    auto load_pa = [&](floatx4 *pa, const float *P, int kb) {
#pragma unroll
        for (int it = 0; it < NKT; ++it)
            pa[it] = *reinterpret_cast<const floatx4 *>(P + (size_t)(16 * it + lr) * K + 16 * kb + 4 * lg);
    };
    auto load_q = [&](floatx4 *q, int j) { // slot j + 1 (from segment j0's) holds Q_{j0 + j} from pass 1
        const float *Q = slot0 + (size_t)(j + 1) * K * V;
#pragma unroll
        for (int it = 0; it < NKT; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i) q[it][i] = Q[(size_t)(16 * it + 4 * lg + i) * V + col];
    };
    floatx4 pa[2][NKT], Nq[NKT];
    if (nsteps > 0) {
        load_q(Nq, 0);
        load_pa(pa[0], P_of(0), 0);
    }
    for (int j = 0; j < nsteps; ++j) {
        float *Q = slot0 + (size_t)(j + 1) * K * V;
        floatx4 N[NKT];
#pragma unroll
        for (int it = 0; it < NKT; ++it) N[it] = Nq[it];
#pragma unroll
        for (int kb = 0; kb < NKT; ++kb) {
            const int cb = kb & 1;
            if (kb + 1 < NKT)
                load_pa(pa[cb ^ 1], P_of(j), kb + 1);
            else if (j + 1 < nsteps)
                load_pa(pa[cb ^ 1], P_of(j + 1), 0);
            if (kb == 0 && j + 1 < nsteps) load_q(Nq, j + 1);
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int it = 0; it < NKT; ++it) N[it] = mfma16(pa[cb][it][st], S[kb][st], N[it]);
        }
#pragma unroll
        for (int it = 0; it < NKT; ++it) {
            S[it] = N[it];
#pragma unroll
            for (int i = 0; i < 4; ++i) Q[(size_t)(16 * it + 4 * lg + i) * V + col] = N[it][i];
        }
    }
}

// The states at the boundaries of caller chunks of Cc = p.st_cc tokens (Cc <
// 64, T a multiple of Cc) from the state S_n entering the 64-token chunk n
// that holds the boundary (stored by chunk-inter in slot j0(n), the first
// caller chunk starting inside chunk n) and the chunk's own tokens: with m
// the boundary's offset in chunk n,
//   S(64 n + m) = diag(exp(G_m)) S_n + sum_{t < m} (k_t exp(G_m - G_{t+1}))^T v_new_t
// with G_j = g_0 + .. + g_{j-1} per key channel from the chunk start, so that
// every exponent is <= 0 (src/kernel/chunk_cube.rs:612-734 returns these
// states for the reference's own chunk size).  One workgroup per (b, hv,
// caller chunk j, 64 value columns).  INPLACE = false: every caller chunk but
// j0(n) (read-only access to slot j0(n)); INPLACE = true, launched after:
// slot j0(n) itself where its boundary is not 64 n (Cc not dividing 64),
// every element read and written by the same thread.
template <int K, bool INPLACE>
__global__ __launch_bounds__(256) void chunk_states_kernel(ChunkParams p) {
    constexpr int KB = K > 64 ? K : 64;
    __shared__ float sA[C][K];  // k rows, then the decayed keys k_t exp(G_m - G_{t+1})
    __shared__ float sB[C][KB]; // g rows, then v_new rows (64 value columns; those past V are zero)
    __shared__ float sGam[K];
    const int cc = p.st_cc, nvs = (p.V + 63) / 64;
    int blk = blockIdx.x;
    const int vs = blk % nvs;
    blk /= nvs;
    int j, n, bh;
    if (INPLACE) { // one workgroup per (b, hv, 64-token chunk)
        n = blk % p.NC;
        bh = blk / p.NC;
        j = (n * C + cc - 1) / cc;
        if (j >= p.st_chunks) return;
    } else {
        j = blk % p.st_chunks;
        bh = blk / p.st_chunks;
        n = j * cc / C;
        if (j == (n * C + cc - 1) / cc) return; // slot j0(n): chunk-inter's (or the in-place pass's)
    }
    const int t0 = n * C, m = j * cc - t0; // tokens of chunk n before the boundary
    if (m == 0) return;                    // (INPLACE: the boundary is the chunk start, already exact)
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int64_t kofs = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + (int64_t)t0 * p.sqt;
    const int tid = threadIdx.x;
    for (int i = tid; i < m * K; i += 256) {
        const int t = i / K, c = i % K;
        sA[t][c] = p.k[kofs + (int64_t)t * p.sqt + c];
        sB[t][c] = p.g[kofs + (int64_t)t * p.sqt + c];
    }
    __syncthreads();
    for (int c = tid; c < K; c += 256) { // a thread per key channel walks the m tokens backwards
        float acc = 0.f;                 // g_{t+1} + .. + g_{m-1}
        for (int t = m - 1; t >= 0; --t) {
            sA[t][c] *= fast_exp2(acc * kLog2e);
            acc += sB[t][c];
        }
        sGam[c] = fast_exp2(acc * kLog2e);
    }
    __syncthreads();
    const float *vn = p.ws_vn + ((size_t)bh * p.T + t0) * p.V + vs * 64;
    const int vw = min(64, p.V - vs * 64); // value columns of this slice
    for (int i = tid; i < m * 64; i += 256) sB[i / 64][i % 64] = (i % 64) < vw ? vn[(size_t)(i / 64) * p.V + i % 64] : 0.f;
    __syncthreads();
    const int v = tid & 63, cg = tid >> 6, col = vs * 64 + v;
    if (v >= vw) return; // (no barrier below)
    const size_t slot0 = (size_t)bh * p.st_chunks + (t0 + cc - 1) / cc; // j0(n)
    const float *Sn = p.ws_sn + slot0 * K * p.V;
    float *So = p.ws_sn + ((size_t)bh * p.st_chunks + j) * K * p.V;
    for (int c = cg; c < K; c += 4) {
        float acc = sGam[c] * Sn[(size_t)c * p.V + col];
        for (int t = 0; t < m; ++t) acc += sA[t][c] * sB[t][v];
        So[(size_t)c * p.V + col] = acc;
    }
}

// The inference output split.  A uniform run of n = NSEG segments (n >= 2)
// walks every segment twice: pass 1 (its local state and transition from 0)
// and pass 3 (with the output).  Segment 0 needs no pass 1, its entering state
// being S0: the split walks it once, with the output, while pass 1 summarises
// segments 1 .. n - 1, then pass 3 walks segments 1 .. n.  With n + 1
// segments in all, pass 3's workgroups stay those of the uniform run's n, and
// segment 0's walk takes one value slice per sequence beside pass 1's.
// Segment 0 gets L0 = r NC / (n + r) chunks and the others L = ceil((NC - L0)
// / n), so that its walk and pass 1 end together: r = 1.1 where pass 1 runs
// eight waves over 128 columns, two per SIMD (the fastest of r = 0.5 .. 1.8
// at B = 1, T = 65536, 16 heads, K = V = 128), else 0.8 (pass 1 cheaper per
// chunk than the walk; the fastest of 0.6 .. 1.6 at B = 8, T = 4096, 4
// heads, K = 64, V = 96).  Only where every segment keeps at least
// kMinSplitChunks chunks; else the uniform run.
constexpr int kMinSplitChunks = 16;

bool split_segments(const ChunkParams &p, bool wide_pass1, ChunkParams *q) {
    if (p.NSEG < 2) return false;
    const int n = p.NSEG, NC = p.NC;
    const double r = wide_pass1 ? 1.1 : 0.8;
    const int L0 = (int)(r * NC / (n + r));
    const int L = (NC - L0 + n - 1) / n;
    const int last = NC - L0 - (n - 1) * L;
    if (L0 < kMinSplitChunks || L < kMinSplitChunks || last < 1) return false;
    *q = p;
    q->NSEG = n + 1;
    q->SEG0 = L0;
    q->SEGL = L;
    q->SLOT0 = 1; // segments 1 .. n in slots 0 .. n - 1 of the uniform run's n
    return true;
}

// A second stream per device (default priority, non-blocking; on the device
// of the caller's stream) with a fork and a join event, for the split's
// segment-0 walk beside pass 1.  Created on first use, never while the
// caller's stream is capturing (then, and if
// creation fails, the two launches run in order on the caller's stream: the
// same kernels and results).  One mutex keeps each record/wait/launch/record/
// wait sequence whole when several host threads launch.
struct AuxStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool tried = false;
};
constexpr int kMaxDevices = 64;
std::mutex g_aux_mu;
AuxStream g_aux[kMaxDevices];

AuxStream *aux_stream(hipStream_t s) { // called with g_aux_mu held
    hipDevice_t dev = 0; // the device of the caller's stream, where its kernels run
    if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    AuxStream &a = g_aux[dev];
    if (a.s) return &a;
    if (a.tried) return nullptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
    a.tried = true;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    bool ok = hipStreamCreateWithFlags(&a.s, hipStreamNonBlocking) == hipSuccess;
    if (!ok) a.s = nullptr;
    ok = ok && hipEventCreateWithFlags(&a.fork, hipEventDisableTiming) == hipSuccess &&
         hipEventCreateWithFlags(&a.join, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        if (a.fork) (void)hipEventDestroy(a.fork);
        if (a.s) (void)hipStreamDestroy(a.s);
        a = AuxStream{};
        a.tried = true;
    }
    if (cur != dev) (void)hipSetDevice(cur);
    return ok ? &a : nullptr;
}

// on_aux(stream) after the work queued on s so far, beside on_s(s); s then
// waits for both.
template <class FA, class FS>
hipError_t fork_join(hipStream_t s, FA on_aux, FS on_s) {
    std::lock_guard<std::mutex> lock(g_aux_mu);
    AuxStream *a = aux_stream(s);
    if (!a) {
        on_aux(s);
        on_s(s);
        return hipGetLastError();
    }
    hipError_t e = hipEventRecord(a->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(a->s, a->fork, 0);
    if (e != hipSuccess) return e;
    on_aux(a->s);
    const hipError_t el = hipGetLastError();
    on_s(s);
    const hipError_t el2 = hipGetLastError();
    e = hipEventRecord(a->join, a->s);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, a->join, 0);
    return e != hipSuccess ? e : el != hipSuccess ? el : el2;
}

// Dynamic LDS that brings a workgroup of chunk_inter_kernel<K, MODE, NW> to
// more than half of a compute unit's 160 KiB, so that no two share one: the
// split's concurrent pair then spreads one workgroup per compute unit instead
// of packing small workgroups of both kernels onto the same ones (two-wave
// workgroups at K = 64 ran 40-60 % slower per chunk packed so).
template <int K, int MODE, int NW>
size_t half_cu_pad() {
    static const size_t pad = [] {
        hipFuncAttributes a{};
        if (hipFuncGetAttributes(&a, reinterpret_cast<const void *>(&chunk_inter_kernel<K, MODE, NW>)) != hipSuccess)
            return size_t(0);
        constexpr size_t half = 80 * 1024 + 256;
        return a.sharedSizeBytes >= half ? size_t(0) : half - a.sharedSizeBytes;
    }();
    return pad;
}

// Pass 3 (or the only pass) of chunk-inter in mode MODE over segments
// seg_base .. seg_base + nseg - 1, with lds bytes of dynamic LDS.
template <int K, int V, int MODE>
void launch_inter(const ChunkParams &p, hipStream_t s, int nseg, int seg_base, size_t lds = 0) {
    constexpr int NWV = inter_nwv(K, V), VSW = 16 * NWV;
    hipLaunchKernelGGL((chunk_inter_kernel<K, MODE, NWV>), dim3(p.B * p.HV * nseg * (V / VSW)), dim3(64 * NWV), lds,
                       s, p, nseg, seg_base);
}

// phases: 1 intra; 2 inter with the output, 4 training (every segment's P and
// the backward's per-chunk states and v_new; with 2 also the output), 8
// output plus v_new and the per-chunk states (2, 4, 8 run every inter pass the
// shape needs); one pass of the segmented inter alone (phase diagnostics):
// 16 segment summaries (with the split, beside segment 0's walk), 32 chain,
// 64 output pass.  The inference output (2 alone, or 16 / 32 / 64) takes the
// split where split_segments allows it; the training and states runs keep
// uniform segments, whose transitions the backward reuses.
template <int K, int V>
hipError_t launch_chunk_t(const ChunkParams &p0, hipStream_t s, int phases) {
    constexpr int NWV = inter_nwv(K, V), VSW = 16 * NWV; // waves and value columns per sequential workgroup
    // Pass 1 (segment summaries: no output, so no q exp(G) or A_qk in LDS) at
    // K = 128 takes 128 columns (V or P) per workgroup of eight waves: the
    // chunk's W and Kd^T are copied once for twice the columns, and two waves
    // per SIMD still fit its registers.
    constexpr int NWL = (K == 128 && V % 128 == 0) ? 8 : NWV, VSWL = 16 * NWL;
    const dim3 blk(64 * NWV), blkl(64 * NWL);
    const int seqs = p0.B * p0.HV;
    const bool infer = (phases & 112) || (phases & 14) == 2;
    ChunkParams ps;
    const bool split = infer && split_segments(p0, NWL == 8, &ps);
    const ChunkParams &p = split ? ps : p0;
    auto summaries = [&](int nl) -> hipError_t { // pass 1 over segments 0 .. nl - 1 (uniform)
        hipLaunchKernelGGL((chunk_inter_kernel<K, kInterLocal, NWL>), dim3(seqs * nl * ((V + K) / VSWL)), blkl, 0, s,
                           p, nl, 0);
        return hipGetLastError();
    };
    auto first_pass = [&]() -> hipError_t { // pass 1, or the split's segment 0 beside it
        if (!split) return p.NSEG > 1 ? summaries(p.NSEG - 1) : hipSuccess;
        return fork_join(
            s, [&](hipStream_t sa) { launch_inter<K, V, kInterOut>(p, sa, 1, 0, half_cu_pad<K, kInterOut, NWV>()); },
            [&](hipStream_t sm) {
                const size_t lds = half_cu_pad<K, kInterLocal, NWL>();
                hipLaunchKernelGGL((chunk_inter_kernel<K, kInterLocal, NWL>),
                                   dim3(seqs * (p.NSEG - 2) * ((V + K) / VSWL)), blkl, lds, sm, p, p.NSEG - 2, 1);
            });
    };
    auto chain = [&]() -> hipError_t {
        hipLaunchKernelGGL((chunk_chain_kernel<K, NWV>), dim3(seqs * (V / VSW)), blk, 0, s, p);
        return hipGetLastError();
    };
    auto output_pass = [&]() -> hipError_t { // pass 3 (split: segments 1 .. NSEG - 1)
        if (split)
            launch_inter<K, V, kInterOut>(p, s, p.NSEG - 1, 1);
        else
            launch_inter<K, V, kInterOut>(p, s, p.NSEG, 0);
        return hipGetLastError();
    };
    hipError_t e = hipSuccess;
    if (phases & 112) {
        if ((phases & 16) && p.NSEG > 1 && (e = first_pass()) != hipSuccess) return e;
        if ((phases & 32) && p.NSEG > 1 && (e = chain()) != hipSuccess) return e;
        if (phases & 64) return output_pass();
        return hipSuccess;
    }
    if (phases & 1) {
        const int nchunks = p.B * p.HV * p.NC;
        if (p.ws_akk) {
            hipLaunchKernelGGL((chunk_intra_kernel<K, V, true>), dim3(nchunks), dim3(512), 0, s, p);
        } else
            hipLaunchKernelGGL((chunk_intra_kernel<K, V, false>), dim3(nchunks), dim3(512), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (phases & 14) {
        if (infer) {
            if (p.NSEG > 1) {
                if ((e = first_pass()) != hipSuccess) return e;
                if ((e = chain()) != hipSuccess) return e;
            }
            return output_pass();
        }
        if (p.NSEG > 1) {
            // the training forward (phases & 4) also takes the last segment's P, which
            // the backward's reverse chain uses
            if ((e = summaries((phases & 4) ? p.NSEG : p.NSEG - 1)) != hipSuccess) return e;
            if ((e = chain()) != hipSuccess) return e;
        }
        if (phases & 8)
            launch_inter<K, V, kInterOutStates>(p, s, p.NSEG, 0);
        else if ((phases & 6) == 6) // the training forward
            launch_inter<K, V, kInterOutTrain>(p, s, p.NSEG, 0);
        else // the backward's states pass
            launch_inter<K, V, kInterStates>(p, s, p.NSEG, 0);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace

bool chunk_supported(int K, int V) {
    return (K == 32 && (V == 32 || V == 64)) || (K == 64 && (V == 64 || V == 96 || V == 128 || V == 256)) ||
           (K == 128 && (V == 64 || V == 128 || V == 192 || V == 256)) || (K == 256 && (V == 128 || V == 256));
}

bool chunk_bwd_supported(int K, int V) { return chunk_supported(K, V); }

template <int K>
hipError_t launch_chunk_states_t(const ChunkParams &p, hipStream_t s) {
    const int nvs = (p.V + 63) / 64;
    const int64_t grid = (int64_t)p.B * p.HV * p.st_chunks * nvs;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL((chunk_states_kernel<K, false>), dim3((unsigned)grid), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || C % p.st_cc == 0) return e; // every j0(n) starts its chunk: nothing in place
    hipLaunchKernelGGL((chunk_states_kernel<K, true>), dim3((unsigned)(p.B * p.HV * p.NC * nvs)), dim3(256),
                       0, s, p);
    return hipGetLastError();
}

hipError_t launch_chunk_states(const ChunkParams &p, hipStream_t s) {
    if (p.st_cc <= 0) return hipSuccess;
    if (p.K == 256) return launch_chunk_states_t<256>(p, s);
    if (p.K == 128) return launch_chunk_states_t<128>(p, s);
    if (p.K == 64) return launch_chunk_states_t<64>(p, s);
    if (p.K == 32) return launch_chunk_states_t<32>(p, s);
    return hipErrorInvalidValue;
}

hipError_t launch_chunk(const ChunkParams &p, hipStream_t s, int phases) {
    if (p.K == 128 && p.V == 128) return launch_chunk_t<128, 128>(p, s, phases);
    if (p.K == 128 && p.V == 192) return launch_chunk_t<128, 192>(p, s, phases);
    if (p.K == 64 && p.V == 96) return launch_chunk_t<64, 96>(p, s, phases);
    if (p.K == 32 && p.V == 32) return launch_chunk_t<32, 32>(p, s, phases);
    if (p.K == 32 && p.V == 64) return launch_chunk_t<32, 64>(p, s, phases);
    if (p.K == 256 && p.V == 256) return launch_chunk_t<256, 256>(p, s, phases);
    if (p.K == 256 && p.V == 128) return launch_chunk_t<256, 128>(p, s, phases);
    if (p.K == 128 && p.V == 256) return launch_chunk_t<128, 256>(p, s, phases);
    if (p.K == 128 && p.V == 64) return launch_chunk_t<128, 64>(p, s, phases);
    if (p.K == 64 && p.V == 64) return launch_chunk_t<64, 64>(p, s, phases);
    if (p.K == 64 && p.V == 128) return launch_chunk_t<64, 128>(p, s, phases);
    if (p.K == 64 && p.V == 256) return launch_chunk_t<64, 256>(p, s, phases);
    return hipErrorInvalidValue;
}

}  // namespace gdn2

using namespace gdn2;

namespace {

struct WsLayout {
    size_t w, qg, u, aqk, kdt, gam, pseg, qseg, total;
};

// Segments per sequence for chunk-inter.  Few long sequences are split so
// that the output pass runs about one workgroup per compute unit (an MI355X
// has 256); a segment keeps at least 4 chunks.  The split only binds where
// the sequences leave most of the chip idle, so the extra passes' work (each
// segment's transition, the chain) costs little beside the shorter walk: at
// 4 value heads x 16 chunks (hidden 256, K = V = 64) chunk-inter takes 57 us
// in 4 segments against 79 us in one.
constexpr int64_t kInterWorkgroups = 256;
constexpr int64_t kMinSegmentChunks = 4;

struct Segments {
    int nseg, segl;
};

Segments inter_segments(int64_t B, int64_t HV, int64_t K, int64_t V, int64_t NC) {
    const int64_t w = (K > 0 && V > 0) ? B * HV * (V / (16 * inter_nwv((int)K, (int)V))) : 0;
    if (w <= 0 || NC <= 0) return {1, (int)NC}; // (K, V) outside the chunk kernels, or no tokens
    int64_t n = kInterWorkgroups / w;
    if (n > NC / kMinSegmentChunks) n = NC / kMinSegmentChunks;
    if (n < 2) return {1, (int)NC};
    const int64_t L = (NC + n - 1) / n;
    return {(int)((NC + L - 1) / L), (int)L};
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

WsLayout ws_layout(int64_t seqs, int64_t NC, int64_t K, int64_t V) {
    const int64_t nchunks = seqs * NC;
    const int64_t nseg = inter_segments(seqs, 1, K, V, NC).nseg;
    const int64_t np = nseg > 1 ? seqs * nseg : 0, nq = np;
    WsLayout L;
    size_t off = 0;
    L.w = off; off = align256(off + sizeof(float) * nchunks * kChunk * K);
    L.qg = off; off = align256(off + sizeof(float) * nchunks * kChunk * K);
    L.u = off; off = align256(off + sizeof(float) * nchunks * kChunk * V);
    L.aqk = off; off = align256(off + sizeof(float) * nchunks * kChunk * kChunk);
    L.kdt = off; off = align256(off + sizeof(float) * nchunks * kChunk * K);
    L.gam = off; off = align256(off + sizeof(float) * nchunks * K);
    L.pseg = off; off = align256(off + sizeof(float) * np * K * K);
    L.qseg = off; off = align256(off + sizeof(float) * nq * K * V);
    L.total = off;
    return L;
}

WsLayout ws_layout(const gdn2_chunk_args *a) {
    return ws_layout(a->batch * a->num_v_heads, (a->seq_len + kChunk - 1) / kChunk, a->head_dim, a->head_v_dim);
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" size_t gdn2_chunk_workspace_bytes(const gdn2_chunk_args *a) {
    if (!a || a->batch <= 0 || a->num_v_heads <= 0 || a->seq_len <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0)
        return 0;
    return ws_layout(a).total;
}

namespace gdn2 {

// Checks shared by the chunked forward and backward; fills p's shapes and
// strides.  Limits: the (K, V) pairs of chunk_supported, 16-byte aligned q,
// k, b with strides that are multiples of 4 elements, token strides within
// the range-checked row loads.
gdn2_status chunk_setup(const gdn2_chunk_args *a, const char *who, bool need_out, ChunkParams *p) {
    const std::string w = std::string(who) + ": ";
    if (!a) return fail(GDN2_EINVAL, w + "null args");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->state || (need_out && !a->out))
        return fail(GDN2_EINVAL, w + "null tensor pointer");
    if (a->batch <= 0 || a->num_heads <= 0 || a->num_v_heads <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0 ||
        a->seq_len < 0)
        return fail(GDN2_EINVAL, w + "invalid dimensions");
    if (a->chunk_size <= 0) return fail(GDN2_EINVAL, w + "chunk_size must be > 0");
    if (a->num_v_heads % a->num_heads != 0) return fail(GDN2_EINVAL, w + "num_v_heads must be a multiple of num_heads");
    if (!chunk_supported((int)a->head_dim, (int)a->head_v_dim))
        return fail(GDN2_NOT_APPLICABLE, w + "(K, V) outside the chunk kernels' instances");
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->b) || (a->stride_qk_b % 4) || (a->stride_qk_h % 4) ||
        (a->stride_qk_t % 4))
        return fail(GDN2_NOT_APPLICABLE, w + "q/k/b need 16-byte aligned rows");
    // The intra kernel reads a chunk's rows through 32-bit range-checked
    // buffer offsets: token rows must not overlap, and one chunk of rows must
    // span less than 2 GiB.
    if (a->stride_qk_t < a->head_dim || a->stride_vw_t < a->head_v_dim ||
        ((kChunk - 1) * a->stride_qk_t + a->head_dim) * 4 >= (int64_t(1) << 31) ||
        ((kChunk - 1) * a->stride_vw_t + a->head_v_dim) * 4 >= (int64_t(1) << 31))
        return fail(GDN2_NOT_APPLICABLE, w + "token strides outside the chunk kernels' range");
    // The output rows of a chunk go through a range-checked buffer resource too.
    if (need_out && (a->stride_o_t < a->head_v_dim ||
                     ((kChunk - 1) * a->stride_o_t + a->head_v_dim) * 4 >= (int64_t(1) << 31)))
        return fail(GDN2_NOT_APPLICABLE, w + "output token stride outside the chunk kernels' range");
    *p = ChunkParams{};
    p->q = a->q; p->k = a->k; p->g = a->g; p->b = a->b; p->v = a->v; p->w = a->w;
    p->state = a->state; p->out = a->out;
    p->B = (int)a->batch; p->HV = (int)a->num_v_heads; p->rep = (int)(a->num_v_heads / a->num_heads);
    p->T = (int)a->seq_len; p->K = (int)a->head_dim; p->V = (int)a->head_v_dim;
    p->NC = (int)((a->seq_len + kChunk - 1) / kChunk);
    p->sqb = a->stride_qk_b; p->sqh = a->stride_qk_h; p->sqt = a->stride_qk_t;
    p->svb = a->stride_vw_b; p->svh = a->stride_vw_h; p->svt = a->stride_vw_t;
    p->sob = a->stride_o_b; p->soh = a->stride_o_h; p->sot = a->stride_o_t;
    p->scale = (float)a->scale;
    const Segments sg = inter_segments(p->B * p->HV, 1, p->K, p->V, p->NC);
    p->NSEG = sg.nseg;
    p->SEGL = sg.segl;
    p->NSLOT = sg.nseg; // uniform runs; the inference split keeps these slots
    p->SEG0 = p->SLOT0 = 0;
    return GDN2_OK;
}

size_t chunk_fwd_ws_bytes(const gdn2_chunk_args *a) { return ws_layout(a).total; }

int chunk_segments(int64_t seqs, int64_t K, int64_t V, int64_t NC) { return inter_segments(seqs, 1, K, V, NC).nseg; }

void chunk_bind_ws(const gdn2_chunk_args *a, char *ws, ChunkParams *p) {
    const WsLayout L = ws_layout(a);
    p->ws_w = reinterpret_cast<float *>(ws + L.w);
    p->ws_qg = reinterpret_cast<float *>(ws + L.qg);
    p->ws_u = reinterpret_cast<float *>(ws + L.u);
    p->ws_aqk = reinterpret_cast<float *>(ws + L.aqk);
    p->ws_kdt = reinterpret_cast<float *>(ws + L.kdt);
    p->ws_gam = reinterpret_cast<float *>(ws + L.gam);
    p->ws_pseg = reinterpret_cast<float *>(ws + L.pseg);
    p->ws_qseg = reinterpret_cast<float *>(ws + L.qseg);
}

}  // namespace gdn2

// fused_chunk_forward (src/kernel/chunk_cube.rs:781-952) / chunk_wy_forward
// (src/forward.rs:44-278).  phases: 1 intra, 2 inter, 8 inter that also
// writes v_new and the per-chunk states.
static gdn2_status chunk_call(const gdn2_chunk_args *a, gdn2_stream_t stream, int phases, const char *who,
                              float *v_new = nullptr, float *states = nullptr, int st_cc = 0) {
    ChunkParams p;
    const gdn2_status st = chunk_setup(a, who, true, &p);
    if (st != GDN2_OK) return st;
    if (a->seq_len == 0) return GDN2_OK;
    if (!a->workspace || a->workspace_bytes < chunk_fwd_ws_bytes(a) || (reinterpret_cast<uintptr_t>(a->workspace) & 255u))
        return fail(GDN2_EINVAL, std::string(who) + ": workspace missing, too small or not 256-byte aligned");
    chunk_bind_ws(a, static_cast<char *>(a->workspace), &p);
    p.ws_vn = v_new;
    p.ws_sn = states;
    if (st_cc) {
        p.st_cc = st_cc;
        p.st_chunks = (int)(a->seq_len / st_cc);
    }
    GDN2_HIP_CHECK(launch_chunk(p, (hipStream_t)stream, phases));
    if (st_cc) GDN2_HIP_CHECK(launch_chunk_states(p, (hipStream_t)stream));
    return GDN2_OK;
}

extern "C" gdn2_status gdn2_chunk_fwd_f32(const gdn2_chunk_args *a, gdn2_stream_t stream) {
    return chunk_call(a, stream, 3, "gdn2_chunk_fwd_f32");
}

extern "C" gdn2_status gdn2_chunk_intra_f32(const gdn2_chunk_args *a, gdn2_stream_t stream) {
    return chunk_call(a, stream, 1, "gdn2_chunk_intra_f32");
}

extern "C" gdn2_status gdn2_chunk_inter_f32(const gdn2_chunk_args *a, gdn2_stream_t stream) {
    return chunk_call(a, stream, 2, "gdn2_chunk_inter_f32");
}

extern "C" int64_t gdn2_chunk_segments(const gdn2_chunk_args *a) {
    if (!a || a->batch <= 0 || a->num_v_heads <= 0 || a->seq_len <= 0 || a->head_dim <= 0 || a->head_v_dim <= 0)
        return 0;
    return chunk_segments(a->batch * a->num_v_heads, a->head_dim, a->head_v_dim, (a->seq_len + kChunk - 1) / kChunk);
}

extern "C" gdn2_status gdn2_chunk_inter_pass_f32(const gdn2_chunk_args *a, int pass, gdn2_stream_t stream) {
    if (pass < 1 || pass > 3) return fail(GDN2_EINVAL, "gdn2_chunk_inter_pass_f32: pass must be 1, 2 or 3");
    return chunk_call(a, stream, 8 << pass, "gdn2_chunk_inter_pass_f32");
}

// The whole tuple of fused_chunk_forward (src/kernel/chunk_cube.rs:781-952):
// out and the state as gdn2_chunk_fwd_f32, plus v_new and the state entering
// every chunk, which it returns for training.
extern "C" gdn2_status gdn2_chunk_fwd_states_f32(const gdn2_chunk_args *a, float *v_new, float *states,
                                                 gdn2_stream_t stream) {
    const char *who = "gdn2_chunk_fwd_states_f32";
    if (!a) return fail(GDN2_EINVAL, std::string(who) + ": null args");
    if (a->seq_len > 0 && (!v_new || !states)) return fail(GDN2_EINVAL, std::string(who) + ": null v_new or states");
    if (a->chunk_size == kChunk) return chunk_call(a, stream, 9, who, v_new, states);
    // smaller caller chunks: the reference's limits (chunk_size <= 64, T a
    // multiple of it, src/kernel/chunk_cube.rs:795-800)
    if (a->chunk_size <= 0 || a->chunk_size > kChunk)
        return fail(GDN2_NOT_APPLICABLE, std::string(who) + ": chunk_size must be in [1, 64]");
    if (a->seq_len % a->chunk_size != 0)
        return fail(GDN2_NOT_APPLICABLE, std::string(who) + ": seq_len must be a multiple of chunk_size");
    return chunk_call(a, stream, 9, who, v_new, states, (int)a->chunk_size);
}

// Layer kernels around the recurrence: the projection epilogue (short conv,
// SiLU, gates, L2 norm; written head-major [B, H, T, D], as the reference's
// project() returns them, so that each chunk of a head is one contiguous
// block), the conv-cache update, the gated RMSNorm and a row fill for Linear
// biases.
#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {
namespace {

__device__ __forceinline__ float sigmoid_(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_(float x) { return x / (1.0f + __expf(-x)); }
// burn's softplus(x, beta = 1) = ln(1 + e^x); above 20 the f32 value is x.
__device__ __forceinline__ float softplus_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
// d silu(x) / dx = s (1 + x (1 - s)), s = sigmoid(x)
__device__ __forceinline__ float dsilu_(float x) {
    const float sg = sigmoid_(x);
    return sg * (1.0f + x * (1.0f - sg));
}

// Causal depthwise conv with four taps at token t of one sequence
// (src/short_conv.rs:22-65): y = sum_i xpad[t + i] * w[c, i] with
// xpad = cat(cache, x); without a cache the first token is replicated.
// `x` points at the sequence's token 0 in column c (row stride ldx).
__device__ __forceinline__ float conv4(const float *x, int64_t ldx, int t, const float *cache, int64_t n_ch,
                                       const float *w) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tp = t + i - 3;
        float xv;
        if (tp >= 0)
            xv = x[(int64_t)tp * ldx];
        else if (cache)
            xv = cache[(int64_t)(3 + tp) * n_ch];
        else
            xv = x[0];
        acc += xv * w[i];
    }
    return acc;
}

// One workgroup per (batch row, block of kProjTB tokens, head), so that every
// raw projection element is read once (plus three tokens of conv history per
// thread's run of tokens) and every output is a contiguous head-major block.
// Key heads (blockIdx.y < H) produce q, k, g, b of their head; the L2 norms
// over K need the whole head, so q and k pass through LDS (heads up to 256
// channels; wider heads keep them in the output rows instead).  Value heads
// produce v and w.  A thread owns one channel and a run of kProjRun tokens,
// sliding the four-tap window along it.  Blocks of 32 tokens give a head of
// 128 channels exactly one (channel, run) per thread, so that every load of a
// thread is requested at once (64-token blocks took two rounds: 876 against
// 717 us at B = 8, T = 4096).
constexpr int kProjTB = 32, kProjRun = 16, kProjLdsMaxK = 256;

// xpad row of token tt (tt < 0: the cache, or token 0 replicated) in column c
__device__ __forceinline__ float conv_row(const float *col, int64_t ld, int tt, const float *cache, int64_t n_ch) {
    if (tt >= 0) return col[(int64_t)tt * ld];
    return cache ? cache[(int64_t)(3 + tt) * n_ch] : col[0];
}

__global__ __launch_bounds__(256) void project_kernel(ProjectParams p) {
    extern __shared__ float sm[];
    const int nb = (p.T + kProjTB - 1) / kProjTB;
    const int bi = blockIdx.x / nb, t0 = (blockIdx.x % nb) * kProjTB;
    const int head = blockIdx.y;
    const int tn = min(kProjTB, p.T - t0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool sc = p.use_short_conv != 0;
    const int kd = p.H * p.K, vd = p.HV * p.V;
    const float *Y0 = p.Y + (int64_t)bi * p.T * p.ldY;  // token 0 of this sequence
    constexpr int NRUN = kProjTB / kProjRun;
    if (head < p.H) {
        const int h = head, K = p.K, K1 = K + 1;
        const int64_t ob = ((int64_t)bi * p.H + h) * p.T * K;  // [B, H, T, K] row of token 0
        // staging of the activated q, k of token t0 + tl, channel c
        const bool lds = K <= kProjLdsMaxK;
        float *sq = lds ? sm : p.q + ob + (int64_t)t0 * K, *sk = lds ? sm + kProjTB * K1 : p.k + ob + (int64_t)t0 * K;
        const int ld = lds ? K1 : K;
        for (int e = tid; e < K * NRUN; e += 256) {
            const int c = e % K, run = e / K, gc = h * K + c;
            const int ta = t0 + run * kProjRun, tb = min(t0 + tn, ta + kProjRun);
            if (ta >= tb) continue;
            const float *qc = Y0 + p.off_q + gc, *kc = Y0 + p.off_k + gc;
            float wq[4] = {0.f, 0.f, 0.f, 0.f}, wk[4] = {0.f, 0.f, 0.f, 0.f};
            float q1 = 0.f, q2 = 0.f, q3 = 0.f, k1 = 0.f, k2 = 0.f, k3 = 0.f;  // x(t-3), x(t-2), x(t-1)
            if (sc) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wq[i] = p.q_conv_w[4 * gc + i];
                    wk[i] = p.k_conv_w[4 * gc + i];
                }
                const int64_t cb = (int64_t)bi * 3 * kd + gc;
                const float *cq = p.conv_q_in ? p.conv_q_in + cb : nullptr;
                const float *ck = p.conv_k_in ? p.conv_k_in + cb : nullptr;
                q1 = conv_row(qc, p.ldY, ta - 3, cq, kd); q2 = conv_row(qc, p.ldY, ta - 2, cq, kd);
                q3 = conv_row(qc, p.ldY, ta - 1, cq, kd);
                k1 = conv_row(kc, p.ldY, ta - 3, ck, kd); k2 = conv_row(kc, p.ldY, ta - 2, ck, kd);
                k3 = conv_row(kc, p.ldY, ta - 1, ck, kd);
            }
            const float dtb = p.dt_bias[gc], A = expf(p.a_log[h]);
            const float dfs = p.decay_factors ? sigmoid_(p.decay_factors[gc]) * p.one_minus_min_decay : 0.f;
            // the run's loads first, all in flight together (rows past the end read row ta)
            float xqs[kProjRun], xks[kProjRun], fs[kProjRun], bs[kProjRun];
#pragma unroll
            for (int j = 0; j < kProjRun; ++j) {
                const int t = ta + j < tb ? ta + j : ta;
                const int64_t row = (int64_t)t * p.ldY;
                xqs[j] = qc[row];
                xks[j] = kc[row];
                fs[j] = p.F[((int64_t)bi * p.T + t) * p.ldF + gc];
                bs[j] = Y0[row + p.off_b + gc];
            }
#pragma unroll
            for (int j = 0; j < kProjRun; ++j) {
                const int t = ta + j;
                if (t >= tb) continue;  // (only the tail of the last block)
                const float xq = xqs[j], xk = xks[j];
                float uq = xq, uk = xk;
                if (sc) {
                    uq = q1 * wq[0] + q2 * wq[1] + q3 * wq[2] + xq * wq[3];
                    uk = k1 * wk[0] + k2 * wk[1] + k3 * wk[2] + xk * wk[3];
                    q1 = q2; q2 = q3; q3 = xq;
                    k1 = k2; k2 = k3; k3 = xk;
                }
                sq[(t - t0) * ld + c] = silu_(uq);
                sk[(t - t0) * ld + c] = silu_(uk);
                // g, b (src/module.rs:417-443, :470-472)
                float gv = -A * softplus_(fs[j] + dtb);
                if (p.decay_factors) gv = logf(dfs * expf(gv) + p.min_decay);
                float bv = sigmoid_(bs[j]);
                if (p.allow_neg_eigval) bv *= 2.0f;
                p.g[ob + (int64_t)t * K + c] = gv;
                p.b[ob + (int64_t)t * K + c] = bv;
            }
        }
        __syncthreads();
        // L2 norm per token over the head's K channels (src/l2norm.rs:13-16): a wave per token
        for (int tl = wave; tl < tn; tl += 4) {
            float ssq = 0.f, ssk = 0.f;
            for (int c = lane; c < K; c += 64) {
                const float a = sq[tl * ld + c], bq = sk[tl * ld + c];
                ssq += a * a;
                ssk += bq * bq;
            }
            ssq = wave_sum(ssq);
            ssk = wave_sum(ssk);
            const float nq = 1.0f / sqrtf(ssq + 1e-6f), nk = 1.0f / sqrtf(ssk + 1e-6f);
            const int64_t o = ob + (int64_t)(t0 + tl) * K;
            for (int c = lane; c < K; c += 64) {
                const float a = sq[tl * ld + c], bq = sk[tl * ld + c];
                p.q[o + c] = a * nq;
                p.k[o + c] = bq * nk;
            }
        }
    } else {
        const int hv = head - p.H, V = p.V;
        const int64_t ob = ((int64_t)bi * p.HV + hv) * p.T * V;  // [B, HV, T, V] row of token 0
        for (int e = tid; e < V * NRUN; e += 256) {
            const int c = e % V, run = e / V, gc = hv * V + c;
            const int ta = t0 + run * kProjRun, tb = min(t0 + tn, ta + kProjRun);
            if (ta >= tb) continue;
            const float *vc = Y0 + p.off_v + gc;
            float wv[4] = {0.f, 0.f, 0.f, 0.f}, v1 = 0.f, v2 = 0.f, v3 = 0.f;
            if (sc) {
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[i] = p.v_conv_w[4 * gc + i];
                const float *cv = p.conv_v_in ? p.conv_v_in + (int64_t)bi * 3 * vd + gc : nullptr;
                v1 = conv_row(vc, p.ldY, ta - 3, cv, vd); v2 = conv_row(vc, p.ldY, ta - 2, cv, vd);
                v3 = conv_row(vc, p.ldY, ta - 1, cv, vd);
            }
            float xvs[kProjRun], xws[kProjRun];
#pragma unroll
            for (int j = 0; j < kProjRun; ++j) {
                const int t = ta + j < tb ? ta + j : ta;
                const int64_t row = (int64_t)t * p.ldY;
                xvs[j] = vc[row];
                xws[j] = Y0[row + p.off_w + gc];
            }
#pragma unroll
            for (int j = 0; j < kProjRun; ++j) {
                const int t = ta + j;
                if (t >= tb) continue;
                const float xv = xvs[j];
                float uv = xv;
                if (sc) {
                    uv = v1 * wv[0] + v2 * wv[1] + v3 * wv[2] + xv * wv[3];
                    v1 = v2; v2 = v3; v3 = xv;
                }
                p.v[ob + (int64_t)t * V + c] = silu_(uv);
                p.w[ob + (int64_t)t * V + c] = sigmoid_(xws[j]);
            }
        }
    }
}

// The reference's GVA layout: a [B, H, T, rep, K] repeat read as
// [B, H rep, T, K].  Destination (b, hv, t2, c), hv = h rep + a, reads source
// (b, h, (a T + t2) / rep, c); one thread per destination element of the four
// tensors.
__global__ __launch_bounds__(256) void gva_expand_kernel(GvaParams p) {
    const int64_t n = p.B * p.H * p.rep * p.T * p.K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < 4 * n; i += (int64_t)gridDim.x * 256) {
        const int which = (int)(i / n);
        const int64_t e = i % n;
        const int64_t c = e % p.K, t2 = (e / p.K) % p.T, hv = (e / (p.K * p.T)) % (p.H * p.rep);
        const int64_t bi = e / (p.K * p.T * p.H * p.rep);
        const int64_t h = hv / p.rep, a = hv % p.rep, t = (a * p.T + t2) / p.rep;
        p.dst[which][e] = p.src[which][((bi * p.H + h) * p.T + t) * p.K + c];
    }
}

// Adjoint of gva_expand_kernel: key element (b, h, t, c) went to the places
// f = t rep + j (j < rep) of the [T rep] run of head h, i.e. value head
// h rep + f / T at time f % T; their gradients are summed in j order.
__global__ __launch_bounds__(256) void gva_fold_kernel(GvaParams p) {
    const int64_t n = p.B * p.H * p.T * p.K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < 4 * n; i += (int64_t)gridDim.x * 256) {
        const int which = (int)(i / n);
        const int64_t e = i % n;
        const int64_t c = e % p.K, t = (e / p.K) % p.T, h = (e / (p.K * p.T)) % p.H, bi = e / (p.K * p.T * p.H);
        float acc = 0.f;
        for (int j = 0; j < p.rep; ++j) {
            const int64_t f = t * p.rep + j, hv = h * p.rep + f / p.T, t2 = f % p.T;
            acc += p.src[which][((bi * p.H * p.rep + hv) * p.T + t2) * p.K + c];
        }
        p.dst[which][e] = acc;
    }
}

// New conv caches: xpad[T .. T + 3) = the last three pre-conv tokens.
__global__ __launch_bounds__(256) void conv_cache_kernel(ConvCacheParams p) {
    const int64_t nq = (int64_t)p.B * 3 * p.kd, nv = (int64_t)p.B * 3 * p.vd;
    const int64_t total = 2 * nq + nv;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t idx = i;
        const float *in;
        float *out;
        int64_t n, off;
        if (idx < nq) {
            in = p.in_q; out = p.out_q; n = p.kd; off = p.off_q;
        } else if (idx < 2 * nq) {
            idx -= nq; in = p.in_k; out = p.out_k; n = p.kd; off = p.off_k;
        } else {
            idx -= 2 * nq; in = p.in_v; out = p.out_v; n = p.vd; off = p.off_v;
        }
        const int64_t c = idx % n, j = (idx / n) % 3, bi = idx / (3 * n);
        const int64_t tp = p.T + j - 3;
        float val;
        if (tp >= 0)
            val = p.Y[(bi * p.T + tp) * p.ldY + off + c];
        else if (in)
            val = in[(bi * 3 + p.T + j) * n + c];
        else
            val = p.Y[(bi * p.T) * p.ldY + off + c];
        out[(bi * 3 + j) * n + c] = val;
    }
}

constexpr int kNormHeld = 4; // row elements per lane held in registers (V <= 256)

// rms_norm_gate_per_head (src/module.rs:501-517): one wave per (token, value head).
__global__ __launch_bounds__(256) void rmsnorm_gate_kernel(float *out, int64_t ld_out, const float *x, int64_t ld_x,
                                                           const float *gate, int64_t ld_gate, const float *gate_bias,
                                                           const float *weight, int64_t rows, int HV, int V, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t m = row / HV;
    const int hv = (int)(row % HV);
    const float *xr = x + m * ld_x + (int64_t)hv * V;
    const float *gr = gate + m * ld_gate + (int64_t)hv * V;
    float *orow = out + m * ld_out + (int64_t)hv * V;
    const float *br = gate_bias ? gate_bias + (int64_t)hv * V : nullptr;
    if (V <= 64 * kNormHeld) {
        // every operand of the row requested before the reduction: one memory
        // round trip per row instead of two
        float xv[kNormHeld], gv[kNormHeld], wv[kNormHeld];
#pragma unroll
        for (int u = 0; u < kNormHeld; ++u) {
            const int i = lane + 64 * u;
            const bool in = i < V;
            xv[u] = in ? xr[i] : 0.f;
            gv[u] = in ? gr[i] + (br ? br[i] : 0.f) : 0.f;
            wv[u] = in ? weight[i] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < kNormHeld; ++u) ss += xv[u] * xv[u];
        ss = wave_sum(ss);
        const float rms = sqrtf(ss / (float)V + eps);
#pragma unroll
        for (int u = 0; u < kNormHeld; ++u) {
            const int i = lane + 64 * u;
            if (i < V) orow[i] = xv[u] / rms * wv[u] * silu_(gv[u]);
        }
        return;
    }
    float ss = 0.f;
    for (int i = lane; i < V; i += 64) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)V + eps);
    for (int i = lane; i < V; i += 64) orow[i] = xr[i] / rms * weight[i] * silu_(gr[i] + (br ? br[i] : 0.f));
}

// The layer's two rank-R up-projections for a few rows (the decode step), in
// one launch instead of two GEMM calls:
//   F[m, n] = sum_j Y[m, off_f0 + j] F1[j, n]              n < kd
//   G[m, n] = sum_j Y[m, off_g0 + j] G1[j, n] (+ bias[n])  n < vd
// Workgroup = (64 columns of F or of G, 16 rows); wave w computes the 16 x 16
// tile of columns 16 w .. 16 w + 15 with v_mfma_f32_16x16x4_f32, operands
// loaded straight into registers (no LDS): lane (g, r) holds row r's
// Y[16 u + 4 g .. + 3] (one float4 per 16-wide block u of j) and its
// column's F1 / G1 [16 u + 4 g + s] (s < 4), all issued before the first
// product.  Requires Y, ldY and the offsets 16-byte aligned (host check).
template <int R>
__global__ __launch_bounds__(256) void lowrank_up_kernel(LowRankParams p) {
    constexpr int NU = R / 16;
    const int nft = (p.kd + 63) / 64;
    const bool isf = (int)blockIdx.x < nft;
    const int N = isf ? p.kd : p.vd;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 15, lg = lane >> 4;
    const int c = 64 * (isf ? blockIdx.x : blockIdx.x - nft) + 16 * wave + lr; // this lane's column
    const int m0 = 16 * blockIdx.y;
    const bool rok = m0 + lr < p.M, cok = c < N;
    const float *arow = p.Y + (isf ? p.off_f0 : p.off_g0) + (int64_t)(rok ? m0 + lr : 0) * p.ldY + 4 * lg;
    const float *bcol = (isf ? p.F1 : p.G1) + (int64_t)(4 * lg) * N + (cok ? c : 0);
    floatx4 a[NU], b[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        a[u] = *reinterpret_cast<const floatx4 *>(arow + 16 * u);
#pragma unroll
        for (int s = 0; s < 4; ++s) b[u][s] = bcol[(int64_t)(16 * u + s) * N];
    }
    // keep every load ahead of the products: left alone, the scheduler
    // interleaves them and each product waits a full memory round trip
    __builtin_amdgcn_sched_barrier(0);
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = mfma16(rok ? a[u][s] : 0.f, b[u][s], acc);
    if (!cok) return;
    const float bias = (!isf && p.g_bias) ? p.g_bias[c] : 0.f;
    float *O = (isf ? p.F : p.G) + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) // accumulator rows 4 g + i, column r
        if (m0 + 4 * lg + i < p.M) O[(int64_t)(m0 + 4 * lg + i) * N] = acc[i] + bias;
}

// Reads n floats (float4 loads, grid-stride) so that earlier data leaves the
// caches without leaving dirty lines behind; the sum is stored only if it
// equals a value it never takes, which keeps every load.
__global__ __launch_bounds__(256) void cache_sweep_kernel(const float *__restrict__ buf, int64_t n4, float *sink) {
    const floatx4 *b = reinterpret_cast<const floatx4 *>(buf);
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) acc += b[i];
    const float t = acc[0] + acc[1] + acc[2] + acc[3];
    if (t == -1.5e38f) sink[0] = t;
}

__global__ __launch_bounds__(256) void fill_rows_kernel(float *y, int64_t ld, const float *row, int64_t M, int64_t N) {
    const int64_t total = M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / N, c = i % N;
        y[r * ld + c] = row ? row[c] : 0.0f;
    }
}


// ---------------------------------------------------------------------------
// Backward (the adjoints of the kernels above)
// ---------------------------------------------------------------------------

// Gated RMSNorm adjoint, one wave per (token, value head) row.  With
// r = (mean O^2 + eps)^-1/2, n = O r, z = silu(G), y = n w z:
//   dn = dy w z,  dO = r dn - O r^3 (sum dy w z O) / V,
//   dG = dy n w silu'(G),  weight-gradient terms dy n z.
__global__ __launch_bounds__(256) void rmsnorm_gate_bwd_kernel(NormBwdParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int64_t o = row * p.V;
    // gate bias of this row's value head (row = token * HV + head)
    const float *gb = p.gate_bias ? p.gate_bias + (row % p.HV) * p.V : nullptr;
    float s1 = 0.f, s2 = 0.f;
    for (int i = lane; i < p.V; i += 64) {
        const float x = p.O[o + i];
        s1 += x * x;
        s2 += p.dy[o + i] * p.weight[i] * silu_(p.G[o + i] + (gb ? gb[i] : 0.f)) * x;
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float r = 1.0f / sqrtf(s1 / (float)p.V + p.eps);
    const float c3 = r * r * r * s2 / (float)p.V;
    for (int i = lane; i < p.V; i += 64) {
        const float x = p.O[o + i], gt = p.G[o + i] + (gb ? gb[i] : 0.f), dyv = p.dy[o + i], w = p.weight[i];
        const float z = silu_(gt), n = x * r;
        p.y[o + i] = n * w * z;
        p.dO[o + i] = r * dyv * w * z - x * c3;
        p.dG[o + i] = dyv * n * w * dsilu_(gt);
        p.dy[o + i] = dyv * n * z;
    }
}

// Projection epilogue adjoint, one workgroup per token m = b * T + t.
__global__ __launch_bounds__(256) void project_bwd_kernel(ProjectBwdParams p) {
    extern __shared__ float sm[];
    const int kd = p.H * p.K, vd = p.HV * p.V;
    float *s_uq = sm, *s_uk = sm + kd;
    const int64_t m = blockIdx.x;
    const int bi = (int)(m / p.T), t = (int)(m % p.T);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)bi * p.T;
    const float *Y = p.Y + m * p.ldY;
    const float *Y0 = p.Y + m0 * p.ldY;
    float *dY = p.dY + m * p.ldY;
    float *DU = p.DU ? p.DU + m * (int64_t)(2 * kd + vd) : nullptr;
    const bool sc = p.use_short_conv != 0;

    // pre-activations of q and k (conv output or raw projection)
    for (int c = tid; c < kd; c += 256) {
        if (sc) {
            const int64_t cb = (int64_t)bi * 3 * kd + c;
            s_uq[c] = conv4(Y0 + p.off_q + c, p.ldY, t, p.conv_q_in ? p.conv_q_in + cb : nullptr, kd, p.q_conv_w + 4 * c);
            s_uk[c] = conv4(Y0 + p.off_k + c, p.ldY, t, p.conv_k_in ? p.conv_k_in + cb : nullptr, kd, p.k_conv_w + 4 * c);
        } else {
            s_uq[c] = Y[p.off_q + c];
            s_uk[c] = Y[p.off_k + c];
        }
    }
    // gates: g = -e^{A_log} softplus(f + dt_bias) (+ min_decay), b = sigmoid (x2)
    for (int c = tid; c < kd; c += 256) {
        const int64_t o = ((int64_t)bi * p.H + c / p.K) * p.T * p.K + (int64_t)t * p.K + c % p.K;
        const float xg = p.F[m * p.ldF + c] + p.dt_bias[c];
        const float A = expf(p.a_log[c / p.K]);
        const float gp = -A * softplus_(xg);
        float dgv = p.dg[o];
        if (p.decay_factors) {
            // g = ln(sd (1 - m) e^{gp} + m), sd = sigmoid(decay_factors)
            const float sd = sigmoid_(p.decay_factors[c]);
            const float eg = expf(gp);
            const float e = sd * p.one_minus_min_decay * eg;
            const float inv = 1.0f / (e + p.min_decay);
            p.PD[m * kd + c] = dgv * eg * p.one_minus_min_decay * sd * (1.0f - sd) * inv;
            dgv *= e * inv;
        }
        p.PA[m * kd + c] = dgv * gp;
        p.dF[m * kd + c] = -dgv * A * sigmoid_(xg);
        const float sb = sigmoid_(Y[p.off_b + c]);
        dY[p.off_b + c] = p.db[o] * (p.allow_neg_eigval ? 2.0f : 1.0f) * sb * (1.0f - sb);
    }
    // v = silu(conv(v_raw)), w = sigmoid(w_raw)
    for (int c = tid; c < vd; c += 256) {
        const int64_t o = ((int64_t)bi * p.HV + c / p.V) * p.T * p.V + (int64_t)t * p.V + c % p.V;
        float uv;
        if (sc) {
            const int64_t cb = (int64_t)bi * 3 * vd + c;
            uv = conv4(Y0 + p.off_v + c, p.ldY, t, p.conv_v_in ? p.conv_v_in + cb : nullptr, vd, p.v_conv_w + 4 * c);
        } else {
            uv = Y[p.off_v + c];
        }
        const float duv = p.dv[o] * dsilu_(uv);
        if (sc)
            DU[2 * kd + c] = duv;
        else
            dY[p.off_v + c] = duv;
        const float sw = sigmoid_(Y[p.off_w + c]);
        dY[p.off_w + c] = p.dw[o] * sw * (1.0f - sw);
    }
    __syncthreads();
    // L2 norm adjoint per key head (one wave per head): with a = silu(u),
    // nrm = sqrt(sum a^2 + 1e-6), q = a / nrm:
    //   da = (dq - a (sum dq a) / nrm^2) / nrm,  du = da silu'(u)
    for (int h = wave; h < p.H; h += 4) {
        const int64_t o = ((int64_t)bi * p.H + h) * p.T * p.K + (int64_t)t * p.K;
        float sq = 0.f, sk = 0.f, dq_a = 0.f, dk_a = 0.f;
        for (int i = lane; i < p.K; i += 64) {
            const float aq = silu_(s_uq[h * p.K + i]), ak = silu_(s_uk[h * p.K + i]);
            sq += aq * aq;
            sk += ak * ak;
            dq_a += p.dq[o + i] * aq;
            dk_a += p.dk[o + i] * ak;
        }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        dq_a = wave_sum(dq_a);
        dk_a = wave_sum(dk_a);
        const float iq = 1.0f / sqrtf(sq + 1e-6f), ik = 1.0f / sqrtf(sk + 1e-6f);
        const float cq = dq_a * iq * iq, ck = dk_a * ik * ik;
        for (int i = lane; i < p.K; i += 64) {
            const int c = h * p.K + i;
            const float uq = s_uq[c], uk = s_uk[c];
            const float duq = (p.dq[o + i] - silu_(uq) * cq) * iq * dsilu_(uq);
            const float duk = (p.dk[o + i] - silu_(uk) * ck) * ik * dsilu_(uk);
            if (sc) {
                DU[c] = duq;
                DU[kd + c] = duk;
            } else {
                dY[p.off_q + c] = duq;
                dY[p.off_k + c] = duk;
            }
        }
    }
}

// Short-conv adjoint.  One thread per (batch row, channel, block of tblock
// tokens); channels [0, kd) are q, [kd, 2 kd) k, [2 kd, 2 kd + vd) v.  With
// xpad = cat(cache or 3 copies of token 0, x) of length T + 3, u[t] =
// sum_i xpad[t + i] w[i] and the new cache xpad[T .. T + 3):
//   dxpad[j] = sum_{i, 0 <= j - i < T} du[j - i] w[i]  (+ d_cache_out[j - T] for j >= T)
//   dx[s] = dxpad[s + 3]  (+ dxpad[0] + dxpad[1] + dxpad[2] at s = 0 without a cache)
//   d_cache_in[j] = dxpad[j] (j < 3, with a cache),  dw[i] = sum_t du[t] xpad[t + i]
__global__ __launch_bounds__(256) void conv_bwd_kernel(ConvBwdParams p) {
    const int kd = p.kd, vd = p.vd, Ctot = 2 * kd + vd;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int blk = blockIdx.y, bi = blockIdx.z, nblk = gridDim.y;
    if (c >= Ctot) return;
    int cc;
    int64_t col, n;
    const float *wc, *cache, *dco;
    float *dci;
    if (c < kd) {
        cc = c; n = kd; col = p.off_q + cc; wc = p.q_conv_w; cache = p.cache_q; dco = p.d_out_q; dci = p.d_in_q;
    } else if (c < 2 * kd) {
        cc = c - kd; n = kd; col = p.off_k + cc; wc = p.k_conv_w; cache = p.cache_k; dco = p.d_out_k; dci = p.d_in_k;
    } else {
        cc = c - 2 * kd; n = vd; col = p.off_v + cc; wc = p.v_conv_w; cache = p.cache_v; dco = p.d_out_v; dci = p.d_in_v;
    }
    const int64_t cb = (int64_t)bi * 3 * n + cc;  // [B, 3, n] offset of this channel
    if (cache) cache += cb;
    if (dco) dco += cb;
    if (dci) dci += cb;
    const float w[4] = {wc[4 * cc], wc[4 * cc + 1], wc[4 * cc + 2], wc[4 * cc + 3]};
    const int T = p.T;
    const int64_t ldu = Ctot;
    const float *__restrict__ du = p.DU + (int64_t)bi * T * ldu + c;
    const float *__restrict__ x = p.Y + (int64_t)bi * T * p.ldY + col;
    float *__restrict__ dx = p.dY + (int64_t)bi * T * p.ldY + col;
    auto xpad = [&](int j) -> float {
        if (j >= 3) return x[(int64_t)(j - 3) * p.ldY];
        return cache ? cache[(int64_t)j * n] : x[0];
    };
    auto dxpad = [&](int j) -> float {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tt = j - i;
            if (tt >= 0 && tt < T) acc += du[(int64_t)tt * ldu] * w[i];
        }
        if (dco && j >= T) acc += dco[(int64_t)(j - T) * n];
        return acc;
    };
    const int t0 = blk * p.tblock, t1 = min(T, t0 + p.tblock);
    float dw0 = 0.f, dw1 = 0.f, dw2 = 0.f, dw3 = 0.f;
    // sliding windows, one new du and one new x per token:
    //   xw_i = xpad[t + i],  g_i = du[t + i] (0 past T), so that
    //   dw_i += g_0 xw_i  and  dxpad[t + 3] = g_3 w_0 + g_2 w_1 + g_1 w_2 + g_0 w_3
    float xw0 = xpad(t0), xw1 = xpad(t0 + 1), xw2 = xpad(t0 + 2);
    float g0 = t0 < T ? du[(int64_t)t0 * ldu] : 0.f;
    float g1 = t0 + 1 < T ? du[(int64_t)(t0 + 1) * ldu] : 0.f;
    float g2 = t0 + 2 < T ? du[(int64_t)(t0 + 2) * ldu] : 0.f;
#pragma unroll 4
    for (int t = t0; t < t1; ++t) {
        const float xw3 = x[(int64_t)t * p.ldY];
        const float g3 = t + 3 < T ? du[(int64_t)(t + 3) * ldu] : 0.f;
        dw0 += g0 * xw0;
        dw1 += g0 * xw1;
        dw2 += g0 * xw2;
        dw3 += g0 * xw3;
        float d = g3 * w[0] + g2 * w[1] + g1 * w[2] + g0 * w[3];
        if (dco && t + 3 >= T) d += dco[(int64_t)(t + 3 - T) * n];
        if (t == 0 && !cache) d += dxpad(0) + dxpad(1) + dxpad(2);
        dx[(int64_t)t * p.ldY] = d;
        xw0 = xw1;
        xw1 = xw2;
        xw2 = xw3;
        g0 = g1;
        g1 = g2;
        g2 = g3;
    }
    if (blk == 0 && cache && dci)
        for (int j = 0; j < 3; ++j) dci[(int64_t)j * n] = dxpad(j);
    float *wp = p.wpart + ((int64_t)(bi * nblk + blk) * Ctot + c) * 4;
    wp[0] = dw0;
    wp[1] = dw1;
    wp[2] = dw2;
    wp[3] = dw3;
}

// Column sums in two deterministic steps: partial sums over `parts` row
// ranges (one thread per column), then one workgroup per output summing the
// parts, `fold` strided column blocks and `group` adjacent columns.
__global__ __launch_bounds__(256) void colsum_part_kernel(const float *A, int64_t rows, int64_t N, int64_t lda,
                                                          int64_t rows_per, float *part) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= N) return;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per, r1 = min(rows, r0 + rows_per);
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        a0 += A[r * lda + c];
        a1 += A[(r + 1) * lda + c];
        a2 += A[(r + 2) * lda + c];
        a3 += A[(r + 3) * lda + c];
    }
    for (; r < r1; ++r) a0 += A[r * lda + c];
    part[(int64_t)blockIdx.y * N + c] = (a0 + a1) + (a2 + a3);
}

__global__ __launch_bounds__(256) void colsum_final_kernel(const float *part, int parts, int64_t N, int group,
                                                           int fold, float *out, int accumulate) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t stride = N / fold, j = blockIdx.x;
    const int64_t terms = (int64_t)parts * fold * group;
    float acc = 0.f;
    for (int64_t e = tid; e < terms; e += 256) {
        const int64_t i = e % group, f = (e / group) % fold, r = e / ((int64_t)group * fold);
        acc += part[r * N + f * stride + j * group + i];
    }
    acc = wave_sum(acc);
    if (lane == 0) red[wave] = acc;
    __syncthreads();
    if (tid == 0) {
        const float t = (red[0] + red[1]) + (red[2] + red[3]);
        out[j] = accumulate ? out[j] + t : t;
    }
}

int grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (int)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

}  // namespace

size_t project_lds_bytes(int kd) { return sizeof(float) * 2 * (size_t)kd; }

size_t project_tile_lds_bytes(int K) { return K <= kProjLdsMaxK ? sizeof(float) * 2 * (size_t)kProjTB * (K + 1) : 0; }

hipError_t launch_project(const ProjectParams &p, hipStream_t s) {
    const int64_t M = (int64_t)p.B * p.T;
    if (M == 0) return hipSuccess;
    const size_t lds = project_tile_lds_bytes(p.K);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&project_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const int nb = (p.T + kProjTB - 1) / kProjTB;
    hipLaunchKernelGGL(project_kernel, dim3((unsigned)(p.B * nb), (unsigned)(p.H + p.HV)), dim3(256), lds, s, p);
    return hipGetLastError();
}

hipError_t launch_gva_expand(const GvaParams &p, hipStream_t s) {
    const int64_t n = 4 * p.B * p.H * p.rep * p.T * p.K;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(gva_expand_kernel, dim3(grid_for(n)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_gva_fold(const GvaParams &p, hipStream_t s) {
    const int64_t n = 4 * p.B * p.H * p.T * p.K;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(gva_fold_kernel, dim3(grid_for(n)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_conv_cache(const ConvCacheParams &p, hipStream_t s) {
    const int64_t total = (int64_t)p.B * 3 * (2 * p.kd + p.vd);
    hipLaunchKernelGGL(conv_cache_kernel, dim3(grid_for(total)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_gate(float *out, int64_t ld_out, const float *x, int64_t ld_x, const float *gate,
                               int64_t ld_gate, const float *gate_bias, const float *weight, int64_t M, int HV, int V,
                               float eps, hipStream_t s) {
    const int64_t rows = M * HV;
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_gate_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, out, ld_out, x, ld_x,
                       gate, ld_gate, gate_bias, weight, rows, HV, V, eps);
    return hipGetLastError();
}

bool lowrank_up_supported(int R, int64_t M, const float *Y, int64_t ldY, int64_t off_f0, int64_t off_g0) {
    const bool aligned = reinterpret_cast<uintptr_t>(Y) % 16 == 0 && ldY % 4 == 0 && off_f0 % 4 == 0 && off_g0 % 4 == 0;
    return M <= kLowRankMaxM && (R == 64 || R == 128 || R == 256) && aligned;
}

hipError_t launch_lowrank_up(const LowRankParams &p, hipStream_t s) {
    if (p.M == 0) return hipSuccess;
    if (!lowrank_up_supported(p.R, p.M, p.Y, p.ldY, p.off_f0, p.off_g0)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.kd + 63) / 64 + (p.vd + 63) / 64), (unsigned)((p.M + 15) / 16));
    if (p.R == 64)
        hipLaunchKernelGGL(lowrank_up_kernel<64>, grid, dim3(256), 0, s, p);
    else if (p.R == 128)
        hipLaunchKernelGGL(lowrank_up_kernel<128>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(lowrank_up_kernel<256>, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_cache_sweep(const float *buf, int64_t n, float *sink, hipStream_t s) {
    if (n < 4) return hipSuccess;
    hipLaunchKernelGGL(cache_sweep_kernel, dim3(2048), dim3(256), 0, s, buf, n / 4, sink);
    return hipGetLastError();
}

hipError_t launch_fill_rows(float *y, int64_t ld, const float *row, int64_t M, int64_t N, hipStream_t s) {
    if (M * N == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_rows_kernel, dim3(grid_for(M * N)), dim3(256), 0, s, y, ld, row, M, N);
    return hipGetLastError();
}

}  // namespace gdn2

namespace gdn2 {

hipError_t launch_rmsnorm_gate_bwd(const NormBwdParams &p, hipStream_t s) {
    if (p.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_gate_bwd_kernel, dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_project_bwd(const ProjectBwdParams &p, hipStream_t s) {
    const int64_t M = (int64_t)p.B * p.T;
    if (M == 0) return hipSuccess;
    hipLaunchKernelGGL(project_bwd_kernel, dim3((unsigned)M), dim3(256), project_lds_bytes(p.H * p.K), s, p);
    return hipGetLastError();
}

int conv_bwd_blocks(int T, int tblock) { return (T + tblock - 1) / tblock; }

hipError_t launch_conv_bwd(const ConvBwdParams &p, hipStream_t s) {
    if (p.B == 0 || p.T == 0) return hipSuccess;
    const int Ctot = 2 * p.kd + p.vd;
    hipLaunchKernelGGL(conv_bwd_kernel, dim3((unsigned)((Ctot + 255) / 256), (unsigned)conv_bwd_blocks(p.T, p.tblock),
                                             (unsigned)p.B),
                       dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_colsum(const float *A, int64_t rows, int64_t N, int64_t lda, int group, int fold, float *out,
                         bool accumulate, float *part, int parts, hipStream_t s) {
    if (N == 0) return hipSuccess;
    if (parts < 1) parts = 1;
    const int64_t rows_per = rows > 0 ? (rows + parts - 1) / parts : 0;
    hipLaunchKernelGGL(colsum_part_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)parts), dim3(256), 0, s, A,
                       rows, N, lda, rows_per, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t nout = N / ((int64_t)group * fold);
    hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)nout), dim3(256), 0, s, part, parts, N, group, fold, out,
                       accumulate ? 1 : 0);
    return hipGetLastError();
}

}  // namespace gdn2

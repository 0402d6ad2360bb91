// Recurrent kernels: the per-token scan (one or many tokens) and the fused
// single-token decode (short conv + gates + L2 norm + step + gated RMSNorm).
//
// Semantics: src/kernel/fused_recurrent.rs:27-52 (scan) and
// src/kernel/fused_recurrent_cube.rs:14-57 (decode step); the fused decode
// adds src/short_conv.rs:22-65, src/module.rs:417-472 and :501-517 around it.
//
// Memory plan.  One workgroup (256 lanes) owns the state slice
// S[b, hv, :, v0 : v0 + VS].  Lane t holds the 4 contiguous columns
// 4 * (t % (VS/4)) of rows r = t / (VS/4) + i * RPP in registers (float4),
// so S is read from HBM exactly once and written exactly once per launch,
// with 16-byte coalesced accesses, however many tokens the launch covers.
// Both K-reductions of a token (the erase term (b*k)^T S' and the read-out
// q^T S') come from the same register pass, using
//   o = scale * (S'^T q + v_new * (k . q)),   S' = diag(exp g) S,
// which is the reference's o = scale * S''^T q with S'' = S' + k v_new^T.
#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {

namespace {

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + __expf(-x)); }
// burn's softplus(x, beta = 1) = ln(1 + e^x); above 20 the f32 value is x.
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Block-wide sum over 256 lanes; `red` holds 4 floats; result returned to all lanes.
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// ---------------------------------------------------------------------------
// Register-resident scan.  K rows x VS columns per workgroup of 256 lanes.
// ---------------------------------------------------------------------------
template <int K, int VS>
__global__ __launch_bounds__(256) void scan_kernel(ScanParams p) {
    constexpr int TPR = VS / 4;    // lanes per state row
    constexpr int RPP = 256 / TPR; // rows covered by one pass of the workgroup
    constexpr int NP = K / RPP;    // float4 registers of S per lane
    static_assert(VS % 4 == 0 && TPR <= 64 && 64 % TPR == 0, "VS");
    static_assert(K % RPP == 0, "K");

    const int nvs = p.V / VS;
    const int bh = blockIdx.x / nvs, vsl = blockIdx.x % nvs;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % TPR, r0 = tid / TPR;

    __shared__ float s_eg[2][K], s_a1[2][K], s_a2[2][K], s_k[2][K];
    __shared__ float s_red[2][4][VS];
    __shared__ float s_vn[VS];
    __shared__ float s_kq[4];

    const size_t sbase = (size_t)bh * K * p.V + (size_t)vsl * VS + cg * 4;
    float4 S[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i)
        S[i] = *reinterpret_cast<const float4 *>(p.state_in + sbase + (size_t)(r0 + i * RPP) * p.V);

    const int64_t koff = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh;
    const int64_t voff = (int64_t)bi * p.svb + (int64_t)hv * p.svh;
    const int64_t ooff = (int64_t)bi * p.sob + (int64_t)hv * p.soh;

    for (int t = 0; t < p.T; ++t) {
        const int buf = t & 1;
        float kq = 0.0f;
        for (int r = tid; r < K; r += 256) {
            const int64_t o = koff + (int64_t)t * p.sqt + r;
            const float qq = p.q[o], kk = p.k[o], gg = p.g[o], bb = p.b[o];
            const float eg = expf(gg);
            s_eg[buf][r] = eg;
            s_a1[buf][r] = eg * (bb * kk);
            s_a2[buf][r] = eg * qq;
            s_k[buf][r] = kk;
            kq += kk * qq;
        }
        kq = wave_sum(kq);
        if (lane == 0) s_kq[wave] = kq;
        __syncthreads();

        float e1[4] = {0.f, 0.f, 0.f, 0.f}, e2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int r = r0 + i * RPP;
            const float a1 = s_a1[buf][r], a2 = s_a2[buf][r];
            e1[0] += S[i].x * a1; e1[1] += S[i].y * a1; e1[2] += S[i].z * a1; e1[3] += S[i].w * a1;
            e2[0] += S[i].x * a2; e2[1] += S[i].y * a2; e2[2] += S[i].z * a2; e2[3] += S[i].w * a2;
        }
#pragma unroll
        for (int off = TPR; off < 64; off <<= 1)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                e1[j] += __shfl_xor(e1[j], off, 64);
                e2[j] += __shfl_xor(e2[j], off, 64);
            }
        if (lane < TPR)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s_red[0][wave][cg * 4 + j] = e1[j];
                s_red[1][wave][cg * 4 + j] = e2[j];
            }
        __syncthreads();
        if (tid < VS) {
            const float E1 = s_red[0][0][tid] + s_red[0][1][tid] + s_red[0][2][tid] + s_red[0][3][tid];
            const float E2 = s_red[1][0][tid] + s_red[1][1][tid] + s_red[1][2][tid] + s_red[1][3][tid];
            const float kqs = s_kq[0] + s_kq[1] + s_kq[2] + s_kq[3];
            const int col = vsl * VS + tid;
            const int64_t vo = voff + (int64_t)t * p.svt + col;
            const float vn = p.w[vo] * p.v[vo] - E1;
            p.out[ooff + (int64_t)t * p.sot + col] = p.scale * (E2 + vn * kqs);
            s_vn[tid] = vn;
        }
        __syncthreads();
        const float4 vn = *reinterpret_cast<const float4 *>(&s_vn[cg * 4]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int r = r0 + i * RPP;
            const float eg = s_eg[buf][r], kk = s_k[buf][r];
            S[i].x = S[i].x * eg + kk * vn.x;
            S[i].y = S[i].y * eg + kk * vn.y;
            S[i].z = S[i].z * eg + kk * vn.z;
            S[i].w = S[i].w * eg + kk * vn.w;
        }
    }
#pragma unroll
    for (int i = 0; i < NP; ++i)
        *reinterpret_cast<float4 *>(p.state_out + sbase + (size_t)(r0 + i * RPP) * p.V) = S[i];
}

// Any K, V (<= 1024): one workgroup per (b, hv), the state is updated in
// place in state_out (copied from state_in first), each column owned by one
// lane for the whole launch.  Used for shapes the register kernel does not
// instantiate (e.g. the reference's K = 16, V = 24 test layer).
__global__ __launch_bounds__(256) void scan_generic_kernel(ScanParams p) {
    extern __shared__ float sm[];
    const int K = p.K, V = p.V;
    float *s_eg = sm, *s_a1 = sm + K, *s_a2 = sm + 2 * K, *s_k = sm + 3 * K;
    __shared__ float red[4];
    const int bh = blockIdx.x;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int tid = threadIdx.x;
    const float *Sin = p.state_in + (size_t)bh * K * V;
    float *S = p.state_out + (size_t)bh * K * V;
    if (Sin != S)
        for (int c = tid; c < V; c += 256)
            for (int r = 0; r < K; ++r) S[(size_t)r * V + c] = Sin[(size_t)r * V + c];
    const int64_t koff = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh;
    const int64_t voff = (int64_t)bi * p.svb + (int64_t)hv * p.svh;
    const int64_t ooff = (int64_t)bi * p.sob + (int64_t)hv * p.soh;
    for (int t = 0; t < p.T; ++t) {
        float kq = 0.0f;
        for (int r = tid; r < K; r += 256) {
            const int64_t o = koff + (int64_t)t * p.sqt + r;
            const float qq = p.q[o], kk = p.k[o], eg = expf(p.g[o]);
            s_eg[r] = eg;
            s_a1[r] = eg * (p.b[o] * kk);
            s_a2[r] = eg * qq;
            s_k[r] = kk;
            kq += kk * qq;
        }
        kq = block_sum256(kq, red); // contains the barrier that publishes s_*
        for (int c = tid; c < V; c += 256) {
            float E1 = 0.f, E2 = 0.f;
            for (int r = 0; r < K; ++r) {
                const float s = S[(size_t)r * V + c];
                E1 += s * s_a1[r];
                E2 += s * s_a2[r];
            }
            const int64_t vo = voff + (int64_t)t * p.svt + c;
            const float vn = p.w[vo] * p.v[vo] - E1;
            p.out[ooff + (int64_t)t * p.sot + c] = p.scale * (E2 + vn * kq);
            for (int r = 0; r < K; ++r) {
                float *sp = S + (size_t)r * V + c;
                *sp = *sp * s_eg[r] + s_k[r] * vn;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Fused single-token decode.  One workgroup per (b, hv) owns all V columns
// (the gated RMSNorm reduces over V).  Prologue computes, for the key head
// hk = hv / rep: q, k = l2norm(silu(conv(raw))), g, b; and for the value
// head: v = silu(conv(raw)), w = sigmoid(raw).  Conv caches are written to
// separate output buffers so that workgroups sharing a key head never see a
// half-updated cache; one workgroup per (b, hk) writes the key-side caches.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float conv_token(const float *cache_in, const float *wconv, int64_t cache_b_off,
                                            int n_ch, int c, float x, float *c0, float *c1, float *c2) {
    float x0, x1, x2;
    if (cache_in) {
        x0 = cache_in[cache_b_off + c];
        x1 = cache_in[cache_b_off + n_ch + c];
        x2 = cache_in[cache_b_off + 2 * n_ch + c];
    } else {
        x0 = x1 = x2 = x;
    }
    *c0 = x1;
    *c1 = x2;
    *c2 = x;
    float acc = 0.0f;
    acc += x0 * wconv[4 * c + 0];
    acc += x1 * wconv[4 * c + 1];
    acc += x2 * wconv[4 * c + 2];
    acc += x * wconv[4 * c + 3];
    return acc;
}

// Key-side prologue for channel r of key head hk; writes s_q/s_k/s_g/s_b (pre-norm q, k).
__device__ __forceinline__ void key_prologue(const DecodeParams &p, int bi, int hk, int r, bool write_cache,
                                             float *s_q, float *s_k, float *s_g, float *s_b, float *sq_part,
                                             float *sk_part) {
    const int kd = p.H * p.K;
    const int c = hk * p.K + r;
    const float qr = p.q_raw[(int64_t)bi * p.ld_q + c], kr = p.k_raw[(int64_t)bi * p.ld_k + c];
    float qa, ka;
    if (p.use_short_conv) {
        const int64_t cb = (int64_t)bi * 3 * kd;
        float a0, a1, a2;
        qa = siluf_(conv_token(p.conv_q_in, p.q_conv_w, cb, kd, c, qr, &a0, &a1, &a2));
        if (write_cache) {
            p.conv_q_out[cb + c] = a0;
            p.conv_q_out[cb + kd + c] = a1;
            p.conv_q_out[cb + 2 * kd + c] = a2;
        }
        ka = siluf_(conv_token(p.conv_k_in, p.k_conv_w, cb, kd, c, kr, &a0, &a1, &a2));
        if (write_cache) {
            p.conv_k_out[cb + c] = a0;
            p.conv_k_out[cb + kd + c] = a1;
            p.conv_k_out[cb + 2 * kd + c] = a2;
        }
    } else {
        qa = siluf_(qr);
        ka = siluf_(kr);
    }
    float gv = -expf(p.a_log[hk]) * softplusf_(p.f_raw[(int64_t)bi * p.ld_f + c] + p.dt_bias[c]);
    if (p.decay_factors) {
        const float f = sigmoidf_(p.decay_factors[c]) * p.one_minus_min_decay;
        gv = logf(f * expf(gv) + p.min_decay);
    }
    float bv = sigmoidf_(p.b_raw[(int64_t)bi * p.ld_b + c]);
    if (p.allow_neg_eigval) bv *= 2.0f;
    s_q[r] = qa;
    s_k[r] = ka;
    s_g[r] = gv;
    s_b[r] = bv;
    *sq_part += qa * qa;
    *sk_part += ka * ka;
}

// Value-side prologue for column col of value head hv: returns v, w; writes conv_v_out.
__device__ __forceinline__ void value_prologue(const DecodeParams &p, int bi, int hv, int col, float *v, float *w) {
    const int vd = p.HV * p.V;
    const int c = hv * p.V + col;
    const float vr = p.v_raw[(int64_t)bi * p.ld_v + c];
    if (p.use_short_conv) {
        const int64_t cb = (int64_t)bi * 3 * vd;
        float a0, a1, a2;
        *v = siluf_(conv_token(p.conv_v_in, p.v_conv_w, cb, vd, c, vr, &a0, &a1, &a2));
        p.conv_v_out[cb + c] = a0;
        p.conv_v_out[cb + vd + c] = a1;
        p.conv_v_out[cb + 2 * vd + c] = a2;
    } else {
        *v = siluf_(vr);
    }
    *w = sigmoidf_(p.w_raw[(int64_t)bi * p.ld_w + c]);
}

template <int K, int V>
__global__ __launch_bounds__(256) void decode_fused_kernel(DecodeParams p) {
    // The V columns are processed in NH parts of VP columns: part h's state
    // is reduced, updated and written back as soon as its own loads have
    // arrived, while the next part's loads are still in flight.
    constexpr int NH = V >= 128 ? 2 : 1, VP = V / NH;
    constexpr int TPR = VP / 4, RPP = 256 / TPR, NP = K / RPP;
    static_assert(VP % 4 == 0 && TPR <= 64 && 64 % TPR == 0, "V");
    static_assert(K % RPP == 0 && K <= 256 && V <= 256, "K, V");
    const int bh = blockIdx.x;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % TPR, r0 = tid / TPR;
    const int kd = p.H * K, vd = p.HV * V;
    const bool sc = p.use_short_conv != 0;

    __shared__ float s_k[K], s_eg[K], s_a1[K], s_a2[K];
    __shared__ float s_red[2][4][VP];
    __shared__ float s_vn[V];
    __shared__ float red[3][4], red_o2[4];

    // Prologue operands first: the memory counter is in order, so anything
    // loaded after the state would wait for the whole 16-row state slice.
    // Every load is unconditional from a valid address (missing optional
    // operands point at an input that is read anyway) and selected after.
    const int r = tid % K;               // key channel (lanes >= K duplicate)
    const int c = hk * K + r;
    const int64_t xq = (int64_t)bi * p.ld_q + c, xk = (int64_t)bi * p.ld_k + c;
    const float qr = p.q_raw[xq], kr = p.k_raw[xk];
    const float fr = p.f_raw[(int64_t)bi * p.ld_f + c], brw = p.b_raw[(int64_t)bi * p.ld_b + c];
    const float dtb = p.dt_bias[c], alog = p.a_log[hk];
    const float dfv = (p.decay_factors ? p.decay_factors : p.dt_bias)[c];
    const int64_t kcb = (int64_t)bi * 3 * kd + c;
    const float *cqi = (sc && p.conv_q_in) ? p.conv_q_in + kcb : p.q_raw + xq;
    const float *cki = (sc && p.conv_k_in) ? p.conv_k_in + kcb : p.k_raw + xk;
    const int64_t cst = (sc && p.conv_q_in) ? kd : 0;
    const float q0 = cqi[0], q1 = cqi[cst], q2 = cqi[2 * cst];
    const float k0 = cki[0], k1 = cki[cst], k2 = cki[2 * cst];
    const float *wq = sc ? p.q_conv_w + 4 * c : p.q_raw + xq;
    const float *wk = sc ? p.k_conv_w + 4 * c : p.k_raw + xk;
    const int wst = sc ? 1 : 0;
    const float wq0 = wq[0], wq1 = wq[wst], wq2 = wq[2 * wst], wq3 = wq[3 * wst];
    const float wk0 = wk[0], wk1 = wk[wst], wk2 = wk[2 * wst], wk3 = wk[3 * wst];

    const int col = tid % V;             // value column (lanes >= V duplicate)
    const int cvc = hv * V + col;
    const int64_t xv = (int64_t)bi * p.ld_v + cvc;
    const float vr = p.v_raw[xv], wr = p.w_raw[(int64_t)bi * p.ld_w + cvc];
    const float gt = p.gate[(int64_t)bi * p.ld_gate + cvc] + (p.gate_bias ? p.gate_bias[cvc] : 0.f),
                onw = p.o_norm_weight[col];
    const int64_t vcb = (int64_t)bi * 3 * vd + cvc;
    const float *cvi = (sc && p.conv_v_in) ? p.conv_v_in + vcb : p.v_raw + xv;
    const int64_t vst = (sc && p.conv_v_in) ? vd : 0;
    const float v0 = cvi[0], v1 = cvi[vst], v2 = cvi[2 * vst];
    const float *wv = sc ? p.v_conv_w + 4 * cvc : p.v_raw + xv;
    const float wv0 = wv[0], wv1 = wv[wst], wv2 = wv[2 * wst], wv3 = wv[3 * wst];

    // The state slice: 16-byte loads, each row read exactly once, part 0 first.
    // State traffic is streamed (non-temporal loads and stores): at B = 64 it
    // is 67 MB per token each way and would only evict the caches' reuse.
    floatx4 S[NH][NP];
    float *Sg = p.state + (size_t)bh * K * V + cg * 4;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int i = 0; i < NP; ++i)
            S[h][i] = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(Sg + (size_t)(r0 + i * RPP) * V + h * VP));

    // Key side: conv + SiLU (src/short_conv.rs:22-65), gates
    // (src/module.rs:417-443), then the L2 norms over K (src/l2norm.rs).
    float qa = 0.f, ka = 0.f;
    {
        float aq = 0.f, ak = 0.f;
        if (sc) {
            aq += q0 * wq0; aq += q1 * wq1; aq += q2 * wq2; aq += qr * wq3;
            ak += k0 * wk0; ak += k1 * wk1; ak += k2 * wk2; ak += kr * wk3;
        } else {
            aq = qr;
            ak = kr;
        }
        qa = siluf_(aq);
        ka = siluf_(ak);
    }
    float gv = -expf(alog) * softplusf_(fr + dtb);
    if (p.decay_factors) gv = logf(sigmoidf_(dfv) * p.one_minus_min_decay * expf(gv) + p.min_decay);
    float bv = sigmoidf_(brw);
    if (p.allow_neg_eigval) bv *= 2.0f;
    const bool klane = tid < K;
    float sq = klane ? qa * qa : 0.f, sk = klane ? ka * ka : 0.f;
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    if (lane == 0) {
        red[0][wave] = sq;
        red[1][wave] = sk;
    }
    __syncthreads();
    const float qn = 1.0f / sqrtf(red[0][0] + red[0][1] + red[0][2] + red[0][3] + 1e-6f);
    const float kn = 1.0f / sqrtf(red[1][0] + red[1][1] + red[1][2] + red[1][3] + 1e-6f);
    float kq = 0.f;
    if (klane) {
        const float qq = qa * qn, kk = ka * kn;
        const float eg = expf(gv);
        s_eg[r] = eg;
        s_a1[r] = eg * (bv * kk);
        s_a2[r] = eg * qq;
        s_k[r] = kk;
        kq = kk * qq;
    }
    kq = wave_sum(kq);
    if (lane == 0) red[2][wave] = kq;
    // Value side: conv + SiLU of v, w = sigmoid.
    float vv;
    {
        float av = 0.f;
        if (sc) {
            av += v0 * wv0; av += v1 * wv1; av += v2 * wv2; av += vr * wv3;
        } else {
            av = vr;
        }
        vv = siluf_(av);
    }
    const float ww = sigmoidf_(wr);
    __syncthreads();

    // Per part: both K-reductions of the step from one pass over the
    // registers, v_new for the part's columns, then its state update and
    // write-back.  Lane c < V holds column c's value-side operands.
    const float kqs = red[2][0] + red[2][1] + red[2][2] + red[2][3];
    const bool vlane = tid < V;
    float o = 0.f;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        float e1[4] = {0.f, 0.f, 0.f, 0.f}, e2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int rr = r0 + i * RPP;
            const float a1 = s_a1[rr], a2 = s_a2[rr];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                e1[j] += S[h][i][j] * a1;
                e2[j] += S[h][i][j] * a2;
            }
        }
#pragma unroll
        for (int off = TPR; off < 64; off <<= 1)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                e1[j] += __shfl_xor(e1[j], off, 64);
                e2[j] += __shfl_xor(e2[j], off, 64);
            }
        if (lane < TPR)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s_red[0][wave][cg * 4 + j] = e1[j];
                s_red[1][wave][cg * 4 + j] = e2[j];
            }
        __syncthreads();
        if (tid >= h * VP && tid < (h + 1) * VP) {
            const int pc = tid - h * VP;
            const float E1 = s_red[0][0][pc] + s_red[0][1][pc] + s_red[0][2][pc] + s_red[0][3][pc];
            const float E2 = s_red[1][0][pc] + s_red[1][1][pc] + s_red[1][2][pc] + s_red[1][3][pc];
            const float vn = ww * vv - E1;
            o = p.scale * (E2 + vn * kqs);
            s_vn[tid] = vn;
        }
        __syncthreads();
        const floatx4 vn4 = *reinterpret_cast<const floatx4 *>(&s_vn[h * VP + cg * 4]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int rr = r0 + i * RPP;
            const float eg = s_eg[rr], kk = s_k[rr];
            __builtin_nontemporal_store(S[h][i] * eg + kk * vn4, reinterpret_cast<floatx4 *>(Sg + (size_t)rr * V + h * VP));
        }
    }
    // gated RMSNorm over the V columns (src/module.rs:501-517)
    const float o2 = wave_sum(vlane ? o * o : 0.f);
    if (lane == 0) red_o2[wave] = o2;
    __syncthreads();
    if (vlane) {
        const float ms = (red_o2[0] + red_o2[1] + red_o2[2] + red_o2[3]) / (float)V;
        p.out[(int64_t)bi * p.ld_out + cvc] = o / sqrtf(ms + p.norm_eps) * onw * siluf_(gt);
    }
    // Conv caches: the last three pre-conv rows, oldest first.  Value caches
    // are owned by this (b, hv); key caches by the first value head of hk.
    if (sc) {
        if (vlane) {
            p.conv_v_out[vcb] = v1;
            p.conv_v_out[vcb + vd] = v2;
            p.conv_v_out[vcb + 2 * vd] = vr;
        }
        if (klane && (hv % p.rep) == 0) {
            p.conv_q_out[kcb] = q1;
            p.conv_q_out[kcb + kd] = q2;
            p.conv_q_out[kcb + 2 * kd] = qr;
            p.conv_k_out[kcb] = k1;
            p.conv_k_out[kcb + kd] = k2;
            p.conv_k_out[kcb + 2 * kd] = kr;
        }
    }
}

// The bare single-token step (src/kernel/fused_recurrent_cube.rs:14-57) at
// the decode kernel's head shapes: one workgroup per (b, hv) owns all V
// columns.  Its q, k, g, b (lane r < K) and v, w (lane c < V) are requested
// before the state, since the memory counter is in order and anything loaded
// after the state would wait for the whole slice; the state is then streamed
// once each way with 16-byte non-temporal accesses, in NH parts so that part
// 0's update and write-back overlap part 1's loads.  state_out may equal
// state_in: every element is read and written by the same lane.
template <int K, int V>
__global__ __launch_bounds__(256) void step_kernel(ScanParams p) {
    constexpr int NH = V >= 128 ? 2 : 1, VP = V / NH;
    constexpr int TPR = VP / 4, RPP = 256 / TPR, NP = K / RPP;
    static_assert(VP % 4 == 0 && TPR <= 64 && 64 % TPR == 0, "V");
    static_assert(K % RPP == 0 && K <= 256 && V <= 256, "K, V");
    const int bh = blockIdx.x;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % TPR, r0 = tid / TPR;

    __shared__ float s_eg[K], s_a1[K], s_a2[K], s_k[K];
    __shared__ float s_red[2][4][VP];
    __shared__ float s_vn[V];
    __shared__ float red[4];

    const int r = tid % K; // key channel (lanes >= K duplicate)
    const int64_t ko = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh + r;
    const float qq = p.q[ko], kk = p.k[ko], gg = p.g[ko], bb = p.b[ko];
    const int col = tid % V; // value column (lanes >= V duplicate)
    const int64_t vo = (int64_t)bi * p.svb + (int64_t)hv * p.svh + col;
    const float vv = p.v[vo], ww = p.w[vo];

    floatx4 S[NH][NP];
    const size_t sb = (size_t)bh * K * V + cg * 4;
    const float *Si = p.state_in + sb;
    float *So = p.state_out + sb;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int i = 0; i < NP; ++i)
            S[h][i] = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(Si + (size_t)(r0 + i * RPP) * V + h * VP));

    const bool klane = tid < K;
    float kq = 0.f;
    if (klane) {
        const float eg = expf(gg);
        s_eg[r] = eg;
        s_a1[r] = eg * (bb * kk);
        s_a2[r] = eg * qq;
        s_k[r] = kk;
        kq = kk * qq;
    }
    kq = wave_sum(kq);
    if (lane == 0) red[wave] = kq;
    __syncthreads();
    const float kqs = red[0] + red[1] + red[2] + red[3];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        float e1[4] = {0.f, 0.f, 0.f, 0.f}, e2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int rr = r0 + i * RPP;
            const float a1 = s_a1[rr], a2 = s_a2[rr];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                e1[j] += S[h][i][j] * a1;
                e2[j] += S[h][i][j] * a2;
            }
        }
#pragma unroll
        for (int off = TPR; off < 64; off <<= 1)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                e1[j] += __shfl_xor(e1[j], off, 64);
                e2[j] += __shfl_xor(e2[j], off, 64);
            }
        if (lane < TPR)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s_red[0][wave][cg * 4 + j] = e1[j];
                s_red[1][wave][cg * 4 + j] = e2[j];
            }
        __syncthreads();
        if (tid >= h * VP && tid < (h + 1) * VP) {
            const int pc = tid - h * VP;
            const float E1 = s_red[0][0][pc] + s_red[0][1][pc] + s_red[0][2][pc] + s_red[0][3][pc];
            const float E2 = s_red[1][0][pc] + s_red[1][1][pc] + s_red[1][2][pc] + s_red[1][3][pc];
            const float vn = ww * vv - E1;
            p.out[(int64_t)bi * p.sob + (int64_t)hv * p.soh + col] = p.scale * (E2 + vn * kqs);
            s_vn[tid] = vn;
        }
        __syncthreads();
        const floatx4 vn4 = *reinterpret_cast<const floatx4 *>(&s_vn[h * VP + cg * 4]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int rr = r0 + i * RPP;
            const float eg = s_eg[rr], k2 = s_k[rr];
            __builtin_nontemporal_store(S[h][i] * eg + k2 * vn4,
                                        reinterpret_cast<floatx4 *>(So + (size_t)rr * V + h * VP));
        }
    }
}

// Any K <= 256, V <= 1024: state in global memory, one column per lane.
__global__ __launch_bounds__(256) void decode_fused_generic_kernel(DecodeParams p) {
    extern __shared__ float sm[];
    const int K = p.K, V = p.V;
    float *s_q = sm, *s_k = sm + K, *s_g = sm + 2 * K, *s_b = sm + 3 * K;
    float *s_eg = sm + 4 * K, *s_a1 = sm + 5 * K, *s_a2 = sm + 6 * K;
    __shared__ float red[4];
    const int bh = blockIdx.x;
    const int bi = bh / p.HV, hv = bh % p.HV, hk = hv / p.rep;
    const int tid = threadIdx.x;
    float *S = p.state + (size_t)bh * K * V;
    float sq = 0.f, sk = 0.f;
    const bool key_writer = (hv % p.rep) == 0;
    if (tid < K) key_prologue(p, bi, hk, tid, key_writer, s_q, s_k, s_g, s_b, &sq, &sk);
    sq = block_sum256(sq, red);
    sk = block_sum256(sk, red);
    const float qn = 1.0f / sqrtf(sq + 1e-6f), kn = 1.0f / sqrtf(sk + 1e-6f);
    float kq = 0.f;
    if (tid < K) {
        const float qq = s_q[tid] * qn, kk = s_k[tid] * kn, eg = expf(s_g[tid]);
        s_eg[tid] = eg;
        s_a1[tid] = eg * (s_b[tid] * kk);
        s_a2[tid] = eg * qq;
        s_k[tid] = kk;
        kq = kk * qq;
    }
    kq = block_sum256(kq, red);
    float o2 = 0.f;
    float ov[4];
    int n = 0;
    for (int c = tid; c < V; c += 256, ++n) {
        float vv, ww;
        value_prologue(p, bi, hv, c, &vv, &ww);
        float E1 = 0.f, E2 = 0.f;
        for (int r = 0; r < K; ++r) {
            const float s = S[(size_t)r * V + c];
            E1 += s * s_a1[r];
            E2 += s * s_a2[r];
        }
        const float vn = ww * vv - E1;
        const float o = p.scale * (E2 + vn * kq);
        for (int r = 0; r < K; ++r) {
            float *sp = S + (size_t)r * V + c;
            *sp = *sp * s_eg[r] + s_k[r] * vn;
        }
        ov[n] = o;
        o2 += o * o;
    }
    o2 = block_sum256(o2, red);
    const float rms = sqrtf(o2 / (float)V + p.norm_eps);
    n = 0;
    for (int c = tid; c < V; c += 256, ++n) {
        const int64_t ch = (int64_t)hv * V + c;
        const float gt = p.gate[bi * p.ld_gate + ch] + (p.gate_bias ? p.gate_bias[ch] : 0.f);
        p.out[bi * p.ld_out + ch] = ov[n] / rms * p.o_norm_weight[c] * siluf_(gt);
    }
}

template <int K, int VS>
hipError_t launch_scan_t(const ScanParams &p, hipStream_t s) {
    const int grid = p.B * p.HV * (p.V / VS);
    hipLaunchKernelGGL((scan_kernel<K, VS>), dim3(grid), dim3(256), 0, s, p);
    return hipGetLastError();
}

template <int K, int V>
hipError_t launch_decode_t(const DecodeParams &p, hipStream_t s) {
    hipLaunchKernelGGL((decode_fused_kernel<K, V>), dim3(p.B * p.HV), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace

template <int K, int V>
hipError_t launch_step_t(const ScanParams &p, hipStream_t s) {
    hipLaunchKernelGGL((step_kernel<K, V>), dim3(p.B * p.HV), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_scan(const ScanParams &p, hipStream_t s) {
    // One token at the decode kernel's head shapes: the streaming step kernel.
    if (p.T == 1) {
        if (p.K == 128 && p.V == 128) return launch_step_t<128, 128>(p, s);
        if (p.K == 128 && p.V == 256) return launch_step_t<128, 256>(p, s);
        if (p.K == 64 && p.V == 64) return launch_step_t<64, 64>(p, s);
        if (p.K == 64 && p.V == 128) return launch_step_t<64, 128>(p, s);
    }
    // Register kernels: VS columns per workgroup.  VS = 64 splits each head's
    // V = 128 columns over two workgroups, which doubles the number of
    // workgroups for small batch x head counts.
    if (p.K == 128 && p.V % 64 == 0) return launch_scan_t<128, 64>(p, s);
    if (p.K == 64 && p.V % 64 == 0) return launch_scan_t<64, 64>(p, s);
    if (p.K == 256 && p.V % 64 == 0) return launch_scan_t<256, 64>(p, s);
    if (p.K == 64 && p.V % 32 == 0) return launch_scan_t<64, 32>(p, s);
    if (p.K == 128 && p.V % 32 == 0) return launch_scan_t<128, 32>(p, s);
    const size_t lds = sizeof(float) * 4 * (size_t)p.K;
    hipLaunchKernelGGL(scan_generic_kernel, dim3(p.B * p.HV), dim3(256), lds, s, p);
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams &p, hipStream_t s) {
    if (p.K == 128 && p.V == 128) return launch_decode_t<128, 128>(p, s);
    if (p.K == 128 && p.V == 256) return launch_decode_t<128, 256>(p, s);
    if (p.K == 64 && p.V == 64) return launch_decode_t<64, 64>(p, s);
    if (p.K == 64 && p.V == 128) return launch_decode_t<64, 128>(p, s);
    const size_t lds = sizeof(float) * 7 * (size_t)p.K;
    hipLaunchKernelGGL(decode_fused_generic_kernel, dim3(p.B * p.HV), dim3(256), lds, s, p);
    return hipGetLastError();
}

}  // namespace gdn2

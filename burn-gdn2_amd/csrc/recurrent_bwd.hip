// Adjoint of the per-token recurrence (src/kernel/fused_recurrent.rs:27-52)
// for the shapes the chunked backward does not cover: the gradients of
// L = <d_out, out> + <d_state_out, S_T> with respect to q, k, g, b, v, w and
// S0, by a forward sweep that keeps S every kCk tokens, then, segment by
// segment from the end, a re-run of the segment's states and the reverse
// recurrence over them.  Per token t, with S1 = diag(e^g) S_prev,
// kb = b k, v_new = w v - S1^T kb, S2 = S1 + k v_new^T = S_t, o = scale S2^T q:
//   dS2 = dS + scale q dO^T            dq = scale S2 dO
//   dk  = dS2 v_new                    dv_new = dS2^T k      dv = dv_new w, dw = dv_new v
//   dkb = -S1 dv_new                   db = dkb k, dk += dkb b
//   dS1 = dS2 - kb dv_new^T            dg = rowsum(dS1 . S1)   dS_prev = diag(e^g) dS1
// One workgroup per (batch row, key head) walks the key head's value heads in
// turn, so that the key-side gradients of GVA sum without atomics.  Column
// work (thread per value column j) and row work (thread per key row i) meet
// in LDS, where S_t and dS live with one padding column.
#include "common.hpp"
#include "kernels.hpp"

namespace gdn2 {
namespace {

constexpr int kCk = 64;  // tokens per checkpoint segment

struct ScanBwdParams {
    const float *q, *k, *g, *b, *v, *w, *S0, *dO, *dST;
    float *dq, *dk, *dg, *db, *dv, *dw, *dS0;
    float *ws;  // per workgroup: (nck + kCk + 1) * K * V floats
    int B, Hk, HV, rep, T, K, V, nck;
    int64_t sqb, sqh, sqt, svb, svh, svt, sob, soh, sot;
    float scale;
};

__global__ __launch_bounds__(256) void scan_bwd_kernel(ScanBwdParams p) {
    extern __shared__ float sm[];
    const int K = p.K, V = p.V, V1 = p.V + 1;
    float *sS = sm;                 // K x (V + 1): S (forward sweeps), S_t (reverse)
    float *sD = sS + K * V1;        // K x (V + 1): dS
    float *sq = sD + K * V1, *sk = sq + K, *se = sk + K, *sb = se + K, *skb = sb + K;
    float *svn = skb + K, *sdvn = svn + V, *sdo = sdvn + V;
    const int tid = threadIdx.x;
    const int bi = blockIdx.x / p.Hk, hk = blockIdx.x % p.Hk;
    const size_t KV = (size_t)K * V;
    float *ck = p.ws + (size_t)blockIdx.x * (p.nck + kCk + 1) * KV;  // checkpoints
    float *seg = ck + (size_t)p.nck * KV;                           // states of one segment
    const int64_t qo = (int64_t)bi * p.sqb + (int64_t)hk * p.sqh;

    // stage token t's key-side rows (and q when wanted) into LDS
    auto stage = [&](int t, bool with_q) {
        const int64_t o = qo + (int64_t)t * p.sqt;
        for (int i = tid; i < K; i += 256) {
            const float kv = p.k[o + i], bv = p.b[o + i];
            sk[i] = kv;
            se[i] = __expf(p.g[o + i]);
            sb[i] = bv;
            skb[i] = bv * kv;
            if (with_q) sq[i] = p.q[o + i];
        }
    };
    // one forward step on the columns this thread owns: S <- S1 + k v_new^T
    auto step = [&](int64_t vo) {
        for (int j = tid; j < V; j += 256) {
            float vn = p.w[vo + j] * p.v[vo + j];
            for (int i = 0; i < K; ++i) {
                const float s1 = se[i] * sS[i * V1 + j];
                sS[i * V1 + j] = s1;
                vn -= s1 * skb[i];
            }
            for (int i = 0; i < K; ++i) sS[i * V1 + j] += sk[i] * vn;
        }
    };
    auto save = [&](float *dst) {  // S -> dst (K x V), coalesced over j
        for (int i = 0; i < K; ++i)
            for (int j = tid; j < V; j += 256) dst[(size_t)i * V + j] = sS[i * V1 + j];
    };
    auto load = [&](float *dstS, const float *src) {
        for (int i = 0; i < K; ++i)
            for (int j = tid; j < V; j += 256) dstS[i * V1 + j] = src ? src[(size_t)i * V + j] : 0.f;
    };

    for (int r = 0; r < p.rep; ++r) {
        const int hv = hk * p.rep + r;
        const size_t bh = (size_t)bi * p.HV + hv;
        const int64_t vbase = (int64_t)bi * p.svb + (int64_t)hv * p.svh;
        const int64_t obase = (int64_t)bi * p.sob + (int64_t)hv * p.soh;
        // forward sweep: the state before tokens 0, kCk, 2 kCk, ...
        load(sS, p.S0 ? p.S0 + bh * KV : nullptr);
        for (int t = 0; t < p.T; ++t) {
            if (t % kCk == 0) save(ck + (size_t)(t / kCk) * KV);
            __syncthreads();  // previous step done with the staged rows
            stage(t, false);
            __syncthreads();
            step(vbase + (int64_t)t * p.svt);
        }
        __syncthreads();
        load(sD, p.dST ? p.dST + bh * KV : nullptr);
        for (int c = p.nck - 1; c >= 0; --c) {
            const int t0 = c * kCk, len = min(kCk, p.T - t0);
            // the segment's states: slot r = S before token t0 + r, slot len = after the last
            __syncthreads();
            load(sS, ck + (size_t)c * KV);
            for (int rr = 0; rr < len; ++rr) {
                save(seg + (size_t)rr * KV);
                __syncthreads();
                stage(t0 + rr, false);
                __syncthreads();
                step(vbase + (int64_t)(t0 + rr) * p.svt);
            }
            save(seg + (size_t)len * KV);
            for (int rr = len - 1; rr >= 0; --rr) {
                const int t = t0 + rr;
                const float *Sprev = seg + (size_t)rr * KV, *S2 = seg + (size_t)(rr + 1) * KV;
                const int64_t vo = vbase + (int64_t)t * p.svt, oo = obase + (int64_t)t * p.sot;
                __syncthreads();  // everyone done with the previous token's LDS
                stage(t, true);
                load(sS, S2);
                __syncthreads();
                // columns: dS2 = dS + scale q dO^T, dv_new, v_new, dv, dw
                for (int j = tid; j < V; j += 256) {
                    const float dOj = p.dO[oo + j];
                    float dvn = 0.f, vn = p.w[vo + j] * p.v[vo + j];
                    for (int i = 0; i < K; ++i) {
                        const float d = sD[i * V1 + j] + p.scale * sq[i] * dOj;
                        sD[i * V1 + j] = d;
                        dvn += d * sk[i];
                        vn -= se[i] * Sprev[(size_t)i * V + j] * skb[i];
                    }
                    svn[j] = vn;
                    sdvn[j] = dvn;
                    sdo[j] = dOj;
                    p.dv[vo + j] = dvn * p.w[vo + j];
                    p.dw[vo + j] = dvn * p.v[vo + j];
                }
                __syncthreads();
                // rows: dq, dk, db, dg and dS_prev = diag(e^g) dS1
                const int64_t to = qo + (int64_t)t * p.sqt;
                for (int i = tid; i < K; i += 256) {
                    const float ki = sk[i], kbi = skb[i], ei = se[i];
                    float dqi = 0.f, dki = 0.f, dkb = 0.f, dgi = 0.f;
                    for (int j = 0; j < V; ++j) {
                        const float s2 = sS[i * V1 + j], d2 = sD[i * V1 + j];
                        const float s1 = s2 - ki * svn[j];
                        const float d1 = d2 - kbi * sdvn[j];
                        dqi += s2 * sdo[j];
                        dki += d2 * svn[j];
                        dkb -= s1 * sdvn[j];
                        dgi += d1 * s1;
                        sD[i * V1 + j] = ei * d1;
                    }
                    dqi *= p.scale;
                    dki += dkb * sb[i];
                    const float dbi = dkb * ki;
                    if (r == 0) {
                        p.dq[to + i] = dqi; p.dk[to + i] = dki; p.db[to + i] = dbi; p.dg[to + i] = dgi;
                    } else {
                        p.dq[to + i] += dqi; p.dk[to + i] += dki; p.db[to + i] += dbi; p.dg[to + i] += dgi;
                    }
                }
            }
        }
        __syncthreads();
        for (int i = 0; i < K; ++i)
            for (int j = tid; j < V; j += 256) p.dS0[bh * KV + (size_t)i * V + j] = sD[i * V1 + j];
        __syncthreads();
    }
}

size_t scan_bwd_lds_bytes(int64_t K, int64_t V) { return sizeof(float) * (2 * K * (V + 1) + 5 * K + 3 * V); }

int nchecks(int64_t T) { return (int)((T + kCk - 1) / kCk); }

}  // namespace
}  // namespace gdn2

using namespace gdn2;

namespace {
gdn2_status check_scan_bwd(const gdn2_recurrent_bwd_args *a, const char *who) {
    if (!a) return fail(GDN2_EINVAL, std::string(who) + ": null args");
    const gdn2_recurrent_args &f = a->fwd;
    if (!f.q || !f.k || !f.g || !f.b || !f.v || !f.w || !a->d_out || !a->dq || !a->dk || !a->dg || !a->db || !a->dv ||
        !a->dw || !a->d_state0)
        return fail(GDN2_EINVAL, std::string(who) + ": null tensor pointer");
    if (f.batch <= 0 || f.num_heads <= 0 || f.num_v_heads <= 0 || f.head_dim <= 0 || f.head_v_dim <= 0 ||
        f.seq_len < 0)
        return fail(GDN2_EINVAL, std::string(who) + ": invalid dimensions");
    if (f.num_v_heads % f.num_heads != 0)
        return fail(GDN2_EINVAL, std::string(who) + ": num_v_heads must be a multiple of num_heads");
    if (scan_bwd_lds_bytes(f.head_dim, f.head_v_dim) > 160 * 1024)
        return fail(GDN2_NOT_APPLICABLE, std::string(who) + ": K x V too large for one workgroup's LDS");
    return GDN2_OK;
}
}  // namespace

extern "C" size_t gdn2_recurrent_bwd_workspace_bytes(const gdn2_recurrent_bwd_args *a) {
    if (!a || a->fwd.batch <= 0 || a->fwd.num_heads <= 0 || a->fwd.seq_len <= 0 || a->fwd.head_dim <= 0 ||
        a->fwd.head_v_dim <= 0)
        return 0;
    const gdn2_recurrent_args &f = a->fwd;
    return sizeof(float) * (size_t)f.batch * f.num_heads * (nchecks(f.seq_len) + kCk + 1) * f.head_dim * f.head_v_dim;
}

extern "C" gdn2_status gdn2_recurrent_bwd_f32(const gdn2_recurrent_bwd_args *a, gdn2_stream_t stream) {
    const char *who = "gdn2_recurrent_bwd_f32";
    gdn2_status st = check_scan_bwd(a, who);
    if (st != GDN2_OK) return st;
    const gdn2_recurrent_args &f = a->fwd;
    hipStream_t s = (hipStream_t)stream;
    const int64_t nS = f.batch * f.num_v_heads * f.head_dim * f.head_v_dim;
    if (f.seq_len == 0) {  // no tokens: dS0 = d_state_out (or 0), by the fill kernel (a copy when a row is given)
        GDN2_HIP_CHECK(launch_fill_rows(a->d_state0, 0, a->d_state_out, 1, nS, s));
        return GDN2_OK;
    }
    const size_t need = gdn2_recurrent_bwd_workspace_bytes(a);
    if (!a->workspace || a->workspace_bytes < need)
        return fail(GDN2_EINVAL, std::string(who) + ": workspace missing or too small");
    ScanBwdParams p{};
    p.q = f.q; p.k = f.k; p.g = f.g; p.b = f.b; p.v = f.v; p.w = f.w; p.S0 = f.state_in;
    p.dO = a->d_out; p.dST = a->d_state_out;
    p.dq = a->dq; p.dk = a->dk; p.dg = a->dg; p.db = a->db; p.dv = a->dv; p.dw = a->dw; p.dS0 = a->d_state0;
    p.ws = static_cast<float *>(a->workspace);
    p.B = (int)f.batch; p.Hk = (int)f.num_heads; p.HV = (int)f.num_v_heads; p.rep = (int)(f.num_v_heads / f.num_heads);
    p.T = (int)f.seq_len; p.K = (int)f.head_dim; p.V = (int)f.head_v_dim; p.nck = nchecks(f.seq_len);
    p.sqb = f.stride_qk_b; p.sqh = f.stride_qk_h; p.sqt = f.stride_qk_t;
    p.svb = f.stride_vw_b; p.svh = f.stride_vw_h; p.svt = f.stride_vw_t;
    p.sob = f.stride_o_b; p.soh = f.stride_o_h; p.sot = f.stride_o_t;
    p.scale = (float)f.scale;
    const size_t lds = scan_bwd_lds_bytes(f.head_dim, f.head_v_dim);
    GDN2_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&scan_bwd_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(scan_bwd_kernel, dim3((unsigned)(f.batch * f.num_heads)), dim3(256), lds, s, p);
    GDN2_HIP_CHECK(hipGetLastError());
    return GDN2_OK;
}

/*
 * gdn2_oracle.c -- CPU restatement of burn-gdn2's forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product path (burn-gdn2_amd/) never links or calls it.
 *
 * Contents and the reference code each function restates:
 *   gdn2o_recurrent_f64   per-token scan, evaluated in double
 *                         (src/kernel/fused_recurrent.rs:27-52)     -- ground truth
 *   gdn2o_recurrent_bwd_f64  its adjoint (gradients of q, k, g, b, v, w,
 *                         S0), in double -- the gradients the reference's
 *                         training path gets from autodiff of the same scan
 *                         (tests/autodiff.rs:153-206; WIP fused backward
 *                         src/kernel/chunk_adjoint_cube.rs:464-707)
 *   gdn2o_recurrent_f32   the same scan with the reference's f32 op order
 *                         (src/kernel/fused_recurrent.rs:25-52)
 *   gdn2o_chunk_wy_f32    chunked WY forward with tile-local (16) log-space
 *                         decay and blocked 16-tile solve, f32
 *                         (src/forward.rs:44-278)
 *   gdn2o_short_conv      causal depthwise conv k=4 + SiLU with replicate
 *                         padding / cache (src/short_conv.rs:22-65)
 *   gdn2o_l2norm_rows     x / sqrt(sum x^2 + eps) (src/l2norm.rs:13-16)
 *   gdn2o_rmsnorm_gate    x / sqrt(mean x^2 + eps) * w * silu(gate)
 *                         (src/module.rs:501-517)
 *   gdn2o_layer_from_raw  the layer from its Linear outputs on: conv, gates,
 *                         L2 norm, GVA, scan, gated RMSNorm, in double
 *                         (src/module.rs:404-476, :244-312)
 *   gdn2o_layer_forward   GatedDeltaNet2::project + forward / forward_train
 *                         in double (src/module.rs:224-495)
 *   gdn2o_scan_d, gdn2o_recurrent_bwd_d  the scan and its adjoint on double
 *                         operands (the layer adjoint in oracle.py feeds them
 *                         its own double values)
 *
 * Pinning (what checks each function against something other than itself):
 *   recurrent_f64/f32  closed forms (b=0,g=0 linear attention; T=1 rank-1
 *                      step; b=0 gated linear attention), golden vectors of
 *                      the reference's own torch model (tests/golden/)
 *   recurrent_bwd_f64  central finite differences of recurrent_f64 on
 *                      every input (tests/test_oracle_bwd.py); the
 *                      b=0, g=0 closed form.  recurrent_bwd_d is the same
 *                      code on double inputs; scan_d is the layer's scan
 *   (layer adjoint)    oracle.py's layer_backward_f64: central finite
 *                      differences of gdn2o_layer_forward on every parameter,
 *                      the input and the state (tests/test_oracle_layer_bwd.py)
 *   chunk_wy_f32       chunk == recurrence invariant for C in {4..128},
 *                      ragged T, non-zero S0, broadcast g/b
 *   short_conv         brute-force convolution on tiny inputs + cache
 *                      continuation invariant + golden vectors
 *   l2norm, rmsnorm    closed forms on hand-made vectors + golden vectors
 *   layer_forward      golden vectors of the reference's torch model
 *   layer_from_raw     (tests/golden/gen_golden.py), decode == prefill;
 *                      layer_forward is Linear layers + layer_from_raw
 *
 * Layouts (all row-major, f32 in / f64 or f32 out):
 *   q,k,g,b  [B][Hk][T][K]   (g, b may be [B][Hk][T][1]: gdim/bdim = 1)
 *   v,w      [B][HV][T][V]
 *   S        [B][HV][K][V]
 *   out      [B][HV][T][V]
 * Value head hv reads key head hv / (HV / Hk).  Hk == HV gives the
 * reference's materialised layout.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define GDN2O_EXPORT __attribute__((visibility("default")))

static inline size_t idx4(size_t a, size_t A1, size_t b, size_t A2, size_t c, size_t A3, size_t d) {
    return ((a * A1 + b) * A2 + c) * A3 + d;
}

GDN2O_EXPORT int gdn2o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

GDN2O_EXPORT void gdn2o_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* Per-token recurrence (src/kernel/fused_recurrent.rs:27-52), double.       */
/*   S <- diag(exp(g_t)) S                                                   */
/*   v_new = w_t * v_t - S^T (b_t * k_t)                                     */
/*   S <- S + k_t v_new^T                                                    */
/*   o_t = scale * S^T q_t                                                   */
/* S0 may be NULL (zero state).                                              */
/* ------------------------------------------------------------------------ */
GDN2O_EXPORT void gdn2o_recurrent_f64(const float *q, const float *k, const float *v, const float *g,
                                      const float *b, const float *w, const double *S0, int B, int HV,
                                      int Hk, int T, int K, int V, int gdim, int bdim, double scale,
                                      double *out, double *S_out) {
    const int rep = HV / Hk;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * HV; ++bh) {
        const int bi = bh / HV, hv = bh % HV, hk = hv / rep;
        double *S = (double *)malloc(sizeof(double) * (size_t)K * V);
        double *vnew = (double *)malloc(sizeof(double) * (size_t)V);
        if (S0)
            memcpy(S, S0 + (size_t)bh * K * V, sizeof(double) * (size_t)K * V);
        else
            memset(S, 0, sizeof(double) * (size_t)K * V);
        for (int t = 0; t < T; ++t) {
            const float *qt = q + idx4(bi, Hk, hk, T, t, K, 0);
            const float *kt = k + idx4(bi, Hk, hk, T, t, K, 0);
            const float *gt = g + idx4(bi, Hk, hk, T, t, gdim, 0);
            const float *bt = b + idx4(bi, Hk, hk, T, t, bdim, 0);
            const float *vt = v + idx4(bi, HV, hv, T, t, V, 0);
            const float *wt = w + idx4(bi, HV, hv, T, t, V, 0);
            for (int i = 0; i < K; ++i) {
                const double eg = exp((double)gt[i % gdim]);
                for (int j = 0; j < V; ++j) S[(size_t)i * V + j] *= eg;
            }
            for (int j = 0; j < V; ++j) vnew[j] = (double)wt[j] * (double)vt[j];
            for (int i = 0; i < K; ++i) {
                const double bk = (double)bt[i % bdim] * (double)kt[i];
                for (int j = 0; j < V; ++j) vnew[j] -= S[(size_t)i * V + j] * bk;
            }
            for (int i = 0; i < K; ++i) {
                const double ki = kt[i];
                for (int j = 0; j < V; ++j) S[(size_t)i * V + j] += ki * vnew[j];
            }
            double *ot = out + idx4(bi, HV, hv, T, t, V, 0);
            for (int j = 0; j < V; ++j) ot[j] = 0.0;
            for (int i = 0; i < K; ++i) {
                const double qi = qt[i];
                for (int j = 0; j < V; ++j) ot[j] += S[(size_t)i * V + j] * qi;
            }
            for (int j = 0; j < V; ++j) ot[j] *= scale;
        }
        if (S_out) memcpy(S_out + (size_t)bh * K * V, S, sizeof(double) * (size_t)K * V);
        free(S);
        free(vnew);
    }
}

/* ------------------------------------------------------------------------ */
/* Adjoint of the per-token recurrence above, in double: the exact gradient  */
/* of L = sum(d_out * out) + sum(d_ST * S_T) with respect to q, k, g, b, v,  */
/* w and S0.  The reference's training path differentiates the same          */
/* recurrence through burn's autodiff (tests/autodiff.rs:153-206), and its   */
/* WIP fused backward (src/kernel/chunk_adjoint_cube.rs:464-707) returns      */
/* the same seven gradients.  Per token t, backwards (S1 = diag(e^g) S_prev, */
/* kb = b*k, S2 = S1 + k vnew^T = S_t):                                      */
/*   dS2 = dS + scale q dO^T;  dq = scale S2 dO                               */
/*   dk += dS2 vnew;  dvnew = dS2^T k;  dw = dvnew*v;  dv = dvnew*w          */
/*   dS1 = dS2 - kb dvnew^T;  dkb = -S1 dvnew;  db = dkb*k;  dk += dkb*b     */
/*   dg = rowsum(dS1 * S1);  dS = diag(e^g) dS1                               */
/* Key-side gradients (dq, dk, dg, db) of a key head sum over its value      */
/* heads; with gdim / bdim = 1 they sum over channels.  d_ST may be NULL     */
/* (zero).  dS0 receives the gradient of S0 (zero S0 when S0 is NULL).       */
/* ------------------------------------------------------------------------ */
static void rec_bwd_d(const double *q, const double *k, const double *v, const double *g,
                                          const double *b, const double *w, const double *S0, const double *d_out,
                                          const double *d_ST, int B, int HV, int Hk, int T, int K, int V, int gdim,
                                          int bdim, double scale, double *dq, double *dk, double *dg, double *db,
                                          double *dv, double *dw, double *dS0) {
    const int rep = HV / Hk;
    memset(dq, 0, sizeof(double) * (size_t)B * Hk * T * K);
    memset(dk, 0, sizeof(double) * (size_t)B * Hk * T * K);
    memset(dg, 0, sizeof(double) * (size_t)B * Hk * T * gdim);
    memset(db, 0, sizeof(double) * (size_t)B * Hk * T * bdim);
#pragma omp parallel for schedule(dynamic, 1)
    for (int bk = 0; bk < B * Hk; ++bk) {
        const int bi = bk / Hk, hk = bk % Hk;
        const size_t KV = (size_t)K * V;
        double *Sall = (double *)malloc(sizeof(double) * KV * (size_t)(T + 1));
        double *S1 = (double *)malloc(sizeof(double) * KV);
        double *dS = (double *)malloc(sizeof(double) * KV);
        double *vnew = (double *)malloc(sizeof(double) * (size_t)V);
        double *dvn = (double *)malloc(sizeof(double) * (size_t)V);
        double *eg = (double *)malloc(sizeof(double) * (size_t)K);
        double *kb = (double *)malloc(sizeof(double) * (size_t)K);
        for (int hv = hk * rep; hv < (hk + 1) * rep; ++hv) {
            const size_t bh = (size_t)bi * HV + hv;
            /* forward, keeping every state S_0 .. S_T */
            if (S0)
                memcpy(Sall, S0 + bh * KV, sizeof(double) * KV);
            else
                memset(Sall, 0, sizeof(double) * KV);
            for (int t = 0; t < T; ++t) {
                const double *kt = k + idx4(bi, Hk, hk, T, t, K, 0);
                const double *gt = g + idx4(bi, Hk, hk, T, t, gdim, 0);
                const double *bt = b + idx4(bi, Hk, hk, T, t, bdim, 0);
                const double *vt = v + idx4(bi, HV, hv, T, t, V, 0);
                const double *wt = w + idx4(bi, HV, hv, T, t, V, 0);
                const double *Sp = Sall + (size_t)t * KV;
                double *Sn = Sall + (size_t)(t + 1) * KV;
                for (int i = 0; i < K; ++i) {
                    const double e = exp((double)gt[i % gdim]);
                    for (int j = 0; j < V; ++j) Sn[(size_t)i * V + j] = Sp[(size_t)i * V + j] * e;
                }
                for (int j = 0; j < V; ++j) vnew[j] = (double)wt[j] * (double)vt[j];
                for (int i = 0; i < K; ++i) {
                    const double bki = (double)bt[i % bdim] * (double)kt[i];
                    for (int j = 0; j < V; ++j) vnew[j] -= Sn[(size_t)i * V + j] * bki;
                }
                for (int i = 0; i < K; ++i)
                    for (int j = 0; j < V; ++j) Sn[(size_t)i * V + j] += (double)kt[i] * vnew[j];
            }
            /* backward */
            if (d_ST)
                memcpy(dS, d_ST + bh * KV, sizeof(double) * KV);
            else
                memset(dS, 0, sizeof(double) * KV);
            for (int t = T - 1; t >= 0; --t) {
                const double *qt = q + idx4(bi, Hk, hk, T, t, K, 0);
                const double *kt = k + idx4(bi, Hk, hk, T, t, K, 0);
                const double *gt = g + idx4(bi, Hk, hk, T, t, gdim, 0);
                const double *bt = b + idx4(bi, Hk, hk, T, t, bdim, 0);
                const double *vt = v + idx4(bi, HV, hv, T, t, V, 0);
                const double *wt = w + idx4(bi, HV, hv, T, t, V, 0);
                const double *dOt = d_out + idx4(bi, HV, hv, T, t, V, 0);
                const double *Sp = Sall + (size_t)t * KV, *S2 = Sall + (size_t)(t + 1) * KV;
                double *dqt = dq + idx4(bi, Hk, hk, T, t, K, 0), *dkt = dk + idx4(bi, Hk, hk, T, t, K, 0);
                double *dgt = dg + idx4(bi, Hk, hk, T, t, gdim, 0), *dbt = db + idx4(bi, Hk, hk, T, t, bdim, 0);
                double *dvt = dv + idx4(bi, HV, hv, T, t, V, 0), *dwt = dw + idx4(bi, HV, hv, T, t, V, 0);
                for (int i = 0; i < K; ++i) {
                    eg[i] = exp((double)gt[i % gdim]);
                    kb[i] = (double)bt[i % bdim] * (double)kt[i];
                    for (int j = 0; j < V; ++j) S1[(size_t)i * V + j] = Sp[(size_t)i * V + j] * eg[i];
                }
                for (int j = 0; j < V; ++j) vnew[j] = (double)wt[j] * (double)vt[j];
                for (int i = 0; i < K; ++i)
                    for (int j = 0; j < V; ++j) vnew[j] -= S1[(size_t)i * V + j] * kb[i];
                /* o_t = scale S2^T q_t */
                for (int i = 0; i < K; ++i) {
                    double a = 0.0;
                    for (int j = 0; j < V; ++j) {
                        dS[(size_t)i * V + j] += scale * (double)qt[i] * dOt[j];
                        a += S2[(size_t)i * V + j] * dOt[j];
                    }
                    dqt[i] += scale * a;
                }
                /* S2 = S1 + k vnew^T */
                for (int j = 0; j < V; ++j) dvn[j] = 0.0;
                for (int i = 0; i < K; ++i) {
                    double a = 0.0;
                    for (int j = 0; j < V; ++j) {
                        a += dS[(size_t)i * V + j] * vnew[j];
                        dvn[j] += dS[(size_t)i * V + j] * (double)kt[i];
                    }
                    dkt[i] += a;
                }
                /* vnew = w v - S1^T kb */
                for (int j = 0; j < V; ++j) {
                    dwt[j] = dvn[j] * (double)vt[j];
                    dvt[j] = dvn[j] * (double)wt[j];
                }
                for (int i = 0; i < K; ++i) {
                    double dkb = 0.0, dgi = 0.0;
                    for (int j = 0; j < V; ++j) {
                        dkb -= S1[(size_t)i * V + j] * dvn[j];
                        dS[(size_t)i * V + j] -= kb[i] * dvn[j];
                        dgi += dS[(size_t)i * V + j] * S1[(size_t)i * V + j];
                        dS[(size_t)i * V + j] *= eg[i];
                    }
                    dbt[i % bdim] += dkb * (double)kt[i];
                    dkt[i] += dkb * (double)bt[i % bdim];
                    dgt[i % gdim] += dgi;
                }
            }
            memcpy(dS0 + bh * KV, dS, sizeof(double) * KV);
        }
        free(Sall);
        free(S1);
        free(dS);
        free(vnew);
        free(dvn);
        free(eg);
        free(kb);
    }
}

/* Inputs in double (the layer adjoint feeds its own double operands). */
GDN2O_EXPORT void gdn2o_recurrent_bwd_d(const double *q, const double *k, const double *v, const double *g,
                                        const double *b, const double *w, const double *S0, const double *d_out,
                                        const double *d_ST, int B, int HV, int Hk, int T, int K, int V, int gdim,
                                        int bdim, double scale, double *dq, double *dk, double *dg, double *db,
                                        double *dv, double *dw, double *dS0) {
    rec_bwd_d(q, k, v, g, b, w, S0, d_out, d_ST, B, HV, Hk, T, K, V, gdim, bdim, scale, dq, dk, dg, db, dv, dw,
              dS0);
}

static double *widen(const float *x, size_t n) {
    double *y = (double *)malloc(sizeof(double) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) y[i] = (double)x[i];
    return y;
}

GDN2O_EXPORT void gdn2o_recurrent_bwd_f64(const float *q, const float *k, const float *v, const float *g,
                                          const float *b, const float *w, const double *S0, const double *d_out,
                                          const double *d_ST, int B, int HV, int Hk, int T, int K, int V, int gdim,
                                          int bdim, double scale, double *dq, double *dk, double *dg, double *db,
                                          double *dv, double *dw, double *dS0) {
    const size_t nk = (size_t)B * Hk * T, nv = (size_t)B * HV * T * V;
    double *qd = widen(q, nk * K), *kd = widen(k, nk * K), *gd = widen(g, nk * gdim), *bd = widen(b, nk * bdim);
    double *vd = widen(v, nv), *wd = widen(w, nv);
    rec_bwd_d(qd, kd, vd, gd, bd, wd, S0, d_out, d_ST, B, HV, Hk, T, K, V, gdim, bdim, scale, dq, dk, dg, db, dv,
              dw, dS0);
    free(qd); free(kd); free(gd); free(bd); free(vd); free(wd);
}

/* Same scan in f32 with the reference's tensor-op order
 * (src/kernel/fused_recurrent.rs:25-52): g pre-exponentiated, state decayed,
 * erase = sum_k(S * (b*k)), v_new = w*v - erase, S += k v_new, o = sum_k(S*q)*scale. */
GDN2O_EXPORT void gdn2o_recurrent_f32(const float *q, const float *k, const float *v, const float *g,
                                      const float *b, const float *w, const float *S0, int B, int HV,
                                      int Hk, int T, int K, int V, int gdim, int bdim, double scale,
                                      float *out, float *S_out) {
    const int rep = HV / Hk;
    const float fscale = (float)scale;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * HV; ++bh) {
        const int bi = bh / HV, hv = bh % HV, hk = hv / rep;
        float *S = (float *)malloc(sizeof(float) * (size_t)K * V);
        float *acc = (float *)malloc(sizeof(float) * (size_t)V);
        if (S0)
            memcpy(S, S0 + (size_t)bh * K * V, sizeof(float) * (size_t)K * V);
        else
            memset(S, 0, sizeof(float) * (size_t)K * V);
        for (int t = 0; t < T; ++t) {
            const float *qt = q + idx4(bi, Hk, hk, T, t, K, 0);
            const float *kt = k + idx4(bi, Hk, hk, T, t, K, 0);
            const float *gt = g + idx4(bi, Hk, hk, T, t, gdim, 0);
            const float *bt = b + idx4(bi, Hk, hk, T, t, bdim, 0);
            const float *vt = v + idx4(bi, HV, hv, T, t, V, 0);
            const float *wt = w + idx4(bi, HV, hv, T, t, V, 0);
            for (int i = 0; i < K; ++i) {
                const float eg = expf(gt[i % gdim]);
                for (int j = 0; j < V; ++j) S[(size_t)i * V + j] *= eg;
            }
            for (int j = 0; j < V; ++j) acc[j] = 0.0f;
            for (int i = 0; i < K; ++i) {
                const float bk = bt[i % bdim] * kt[i];
                for (int j = 0; j < V; ++j) acc[j] += S[(size_t)i * V + j] * bk;
            }
            for (int j = 0; j < V; ++j) acc[j] = wt[j] * vt[j] - acc[j];
            for (int i = 0; i < K; ++i) {
                const float ki = kt[i];
                for (int j = 0; j < V; ++j) S[(size_t)i * V + j] += ki * acc[j];
            }
            float *ot = out + idx4(bi, HV, hv, T, t, V, 0);
            for (int j = 0; j < V; ++j) ot[j] = 0.0f;
            for (int i = 0; i < K; ++i) {
                const float qi = qt[i];
                for (int j = 0; j < V; ++j) ot[j] += S[(size_t)i * V + j] * qi;
            }
            for (int j = 0; j < V; ++j) ot[j] *= fscale;
        }
        if (S_out) memcpy(S_out + (size_t)bh * K * V, S, sizeof(float) * (size_t)K * V);
        free(S);
        free(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* Chunked WY forward (src/forward.rs:44-278), f32, restated per (b, hv).     */
/* Every quantity below is the reference's, with the same tile-local decay:  */
/*   G       = cumsum_t g            (per channel, over the padded chunk)    */
/*   Gb[p]   = G at the last row of tile p-1 (0 for p = 0)   (:109-129)      */
/*   gre     = exp(G - Gb[tile])                             (:138-139)      */
/*   gamma   = exp(G)                                        (:141-142)      */
/*   eblk    = exp(min(Gb[p_r] - Gb[p_s], 0))                (:146-157)      */
/*   Aqk[r,s]= scale*sum_c q_r gre_r (k_s/gre_s) eblk, causal (:163-186)     */
/*   Akk[r,s]= sum_c b_r k_r gre_r (k_s/gre_s) eblk, strict   (:183-187)     */
/*   (I+Akk)[W|U] = [b k gamma | w v] by 16-tile blocks       (:189-261)     */
/*   v_new = U - W S; out = Aqk v_new + scale (q gamma) S     (:263-268)     */
/*   S <- gamma_last S + (k exp(G_last - G))^T v_new          (:271-274)     */
/* The k/gre factor overflows when 16 |g| > 88 (as in the reference).        */
/* ------------------------------------------------------------------------ */
GDN2O_EXPORT void gdn2o_chunk_wy_f32(const float *q, const float *k, const float *v, const float *g,
                                     const float *b, const float *w, const float *S0, int B, int HV,
                                     int Hk, int T, int K, int V, int gdim, int bdim, double scale,
                                     int chunk_size, float *out, float *S_out) {
    const int rep = HV / Hk;
    const int TILE = 16;
    const int cmax_pad = ((chunk_size + TILE - 1) / TILE) * TILE;
    const float fscale = (float)scale;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * HV; ++bh) {
        const int bi = bh / HV, hv = bh % HV, hk = hv / rep;
        const int CP = cmax_pad;
        float *S = (float *)malloc(sizeof(float) * (size_t)K * V);
        float *qp = (float *)calloc((size_t)CP * K, sizeof(float));
        float *kp = (float *)calloc((size_t)CP * K, sizeof(float));
        float *gp = (float *)calloc((size_t)CP * gdim, sizeof(float));
        float *bp = (float *)calloc((size_t)CP * bdim, sizeof(float));
        float *vp = (float *)calloc((size_t)CP * V, sizeof(float));
        float *wp = (float *)calloc((size_t)CP * V, sizeof(float));
        float *G = (float *)malloc(sizeof(float) * (size_t)CP * gdim);
        float *gre = (float *)malloc(sizeof(float) * (size_t)CP * gdim);
        float *gam = (float *)malloc(sizeof(float) * (size_t)CP * gdim);
        float *Gb = (float *)malloc(sizeof(float) * (size_t)(CP / TILE) * gdim);
        float *aqk = (float *)malloc(sizeof(float) * (size_t)CP * CP);
        float *akk = (float *)malloc(sizeof(float) * (size_t)CP * CP);
        float *Ww = (float *)malloc(sizeof(float) * (size_t)CP * K);
        float *U = (float *)malloc(sizeof(float) * (size_t)CP * V);
        float *vn = (float *)malloc(sizeof(float) * (size_t)CP * V);
        float *kq = (float *)malloc(sizeof(float) * (size_t)CP);
        if (S0)
            memcpy(S, S0 + (size_t)bh * K * V, sizeof(float) * (size_t)K * V);
        else
            memset(S, 0, sizeof(float) * (size_t)K * V);

        for (int cs = 0; cs < T; cs += chunk_size) {
            const int ce = cs + chunk_size < T ? cs + chunk_size : T;
            const int c = ce - cs;
            const int cp = ((c + TILE - 1) / TILE) * TILE;
            const int nt = cp / TILE;
            /* pad_time (:34-41, :94-99) */
            memset(qp, 0, sizeof(float) * (size_t)cp * K);
            memset(kp, 0, sizeof(float) * (size_t)cp * K);
            memset(gp, 0, sizeof(float) * (size_t)cp * gdim);
            memset(bp, 0, sizeof(float) * (size_t)cp * bdim);
            memset(vp, 0, sizeof(float) * (size_t)cp * V);
            memset(wp, 0, sizeof(float) * (size_t)cp * V);
            for (int t = 0; t < c; ++t) {
                memcpy(qp + (size_t)t * K, q + idx4(bi, Hk, hk, T, cs + t, K, 0), sizeof(float) * K);
                memcpy(kp + (size_t)t * K, k + idx4(bi, Hk, hk, T, cs + t, K, 0), sizeof(float) * K);
                memcpy(gp + (size_t)t * gdim, g + idx4(bi, Hk, hk, T, cs + t, gdim, 0), sizeof(float) * gdim);
                memcpy(bp + (size_t)t * bdim, b + idx4(bi, Hk, hk, T, cs + t, bdim, 0), sizeof(float) * bdim);
                memcpy(vp + (size_t)t * V, v + idx4(bi, HV, hv, T, cs + t, V, 0), sizeof(float) * V);
                memcpy(wp + (size_t)t * V, w + idx4(bi, HV, hv, T, cs + t, V, 0), sizeof(float) * V);
            }
            /* cumsum via tril matmul (:104-108) */
            for (int ch = 0; ch < gdim; ++ch) {
                float acc = 0.0f;
                for (int t = 0; t < cp; ++t) {
                    acc += gp[(size_t)t * gdim + ch];
                    G[(size_t)t * gdim + ch] = acc;
                }
            }
            for (int ch = 0; ch < gdim; ++ch) {
                Gb[ch] = 0.0f;
                for (int p = 1; p < nt; ++p) Gb[(size_t)p * gdim + ch] = G[(size_t)(p * TILE - 1) * gdim + ch];
            }
            for (int t = 0; t < cp; ++t)
                for (int ch = 0; ch < gdim; ++ch) {
                    const float Gt = G[(size_t)t * gdim + ch];
                    gre[(size_t)t * gdim + ch] = expf(Gt - Gb[(size_t)(t / TILE) * gdim + ch]);
                    gam[(size_t)t * gdim + ch] = expf(Gt);
                }
            /* A_qk, A_kk channel sums (:159-187) */
            for (int r = 0; r < cp; ++r)
                for (int s = 0; s < cp; ++s) {
                    float a1 = 0.0f, a2 = 0.0f;
                    const int pr = r / TILE, ps = s / TILE;
                    for (int kk = 0; kk < K; ++kk) {
                        const int gc = kk % gdim, bc = kk % bdim;
                        float d = Gb[(size_t)pr * gdim + gc] - Gb[(size_t)ps * gdim + gc];
                        if (d > 0.0f) d = 0.0f;
                        const float e = expf(d);
                        const float gr = gre[(size_t)r * gdim + gc];
                        const float ks = kp[(size_t)s * K + kk] / gre[(size_t)s * gdim + gc];
                        a1 += (qp[(size_t)r * K + kk] * gr) * ks * e;
                        a2 += ((bp[(size_t)r * bdim + bc] * kp[(size_t)r * K + kk]) * gr) * ks * e;
                    }
                    aqk[(size_t)r * cp + s] = (s <= r) ? a1 * fscale : 0.0f;
                    akk[(size_t)r * cp + s] = (s < r) ? a2 : 0.0f;
                }
            /* rhs (:189-190) and blocked WY solve (:197-261) */
            for (int t = 0; t < cp; ++t) {
                for (int kk = 0; kk < K; ++kk)
                    Ww[(size_t)t * K + kk] =
                        bp[(size_t)t * bdim + kk % bdim] * kp[(size_t)t * K + kk] * gam[(size_t)t * gdim + kk % gdim];
                for (int j = 0; j < V; ++j) U[(size_t)t * V + j] = wp[(size_t)t * V + j] * vp[(size_t)t * V + j];
            }
            for (int p = 0; p < nt; ++p) {
                const int r0 = p * TILE;
                /* inter-tile: wb = rhs - T_pq W_prev (rows of previous tiles are final) */
                for (int i = 0; i < TILE; ++i) {
                    const int r = r0 + i;
                    for (int s = 0; s < r0; ++s) {
                        const float a = akk[(size_t)r * cp + s];
                        if (a == 0.0f) continue;
                        for (int kk = 0; kk < K; ++kk) Ww[(size_t)r * K + kk] -= a * Ww[(size_t)s * K + kk];
                        for (int j = 0; j < V; ++j) U[(size_t)r * V + j] -= a * U[(size_t)s * V + j];
                    }
                }
                /* in-tile forward substitution */
                for (int i = 1; i < TILE; ++i) {
                    const int r = r0 + i;
                    for (int jj = 0; jj < i; ++jj) {
                        const int s = r0 + jj;
                        const float a = akk[(size_t)r * cp + s];
                        for (int kk = 0; kk < K; ++kk) Ww[(size_t)r * K + kk] -= a * Ww[(size_t)s * K + kk];
                        for (int j = 0; j < V; ++j) U[(size_t)r * V + j] -= a * U[(size_t)s * V + j];
                    }
                }
            }
            /* v_new = U - W S (:264) */
            for (int t = 0; t < cp; ++t) {
                float *vr = vn + (size_t)t * V;
                for (int j = 0; j < V; ++j) vr[j] = 0.0f;
                for (int kk = 0; kk < K; ++kk) {
                    const float a = Ww[(size_t)t * K + kk];
                    const float *Sr = S + (size_t)kk * V;
                    for (int j = 0; j < V; ++j) vr[j] += a * Sr[j];
                }
                for (int j = 0; j < V; ++j) vr[j] = U[(size_t)t * V + j] - vr[j];
            }
            /* out = Aqk v_new + scale (q gamma) S (:265-268) */
            for (int t = 0; t < c; ++t) {
                float *ot = out + idx4(bi, HV, hv, T, cs + t, V, 0);
                float *tmp = U + (size_t)t * V; /* U row t no longer needed: reuse as scratch */
                for (int j = 0; j < V; ++j) ot[j] = 0.0f;
                for (int s = 0; s <= t; ++s) {
                    const float a = aqk[(size_t)t * cp + s];
                    const float *vr = vn + (size_t)s * V;
                    for (int j = 0; j < V; ++j) ot[j] += a * vr[j];
                }
                for (int j = 0; j < V; ++j) tmp[j] = 0.0f;
                for (int kk = 0; kk < K; ++kk) {
                    const float a = qp[(size_t)t * K + kk] * gam[(size_t)t * gdim + kk % gdim];
                    const float *Sr = S + (size_t)kk * V;
                    for (int j = 0; j < V; ++j) tmp[j] += a * Sr[j];
                }
                for (int j = 0; j < V; ++j) ot[j] += tmp[j] * fscale;
            }
            /* S <- gamma_last S + (k decay_last)^T v_new (:271-274) */
            for (int kk = 0; kk < K; ++kk) {
                const int gc = kk % gdim;
                const float gl = gam[(size_t)(c - 1) * gdim + gc];
                const float Gl = G[(size_t)(c - 1) * gdim + gc];
                for (int t = 0; t < cp; ++t) kq[t] = kp[(size_t)t * K + kk] * expf(Gl - G[(size_t)t * gdim + gc]);
                float *Sr = S + (size_t)kk * V;
                for (int j = 0; j < V; ++j) Sr[j] *= gl;
                for (int t = 0; t < cp; ++t) {
                    const float a = kq[t];
                    const float *vr = vn + (size_t)t * V;
                    for (int j = 0; j < V; ++j) Sr[j] += a * vr[j];
                }
            }
        }
        if (S_out) memcpy(S_out + (size_t)bh * K * V, S, sizeof(float) * (size_t)K * V);
        free(S); free(qp); free(kp); free(gp); free(bp); free(vp); free(wp);
        free(G); free(gre); free(gam); free(Gb); free(aqk); free(akk);
        free(Ww); free(U); free(vn); free(kq);
    }
}

/* ------------------------------------------------------------------------ */
/* Layer glue in double (src/module.rs, src/short_conv.rs, src/l2norm.rs).   */
/* ------------------------------------------------------------------------ */
static inline double silu_d(double x) { return x / (1.0 + exp(-x)); }
static inline double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }
static inline double softplus_d(double x) { return x > 30.0 ? x + log1p(exp(-x)) : log1p(exp(x)); }

/* Causal depthwise conv k=4 + SiLU (src/short_conv.rs:22-65).
 * x [B][T][Cn], w [Cn][4], cache [B][3][Cn] or NULL (replicate first row).
 * Writes y [B][T][Cn] and new_cache [B][3][Cn] = last 3 rows of cat(pad|cache, x). */
GDN2O_EXPORT void gdn2o_short_conv(const double *x, const float *wconv, const double *cache, int B, int T,
                                   int Cn, double *y, double *new_cache) {
    for (int bi = 0; bi < B; ++bi) {
        const int L = T + 3;
        double *xp = (double *)malloc(sizeof(double) * (size_t)L * Cn);
        for (int r = 0; r < 3; ++r)
            for (int c = 0; c < Cn; ++c)
                xp[(size_t)r * Cn + c] = cache ? cache[((size_t)bi * 3 + r) * Cn + c] : x[((size_t)bi * T + 0) * Cn + c];
        memcpy(xp + (size_t)3 * Cn, x + (size_t)bi * T * Cn, sizeof(double) * (size_t)T * Cn);
        for (int t = 0; t < T; ++t)
            for (int c = 0; c < Cn; ++c) {
                double acc = 0.0;
                for (int i = 0; i < 4; ++i) acc += xp[(size_t)(t + i) * Cn + c] * (double)wconv[(size_t)c * 4 + i];
                y[((size_t)bi * T + t) * Cn + c] = silu_d(acc);
            }
        if (new_cache)
            memcpy(new_cache + (size_t)bi * 3 * Cn, xp + (size_t)T * Cn, sizeof(double) * 3 * (size_t)Cn);
        free(xp);
    }
}

/* rows of length n: x / sqrt(sum x^2 + eps) (src/l2norm.rs:13-16) */
GDN2O_EXPORT void gdn2o_l2norm_rows(double *x, long rows, int n, double eps) {
    for (long r = 0; r < rows; ++r) {
        double s = 0.0;
        for (int i = 0; i < n; ++i) s += x[r * n + i] * x[r * n + i];
        const double inv = 1.0 / sqrt(s + eps);
        for (int i = 0; i < n; ++i) x[r * n + i] *= inv;
    }
}

/* y = x / sqrt(mean x^2 + eps) * w * silu(gate), rows of length n
 * (src/module.rs:501-517). */
GDN2O_EXPORT void gdn2o_rmsnorm_gate(const double *x, const double *gate, const float *wn, long rows, int n,
                                     double eps, double *y) {
    for (long r = 0; r < rows; ++r) {
        double s = 0.0;
        for (int i = 0; i < n; ++i) s += x[r * n + i] * x[r * n + i];
        const double rms = sqrt(s / n + eps);
        for (int i = 0; i < n; ++i) y[r * n + i] = x[r * n + i] / rms * (double)wn[i] * silu_d(gate[r * n + i]);
    }
}

/* y[M][N] = x[M][Kd] W[Kd][N] (+ bias[N]); W in burn's [in, out] layout.
 * Every element is bias + sum over kk = 0, 1, .. of x[m][kk] W[kk][n], added in
 * that order.  Blocks of LIN_MB rows x LIN_NB columns keep their W rows in cache
 * across the block's rows (one pass over W per LIN_MB rows, not per row), which
 * keeps D = 2048 layers over thousands of tokens at seconds. */
#define LIN_MB 8
#define LIN_NB 256
static void linear_d(const double *x, const float *W, const float *bias, long M, int Kd, int N, double *y) {
    const long nmb = (M + LIN_MB - 1) / LIN_MB, nnb = (N + LIN_NB - 1) / LIN_NB;
#pragma omp parallel for schedule(dynamic, 1)
    for (long blk = 0; blk < nmb * nnb; ++blk) {
        const long m0 = (blk / nnb) * LIN_MB, n0 = (blk % nnb) * LIN_NB;
        const int mb = (int)(M - m0 < LIN_MB ? M - m0 : LIN_MB), nb = (int)(N - n0 < LIN_NB ? N - n0 : LIN_NB);
        double acc[LIN_MB][LIN_NB];
        for (int i = 0; i < mb; ++i)
            for (int n = 0; n < nb; ++n) acc[i][n] = bias ? (double)bias[n0 + n] : 0.0;
        for (int kk = 0; kk < Kd; ++kk) {
            const float *Wr = W + (size_t)kk * N + n0;
            for (int i = 0; i < mb; ++i) {
                const double a = x[(m0 + i) * Kd + kk];
                for (int n = 0; n < nb; ++n) acc[i][n] += a * (double)Wr[n];
            }
        }
        for (int i = 0; i < mb; ++i) memcpy(y + (m0 + i) * N + n0, acc[i], sizeof(double) * nb);
    }
}

/* Layer configuration (src/config.rs:23-58) in the oracle's own terms. */
typedef struct {
    int hidden, heads, head_dim, num_v_heads, head_v_dim;
    int use_short_conv, allow_neg_eigval, mode_chunk, chunk_size;
    int has_min_decay;
    double min_decay, norm_eps;
    int gva_scrambled; /* 1: reproduce the reference's unsqueeze/repeat/reshape (src/module.rs:456-468) */
} gdn2o_cfg;

/* Parameters in burn layout: Linear weights [in][out]. */
typedef struct {
    const float *q_proj, *k_proj, *v_proj, *f_proj_0, *f_proj_1, *b_proj, *w_proj, *g_proj_0, *g_proj_1,
        *g_proj_1_bias, *a_log, *dt_bias, *o_norm_weight, *o_proj, *q_conv_w, *k_conv_w, *v_conv_w,
        *decay_factors;
} gdn2o_weights;

/* [B][T][n][d] -> [B][n][T][d] (to_4d, src/module.rs:395-398) */
static void to_4d(const double *x, int B, int T, int n, int d, double *y) {
    for (int bi = 0; bi < B; ++bi)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < n; ++h)
                memcpy(y + (((size_t)bi * n + h) * T + t) * d, x + (((size_t)bi * T + t) * n + h) * d,
                       sizeof(double) * d);
}

/* GVA repeat of [B][H][T][K] into [B][HV][T][K] with the reference's
 * row-major reshape (src/module.rs:459-463): element (b,h,t,j,:) of the
 * [B,H,T,rep,K] view lands at flat row (h*T + t)*rep + j of [B,HV*T]. */
static void gva_scramble(const double *x, int B, int H, int HV, int T, int K, double *y) {
    const int rep = HV / H;
    for (int bi = 0; bi < B; ++bi)
        for (int h = 0; h < H; ++h)
            for (int t = 0; t < T; ++t)
                for (int j = 0; j < rep; ++j) {
                    const size_t flat = ((size_t)h * T + t) * rep + j;
                    memcpy(y + ((size_t)bi * HV * T + flat) * K, x + (((size_t)bi * H + h) * T + t) * K,
                           sizeof(double) * K);
                }
}

/* Double-precision per-token scan on double inputs (used by the layer). */
static void scan_d(const double *q, const double *k, const double *v, const double *g, const double *b,
                   const double *w, double *S, int B, int HV, int Hk, int T, int K, int V, double scale,
                   double *out) {
    const int rep = HV / Hk;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * HV; ++bh) {
        const int bi = bh / HV, hv = bh % HV, hk = hv / rep;
        double *Sh = S + (size_t)bh * K * V;
        double *vnew = (double *)malloc(sizeof(double) * V);
        for (int t = 0; t < T; ++t) {
            const size_t ko = idx4(bi, Hk, hk, T, t, K, 0), vo = idx4(bi, HV, hv, T, t, V, 0);
            for (int i = 0; i < K; ++i) {
                const double eg = exp(g[ko + i]);
                for (int j = 0; j < V; ++j) Sh[(size_t)i * V + j] *= eg;
            }
            for (int j = 0; j < V; ++j) vnew[j] = w[vo + j] * v[vo + j];
            for (int i = 0; i < K; ++i) {
                const double bk = b[ko + i] * k[ko + i];
                for (int j = 0; j < V; ++j) vnew[j] -= Sh[(size_t)i * V + j] * bk;
            }
            for (int i = 0; i < K; ++i)
                for (int j = 0; j < V; ++j) Sh[(size_t)i * V + j] += k[ko + i] * vnew[j];
            double *ot = out + vo;
            for (int j = 0; j < V; ++j) ot[j] = 0.0;
            for (int i = 0; i < K; ++i)
                for (int j = 0; j < V; ++j) ot[j] += Sh[(size_t)i * V + j] * q[ko + i];
            for (int j = 0; j < V; ++j) ot[j] *= scale;
        }
        free(vnew);
    }
}

/* scan_d for callers: S [B][HV][K][V] in/out, out [B][HV][T][V]. */
GDN2O_EXPORT void gdn2o_scan_d(const double *q, const double *k, const double *v, const double *g, const double *b,
                               const double *w, double *S, int B, int HV, int Hk, int T, int K, int V,
                               double scale, double *out) {
    scan_d(q, k, v, g, b, w, S, B, HV, Hk, T, K, V, scale, out);
}

/*
 * The layer after its Linear layers, in double (src/module.rs:404-476 from
 * the raw projections on, then :244-315 without o_proj):
 *   short conv or SiLU, g = -exp(A_log) softplus(f + dt_bias) (+ min_decay),
 *   b = sigmoid (x2 if allow_neg_eigval), w = sigmoid, head split, L2 norm,
 *   GVA, the exact scan, permute, gated RMSNorm.
 * Raw inputs (Linear outputs, [B][T][n]): q_raw, k_raw, f_raw, b_raw (n = kd),
 * v_raw, w_raw, gate (n = vd; gate includes the g_proj_1 bias).
 * state_S [B][HV][K][V], conv_{q,k,v} [B][3][kd|vd]: in/out (has_state 0 =
 * Option::None on entry).  o_norm [B][T][vd] = input of o_proj.
 * Optional outputs (NULL to skip): o_core [B][HV][T][V] (pre-norm scan
 * output) and the activated operands proj_q/k/g/b [B][Hk][T][K]
 * (Hk = H, or HV with gva_scrambled), proj_v/w [B][HV][T][V].
 */
GDN2O_EXPORT void gdn2o_layer_from_raw(const gdn2o_cfg *cfg, const gdn2o_weights *W, const double *q_raw,
                                       const double *k_raw, const double *f_raw, const double *b_raw,
                                       const double *v_raw, const double *w_raw, const double *gate, int B,
                                       int T, int has_state, double *state_S, double *conv_q, double *conv_k,
                                       double *conv_v, double *o_norm, double *o_core, double *proj_q,
                                       double *proj_k, double *proj_g, double *proj_b, double *proj_v,
                                       double *proj_w) {
    const int H = cfg->heads, K = cfg->head_dim, HV = cfg->num_v_heads, V = cfg->head_v_dim;
    const int kd = H * K, vd = HV * V;
    const long M = (long)B * T;
    double *qa = (double *)malloc(sizeof(double) * M * kd), *ka = (double *)malloc(sizeof(double) * M * kd);
    double *va = (double *)malloc(sizeof(double) * M * vd);
    double *ncq = NULL, *nck = NULL, *ncv = NULL;
    if (cfg->use_short_conv) {
        ncq = (double *)malloc(sizeof(double) * B * 3 * kd);
        nck = (double *)malloc(sizeof(double) * B * 3 * kd);
        ncv = (double *)malloc(sizeof(double) * B * 3 * vd);
        gdn2o_short_conv(q_raw, W->q_conv_w, has_state ? conv_q : NULL, B, T, kd, qa, ncq);
        gdn2o_short_conv(k_raw, W->k_conv_w, has_state ? conv_k : NULL, B, T, kd, ka, nck);
        gdn2o_short_conv(v_raw, W->v_conv_w, has_state ? conv_v : NULL, B, T, vd, va, ncv);
    } else {
        for (long i = 0; i < M * kd; ++i) { qa[i] = silu_d(q_raw[i]); ka[i] = silu_d(k_raw[i]); }
        for (long i = 0; i < M * vd; ++i) va[i] = silu_d(v_raw[i]);
    }
    /* gates (src/module.rs:417-443) */
    double *gg = (double *)malloc(sizeof(double) * M * kd);
    for (long m = 0; m < M; ++m)
        for (int c = 0; c < kd; ++c) {
            const double a = exp((double)W->a_log[c / K]);
            double gv = -a * softplus_d(f_raw[m * kd + c] + (double)W->dt_bias[c]);
            if (cfg->has_min_decay) {
                const double f = sigmoid_d((double)W->decay_factors[c]) * (1.0 - cfg->min_decay);
                gv = log(f * exp(gv) + cfg->min_decay);
            }
            gg[m * kd + c] = gv;
        }
    double *bb = (double *)malloc(sizeof(double) * M * kd), *ww = (double *)malloc(sizeof(double) * M * vd);
    for (long i = 0; i < M * kd; ++i) bb[i] = sigmoid_d(b_raw[i]);
    for (long i = 0; i < M * vd; ++i) ww[i] = sigmoid_d(w_raw[i]);

    /* heads split, l2norm, GVA, neg-eig (src/module.rs:445-472) */
    double *q4 = (double *)malloc(sizeof(double) * M * kd), *k4 = (double *)malloc(sizeof(double) * M * kd);
    double *g4 = (double *)malloc(sizeof(double) * M * kd), *b4 = (double *)malloc(sizeof(double) * M * kd);
    double *v4 = (double *)malloc(sizeof(double) * M * vd), *w4 = (double *)malloc(sizeof(double) * M * vd);
    to_4d(qa, B, T, H, K, q4);
    to_4d(ka, B, T, H, K, k4);
    to_4d(va, B, T, HV, V, v4);
    to_4d(gg, B, T, H, K, g4);
    to_4d(bb, B, T, H, K, b4);
    to_4d(ww, B, T, HV, V, w4);
    gdn2o_l2norm_rows(q4, M * H, K, 1e-6);
    gdn2o_l2norm_rows(k4, M * H, K, 1e-6);
    int Hk = H;
    if (HV > H && cfg->gva_scrambled) {
        double *t;
        t = (double *)malloc(sizeof(double) * (size_t)B * HV * T * K); gva_scramble(q4, B, H, HV, T, K, t); free(q4); q4 = t;
        t = (double *)malloc(sizeof(double) * (size_t)B * HV * T * K); gva_scramble(k4, B, H, HV, T, K, t); free(k4); k4 = t;
        t = (double *)malloc(sizeof(double) * (size_t)B * HV * T * K); gva_scramble(g4, B, H, HV, T, K, t); free(g4); g4 = t;
        t = (double *)malloc(sizeof(double) * (size_t)B * HV * T * K); gva_scramble(b4, B, H, HV, T, K, t); free(b4); b4 = t;
        Hk = HV;
    }
    const long nk = (long)B * Hk * T * K;
    if (cfg->allow_neg_eigval)
        for (long i = 0; i < nk; ++i) b4[i] *= 2.0;
    if (proj_q) memcpy(proj_q, q4, sizeof(double) * nk);
    if (proj_k) memcpy(proj_k, k4, sizeof(double) * nk);
    if (proj_g) memcpy(proj_g, g4, sizeof(double) * nk);
    if (proj_b) memcpy(proj_b, b4, sizeof(double) * nk);
    if (proj_v) memcpy(proj_v, v4, sizeof(double) * M * vd);
    if (proj_w) memcpy(proj_w, w4, sizeof(double) * M * vd);

    /* recurrence (src/module.rs:244-296, :336-367) */
    double *S = (double *)calloc((size_t)B * HV * K * V, sizeof(double));
    if (has_state && state_S) memcpy(S, state_S, sizeof(double) * (size_t)B * HV * K * V);
    double *oc = (double *)malloc(sizeof(double) * M * vd);
    scan_d(q4, k4, v4, g4, b4, w4, S, B, HV, Hk, T, K, V, pow((double)K, -0.5), oc);
    if (o_core) memcpy(o_core, oc, sizeof(double) * M * vd);
    if (state_S) memcpy(state_S, S, sizeof(double) * (size_t)B * HV * K * V);
    if (cfg->use_short_conv) {
        if (conv_q) memcpy(conv_q, ncq, sizeof(double) * B * 3 * kd);
        if (conv_k) memcpy(conv_k, nck, sizeof(double) * B * 3 * kd);
        if (conv_v) memcpy(conv_v, ncv, sizeof(double) * B * 3 * vd);
    }

    /* permute -> rmsnorm gate (src/module.rs:310-312) */
    double *o_btv = (double *)malloc(sizeof(double) * M * vd);
    for (int bi = 0; bi < B; ++bi)
        for (int h = 0; h < HV; ++h)
            for (int t = 0; t < T; ++t)
                memcpy(o_btv + (((size_t)bi * T + t) * HV + h) * V, oc + (((size_t)bi * HV + h) * T + t) * V,
                       sizeof(double) * V);
    gdn2o_rmsnorm_gate(o_btv, gate, W->o_norm_weight, M * HV, V, cfg->norm_eps, o_norm);

    free(qa); free(ka); free(va); free(ncq); free(nck); free(ncv); free(gg); free(bb); free(ww);
    free(q4); free(k4); free(g4); free(b4); free(v4); free(w4); free(S); free(oc); free(o_btv);
}

/*
 * GatedDeltaNet2::forward(x, &mut state, true) / forward_train(x) in double
 * (src/module.rs:224-375): the Linear layers (:400-402, :417-418, :442-443,
 * :474-475), gdn2o_layer_from_raw, then o_proj (:313-315).  The chunk and
 * recurrent modes compute the same map, so the oracle evaluates both with
 * the exact double scan; the f32 chunk restatement is checked against it
 * separately.  x [B][T][D] -> out [B][T][D].  Optional raw outputs
 * (q_raw..gate, NULL to skip) expose the Linear outputs.
 */
GDN2O_EXPORT void gdn2o_layer_forward(const gdn2o_cfg *cfg, const gdn2o_weights *W, const float *x, int B,
                                      int T, int has_state, double *state_S, double *conv_q, double *conv_k,
                                      double *conv_v, double *out, double *o_core, double *proj_q,
                                      double *proj_k, double *proj_g, double *proj_b, double *proj_v,
                                      double *proj_w, double *proj_gate) {
    const int D = cfg->hidden, H = cfg->heads, K = cfg->head_dim, HV = cfg->num_v_heads, V = cfg->head_v_dim;
    const int kd = H * K, vd = HV * V;
    const long M = (long)B * T;
    double *xd = (double *)malloc(sizeof(double) * M * D);
    for (long i = 0; i < M * D; ++i) xd[i] = x[i];
    double *qr = (double *)malloc(sizeof(double) * M * kd), *kr = (double *)malloc(sizeof(double) * M * kd);
    double *vr = (double *)malloc(sizeof(double) * M * vd), *br = (double *)malloc(sizeof(double) * M * kd);
    double *wr = (double *)malloc(sizeof(double) * M * vd), *fo = (double *)malloc(sizeof(double) * M * kd);
    double *fh = (double *)malloc(sizeof(double) * M * V), *gh = (double *)malloc(sizeof(double) * M * V);
    double *gate = (double *)malloc(sizeof(double) * M * vd), *on = (double *)malloc(sizeof(double) * M * vd);
    linear_d(xd, W->q_proj, NULL, M, D, kd, qr);
    linear_d(xd, W->k_proj, NULL, M, D, kd, kr);
    linear_d(xd, W->v_proj, NULL, M, D, vd, vr);
    linear_d(xd, W->f_proj_0, NULL, M, D, V, fh);
    linear_d(fh, W->f_proj_1, NULL, M, V, kd, fo);
    linear_d(xd, W->b_proj, NULL, M, D, kd, br);
    linear_d(xd, W->w_proj, NULL, M, D, vd, wr);
    linear_d(xd, W->g_proj_0, NULL, M, D, V, gh);
    linear_d(gh, W->g_proj_1, W->g_proj_1_bias, M, V, vd, gate);
    gdn2o_layer_from_raw(cfg, W, qr, kr, fo, br, vr, wr, gate, B, T, has_state, state_S, conv_q, conv_k, conv_v, on,
                         o_core, proj_q, proj_k, proj_g, proj_b, proj_v, proj_w);
    if (proj_gate) memcpy(proj_gate, gate, sizeof(double) * M * vd);
    if (out) linear_d(on, W->o_proj, NULL, M, vd, D, out);
    free(xd); free(qr); free(kr); free(vr); free(br); free(wr); free(fo); free(fh); free(gh); free(gate); free(on);
}

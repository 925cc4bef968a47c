/*
 * C restatement of the three recurrent operators (SelectiveScanFn,
 * GatedDeltaNet2Fn, Mamba3SisoFn).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle: tests/, the smoke check
 * and the benchmark's cpu_baseline leg load the shared object built from it
 * as the checker.  The product library never links or calls it.
 *
 * The file is compiled twice: with -DXMO_REAL=float -DXMO_SFX=_f32 (every
 * intermediate in fp32, the reference's operation order) and with
 * -DXMO_REAL=double -DXMO_SFX=_f64 (the accuracy yardstick).  Inputs are
 * always fp32 arrays, as the operators receive them; outputs are XMO_REAL.
 *
 * Each function cites the reference file:line it restates.  What pins each
 * function (closed forms, invariants, brute force) is listed in
 * tests/test_oracle_pins.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef XMO_REAL
#define XMO_REAL double
#define XMO_SFX _f64
#endif

#define XMO_CAT2(a, b) a##b
#define XMO_CAT(a, b) XMO_CAT2(a, b)
#define XMO_NAME(base) XMO_CAT(base, XMO_SFX)

typedef XMO_REAL real;

static const float kLog2eF = 1.4426950408889634f;  /* M_LOG2E as float (selective_scan_fwd_kernel.cuh:172) */
static const float kPiF = 3.14159265358979323846f;   /* mamba3_siso_fwd.cu:15 */
static const float kL2EpsF = 1.0e-6f;                /* gated_deltanet2_fwd.cu:14 */

#define IS_F32 (sizeof(real) == sizeof(float))

static real r_exp(real x) { return IS_F32 ? (real)expf((float)x) : (real)exp((double)x); }
static real r_exp2(real x) { return IS_F32 ? (real)exp2f((float)x) : (real)exp2((double)x); }
static real r_log1p(real x) { return IS_F32 ? (real)log1pf((float)x) : (real)log1p((double)x); }
static real r_sqrt(real x) { return IS_F32 ? (real)sqrtf((float)x) : (real)sqrt((double)x); }
static real r_tanh(real x) { return IS_F32 ? (real)tanhf((float)x) : (real)tanh((double)x); }
static real r_floor(real x) { return IS_F32 ? (real)floorf((float)x) : (real)floor((double)x); }
static real r_sin(real x) { return IS_F32 ? (real)sinf((float)x) : (real)sin((double)x); }
static real r_cos(real x) { return IS_F32 ? (real)cosf((float)x) : (real)cos((double)x); }

/* ------------------------------------------------------------------------ */
/* SelectiveScanFn                                                           */
/* ------------------------------------------------------------------------ */

/*
 * Output 0 of SelectiveScanFn for one call.
 *   u, delta: [batch, dim, seqlen]; A: [dim, dstate]
 *   B: b_var ? [batch, groups_b, dstate, seqlen] : [dim, dstate]
 *   C: c_var ? [batch, groups_c, dstate, seqlen] : [dim, dstate]
 *   D, delta_bias: [dim] or NULL.
 *   last_state: [batch, dim, dstate] or NULL; receives h after the last token
 *   (zeros when seqlen == 0), the state the scan carries (the Mamba
 *   selective_scan_fn's last_state).
 * Restates selective_scan_fwd_kernel.cuh:114-127, :150-163, :166-270,
 * :272-281 and selective_scan_fn_ort.cpp:107-117 (n_groups comes from B; when B
 * is constant the group index is 0 for every channel, so a variable C reads
 * group 0).  z never reaches output 0 and is not an argument here.
 */
void XMO_NAME(xmo_selective_scan)(const float *u, const float *delta, const float *A, const float *B,
                                  const float *C, const float *D, const float *delta_bias, int batch,
                                  int dim, int seqlen, int dstate, int b_var, int c_var, int groups_b,
                                  int groups_c, int delta_softplus, real *out, real *last_state) {
    const int ngroups = b_var ? groups_b : 1;
    const int ratio = dim / ngroups;
    const long long nbd = (long long)batch * dim;
#pragma omp parallel
    {
        real *dl = (real *)malloc(sizeof(real) * (size_t)seqlen);
        real *du = (real *)malloc(sizeof(real) * (size_t)seqlen);
#pragma omp for schedule(static)
        for (long long bd = 0; bd < nbd; ++bd) {
            const int b = (int)(bd / dim);
            const int d = (int)(bd % dim);
            const int g = d / ratio;
            const float *ur = u + (size_t)bd * seqlen;
            const float *dr = delta + (size_t)bd * seqlen;
            real *yr = out + (size_t)bd * seqlen;
            const real dval = D ? (real)D[d] : (real)0;
            const real bias = delta_bias ? (real)delta_bias[d] : (real)0;
            for (int t = 0; t < seqlen; ++t) {
                real x = (real)dr[t] + bias;
                if (delta_softplus) x = x <= (real)20 ? r_log1p(r_exp(x)) : x;
                dl[t] = x;
                du[t] = x * (real)ur[t];
                yr[t] = dval * (real)ur[t];
            }
            for (int n = 0; n < dstate; ++n) {
                real a2;
                if (IS_F32) a2 = (real)((float)A[(size_t)d * dstate + n] * kLog2eF);
                else a2 = (real)A[(size_t)d * dstate + n] * (real)1.4426950408889634073599;
                const float *brow = b_var ? B + (((size_t)b * groups_b + g) * dstate + n) * seqlen : NULL;
                const float *crow = NULL;
                if (c_var) {
                    const int gc = b_var ? g : 0;
                    crow = C + (((size_t)b * groups_c + gc) * dstate + n) * seqlen;
                }
                const real bconst = b_var ? (real)0 : (real)B[(size_t)d * dstate + n];
                const real cconst = c_var ? (real)0 : (real)C[(size_t)d * dstate + n];
                const real bc = bconst * cconst;
                real h = 0;
                for (int t = 0; t < seqlen; ++t) {
                    const real a = r_exp2(dl[t] * a2);
                    const real bt = b_var ? (real)brow[t] * du[t] : du[t];
                    h = a * h + bt;
                    real cv;
                    if (c_var) cv = b_var ? (real)crow[t] : bconst * (real)crow[t];
                    else cv = b_var ? cconst : bc;
                    yr[t] += h * cv;
                }
                if (last_state) last_state[(size_t)bd * dstate + n] = h;
            }
        }
        free(dl);
        free(du);
    }
}

/* ------------------------------------------------------------------------ */
/* GatedDeltaNet2Fn                                                          */
/* ------------------------------------------------------------------------ */

/*
 * Output of GatedDeltaNet2Fn.  q, k, g, beta: [batch, seqlen, nheads, dk];
 * v, w: [batch, seqlen, nheads, dv]; s0: [batch, nheads, dk, dv] or NULL;
 * final_state: [batch, nheads, dk, dv] or NULL, receives S after the last
 * token (s0, or zeros, when seqlen == 0).
 * Preparation restates gated_deltanet2_fwd.cu:39-76 (q_mul = scale *
 * rsqrt(sum q^2 + 1e-6), k_mul = rsqrt(sum k^2 + 1e-6), exp(g), beta * khat);
 * the recurrence restates :82-140 (decay, erase, write = w*v - erase, update,
 * readout), which the generic path :142-233 computes identically.
 */
void XMO_NAME(xmo_gated_deltanet2)(const float *q, const float *k, const float *v, const float *g,
                                   const float *beta, const float *w, const float *s0, int batch,
                                   int seqlen, int nheads, int dk, int dv, float scale, int l2norm,
                                   real *out, real *final_state) {
    const int nbh = batch * nheads;
#pragma omp parallel
    {
        real *S = (real *)malloc(sizeof(real) * (size_t)dk * dv);
        real *qn = (real *)malloc(sizeof(real) * (size_t)dk);
        real *kn = (real *)malloc(sizeof(real) * (size_t)dk);
        real *dec = (real *)malloc(sizeof(real) * (size_t)dk);
        real *bk = (real *)malloc(sizeof(real) * (size_t)dk);
        real *er = (real *)malloc(sizeof(real) * (size_t)dv);
        real *ov = (real *)malloc(sizeof(real) * (size_t)dv);
#pragma omp for schedule(dynamic, 1)
        for (int bh = 0; bh < nbh; ++bh) {
            const int b = bh / nheads;
            const int h = bh % nheads;
            if (s0) {
                for (size_t i = 0; i < (size_t)dk * dv; ++i) S[i] = (real)s0[(size_t)bh * dk * dv + i];
            } else {
                memset(S, 0, sizeof(real) * (size_t)dk * dv);
            }
            for (int t = 0; t < seqlen; ++t) {
                const size_t row = ((size_t)b * seqlen + t) * nheads + h;
                const float *qr = q + row * dk, *kr = k + row * dk, *gr = g + row * dk, *br = beta + row * dk;
                const float *vr = v + row * dv, *wr = w + row * dv;
                real qs = 0, ks = 0;
                for (int i = 0; i < dk; ++i) {
                    qs += (real)qr[i] * (real)qr[i];
                    ks += (real)kr[i] * (real)kr[i];
                }
                real qm = (real)scale, km = 1;
                if (l2norm) {
                    qm = (real)scale * ((real)1 / r_sqrt(qs + (real)kL2EpsF));
                    km = (real)1 / r_sqrt(ks + (real)kL2EpsF);
                }
                for (int i = 0; i < dk; ++i) {
                    qn[i] = (real)qr[i] * qm;
                    kn[i] = (real)kr[i] * km;
                    dec[i] = r_exp((real)gr[i]);
                    bk[i] = (real)br[i] * kn[i];
                }
                for (int j = 0; j < dv; ++j) er[j] = 0;
                for (int i = 0; i < dk; ++i) {
                    real *Si = S + (size_t)i * dv;
                    const real di = dec[i], bi = bk[i];
                    for (int j = 0; j < dv; ++j) {
                        Si[j] *= di;
                        er[j] += bi * Si[j];
                    }
                }
                for (int j = 0; j < dv; ++j) {
                    er[j] = (real)wr[j] * (real)vr[j] - er[j]; /* write */
                    ov[j] = 0;
                }
                for (int i = 0; i < dk; ++i) {
                    real *Si = S + (size_t)i * dv;
                    const real ki = kn[i], qi = qn[i];
                    for (int j = 0; j < dv; ++j) {
                        Si[j] += ki * er[j];
                        ov[j] += qi * Si[j];
                    }
                }
                real *orow = out + row * dv;
                for (int j = 0; j < dv; ++j) orow[j] = ov[j];
            }
            if (final_state)
                for (size_t i = 0; i < (size_t)dk * dv; ++i) final_state[(size_t)bh * dk * dv + i] = S[i];
        }
        free(S); free(qn); free(kn); free(dec); free(bk); free(er); free(ov);
    }
}

/* ------------------------------------------------------------------------ */
/* Mamba3SisoFn                                                              */
/* ------------------------------------------------------------------------ */

static real sigmoid_r(real x) { return (real)1 / ((real)1 + r_exp(-x)); }

/*
 * Output of Mamba3SisoFn.  Q, K: [batch, seqlen, nheads_qk, n]; V, Z:
 * [batch, seqlen, nheads, p]; ADT, DT, Trap: [batch, nheads, seqlen];
 * Q_bias, K_bias: [nheads, n]; Angles: [batch, seqlen, nheads, a]; D: [nheads]
 * or NULL; Z may be NULL.  Restates mamba3_siso_fwd.cu:79-171 including the
 * per-step wrap of the angle state (:26-28, :82-86), the unrotated q.k diagonal
 * term (:89-106), rotation of pairs below A (:108-123), the trapezoid look-ahead
 * (:126-134), decay before readout (:140-161) and the update after it (:164-169).
 *
 * States (a widening: the reference rejects has_input_states and
 * return_final_states, mamba3_siso_fn_ort.cpp:50-55).  The state after a call
 * is (ssm [B,H,P,N], angle [B,H,A], k [B,H,N], v [B,H,P]): S and the angle
 * state after the last token (whose look-ahead is 0, :126-134), and that
 * token's rotated k and its v.  A call given these states starts from
 * S = ssm + v (x) k * DT_0 (1 - sigmoid(Trap_0)), the last token's look-ahead
 * now that its successor is known, and the angle state; so two calls chained
 * through the states give the outputs and states of one call.  in_* may be
 * NULL (zero state); f_* may be NULL (not written).
 */
void XMO_NAME(xmo_mamba3_siso)(const float *Q, const float *K, const float *V, const float *ADT,
                               const float *DT, const float *Trap, const float *Qb, const float *Kb,
                               const float *Ang, const float *D, const float *Z, int batch, int seqlen,
                               int nheads, int nheads_qk, int n, int p, int a_dim,
                               const float *in_ssm, const float *in_ang, const float *in_k,
                               const float *in_v, real *out, real *f_ssm, real *f_ang, real *f_k,
                               real *f_v) {
    const int nbh = batch * nheads;
    const int grp = nheads / nheads_qk;
    const real pi = (real)kPiF;
    const real two_pi = IS_F32 ? (real)(2.0f * kPiF) : (real)2 * (real)kPiF;
#pragma omp parallel
    {
        real *S = (real *)malloc(sizeof(real) * (size_t)p * n);
        real *th = (real *)malloc(sizeof(real) * (size_t)(a_dim > 0 ? a_dim : 1));
        real *qv = (real *)malloc(sizeof(real) * (size_t)n);
        real *kv = (real *)malloc(sizeof(real) * (size_t)n);
#pragma omp for schedule(dynamic, 1)
        for (int bh = 0; bh < nbh; ++bh) {
            const int b = bh / nheads;
            const int h = bh % nheads;
            const int gq = h / grp;
            const float *dtr = DT + (size_t)bh * seqlen, *trr = Trap + (size_t)bh * seqlen, *adr = ADT + (size_t)bh * seqlen;
            if (in_ssm) {
                const real look0 = seqlen > 0 ? (real)dtr[0] * ((real)1 - sigmoid_r((real)trr[0])) : (real)0;
                for (int r = 0; r < p; ++r)
                    for (int i = 0; i < n; ++i)
                        S[(size_t)r * n + i] = (real)in_ssm[((size_t)bh * p + r) * n + i] +
                                               (real)in_v[(size_t)bh * p + r] * ((real)in_k[(size_t)bh * n + i] * look0);
                for (int a = 0; a < a_dim; ++a) th[a] = (real)in_ang[(size_t)bh * a_dim + a];
            } else {
                memset(S, 0, sizeof(real) * (size_t)p * n);
                for (int a = 0; a < a_dim; ++a) th[a] = 0;
            }
            for (int t = 0; t < seqlen; ++t) {
                const real dt = (real)dtr[t];
                const float *angr = Ang + (((size_t)b * seqlen + t) * nheads + h) * a_dim;
                for (int a = 0; a < a_dim; ++a) {
                    const real nx = th[a] + r_tanh((real)angr[a]) * dt * pi;
                    th[a] = nx - two_pi * r_floor(nx / two_pi);
                }
                const float *qr = Q + (((size_t)b * seqlen + t) * nheads_qk + gq) * n;
                const float *kr = K + (((size_t)b * seqlen + t) * nheads_qk + gq) * n;
                real qk = 0;
                for (int i = 0; i < n; ++i) {
                    qv[i] = (real)qr[i] + (real)Qb[(size_t)h * n + i];
                    kv[i] = (real)kr[i] + (real)Kb[(size_t)h * n + i];
                    qk += qv[i] * kv[i];
                }
                for (int pr = 0; pr < n / 2; ++pr) {
                    const real phi = pr < a_dim ? th[pr] : (real)0;
                    const real c = r_cos(phi), s = r_sin(phi);
                    const real q0 = qv[2 * pr], q1 = qv[2 * pr + 1];
                    const real k0 = kv[2 * pr], k1 = kv[2 * pr + 1];
                    qv[2 * pr] = q0 * c - q1 * s;
                    qv[2 * pr + 1] = q0 * s + q1 * c;
                    kv[2 * pr] = k0 * c - k1 * s;
                    kv[2 * pr + 1] = k0 * s + k1 * c;
                }
                const real gamma = dt * sigmoid_r((real)trr[t]);
                real shifted = 0;
                if (t + 1 < seqlen) shifted = (real)dtr[t + 1] * ((real)1 - sigmoid_r((real)trr[t + 1]));
                const real ksc = gamma + shifted;
                const real decay = r_exp((real)adr[t]);
                const real diag = (D ? (real)D[h] : (real)0) + qk * gamma;
                const float *vr = V + (((size_t)b * seqlen + t) * nheads + h) * p;
                const float *zr = Z ? Z + (((size_t)b * seqlen + t) * nheads + h) * p : NULL;
                real *orow = out + (((size_t)b * seqlen + t) * nheads + h) * p;
                for (int r = 0; r < p; ++r) {
                    real *Sr = S + (size_t)r * n;
                    real acc = 0;
                    for (int i = 0; i < n; ++i) {
                        Sr[i] *= decay;
                        acc += qv[i] * Sr[i];
                    }
                    real y = acc + diag * (real)vr[r];
                    if (zr) {
                        const real zz = (real)zr[r];
                        y *= zz * sigmoid_r(zz);
                    }
                    orow[r] = y;
                    const real vv = (real)vr[r];
                    for (int i = 0; i < n; ++i) Sr[i] += vv * (kv[i] * ksc);
                }
            }
            if (f_ssm) memcpy(f_ssm + (size_t)bh * p * n, S, sizeof(real) * (size_t)p * n);
            if (f_ang)
                for (int a = 0; a < a_dim; ++a) f_ang[(size_t)bh * a_dim + a] = th[a];
            if (f_k && seqlen > 0)
                for (int i = 0; i < n; ++i) f_k[(size_t)bh * n + i] = kv[i];   /* rotated k of the last token */
            if (f_v && seqlen > 0)
                for (int r = 0; r < p; ++r) f_v[(size_t)bh * p + r] = (real)V[(((size_t)b * seqlen + seqlen - 1) * nheads + h) * p + r];
        }
        free(S); free(th); free(qv); free(kv);
    }
}

/* ---------------------------------------------------------------------------
 * SoftmaxCPU, softmax_cpu_ort.cpp:38-77: one line at a time along the axis,
 * max, then e = exp(x - max) summed in axis order, then e * inv_sum with
 * inv_sum = sum > 0 ? 1 / sum : 0 (:75).  In the fp32 build every operation
 * is the reference's fp32 operation in the reference's order.
 * ------------------------------------------------------------------------- */
void XMO_NAME(xmo_softmax_cpu)(const float *in, size_t outer, size_t axis_dim, size_t inner, real *out) {
    for (size_t o = 0; o < outer; ++o) {
        for (size_t i = 0; i < inner; ++i) {
            const size_t base = o * axis_dim * inner + i;
            real mx = -(real)INFINITY;
            for (size_t a = 0; a < axis_dim; ++a) {
                const real x = (real)in[base + a * inner];
                mx = x > mx ? x : mx;   /* std::max(max, x): keeps max unless x is larger */
            }
            real sum = 0;
            for (size_t a = 0; a < axis_dim; ++a) {
                const real e = r_exp((real)in[base + a * inner] - mx);
                out[base + a * inner] = e;
                sum += e;
            }
            const real inv = sum > 0 ? (real)1 / sum : (real)0;
            for (size_t a = 0; a < axis_dim; ++a) out[base + a * inner] *= inv;
        }
    }
}

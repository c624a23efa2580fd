/*
 * rqf_oracle.c -- fp64 CPU restatement of the reference's complex
 * linear-recurrence scans.  TEST INFRASTRUCTURE ONLY: it is the checker that
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the
 * HIP library against.  Nothing in prospective_rqf_amd/ links or calls it.
 *
 * Every routine is a plain sequential (time-major) loop in double precision,
 * written from the recurrences the reference defines:
 *
 *   two-tap / time-invariant scan   y[t] = c1*y[t-1] + k0*x[t] + k1*x[t-1]
 *     - k1 = 0, k0 = C2 is `_sequential_scan_cpu`   (rqf_models/ops/scan.py:252-287)
 *     - two-tap drive is `_apply_prospective_taps`  (rqf_models/backbones/rqf/block.py:644-682)
 *     - adjoint formulas of `_chunked_scan_backward_kernel`
 *       (rqf_models/ops/chunked_scan_kernel.py:135-137) and of the FBT backward
 *       (rqf_models/ops/fbt_scan_kernel.py:130-146), including the split-ReLU
 *       mask convention relu'(0) = 0 (fbt_scan_kernel.py:180-185).
 *
 *   multi-oscillator scan with C-weight reduction (BTF)
 *     - x_n[t] = C1_n x_n[t-1] + C2_n u[t], y[t] = sum_n cw_n x_n[t]:
 *       `_sequential_scan_multi_osc_kernel` (rqf_models/ops/triton_scan_kernel.py:1826-1940),
 *       the same as the expand -> scan -> C-weighted sum of
 *       `_scan_standard_fallback` / `_c_weighted_sum` (rqf_models/backbones/rqf/block.py:599-630)
 *     - adjoint and gradients of `_sequential_scan_multi_osc_backward_kernel`
 *       (triton_scan_kernel.py:2089-2279)
 *
 *   selective scan
 *     - coefficients: `selective_coefficients` (rqf_models/ops/selective_scan.py:26-68)
 *     - recurrence:   `reference_layer_scan`   (rqf_models/ops/selective_scan.py:71-104)
 *     - spec:         docs/selective_rqf.md:84-114
 *     - gradients:    derived by hand (reverse mode of the two routines above,
 *       PyTorch's conjugate-Wirtinger convention grad = dL/dRe + i dL/dIm);
 *       the layout of the returned tensors follows `selective_backward`
 *       (rqf_models/ops/selective_scan_kernel.py:517-561).
 *
 * Complex arrays are interleaved (re, im) doubles.  Layout codes:
 *   RQF_LAYOUT_BTF: element (b,t,f) at (b*T + t)*F + f   (the (B,T,F) API)
 *   RQF_LAYOUT_FBT: element (f,b,t) at (f*B + b)*T + t   (channel-outermost)
 */
#include <complex.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef double complex cd;

enum { RQF_LAYOUT_BTF = 0, RQF_LAYOUT_FBT = 1 };

static inline cd ld(const double *p, int64_t i) { return p[2 * i] + I * p[2 * i + 1]; }
static inline void st(double *p, int64_t i, cd v) {
    p[2 * i] = creal(v);
    p[2 * i + 1] = cimag(v);
}
static inline void acc(double *p, int64_t i, cd v) {
    p[2 * i] += creal(v);
    p[2 * i + 1] += cimag(v);
}

/* Element index of (row = (b, f), t) in either layout. */
static inline int64_t at(int layout, int64_t B, int64_t T, int64_t F, int64_t b, int64_t f,
                         int64_t t) {
    return layout == RQF_LAYOUT_BTF ? (b * T + t) * F + f : (f * B + b) * T + t;
}

/* ------------------------------------------------------------------------ */
/* Two-tap / time-invariant scan                                             */
/* ------------------------------------------------------------------------ */

/* y[t] = c1*y[t-1] + k0*x[t] + k1*x[t-1], y[-1] = x[-1] = 0.
 * k1 may be NULL (plain C2 scan).  act (nullable) receives the split-ReLU. */
void orc_twotap_fwd(int layout, int64_t B, int64_t T, int64_t F, const double *c1,
                    const double *k0, const double *k1, const double *x, double *y,
                    double *act) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t f = 0; f < F; ++f) {
            cd a = ld(c1, f), p = ld(k0, f), n = k1 ? ld(k1, f) : 0;
            cd prev = 0, xprev = 0;
            for (int64_t t = 0; t < T; ++t) {
                int64_t i = at(layout, B, T, F, b, f, t);
                cd xt = ld(x, i);
                prev = a * prev + p * xt + n * xprev;
                xprev = xt;
                st(y, i, prev);
                if (act) st(act, i, fmax(creal(prev), 0.0) + I * fmax(cimag(prev), 0.0));
            }
        }
}

/* Adjoint of orc_twotap_fwd for the cotangent gy on its output.  With
 * mask_act the cotangent is on the split-ReLU output instead (relu'(0)=0,
 * mask taken from the raw state).  Coefficient gradients are summed over
 * (b, t) into gc1 / gk0 / gk1 (each (F,) complex, overwritten; gk1 may be
 * NULL).  g[t] = e[t] + conj(c1) g[t+1]; gx[t] = conj(k0) g[t] + conj(k1) g[t+1];
 * gc1 = sum conj(y[t-1]) g[t]; gk0 = sum conj(x[t]) g[t]; gk1 = sum conj(x[t-1]) g[t]. */
void orc_twotap_bwd(int layout, int64_t B, int64_t T, int64_t F, const double *c1,
                    const double *k0, const double *k1, const double *x, const double *y,
                    const double *gy, int mask_act, double *gx, double *gc1, double *gk0,
                    double *gk1) {
    memset(gc1, 0, sizeof(double) * 2 * F);
    memset(gk0, 0, sizeof(double) * 2 * F);
    if (gk1) memset(gk1, 0, sizeof(double) * 2 * F);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t f = 0; f < F; ++f) {
            cd a = ld(c1, f), p = ld(k0, f), n = k1 ? ld(k1, f) : 0;
            cd gnext = 0, s1 = 0, s0 = 0, sk1 = 0;
            for (int64_t t = T - 1; t >= 0; --t) {
                int64_t i = at(layout, B, T, F, b, f, t);
                cd e = ld(gy, i);
                if (mask_act) {
                    cd r = ld(y, i);
                    e = (creal(r) > 0 ? creal(e) : 0.0) + I * (cimag(r) > 0 ? cimag(e) : 0.0);
                }
                cd g = e + conj(a) * gnext;
                st(gx, i, conj(p) * g + conj(n) * gnext);
                cd yprev = t ? ld(y, at(layout, B, T, F, b, f, t - 1)) : 0;
                cd xprev = t ? ld(x, at(layout, B, T, F, b, f, t - 1)) : 0;
                s1 += conj(yprev) * g;
                s0 += conj(ld(x, i)) * g;
                sk1 += conj(xprev) * g;
                gnext = g;
            }
            acc(gc1, f, s1);
            acc(gk0, f, s0);
            if (gk1) acc(gk1, f, sk1);
        }
}

/* ------------------------------------------------------------------------ */
/* Multi-oscillator scan with C-weight reduction (BTF layout)                */
/* ------------------------------------------------------------------------ */

/* N oscillators per filter f, coefficient index f*N + n:
 *   x_n[t] = c1_n x_n[t-1] + c2_n u[t],   y[t] = sum_n cw_n x_n[t]
 * cw NULL means y = x_0 (N = 1).  u, y: (B,T,F) complex; yabs (nullable)
 * receives |y|; y may be NULL when only yabs is wanted. */
void orc_mosc_fwd(int64_t B, int64_t T, int64_t F, int64_t N, const double *c1,
                  const double *c2, const double *cw, const double *u, double *y,
                  double *yabs) {
    cd *x = calloc((size_t)N, sizeof(cd));
    for (int64_t b = 0; b < B; ++b)
        for (int64_t f = 0; f < F; ++f) {
            for (int64_t n = 0; n < N; ++n) x[n] = 0;
            for (int64_t t = 0; t < T; ++t) {
                int64_t i = (b * T + t) * F + f;
                cd ut = ld(u, i), out = 0;
                for (int64_t n = 0; n < N; ++n) {
                    x[n] = ld(c1, f * N + n) * x[n] + ld(c2, f * N + n) * ut;
                    out += cw ? ld(cw, f * N + n) * x[n] : (n == 0 ? x[0] : 0);
                }
                if (y) st(y, i, out);
                if (yabs) yabs[i] = cabs(out);
            }
        }
    free(x);
}

/* Adjoint of orc_mosc_fwd (cw required) for the cotangent gy on y:
 *   d_n[t] = conj(c1_n) d_n[t+1] + conj(cw_n) gy[t]
 *   gu[t]  = sum_n conj(c2_n) d_n[t]
 *   gc1_n  = sum_{b,t} d_n[t] conj(x_n[t-1]),  gc2_n = sum d_n[t] conj(u[t]),
 *   gcw_n  = sum gy[t] conj(x_n[t])
 * Forward states are recomputed and kept per row (T*N complex). */
void orc_mosc_bwd(int64_t B, int64_t T, int64_t F, int64_t N, const double *c1,
                  const double *c2, const double *cw, const double *u, const double *gy,
                  double *gu, double *gc1, double *gc2, double *gcw) {
    memset(gc1, 0, sizeof(double) * 2 * F * N);
    memset(gc2, 0, sizeof(double) * 2 * F * N);
    memset(gcw, 0, sizeof(double) * 2 * F * N);
    cd *xs = malloc(sizeof(cd) * (size_t)(T * N + 1));
    cd *d = calloc((size_t)N, sizeof(cd));
    for (int64_t b = 0; b < B; ++b)
        for (int64_t f = 0; f < F; ++f) {
            for (int64_t n = 0; n < N; ++n) {
                cd x = 0;
                for (int64_t t = 0; t < T; ++t) {
                    x = ld(c1, f * N + n) * x + ld(c2, f * N + n) * ld(u, (b * T + t) * F + f);
                    xs[t * N + n] = x;
                }
                d[n] = 0;
            }
            for (int64_t t = T - 1; t >= 0; --t) {
                int64_t i = (b * T + t) * F + f;
                cd g = ld(gy, i), ut = ld(u, i), gsum = 0;
                for (int64_t n = 0; n < N; ++n) {
                    int64_t k = f * N + n;
                    d[n] = conj(ld(c1, k)) * d[n] + conj(ld(cw, k)) * g;
                    gsum += conj(ld(c2, k)) * d[n];
                    cd xprev = t ? xs[(t - 1) * N + n] : 0;
                    acc(gc1, k, d[n] * conj(xprev));
                    acc(gc2, k, d[n] * conj(ut));
                    acc(gcw, k, g * conj(xs[t * N + n]));
                }
                st(gu, i, gsum);
            }
        }
    free(d);
    free(xs);
}

/* ------------------------------------------------------------------------ */
/* Selective scan                                                            */
/* ------------------------------------------------------------------------ */

/* Mirrors SelectiveScanInputs (rqf_models/ops/selective_scan.py:10-23) in fp64,
 * with the options tuple unpacked (rqf_models/backbones/rqf/selective.py:245-262). */
typedef struct {
    int64_t F, B, T, G;
    const double *gamma_logits; /* (F,B,T) or NULL */
    const double *warp_logits;  /* (G,B,T) or NULL */
    const double *write_logits; /* (F,B,T) or NULL */
    const double *bias, *theta, *minimum, *span, *step, *horizon, *theta_minimum,
        *theta_maximum;       /* (F,) */
    const int64_t *groups;    /* (F,) or NULL */
    int32_t has_gamma, has_warp, has_write, log_shift;
    double gamma_scale, warp_scale;
    int32_t prospective, gamma_horizon, write_sigmoid;
    double write_max, write_bias;
    int32_t bound_warp;
} orc_selective_inputs;

typedef struct {
    double gamma, sig, theta, warp, inside, gate, eta, ratio;
    cd a, A, phi, bp, bn; /* bp, bn: un-gated taps */
} sel_elem;

static double sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

/* (exp(a) - 1)/a with the reference's |a| < 1e-4 cubic series
 * (selective_scan.py:49-54); expm1 formed without cancellation. */
static cd exprel(cd a) {
    if (cabs(a) < 1e-4) return 1 + a * (0.5 + a * (1.0 / 6 + a / 24));
    double ar = creal(a), ai = cimag(a), h = sin(0.5 * ai);
    cd em1 = (expm1(ar) * cos(ai) - 2 * h * h) + I * (exp(ar) * sin(ai));
    return em1 / a;
}

static void sel_eval(const orc_selective_inputs *s, int64_t f, int64_t b, int64_t t,
                     sel_elem *e) {
    int64_t i = (f * s->B + b) * s->T + t;
    e->gamma = s->bias[f];
    e->sig = 0;
    if (s->has_gamma) {
        double v = s->gamma_logits[i];
        if (s->log_shift) {
            e->sig = tanh(v);
            e->gamma = exp(s->bias[f] + s->gamma_scale * e->sig);
        } else {
            e->sig = sigmoid(s->bias[f] + v);
            e->gamma = s->minimum[f] + s->span[f] * e->sig;
        }
    }
    e->theta = s->theta[f];
    e->warp = 0;
    e->inside = 1;
    if (s->has_warp) {
        e->warp = tanh(s->warp_logits[(s->groups[f] * s->B + b) * s->T + t]);
        e->theta *= exp(s->warp_scale * e->warp);
        if (s->bound_warp) {
            double lo = s->theta_minimum[f], hi = s->theta_maximum[f];
            e->inside = (e->theta >= lo && e->theta <= hi);
            e->theta = fmin(fmax(e->theta, lo), hi);
        }
    }
    e->gate = 1;
    if (s->has_write) {
        double w = s->write_logits[i];
        e->gate = s->write_sigmoid ? s->write_max * sigmoid(w + s->write_bias) : 1 + w;
    }
    e->eta = s->step[f];
    e->a = e->eta * (-e->gamma + I * (1 - e->gamma) * e->theta);
    e->A = cexp(e->a);
    e->phi = exprel(e->a);
    e->bp = e->gamma * e->eta * e->phi;
    e->bn = 0;
    e->ratio = 0;
    if (s->prospective) {
        e->ratio = s->gamma_horizon ? 1 / e->gamma : s->horizon[f];
        cd extra = e->ratio * e->gamma * e->A;
        e->bp += extra;
        e->bn = -extra;
    }
}

/* Explicit (A, gated p, gated n) in (F,B,T) layout (selective_scan.py:26-68). */
void orc_selective_coefficients(const orc_selective_inputs *s, double *A, double *p,
                                double *n) {
    for (int64_t f = 0; f < s->F; ++f)
        for (int64_t b = 0; b < s->B; ++b)
            for (int64_t t = 0; t < s->T; ++t) {
                sel_elem e;
                sel_eval(s, f, b, t, &e);
                int64_t i = (f * s->B + b) * s->T + t;
                st(A, i, e.A);
                st(p, i, e.gate * e.bp);
                st(n, i, e.gate * e.bn);
            }
}

/* Forward of reference_layer_scan after the drive GEMM: z (F,B,T) -> raw, act
 * (either nullable).  y[t] = A y[t-1] + p z[t] + n z[t-1] (the lag term only
 * for t > 0 and prospective input). */
void orc_selective_fwd(const orc_selective_inputs *s, const double *z, double *raw,
                       double *act) {
    for (int64_t f = 0; f < s->F; ++f)
        for (int64_t b = 0; b < s->B; ++b) {
            cd y = 0, zprev = 0;
            for (int64_t t = 0; t < s->T; ++t) {
                sel_elem e;
                sel_eval(s, f, b, t, &e);
                int64_t i = (f * s->B + b) * s->T + t;
                cd zt = ld(z, i);
                y = e.A * y + e.gate * (e.bp * zt + e.bn * zprev);
                zprev = zt;
                if (raw) st(raw, i, y);
                if (act) st(act, i, fmax(creal(y), 0.0) + I * fmax(cimag(y), 0.0));
            }
        }
}

/* Reverse mode of orc_selective_fwd.  Cotangents gy (on raw) and gx (on the
 * split-ReLU output) are nullable.  Outputs (all overwritten):
 *   dz   (F,B,T) c  gradient reaching x through the current tap p[t] z[t]; in
 *                   full BPTT it also carries the lag tap (then equal to dzw)
 *   dzw  (F,B,T) c  gradient reaching W: current + lag tap
 *   dg   (F,B,T)    gamma logits (if has_gamma)
 *   dd   (G,B,T)    warp logits, summed over the channels of each group
 *   dw   (F,B,T)    write logits (if has_write)
 *   dbias, dtheta (F,)
 * truncated = TBPTT(1): y[t-1] is detached (no reverse recursion) and the lag
 * tap's gradient reaches W only (docs/selective_rqf.md:100-104). */
void orc_selective_bwd(const orc_selective_inputs *s, const double *z, const double *gy,
                       const double *gx, int truncated, double *dz, double *dzw, double *dg,
                       double *dd, double *dw, double *dbias, double *dtheta) {
    const int64_t F = s->F, B = s->B, T = s->T;
    if (dd) memset(dd, 0, sizeof(double) * s->G * B * T);
    memset(dbias, 0, sizeof(double) * F);
    memset(dtheta, 0, sizeof(double) * F);
    sel_elem *el = (sel_elem *)malloc(sizeof(sel_elem) * (T > 0 ? T : 1));
    cd *y = (cd *)malloc(sizeof(cd) * (T > 0 ? T : 1));
    for (int64_t f = 0; f < F; ++f)
        for (int64_t b = 0; b < B; ++b) {
            const int64_t row = (f * B + b) * T;
            cd state = 0;
            for (int64_t t = 0; t < T; ++t) {
                sel_eval(s, f, b, t, &el[t]);
                cd zp = t ? ld(z, row + t - 1) : 0;
                state = el[t].A * state + el[t].gate * (el[t].bp * ld(z, row + t) + el[t].bn * zp);
                y[t] = state;
            }
            cd dnext = 0;
            double sb = 0, sth = 0;
            for (int64_t t = T - 1; t >= 0; --t) {
                const sel_elem *e = &el[t];
                cd ecot = gy ? ld(gy, row + t) : 0;
                if (gx) {
                    cd c = ld(gx, row + t);
                    ecot += (creal(y[t]) > 0 ? creal(c) : 0.0) + I * (cimag(y[t]) > 0 ? cimag(c) : 0.0);
                }
                cd Anext = (t + 1 < T) ? el[t + 1].A : 0;
                cd nnext = (t + 1 < T) ? el[t + 1].gate * el[t + 1].bn : 0;
                cd d = truncated ? ecot : ecot + conj(Anext) * dnext;
                cd p = e->gate * e->bp;
                cd cur = conj(p) * d;
                cd lag = conj(nnext) * dnext;
                st(dzw, row + t, cur + lag);
                st(dz, row + t, truncated ? cur : cur + lag);
                /* gradients of the gated taps and of A */
                cd zt = ld(z, row + t), zp = t ? ld(z, row + t - 1) : 0;
                cd ypv = t ? y[t - 1] : 0;
                cd gp = conj(zt) * d, gn = conj(zp) * d, gA = conj(ypv) * d;
                double ggate = creal(conj(e->bp) * gp + conj(e->bn) * gn);
                cd gbp = e->gate * gp, gbn = e->gate * gn;
                /* bp = gamma*eta*phi(a) + ratio*gamma*A, bn = -ratio*gamma*A */
                double ggamma = 0;
                if (s->prospective) {
                    cd q = gbp - gbn;
                    gA += e->ratio * e->gamma * q; /* ratio*gamma is real */
                    if (!s->gamma_horizon) ggamma += e->ratio * creal(conj(e->A) * q);
                }
                ggamma += e->eta * creal(conj(e->phi) * gbp);
                /* phi'(a) = (A - phi)/a, with its series near 0 */
                cd dphi;
                if (cabs(e->a) < 1e-3) {
                    cd a = e->a;
                    dphi = 0.5 + a * (1.0 / 3 + a * (1.0 / 8 + a * (1.0 / 30 + a * (1.0 / 144 + a * (1.0 / 840)))));
                } else {
                    dphi = (e->A - e->phi) / e->a;
                }
                cd ga = conj(e->A) * gA + e->gamma * e->eta * conj(dphi) * gbp;
                /* a = eta*(-gamma + i*(1-gamma)*theta) */
                ggamma += e->eta * (-creal(ga) - e->theta * cimag(ga));
                double gth = e->eta * (1 - e->gamma) * cimag(ga);
                /* controller chain rules */
                int64_t i = row + t;
                if (s->has_gamma) {
                    double glog;
                    if (s->log_shift) {
                        double gb = ggamma * e->gamma; /* d gamma / d bias = gamma */
                        sb += gb;
                        glog = gb * s->gamma_scale * (1 - e->sig * e->sig);
                    } else {
                        glog = ggamma * s->span[f] * e->sig * (1 - e->sig);
                        sb += glog;
                    }
                    if (dg) dg[i] = glog;
                } else {
                    sb += ggamma;
                }
                if (s->has_warp) {
                    double scale = exp(s->warp_scale * e->warp);
                    double gin = e->inside ? gth : 0.0;
                    if (dd)
                        dd[(s->groups[f] * B + b) * T + t] +=
                            gin * e->theta * s->warp_scale * (1 - e->warp * e->warp);
                    sth += gin * scale;
                } else {
                    sth += gth;
                }
                if (s->has_write && dw) {
                    double gw = ggate;
                    if (s->write_sigmoid) gw *= e->gate * (1 - e->gate / s->write_max);
                    dw[i] = gw;
                }
                dnext = d;
            }
            dbias[f] += sb;
            dtheta[f] += sth;
        }
    free(el);
    free(y);
}

/* Static two-tap ZOH coefficients of RQF.compute_two_tap_coefficients
 * (rqf_models/backbones/rqf/filter.py:630-646) for per-channel
 * (gamma, theta, eta = dt/tau, ratio): C1 = e^a, tap0 = gamma*eta*phi(a) +
 * gamma*ratio*C1, tap1 = -gamma*ratio*C1 with a = eta*(-gamma + i(1-gamma)theta). */
void orc_zoh_two_tap(int64_t F, const double *gamma, const double *theta, const double *eta,
                     const double *ratio, double *c1, double *tap0, double *tap1) {
    for (int64_t f = 0; f < F; ++f) {
        cd a = eta[f] * (-gamma[f] + I * (1 - gamma[f]) * theta[f]);
        cd C1 = cexp(a);
        cd extra = gamma[f] * ratio[f] * C1;
        st(c1, f, C1);
        st(tap0, f, gamma[f] * eta[f] * exprel(a) + extra);
        st(tap1, f, -extra);
    }
}

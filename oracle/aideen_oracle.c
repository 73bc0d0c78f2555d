/*
 * aideen_oracle.c -- CPU restatement of the AIDEEN DEQ forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared against; it is
 * never linked into, called by or shipped with the product library.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Arithmetic order follows the reference's f32 code (nalgebra gemv accumulates each output
 * sequentially over the input index; sums and means fold left to right).  Build with
 * -ffp-contract=off so no multiply-add is fused, as Rust never fuses them.
 *
 * Pinning (how each function is checked; tests/test_oracle_pins.py):
 *   orc_spectral_norm / normalize*  -- the reference's own unit tests (spectral_norm.rs:98-149)
 *                                      plus sigma of matrices with a known SVD.
 *   orc_picard_step / orc_solve_token -- zero-attention closed form (iteration count known
 *                                      exactly), H=1 closed form, uniform-attention closed form,
 *                                      float64 brute force at d<=16, slot-permutation
 *                                      equivariance, fixed-point residual invariant.
 *   orc_lm_head_token / orc_argmax   -- lm_head.rs:249-310 tests, closed-form W entries,
 *                                      RMSNorm scale invariance, last-max tie rule.
 *   orc_scan_seq / recirculate       -- geometric-series closed form, readout==recirculate at
 *                                      W_out=0, sequential==chunked invariants.
 *   Anderson mixing                  -- m=1 equals Picard; the solved coefficients satisfy the
 *                                      regularised system; convergence on a linear map.
 *   orc_zoh_step / orc_gemv_colmajor -- closed forms of gpu_backend.rs:18-56 and the engine
 *                                      GEMV known answer (aideen-engine/src/gpu/mod.rs:229-257).
 */
#include "aideen_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* small linear algebra in reference order                                    */
/* ------------------------------------------------------------------------- */

/* y = W x, W row-major [out][in]; y[o] accumulates sequentially over i (nalgebra gemv). */
static void gemv_rm(const float *W, int out, int in, const float *x, float *y) {
    for (int o = 0; o < out; ++o) {
        const float *row = W + (size_t)o * in;
        float acc = 0.0f;
        for (int i = 0; i < in; ++i) acc += row[i] * x[i];
        y[o] = acc;
    }
}

/* y = W x with W given transposed, Wt [in][out]: same per-output order as gemv_rm, but the
 * loop runs across outputs so it vectorises.  Bit-identical to gemv_rm without FP contraction. */
static void gemv_t(const float *Wt, int out, int in, const float *x, float *y) {
    for (int o = 0; o < out; ++o) y[o] = 0.0f;
    for (int i = 0; i < in; ++i) {
        const float xi = x[i];
        const float *col = Wt + (size_t)i * out;
        for (int o = 0; o < out; ++o) y[o] += col[o] * xi;
    }
}

static float dot_seq(const float *a, const float *b, int n) {
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

static void transpose(const float *src, int rows, int cols, float *dst) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) dst[(size_t)c * rows + r] = src[(size_t)r * cols + c];
}

/* ------------------------------------------------------------------------- */
/* spectral_norm.rs                                                           */
/* ------------------------------------------------------------------------- */

static float norm2(const float *v, int n) { return sqrtf(dot_seq(v, v, n)); }

/* spectral_norm.rs:25-59 -- power iteration from u0 = 1/sqrt(rows). */
float orc_spectral_norm(const float *w, int rows, int cols, int n_iter) {
    if (rows == 0 || cols == 0) return 1.0f;
    float *u = (float *)malloc(sizeof(float) * rows);
    float *v = (float *)malloc(sizeof(float) * cols);
    float *wv = (float *)malloc(sizeof(float) * rows);
    const float inv = 1.0f / sqrtf((float)rows);
    for (int i = 0; i < rows; ++i) u[i] = inv;
    float sigma = 1.0f;
    for (int it = 0; it < n_iter; ++it) {
        /* v = W^T u / ||W^T u||; each output of W^T u accumulates over rows in order */
        for (int j = 0; j < cols; ++j) {
            float acc = 0.0f;
            for (int i = 0; i < rows; ++i) acc += w[(size_t)i * cols + j] * u[i];
            v[j] = acc;
        }
        float nv = norm2(v, cols);
        if (nv < 1e-12f) { sigma = 0.0f; goto done_zero; }
        for (int j = 0; j < cols; ++j) v[j] = v[j] / nv;
        gemv_rm(w, rows, cols, v, wv);
        float nu = norm2(wv, rows);
        if (nu < 1e-12f) { sigma = 0.0f; goto done_zero; }
        for (int i = 0; i < rows; ++i) u[i] = wv[i] / nu;
        /* sigma = (u^T W) v: nalgebra evaluates the row vector u^T W first */
        float acc_s = 0.0f;
        for (int j = 0; j < cols; ++j) {
            float z = 0.0f;
            for (int i = 0; i < rows; ++i) z += u[i] * w[(size_t)i * cols + j];
            acc_s += z * v[j];
        }
        sigma = acc_s;
    }
    free(u); free(v); free(wv);
    sigma = fabsf(sigma);
    return sigma > 1e-12f ? sigma : 1e-12f;
done_zero:
    free(u); free(v); free(wv);
    return 0.0f;
}

/* spectral_norm.rs:65-71 */
void orc_normalize(float *w, int rows, int cols, float target, int n_iter) {
    float sigma = orc_spectral_norm(w, rows, cols, n_iter);
    if (sigma < 1e-12f) return;
    const float s = target / sigma;
    for (size_t i = 0; i < (size_t)rows * cols; ++i) w[i] *= s;
}

/* spectral_norm.rs:75-80 */
void orc_normalize_if_needed(float *w, int rows, int cols, float threshold, int n_iter) {
    float sigma = orc_spectral_norm(w, rows, cols, n_iter);
    if (sigma > threshold) {
        const float s = threshold / sigma;
        for (size_t i = 0; i < (size_t)rows * cols; ++i) w[i] *= s;
    }
}

/* spectral_norm.rs:93-95: f*beta + h*(1-beta) */
void orc_damped_update(const float *h, const float *f, float beta, int n, float *out) {
    const float omb = 1.0f - beta;
    for (int i = 0; i < n; ++i) out[i] = f[i] * beta + h[i] * omb;
}

/* ------------------------------------------------------------------------- */
/* prepared (transposed) weights for the fast per-token path                  */
/* ------------------------------------------------------------------------- */

typedef struct prep {
    orc_cfg c;
    const orc_weights *w;
    float *wq_t, *wk_t, *wv_t, *wo_t, *win_t; /* [H][in][out] */
} prep;

static void prep_init(prep *p, const orc_cfg *c, const orc_weights *w) {
    const int d = c->d, H = c->H;
    const size_t mat = (size_t)d * d;
    p->c = *c;
    p->w = w;
    float **dst[5] = {&p->wq_t, &p->wk_t, &p->wv_t, &p->wo_t, &p->win_t};
    const float *src[5] = {w->w_q, w->w_k, w->w_v, w->w_o, w->w_in};
    for (int m = 0; m < 5; ++m) {
        *dst[m] = (float *)malloc(sizeof(float) * mat * H);
        for (int s = 0; s < H; ++s) {
            if (m == 4 && (c->flags & ORC_F_WIN_TRANSPOSED)) {
                /* signal = W_in^T x: the transposed matrix of W_in^T is W_in itself */
                memcpy(*dst[m] + s * mat, src[m] + s * mat, sizeof(float) * mat);
            } else {
                transpose(src[m] + s * mat, d, d, *dst[m] + s * mat);
            }
        }
    }
}

static void prep_free(prep *p) {
    free(p->wq_t); free(p->wk_t); free(p->wv_t); free(p->wo_t); free(p->win_t);
}

/* per-thread scratch */
typedef struct scratch {
    float *q, *k, *v, *mix, *o, *comb, *hn, *hist; /* hist: Anderson ring [m][H*d] */
    float *scores, *attn;
    float *rms; /* [H] each slot's RMSNorm denominator in the last step (relative residual) */
} scratch;

static void scratch_init(scratch *s, const orc_cfg *c) {
    const size_t hd = (size_t)c->H * c->d;
    s->q = (float *)malloc(sizeof(float) * hd);
    s->k = (float *)malloc(sizeof(float) * hd);
    s->v = (float *)malloc(sizeof(float) * hd);
    s->mix = (float *)malloc(sizeof(float) * c->d);
    s->o = (float *)malloc(sizeof(float) * c->d);
    s->comb = (float *)malloc(sizeof(float) * c->d);
    s->hn = (float *)malloc(sizeof(float) * hd);
    int m = c->anderson_m > 0 ? c->anderson_m : 1;
    s->hist = (float *)malloc(sizeof(float) * hd * m);
    s->scores = (float *)malloc(sizeof(float) * c->H);
    s->attn = (float *)malloc(sizeof(float) * c->H * c->H);
    s->rms = (float *)malloc(sizeof(float) * c->H);
}

static void scratch_free(scratch *s) {
    free(s->q); free(s->k); free(s->v); free(s->mix); free(s->o); free(s->comb); free(s->hn);
    free(s->hist); free(s->scores); free(s->attn); free(s->rms);
}

/* FPMR:1305-1315 project_input_signal (per slot: signal_s = W_in[s] x). */
static void signal_p(const prep *p, const float *x, float *signal) {
    const int d = p->c.d;
    for (int s = 0; s < p->c.H; ++s)
        gemv_t(p->win_t + (size_t)s * d * d, d, d, x, signal + (size_t)s * d);
}

/* FPMR:1432-1448 init (h0 = x + anchor); UWGSL:900-943 signal/rms variant. */
static void init_p(const prep *p, const float *x, const float *signal, float *h0) {
    const int d = p->c.d, H = p->c.H;
    for (int s = 0; s < H; ++s) {
        float *hs = h0 + (size_t)s * d;
        if (p->c.flags & ORC_F_INIT_SIGNAL_RMS) {
            const float *sg = signal + (size_t)s * d;
            float ss = 0.0f;
            for (int i = 0; i < d; ++i) ss += sg[i] * sg[i];
            const float rms = sqrtf(ss / (float)d + 1e-6f);
            for (int i = 0; i < d; ++i) hs[i] = sg[i] / rms;
        } else {
            const float *an = p->w->anchor + (size_t)s * d;
            for (int i = 0; i < d; ++i) hs[i] = x[i] + an[i];
        }
    }
}

/* FPMR:1397-1424 cross_slot_attn followed by FPMR:1372-1395 step_with_fixed_hist_ctx
 * (hist = NULL is the zero context of FPMR:1450-1453), FPMR:1300-1303 rms_norm and
 * spectral_norm.rs:93 damped_update. */
static void step_p(const prep *p, scratch *sc, const float *h, const float *signal,
                   const float *hist, float *h_next, float *attn_out) {
    const int d = p->c.d, H = p->c.H;
    const orc_weights *w = p->w;
    const size_t mat = (size_t)d * d;
    for (int s = 0; s < H; ++s) {
        const float *hs = h + (size_t)s * d;
        gemv_t(p->wq_t + s * mat, d, d, hs, sc->q + (size_t)s * d);
        gemv_t(p->wk_t + s * mat, d, d, hs, sc->k + (size_t)s * d);
        gemv_t(p->wv_t + s * mat, d, d, hs, sc->v + (size_t)s * d);
        if (w->q_bias)
            for (int i = 0; i < d; ++i) sc->q[(size_t)s * d + i] += w->q_bias[(size_t)s * d + i];
        if (w->k_bias)
            for (int i = 0; i < d; ++i) sc->k[(size_t)s * d + i] += w->k_bias[(size_t)s * d + i];
    }
    const float scale = 1.0f / sqrtf((float)d);
    for (int a = 0; a < H; ++a) {
        /* raw scores, max-subtracted softmax (FPMR:1405-1413) */
        float mx = -INFINITY;
        for (int cc = 0; cc < H; ++cc) {
            float sc_ = dot_seq(sc->q + (size_t)a * d, sc->k + (size_t)cc * d, d) * scale;
            if (p->c.flags & ORC_F_SCORE_CLAMP4) sc_ = fminf(fmaxf(sc_, -4.0f), 4.0f);
            sc->scores[cc] = sc_;
            mx = fmaxf(mx, sc_);
        }
        float sum = 0.0f;
        for (int cc = 0; cc < H; ++cc) {
            sc->scores[cc] = expf(sc->scores[cc] - mx);
            sum += sc->scores[cc];
        }
        for (int cc = 0; cc < H; ++cc) sc->attn[a * H + cc] = sc->scores[cc] / sum;
        /* mixed = fold(0, acc + v_c * attn_c) (FPMR:1415-1419) */
        for (int i = 0; i < d; ++i) sc->mix[i] = 0.0f;
        for (int cc = 0; cc < H; ++cc) {
            const float at = sc->attn[a * H + cc];
            const float *vc = sc->v + (size_t)cc * d;
            for (int i = 0; i < d; ++i) sc->mix[i] = sc->mix[i] + vc[i] * at;
        }
        gemv_t(p->wo_t + a * mat, d, d, sc->mix, sc->o);
        /* combined = attn + signal + hist(0) + anchor; f = g*c/rms (FPMR:1386-1391) */
        const float *sg = signal + (size_t)a * d;
        const float *an = w->anchor + (size_t)a * d;
        const float *hc = hist ? hist + (size_t)a * d : NULL;
        float ss = 0.0f;
        if (p->c.flags & ORC_F_RMS_EXCL_ANCHOR) {
            for (int i = 0; i < d; ++i) {
                const float as_ = (sc->o[i] + sg[i]) + (hc ? hc[i] : 0.0f);
                ss += as_ * as_;
                sc->comb[i] = as_ + an[i];
            }
        } else {
            /* combined = attn + input_signal + hist_k, then + slot_bias (FPMR:1386-1389) */
            for (int i = 0; i < d; ++i) {
                sc->comb[i] = ((sc->o[i] + sg[i]) + (hc ? hc[i] : 0.0f)) + an[i];
                ss += sc->comb[i] * sc->comb[i];
            }
        }
        const float rms = sqrtf(ss / (float)d + 1e-6f);
        sc->rms[a] = rms;
        const float beta = p->c.beta, omb = 1.0f - p->c.beta;
        const float *ha = h + (size_t)a * d;
        float *hn = h_next + (size_t)a * d;
        for (int i = 0; i < d; ++i) {
            const float f = w->norm_scale[i] * sc->comb[i] / rms;
            hn[i] = f * beta + ha[i] * omb;
        }
    }
    if (attn_out) memcpy(attn_out, sc->attn, sizeof(float) * H * H);
}

/* Residual between consecutive iterates: max-abs (ARCHITECTURE.md:178-185), L2 over the
 * token's flat [H*d] state (aideen-node/src/inference.rs:214-221), or the largest per-slot
 * relative RMS change sqrt(mean (a-b)^2 + 1e-12) / max(rms, 1e-6) with rms the slot's RMSNorm
 * denominator of the step that produced a (the GPU reference's err_h,
 * deq_slot_attn_unified_clean.wgsl:1654-1695). */
/* A non-finite value (a NaN or inf state) counts as an infinite residual, so the token never
 * passes the exit test (the reference's finite_or guards, UWGSL:99-108); fmaxf alone would drop
 * a NaN and report such a token converged. */
static float nan_to_inf(float v) { return v != v ? INFINITY : v; }

static float residual(const orc_cfg *c, const float *rms, const float *a, const float *b) {
    const int n = c->H * c->d;
    if (c->flags & ORC_F_RESID_RELRMS) {
        const int d = c->d;
        float mx = 0.0f;
        for (int s = 0; s < c->H; ++s) {
            float acc = 0.0f;
            for (int i = 0; i < d; ++i) {
                const float df = a[(size_t)s * d + i] - b[(size_t)s * d + i];
                acc += df * df;
            }
            mx = fmaxf(mx, nan_to_inf(sqrtf(acc / (float)d + 1e-12f) / fmaxf(rms[s], 1e-6f)));
        }
        return mx;
    }
    if (c->flags & ORC_F_RESID_L2) {
        float acc = 0.0f;
        for (int i = 0; i < n; ++i) {
            const float df = a[i] - b[i];
            acc += df * df;
        }
        return nan_to_inf(sqrtf(acc));
    }
    float mx = 0.0f;
    for (int i = 0; i < n; ++i) mx = fmaxf(mx, nan_to_inf(fabsf(a[i] - b[i])));
    return mx;
}

/* Anderson coefficients: the reference's iterate-difference scheme
 * (staged_adjoint_picard_clean.wgsl:1043-1121).  g[n*n] is the Gram matrix of the pseudo-
 * residuals; solves (G + reg I) beta = 1 by Cramer's rule for n = 2, 3 (the reference's
 * formulas) and by cofactor expansion for n = 4 (build extension, same determinant clamp),
 * clamps to [-2, 3] and normalises to sum 1. */
void orc_anderson_coeffs(int n, const float *g_in, float *beta) {
    float g[16];
    memcpy(g, g_in, sizeof(float) * n * n);
    if (n == 2) {
        const float reg = fmaxf(1e-8f, 1e-4f * (fabsf(g[0]) + fabsf(g[3])));
        const float g00 = g[0] + reg, g01 = g[1], g10 = g[2], g11 = g[3] + reg;
        const float det = g00 * g11 - g01 * g10;
        const float sdet = det < 0.0f ? fminf(det, -1e-10f) : fmaxf(det, 1e-10f);
        beta[0] = (g11 - g01) / sdet;
        beta[1] = (g00 - g10) / sdet;
    } else if (n == 3) {
        const float reg = fmaxf(1e-8f, 1e-4f * (fabsf(g[0]) + fabsf(g[4]) + fabsf(g[8])));
        const float g00 = g[0] + reg, g01 = g[1], g02 = g[2];
        const float g10 = g[3], g11 = g[4] + reg, g12 = g[5];
        const float g20 = g[6], g21 = g[7], g22 = g[8] + reg;
        const float det = g00 * (g11 * g22 - g12 * g21) - g01 * (g10 * g22 - g12 * g20) +
                          g02 * (g10 * g21 - g11 * g20);
        const float sdet = det < 0.0f ? fminf(det, -1e-8f) : fmaxf(det, 1e-8f);
        beta[0] = (1.0f * (g11 * g22 - g12 * g21) - g01 * (g22 - g12) + g02 * (g21 - g11)) / sdet;
        beta[1] = (g00 * (g22 - g12) - 1.0f * (g10 * g22 - g12 * g20) + g02 * (g10 - g20)) / sdet;
        beta[2] = (g00 * (g11 - g21) - g01 * (g10 - g20) + 1.0f * (g10 * g21 - g11 * g20)) / sdet;
    } else { /* n == 4: Cramer by 3x3 cofactors */
        float a[16];
        float tr = 0.0f;
        for (int i = 0; i < 4; ++i) tr += fabsf(g[i * 4 + i]);
        const float reg = fmaxf(1e-8f, 1e-4f * tr);
        memcpy(a, g, sizeof(a));
        for (int i = 0; i < 4; ++i) a[i * 4 + i] += reg;
#define M3(r0, r1, r2, c0, c1, c2)                                                   \
    (m[r0 * 4 + c0] * (m[r1 * 4 + c1] * m[r2 * 4 + c2] - m[r1 * 4 + c2] * m[r2 * 4 + c1]) - \
     m[r0 * 4 + c1] * (m[r1 * 4 + c0] * m[r2 * 4 + c2] - m[r1 * 4 + c2] * m[r2 * 4 + c0]) + \
     m[r0 * 4 + c2] * (m[r1 * 4 + c0] * m[r2 * 4 + c1] - m[r1 * 4 + c1] * m[r2 * 4 + c0]))
        const float *m = a;
        const float det = a[0] * M3(1, 2, 3, 1, 2, 3) - a[1] * M3(1, 2, 3, 0, 2, 3) +
                          a[2] * M3(1, 2, 3, 0, 1, 3) - a[3] * M3(1, 2, 3, 0, 1, 2);
        const float sdet = det < 0.0f ? fminf(det, -1e-8f) : fmaxf(det, 1e-8f);
        for (int col = 0; col < 4; ++col) {
            float b[16];
            memcpy(b, a, sizeof(b));
            for (int r = 0; r < 4; ++r) b[r * 4 + col] = 1.0f;
            m = b;
            const float dc = b[0] * M3(1, 2, 3, 1, 2, 3) - b[1] * M3(1, 2, 3, 0, 2, 3) +
                             b[2] * M3(1, 2, 3, 0, 1, 3) - b[3] * M3(1, 2, 3, 0, 1, 2);
            beta[col] = dc / sdet;
        }
#undef M3
    }
    float s = 0.0f;
    for (int i = 0; i < n; ++i) {
        beta[i] = fminf(fmaxf(beta[i], -2.0f), 3.0f);
        s += beta[i];
    }
    if (fabsf(s) < 1e-6f) {
        for (int i = 0; i < n; ++i) beta[i] = 0.0f;
        beta[0] = 1.0f;
    } else {
        for (int i = 0; i < n; ++i) beta[i] = beta[i] / s;
    }
}

/* Per-token solve.  Loop/exit: aideen-node/src/inference.rs:196-228 (apply the step, then
 * exit when the residual between consecutive iterates is below eps); iteration count = number
 * of updates applied.  Converged tokens are frozen.  Optional Anderson mixing after each step
 * (staged_adjoint_picard_clean.wgsl:1012-1134, gpu_deq.rs:4278-4293): the ring stores the
 * un-mixed Picard iterate; mixing starts at k >= 2 with n_res = min(k, m-1) >= 2. */
/* warm != 0: h already holds the starting iterate (token carry), init_p is skipped.
 * *conv (when given) = 1 if the solve exited on the tolerance or the plateau, 0 if it stopped at
 * max_iters unconverged. */
static int solve_p(const prep *p, scratch *sc, const float *x, const float *hist, float *h,
                   float *resid_trace, int warm, int *conv) {
    const orc_cfg *c = &p->c;
    const int d = c->d, H = c->H;
    const size_t hd = (size_t)H * d;
    float *signal = (float *)malloc(sizeof(float) * hd);
    signal_p(p, x, signal);
    if (!warm) init_p(p, x, signal, h);
    int iters = 0;
    if (conv) *conv = 0;
    const int m = c->anderson_m;
    float r_prev = 1.0f; /* homeostatic exit: the previous update's residual (1 before the first) */
    for (int k = 0; k < c->max_iters; ++k) {
        step_p(p, sc, h, signal, hist, sc->hn, NULL);
        const float r = residual(c, sc->rms, sc->hn, h);
        if (resid_trace) resid_trace[k] = r;
        iters = k + 1;
        /* exit below eps, or (ORC_F_HOMEOSTATIC_EXIT) on the plateau of
         * deq_slot_attn_unified_clean.wgsl:1786-1793: k+1 >= 4, r <= max(eps, 0.15 * 0.2) and
         * |r - r_prev| <= 0.10 max(r_prev, eps) */
        int stop = r < c->eps;
        if ((c->flags & ORC_F_HOMEOSTATIC_EXIT) && k + 1 >= 4 && r <= fmaxf(c->eps, 0.15f * 0.2f) &&
            fabsf(r - r_prev) / fmaxf(r_prev, c->eps) <= 0.10f)
            stop = 1;
        r_prev = r;
        if (stop && conv) *conv = 1;
        if (stop || m <= 0) {
            memcpy(h, sc->hn, sizeof(float) * hd);
            if (stop) break;
            continue;
        }
        /* Anderson: store g into ring slot k % m, then mix */
        memcpy(sc->hist + (size_t)(k % m) * hd, sc->hn, sizeof(float) * hd);
        const int n_res = k < m - 1 ? k : m - 1;
        if (k >= 2 && n_res >= 2) {
            float g[16], beta[4];
            for (int ri = 0; ri < n_res; ++ri) {
                for (int rj = ri; rj < n_res; ++rj) {
                    const float *xi = sc->hist + (size_t)((k + m - ri) % m) * hd;
                    const float *xi1 = sc->hist + (size_t)((k + m - ri - 1) % m) * hd;
                    const float *xj = sc->hist + (size_t)((k + m - rj) % m) * hd;
                    const float *xj1 = sc->hist + (size_t)((k + m - rj - 1) % m) * hd;
                    float acc = 0.0f;
                    for (size_t e = 0; e < hd; ++e) acc += (xi[e] - xi1[e]) * (xj[e] - xj1[e]);
                    g[ri * n_res + rj] = acc;
                    g[rj * n_res + ri] = acc;
                }
            }
            orc_anderson_coeffs(n_res, g, beta);
            for (size_t e = 0; e < hd; ++e) {
                float acc = 0.0f;
                for (int i = 0; i < n_res; ++i)
                    acc += beta[i] * sc->hist[(size_t)((k + m - i) % m) * hd + e];
                h[e] = acc;
            }
        } else {
            memcpy(h, sc->hn, sizeof(float) * hd);
        }
    }
    free(signal);
    return iters;
}

/* ------------------------------------------------------------------------- */
/* public per-token API                                                       */
/* ------------------------------------------------------------------------- */

void orc_signal(const orc_cfg *c, const orc_weights *w, const float *x, float *signal) {
    prep p;
    prep_init(&p, c, w);
    signal_p(&p, x, signal);
    prep_free(&p);
}

void orc_init(const orc_cfg *c, const orc_weights *w, const float *x, const float *signal,
              float *h0) {
    prep p;
    p.c = *c;
    p.w = w;
    init_p(&p, x, signal, h0);
}

void orc_picard_step(const orc_cfg *c, const orc_weights *w, const float *h, const float *signal,
                     float *h_next, float *attn) {
    prep p;
    scratch sc;
    prep_init(&p, c, w);
    scratch_init(&sc, c);
    step_p(&p, &sc, h, signal, NULL, h_next, attn);
    scratch_free(&sc);
    prep_free(&p);
}

int orc_solve_token(const orc_cfg *c, const orc_weights *w, const float *x, float *h_star,
                    float *resid_trace) {
    prep p;
    scratch sc;
    prep_init(&p, c, w);
    scratch_init(&sc, c);
    int it = solve_p(&p, &sc, x, NULL, h_star, resid_trace, 0, NULL);
    scratch_free(&sc);
    prep_free(&p);
    return it;
}

/* ------------------------------------------------------------------------- */
/* lm_head.rs                                                                 */
/* ------------------------------------------------------------------------- */

/* lm_head.rs:35-54: pooled = fold(0, acc + slot)/H; rmsnorm(eps 1e-5): (v/rms)*g; W x + b. */
static void lm_head_tok(const orc_cfg *c, const orc_weights *w, const float *lm_wt,
                        const float *h_star, float *pooled, float *logits, float *tmp) {
    const int d = c->d, H = c->H, V = c->V;
    for (int i = 0; i < d; ++i) tmp[i] = 0.0f;
    for (int s = 0; s < H; ++s)
        for (int i = 0; i < d; ++i) tmp[i] = tmp[i] + h_star[(size_t)s * d + i];
    for (int i = 0; i < d; ++i) tmp[i] = tmp[i] / (float)H;
    if (pooled) memcpy(pooled, tmp, sizeof(float) * d);
    if (!logits) return;
    float ss = 0.0f;
    for (int i = 0; i < d; ++i) ss += tmp[i] * tmp[i];
    const float rms = sqrtf(ss / (float)d + 1e-5f);
    for (int i = 0; i < d; ++i) tmp[i] = (tmp[i] / rms) * (w->lm_g ? w->lm_g[i] : 1.0f);
    if (lm_wt)
        gemv_t(lm_wt, V, d, tmp, logits);
    else
        gemv_rm(w->lm_w, V, d, tmp, logits);
    if (w->lm_b)
        for (int v = 0; v < V; ++v) logits[v] = logits[v] + w->lm_b[v];
}

void orc_lm_head_token(const orc_cfg *c, const orc_weights *w, const float *h_star, float *pooled,
                       float *logits) {
    float *tmp = (float *)malloc(sizeof(float) * c->d);
    lm_head_tok(c, w, NULL, h_star, pooled, logits, tmp);
    free(tmp);
}

/* lm_head.rs:62-69: Iterator::max_by keeps the LAST maximal element; NaN compares Equal. */
int orc_argmax(const float *logits, int V) {
    if (V <= 0) return 0;
    int best = 0;
    float bv = logits[0];
    for (int v = 1; v < V; ++v) {
        const float x = logits[v];
        /* max_by replaces the running max when the new element is >= it (or unordered) */
        if (!(x < bv)) {
            best = v;
            bv = x;
        }
    }
    return best;
}

/* spectral_renorm.wgsl:26-47: the workgroup reduction (256 partial sums folded at strides
 * 128, 64, ..., 1). */
static float wg_tree_sum(float *part) {
    for (int stride = 128; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; ++t) part[t] += part[t + stride];
    return part[0];
}

/* spectral_renorm.wgsl:83-160: thread tid of 256 owns rows tid, tid + 256, ...; its partial sum of
 * squares runs over those rows in order. */
float orc_spectral_norm_gpu(const float *wg, int d, int n_iters) {
    float *u = (float *)malloc(sizeof(float) * d);
    float *v = (float *)malloc(sizeof(float) * d);
    float part[256];
    const int items = (d + 255) / 256;
    for (int i = 0; i < d; ++i) u[i] = 1.0f / sqrtf((float)d);
    float sigma = 1.0f;
    for (int it = 0; it < n_iters; ++it) {
        for (int row = 0; row < d; ++row) {
            float vt = 0.0f;
            for (int j = 0; j < d; ++j) vt += wg[(size_t)j * d + row] * u[j];
            v[row] = vt;
        }
        for (int t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int i = 0; i < items; ++i) {
                const int row = t + i * 256;
                if (row < d) acc += v[row] * v[row];
            }
            part[t] = acc;
        }
        const float vn = sqrtf(wg_tree_sum(part) + 1e-12f);
        for (int row = 0; row < d; ++row) v[row] = v[row] / vn;
        for (int t = 0; t < 256; ++t) part[t] = 0.0f;
        for (int row = 0; row < d; ++row) {
            float ut = 0.0f;
            for (int j = 0; j < d; ++j) ut += wg[(size_t)row * d + j] * v[j];
            u[row] = ut;
        }
        for (int t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int i = 0; i < items; ++i) {
                const int row = t + i * 256;
                if (row < d) acc += u[row] * u[row];
            }
            part[t] = acc;
        }
        sigma = sqrtf(wg_tree_sum(part) + 1e-12f);
        for (int row = 0; row < d; ++row) u[row] = u[row] / sigma;
    }
    free(u);
    free(v);
    return sigma;
}

/* spectral_renorm.wgsl:162-195: rescale when sigma exceeds the matrix's threshold. */
float orc_renorm_gpu(float *w, long n, const float *wg, int d, float threshold, int n_iters) {
    const float sigma = orc_spectral_norm_gpu(wg, d, n_iters);
    if (sigma > threshold) {
        const float scale = threshold / sigma;
        for (long i = 0; i < n; ++i) w[i] = w[i] * scale;
    }
    return sigma;
}

/* ------------------------------------------------------------------------- */
/* temporal carrier (selective scan)                                          */
/* ------------------------------------------------------------------------- */

/* One slot-token of the carrier prologue: u = h/rms(h) (FPMR:1462-1464), x = u + 0.5 tanh(wx) u
 * (FPMR:1471-1477), abar per FPMR:1468-1470 or the selective form of gpu_deq.rs:6172-6199,
 * B/C = W_B u, W_C u (rank-N readout, build-defined beyond N=1). */
static void carrier_inputs(const orc_cfg *c, const orc_weights *w, int s, const float *h,
                           float *x, float *abar, float *Bv, float *Cv, float *bn) {
    const int d = c->d, N = c->N, r = c->r;
    float ss = 0.0f;
    for (int i = 0; i < d; ++i) ss += h[i] * h[i];
    const float rms = sqrtf(ss / (float)d + 1e-6f);
    float *u = (float *)malloc(sizeof(float) * d);
    for (int i = 0; i < d; ++i) u[i] = h[i] / rms;
    for (int i = 0; i < d; ++i) {
        const float wx = 0.5f * tanhf(w->wx_diag[(size_t)s * d + i]);
        x[i] = u[i] + wx * u[i];
    }
    if (c->flags & ORC_F_SCAN_SELECTIVE) {
        const float *wkw = w->w_kw + (size_t)s * d * r;
        const float *wvw = w->w_vw + (size_t)s * r * d;
        for (int j = 0; j < r; ++j) bn[j] = 0.0f;
        for (int i = 0; i < d; ++i)
            for (int j = 0; j < r; ++j) bn[j] += wkw[(size_t)i * r + j] * u[i];
        for (int i = 0; i < d; ++i) {
            float pre = w->b_delta ? w->b_delta[(size_t)s * d + i] : 0.0f;
            for (int j = 0; j < r; ++j) pre += wvw[(size_t)j * d + i] * bn[j];
            const float delta = logf(1.0f + expf(pre));
            const float abase = 1.0f / (1.0f + expf(w->a_log[(size_t)s * d + i]));
            const float acore = expf(delta * logf(fmaxf(abase, 1.0e-6f)));
            abar[i] = 0.10f + (1.0f - 0.10f) * acore;
        }
    } else {
        for (int i = 0; i < d; ++i) abar[i] = 1.0f / (1.0f + expf(w->a_log[(size_t)s * d + i]));
    }
    for (int n = 0; n < N; ++n) {
        Bv[n] = w->w_b ? dot_seq(w->w_b + ((size_t)s * N + n) * d, u, d) : 1.0f;
        Cv[n] = w->w_c ? dot_seq(w->w_c + ((size_t)s * N + n) * d, u, d) : 1.0f;
    }
    free(u);
}

/* Readout carrier over one sequence: m_t[n] = abar m_{t-1}[n] + (1-abar) B_t[n] x_t,
 * y_t = sum_n C_t[n] m_t[n], Y_t = y_t + W_out y_t (FPMR:1478-1482 with the recurrent state kept
 * before W_out, UWGSL:2121-2140).  h_star [T][H][d]; state [H][d][N]; y [T][H][d]. */
void orc_scan_seq(const orc_cfg *c, const orc_weights *w, int T, const float *h_star,
                  const float *state_in, float *y, float *state_out) {
    const int d = c->d, H = c->H, N = c->N, r = c->r > 0 ? c->r : 1;
    /* The slots are independent carriers: they run in parallel (OpenMP; inside a caller's
     * parallel region the nested region runs on one thread), each with its own buffers.  W_out
     * is applied through its transpose (gemv_t, bit-identical to gemv_rm: the same per-output
     * order). */
#pragma omp parallel for schedule(dynamic, 1)
    for (int s = 0; s < H; ++s) {
        float *m = (float *)malloc(sizeof(float) * (size_t)d * N);
        float *x = (float *)malloc(sizeof(float) * d);
        float *ab = (float *)malloc(sizeof(float) * d);
        float *yt = (float *)malloc(sizeof(float) * d);
        float *wy = (float *)malloc(sizeof(float) * d);
        float *Bv = (float *)malloc(sizeof(float) * N);
        float *Cv = (float *)malloc(sizeof(float) * N);
        float *bn = (float *)malloc(sizeof(float) * r);
        float *wt = NULL;
        if (w->w_out) {
            wt = (float *)malloc(sizeof(float) * (size_t)d * d);
            transpose(w->w_out + (size_t)s * d * d, d, d, wt);
        }
        if (state_in)
            memcpy(m, state_in + (size_t)s * d * N, sizeof(float) * d * N);
        else
            memset(m, 0, sizeof(float) * d * N);
        for (int t = 0; t < T; ++t) {
            const float *h = h_star + ((size_t)t * H + s) * d;
            carrier_inputs(c, w, s, h, x, ab, Bv, Cv, bn);
            for (int i = 0; i < d; ++i) {
                const float bb = 1.0f - ab[i];
                float acc = 0.0f;
                for (int n = 0; n < N; ++n) {
                    float *mi = m + (size_t)i * N + n;
                    *mi = ab[i] * *mi + bb * (Bv[n] * x[i]);
                    acc += Cv[n] * *mi;
                }
                yt[i] = acc;
            }
            float *out = y + ((size_t)t * H + s) * d;
            if (wt) {
                gemv_t(wt, d, d, yt, wy);
                for (int i = 0; i < d; ++i) out[i] = yt[i] + wy[i];
            } else {
                memcpy(out, yt, sizeof(float) * d);
            }
        }
        if (state_out) memcpy(state_out + (size_t)s * d * N, m, sizeof(float) * d * N);
        free(m); free(x); free(ab); free(yt); free(wy); free(Bv); free(Cv); free(bn); free(wt);
    }
}

/* FPMR:1455-1486 temporal_step iterated over a sequence: the carried state is the output
 * (I + W_out) m (dense recirculation, N = 1, B = C = 1). */
void orc_scan_recirculate(const orc_cfg *c, const orc_weights *w, int T, const float *h_star,
                          const float *m_in, float *y) {
    const int d = c->d, H = c->H, r = c->r > 0 ? c->r : 1;
    float *m = (float *)malloc(sizeof(float) * d);
    float *mn = (float *)malloc(sizeof(float) * d);
    float *x = (float *)malloc(sizeof(float) * d);
    float *ab = (float *)malloc(sizeof(float) * d);
    float *wy = (float *)malloc(sizeof(float) * d);
    float Bv[1], Cv[1];
    float *bn = (float *)malloc(sizeof(float) * r);
    orc_cfg c1 = *c;
    c1.N = 1;
    orc_weights w1 = *w;
    w1.w_b = NULL;
    w1.w_c = NULL;
    for (int s = 0; s < H; ++s) {
        if (m_in)
            memcpy(m, m_in + (size_t)s * d, sizeof(float) * d);
        else
            memset(m, 0, sizeof(float) * d);
        for (int t = 0; t < T; ++t) {
            carrier_inputs(&c1, &w1, s, h_star + ((size_t)t * H + s) * d, x, ab, Bv, Cv, bn);
            for (int i = 0; i < d; ++i) mn[i] = ab[i] * m[i] + (1.0f - ab[i]) * x[i];
            float *out = y + ((size_t)t * H + s) * d;
            if (w->w_out) {
                gemv_rm(w->w_out + (size_t)s * d * d, d, d, mn, wy);
                for (int i = 0; i < d; ++i) out[i] = mn[i] + wy[i];
            } else {
                memcpy(out, mn, sizeof(float) * d);
            }
            memcpy(m, out, sizeof(float) * d);
        }
    }
    free(m); free(mn); free(x); free(ab); free(wy); free(bn);
}

/* ------------------------------------------------------------------------- */
/* whole forward                                                              */
/* ------------------------------------------------------------------------- */

/* A model with its weights laid out for the CPU loops (transposed once). */
struct orc_model {
    prep p;
    float *lm_wt; /* [d][V] */
};

orc_model *orc_model_create(const orc_cfg *c, const orc_weights *w) {
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    prep_init(&m->p, c, w);
    m->lm_wt = (float *)malloc(sizeof(float) * (size_t)c->V * c->d);
    transpose(w->lm_w, c->V, c->d, m->lm_wt);
    return m;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    prep_free(&m->p);
    free(m->lm_wt);
    free(m);
}

/* Canonical forward (TRAINER:4677-4731 per-token structure with x_t = E[tok] as in the
 * fixed-history query, tokenizer.rs:117-119): solve every token independently, pool, LM head,
 * greedy argmax; then the carrier over each sequence. */
void orc_model_forward(orc_model *mdl, int B, int T, const int32_t *tokens, float *h_star,
                       float *pooled, float *logits, int32_t *iters, int32_t *converged,
                       int32_t *argmax, float *scan_y, float *scan_state, int nthreads) {
    const orc_cfg *c = &mdl->p.c;
    const orc_weights *w = mdl->p.w;
    const int d = c->d, H = c->H, V = c->V;
    const size_t hd = (size_t)H * d;
    const long ntok = (long)B * T;
    const prep *p = &mdl->p;
    const float *lm_wt = mdl->lm_wt;
    float *hs_all = h_star;
    int own_h = 0;
    if (!hs_all) {
        hs_all = (float *)malloc(sizeof(float) * hd * ntok);
        own_h = 1;
    }
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        scratch sc;
        scratch_init(&sc, c);
        float *tmp = (float *)malloc(sizeof(float) * d);
        float *lg = (float *)malloc(sizeof(float) * V);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (long t = 0; t < ntok; ++t) {
            const int32_t tok = tokens[t];
            float *h = hs_all + hd * t;
            int cv = 0;
            int it = solve_p(p, &sc, w->embed + (size_t)tok * d, NULL, h, NULL, 0, &cv);
            if (iters) iters[t] = it;
            if (converged) converged[t] = cv;
            if (pooled || logits || argmax) {
                float *lt = logits ? logits + (size_t)V * t : lg;
                lm_head_tok(c, w, lm_wt, h, pooled ? pooled + (size_t)d * t : NULL,
                            (logits || argmax) ? lt : NULL, tmp);
                if (argmax) argmax[t] = orc_argmax(lt, V);
            }
        }
        free(tmp);
        free(lg);
        scratch_free(&sc);
    }
    if (scan_y || scan_state) {
        float *ybuf = scan_y;
        if (!ybuf) ybuf = (float *)malloc(sizeof(float) * hd * ntok);
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1)
#endif
        for (int b = 0; b < B; ++b)
            orc_scan_seq(c, w, T, hs_all + hd * (size_t)b * T, NULL, ybuf + hd * (size_t)b * T,
                         scan_state ? scan_state + (size_t)b * hd * c->N : NULL);
        if (!scan_y) free(ybuf);
    }
    if (own_h) free(hs_all);
}

void orc_forward(const orc_cfg *c, const orc_weights *w, int B, int T, const int32_t *tokens,
                 float *h_star, float *pooled, float *logits, int32_t *iters, int32_t *converged,
                 int32_t *argmax, float *scan_y, float *scan_state, int nthreads) {
    orc_model *m = orc_model_create(c, w);
    orc_model_forward(m, B, T, tokens, h_star, pooled, logits, iters, converged, argmax, scan_y, scan_state,
                      nthreads);
    orc_model_free(m);
}

/* ------------------------------------------------------------------------- */
/* memory-coupled solve (fixed history context)                               */
/* ------------------------------------------------------------------------- */

/* FPMR:1317-1329: alpha_k = 0.07 + (0.20 - 0.07) * sigmoid(hist_gate_logit[k]). */
static float hist_gate_alpha(const orc_hist_weights *hw, int k) {
    const float sigma = 1.0f / (1.0f + expf(-hw->gate_logit[k]));
    return 0.070f + (0.20f - 0.070f) * sigma;
}

/* FPMR:1337-1370 fixed_hist_ctx, with the input-signal RMS taken per slot (the reference has one
 * shared W_in, so its signal is the same for every slot; per-slot W_in generalises it).
 *   u_k = W_hist m_k + slot_scale_k * m_k / rms(m_k);  hist_k = u_k * (alpha_k * min(1, rms(sig_k)/rms(u_k)))
 * (scale 1 when rms(u_k) <= 1e-6).  m_prev == NULL gives the zero context. */
void orc_hist_ctx(const orc_cfg *c, const orc_hist_weights *hw, const float *m_prev,
                  const float *signal, float *hist) {
    const int d = c->d, H = c->H;
    if (!m_prev) {
        memset(hist, 0, sizeof(float) * (size_t)H * d);
        return;
    }
    float *u = (float *)malloc(sizeof(float) * d);
    for (int k = 0; k < H; ++k) {
        const float *sg = signal + (size_t)k * d;
        const float *pm = m_prev + (size_t)k * d;
        float ss = 0.0f;
        for (int i = 0; i < d; ++i) ss += sg[i] * sg[i];
        const float inj_rms = sqrtf(ss / (float)d + 1e-6f);
        float sp = 0.0f;
        for (int i = 0; i < d; ++i) sp += pm[i] * pm[i];
        const float prev_rms = sqrtf(sp / (float)d + 1e-6f);
        gemv_rm(hw->w_hist, d, d, pm, u);
        const float *sc = hw->slot_scale + (size_t)k * d;
        for (int i = 0; i < d; ++i) u[i] += sc[i] * (pm[i] / prev_rms);
        float su = 0.0f;
        for (int i = 0; i < d; ++i) su += u[i] * u[i];
        const float u_rms = sqrtf(su / (float)d + 1e-6f);
        const float scale = u_rms > 1e-6f ? fminf(inj_rms / u_rms, 1.0f) : 1.0f;
        const float g = hist_gate_alpha(hw, k) * scale;
        for (int i = 0; i < d; ++i) hist[(size_t)k * d + i] = u[i] * g;
    }
    free(u);
}

/* FPMR:1454-1485 temporal_step: m_next = (I + W_out)(abar m + (1 - abar) x), x = u(1 + 0.5 tanh wx),
 * u = h/rms(h), abar = sigmoid(-a_log) (or the selective decay when the flag is set).
 * m_prev == NULL is the zero state. */
void orc_temporal_step(const orc_cfg *c, const orc_weights *w, const float *m_prev,
                       const float *h_star, float *m_next) {
    const int d = c->d, H = c->H, r = c->r > 0 ? c->r : 1;
    float *x = (float *)malloc(sizeof(float) * d);
    float *ab = (float *)malloc(sizeof(float) * d);
    float *mn = (float *)malloc(sizeof(float) * d);
    float *wy = (float *)malloc(sizeof(float) * d);
    float *bn = (float *)malloc(sizeof(float) * r);
    float Bv[1], Cv[1];
    orc_cfg c1 = *c;
    c1.N = 1;
    orc_weights w1 = *w;
    w1.w_b = NULL;
    w1.w_c = NULL;
    for (int s = 0; s < H; ++s) {
        carrier_inputs(&c1, &w1, s, h_star + (size_t)s * d, x, ab, Bv, Cv, bn);
        const float *m = m_prev ? m_prev + (size_t)s * d : NULL;
        for (int i = 0; i < d; ++i) mn[i] = ab[i] * (m ? m[i] : 0.0f) + (1.0f - ab[i]) * x[i];
        float *out = m_next + (size_t)s * d;
        if (w->w_out) {
            gemv_rm(w->w_out + (size_t)s * d * d, d, d, mn, wy);
            for (int i = 0; i < d; ++i) out[i] = mn[i] + wy[i];
        } else {
            memcpy(out, mn, sizeof(float) * d);
        }
    }
    free(x); free(ab); free(mn); free(wy); free(bn);
}

/* Memory-coupled forward, the fixed-history reference mode of the trainer (TRAINER:677-720).
 * With ORC_F_TOKEN_CARRY the solve of position t > 0 starts from h*_{t-1} of the same sequence
 * instead of the init rule (the GPU reference's default warm start, UWGSL:898, BRIDGE:167-173):
 * per sequence and token, hist = fixed_hist_ctx(m_{t-1}, signal_t) (zero at the first token
 * unless m_in is given), h* = the Picard solve with hist added (FPMR:1372-1395), then
 * m_t = temporal_step(m_{t-1}, h*).  The solve keeps this library's exit rule (eps = 0 runs
 * exactly max_iters steps, as solve_query_with_fixed_history does).  m_seq [B][T][H][d] receives
 * every m_t; pooled/logits/argmax as in the canonical forward. */
void orc_forward_memory(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B,
                        int T, const int32_t *tokens, const float *m_in, float *h_star, float *pooled,
                        float *logits, int32_t *iters, int32_t *converged, int32_t *argmax, float *m_seq,
                        int nthreads) {
    const int d = c->d, H = c->H, V = c->V;
    const size_t hd = (size_t)H * d;
    prep p;
    prep_init(&p, c, w);
    float *lm_wt = (float *)malloc(sizeof(float) * (size_t)V * d);
    transpose(w->lm_w, V, d, lm_wt);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        scratch sc;
        scratch_init(&sc, c);
        float *sig = (float *)malloc(sizeof(float) * hd);
        float *hist = (float *)malloc(sizeof(float) * hd);
        float *h = (float *)malloc(sizeof(float) * hd);
        float *m = (float *)malloc(sizeof(float) * hd);
        float *mn = (float *)malloc(sizeof(float) * hd);
        float *tmp = (float *)malloc(sizeof(float) * d);
        float *lg = (float *)malloc(sizeof(float) * V);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int b = 0; b < B; ++b) {
            int have_m = 0;
            if (m_in) {
                memcpy(m, m_in + hd * b, sizeof(float) * hd);
                have_m = 1;
            }
            for (int t = 0; t < T; ++t) {
                const size_t row = (size_t)b * T + t;
                const float *x = w->embed + (size_t)tokens[row] * d;
                signal_p(&p, x, sig);
                orc_hist_ctx(c, hw, have_m ? m : NULL, sig, hist);
                /* token carry: h still holds h*_{t-1} of this sequence (UWGSL:898
                 * should_init_h = t == 0 || !ENABLE_TOKEN_CARRY) */
                const int warm = (c->flags & ORC_F_TOKEN_CARRY) && t > 0;
                int cv = 0;
                const int it = solve_p(&p, &sc, x, hist, h, NULL, warm, &cv);
                if (iters) iters[row] = it;
                if (converged) converged[row] = cv;
                if (h_star) memcpy(h_star + hd * row, h, sizeof(float) * hd);
                orc_temporal_step(c, w, have_m ? m : NULL, h, mn);
                memcpy(m, mn, sizeof(float) * hd);
                have_m = 1;
                if (m_seq) memcpy(m_seq + hd * row, m, sizeof(float) * hd);
                if (pooled || logits || argmax) {
                    float *lt = logits ? logits + (size_t)V * row : lg;
                    lm_head_tok(c, w, lm_wt, h, pooled ? pooled + (size_t)d * row : NULL, lt, tmp);
                    if (argmax) argmax[row] = orc_argmax(lt, V);
                }
            }
        }
        free(sig); free(hist); free(h); free(m); free(mn); free(tmp); free(lg);
        scratch_free(&sc);
    }
    free(lm_wt);
    prep_free(&p);
}

/* tokenizer.rs:133-149 embed_context over one window ctx[0..len) (len <= max_ctx, so the whole
 * window is used): result += emb * pos_weight in window order, pos_weight = (pos + 1) as f32 /
 * len as f32 (f32 division), then result / result.norm() when the norm exceeds 1e-6.  The norm's
 * summation order (nalgebra) is restated as a sequential sum of squares: ulp-level, unpinned. */
static void embed_window(int d, const float *embed, const int32_t *ctx, int len, float *r, float *out) {
    for (int j = 0; j < d; ++j) r[j] = 0.0f;
    for (int pos = 0; pos < len; ++pos) {
        const float w = (float)(pos + 1) / (float)len;
        const float *e = embed + (size_t)ctx[pos] * d;
        for (int j = 0; j < d; ++j) {
            const float t = e[j] * w;
            r[j] = r[j] + t;
        }
    }
    float ss = 0.0f;
    for (int j = 0; j < d; ++j) ss += r[j] * r[j];
    const float nrm = sqrtf(ss);
    for (int j = 0; j < d; ++j) out[j] = nrm > 1e-6f ? r[j] / nrm : r[j];
}

/* LmHead::sample's repetition penalty (lm_head.rs:81-99): every distinct token of the context has
 * its logit multiplied by the penalty when negative, divided by it otherwise; nothing happens when
 * |penalty - 1| <= 1e-4 or the context is empty.  Greedy sampling (temperature <= 0) then takes
 * the arg-max of the penalised logits (lm_head.rs:104-111). */
static void repetition_penalty(float *logits, int V, const int32_t *ctx, int len, float pen) {
    if (!(fabsf(pen - 1.0f) > 1e-4f) || len == 0) return;
    for (int p = 0; p < len; ++p) {
        const int tok = ctx[p];
        int seen = 0;
        for (int q = 0; q < p && !seen; ++q) seen = ctx[q] == tok;
        if (seen || tok < 0 || tok >= V) continue;
        const float sc = logits[tok];
        logits[tok] = sc < 0.0f ? sc * pen : sc / pen;
    }
}

/* Greedy decode as Trainer::generate (TRAINER:4219-4431) with LmHead::sample at temperature
 * <= 1e-4.  prompt [B][T0] (T0 >= 1), out_tokens [B][n_new].  At step j of sequence b the context
 * is the last ctx_len of its T0 + j tokens (TRAINER:4248-4249), and
 *   - canonical (TRAINER:4388-4392, 4402-4406): query = embed_context(context, ctx_len), h = the
 *     solve from init(query) under c's iteration cap and exit rule (generate itself runs exactly 10
 *     steps: max_iters = 10, eps = 0);
 *   - ORC_F_MEMORY, the fixed-history reference mode (TRAINER:4395-4400 with 677-735): the memory is
 *     first primed over every prompt token (prime_fixed_history_state, :718-733), then each step
 *     solves query = embed(last context token) with hist = fixed_hist_ctx(m, signal) and advances
 *     m = temporal_step(m, h*) (each solve from the init rule, as solve_query_with_fixed_history);
 * then logits = LmHead::forward(h) (lm_head.rs:50-54), the repetition penalty over the context,
 * and the arg-max with the last-max tie rule; the token is appended. */
int orc_lm_sample(const float *logits_in, int V, const int32_t *ctx, int L, float temperature, float top_p,
                  int top_k, float rep_penalty, float r, double *cond);

/* smp: temperature, top_p, top_k (as a float) per LmHead::sample, uniforms [B][n_new] the draws and
 * cond [B][n_new] (or NULL) each step's conditioning; NULL = greedy */
typedef struct {
    float temperature, top_p;
    int top_k;
    const float *uniforms;
    double *cond;
} samp_cfg;

static void decode_run(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B, int T0,
                       const int32_t *prompt, int n_new, int ctx_len, float rep_penalty, const samp_cfg *smp,
                       int32_t *out_tokens, int nthreads) {
    const int d = c->d, H = c->H, V = c->V;
    const size_t hd = (size_t)H * d;
    const int memory = (c->flags & ORC_F_MEMORY) != 0;
    prep p;
    prep_init(&p, c, w);
    float *lm_wt = (float *)malloc(sizeof(float) * (size_t)V * d);
    transpose(w->lm_w, V, d, lm_wt);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        scratch sc;
        scratch_init(&sc, c);
        int32_t *toks = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T0 + n_new));
        float *q = (float *)malloc(sizeof(float) * d);
        float *r = (float *)malloc(sizeof(float) * d);
        float *tmp = (float *)malloc(sizeof(float) * d);
        float *h = (float *)malloc(sizeof(float) * hd);
        float *sig = (float *)malloc(sizeof(float) * hd);
        float *hist = (float *)malloc(sizeof(float) * hd);
        float *m = (float *)malloc(sizeof(float) * hd);
        float *mn = (float *)malloc(sizeof(float) * hd);
        float *lg = (float *)malloc(sizeof(float) * V);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int b = 0; b < B; ++b) {
            memcpy(toks, prompt + (size_t)b * T0, sizeof(int32_t) * T0);
            int have_m = 0;
            if (memory) {
                for (int t = 0; t < T0; ++t) {
                    const float *x = w->embed + (size_t)toks[t] * d;
                    signal_p(&p, x, sig);
                    orc_hist_ctx(c, hw, have_m ? m : NULL, sig, hist);
                    solve_p(&p, &sc, x, hist, h, NULL, 0, NULL);
                    orc_temporal_step(c, w, have_m ? m : NULL, h, mn);
                    memcpy(m, mn, sizeof(float) * hd);
                    have_m = 1;
                }
            }
            for (int j = 0; j < n_new; ++j) {
                const int len = T0 + j;
                const int start = len > ctx_len ? len - ctx_len : 0;
                const int32_t *ctx = toks + start;
                const int L = len - start;
                if (memory) {
                    const float *x = w->embed + (size_t)ctx[L - 1] * d;
                    signal_p(&p, x, sig);
                    orc_hist_ctx(c, hw, have_m ? m : NULL, sig, hist);
                    solve_p(&p, &sc, x, hist, h, NULL, 0, NULL);
                    orc_temporal_step(c, w, have_m ? m : NULL, h, mn);
                    memcpy(m, mn, sizeof(float) * hd);
                    have_m = 1;
                } else {
                    embed_window(d, w->embed, ctx, L, r, q);
                    solve_p(&p, &sc, q, NULL, h, NULL, 0, NULL);
                }
                lm_head_tok(c, w, lm_wt, h, NULL, lg, tmp);
                int32_t tok;
                if (smp) {
                    const size_t jb = (size_t)b * n_new + j;
                    double cd[2];
                    tok = orc_lm_sample(lg, V, ctx, L, smp->temperature, smp->top_p, smp->top_k, rep_penalty,
                                        smp->uniforms[jb], cd);
                    if (smp->cond) smp->cond[jb] = cd[0];
                } else {
                    repetition_penalty(lg, V, ctx, L, rep_penalty);
                    tok = orc_argmax(lg, V);
                }
                toks[len] = tok;
                out_tokens[(size_t)b * n_new + j] = tok;
            }
        }
        free(toks); free(q); free(r); free(tmp); free(h); free(sig); free(hist); free(m); free(mn); free(lg);
        scratch_free(&sc);
    }
    free(lm_wt);
    prep_free(&p);
}

void orc_decode_greedy(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B, int T0,
                       const int32_t *prompt, int n_new, int ctx_len, float rep_penalty,
                       int32_t *out_tokens, int nthreads) {
    decode_run(c, w, hw, B, T0, prompt, n_new, ctx_len, rep_penalty, NULL, out_tokens, nthreads);
}

/* The same loop with LmHead::sample (lm_head.rs:78-168) in place of the arg-max (TRAINER:4410-4417):
 * step j of sequence b draws with uniforms[b][j]; cond [B][n_new] (or NULL) receives each step's
 * conditioning as orc_lm_sample gives it. */
void orc_decode_sample(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B, int T0,
                       const int32_t *prompt, int n_new, int ctx_len, float temperature, float top_p, int top_k,
                       float rep_penalty, const float *uniforms, int32_t *out_tokens, double *cond,
                       int nthreads) {
    const samp_cfg smp = {temperature, top_p, top_k, uniforms, cond};
    decode_run(c, w, hw, B, T0, prompt, n_new, ctx_len, rep_penalty, &smp, out_tokens, nthreads);
}

/* LmHead::sample's sorted list (lm_head.rs:115-117): probability descending by a stable sort,
 * so equal probabilities keep index order. */
typedef struct {
    float p;
    int32_t i;
} samp_item;

static int samp_cmp(const void *a, const void *b) {
    const samp_item *x = (const samp_item *)a, *y = (const samp_item *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return (x->i > y->i) - (x->i < y->i);
}

/* Conditioning of one decision, for the tests: the smallest ratio of a decisive distance to the
 * rounding that could move it on a device with its own exp (within an ulp) and summation orders.
 * >= 1: that device takes the same decision.  Order: the scaled logits of adjacent list items
 * whose order decides differ by at least 5e-7 (four ulps of relative probability; equal logits
 * give equal probabilities everywhere).  Cuts: where rounding could move the top-k cut (its two
 * items' logits closer than that) or the top-p cut (the running sum within its own float error,
 * twice, plus top_p times the float error of the softmax sum, plus 1e-7, of top_p), the kept
 * weight may change by the items involved and the items from the first of them on may enter or
 * leave: a draw landing there reads 0, any other has that weight added to its tolerance.  Draw:
 * the normalised running sum lies from the draw by at least twice its float error plus 1e-7 plus
 * that weight.  0 when the float running sums take another decision than the same sums in double. */
static double samp_dw(const float *w, float mx, const samp_item *it, int a, int b) {
    const float x = w[it[a].i], y = w[it[b].i];
    if (x == y) return INFINITY;
    /* exp(l - max) below 2^-150 is 0 on every device: such items are ordered by index alone */
    if (it[a].p == 0.0f && it[b].p == 0.0f && fmaxf(x, y) - mx < -105.0f) return INFINITY;
    return fabs((double)x - (double)y) / 5e-7;
}

/* LmHead::sample (lm_head.rs:78-168) with the draw r = rng.gen::<f32>() given (the reference
 * draws it from thread_rng).  ctx [L] the context.  cond (or NULL) receives [2]: the
 * conditioning above (INFINITY where no rounding enters: greedy, the fallback arg-max) and the
 * length of the kept list (0 where there is none). */
int orc_lm_sample(const float *logits_in, int V, const int32_t *ctx, int L, float temperature, float top_p,
                  int top_k, float rep_penalty, float r, double *cond) {
    if (cond) {
        cond[0] = INFINITY;
        cond[1] = 0.0;
    }
    if (V <= 0) return 0;
    float *w = (float *)malloc(sizeof(float) * (size_t)V);
    memcpy(w, logits_in, sizeof(float) * (size_t)V);
    /* 1. repetition penalty (:81-99) */
    repetition_penalty(w, V, ctx, L, rep_penalty);
    /* 2. temperature (:103-111): a temperature in (0, 1e-4] takes the first branch */
    if (temperature > 0.0f && fabsf(temperature - 1.0f) > 1e-4f) {
        for (int v = 0; v < V; ++v) w[v] /= temperature;
    } else if (temperature <= 1e-4f) {
        const int t = orc_argmax(w, V);
        free(w);
        return t;
    }
    /* 3. softmax (:71-76): max by f32::max (NaN skipped), exp(l - max), the sum folded in index
     * order, each exp divided by it */
    float mx = -INFINITY;
    for (int v = 0; v < V; ++v) mx = fmaxf(mx, w[v]);
    samp_item *it = (samp_item *)malloc(sizeof(samp_item) * (size_t)V);
    float S = 0.0f;
    double S_d = 0.0;
    for (int v = 0; v < V; ++v) {
        it[v].p = expf(w[v] - mx);
        it[v].i = v;
    }
    for (int v = 0; v < V; ++v) {
        S += it[v].p;
        S_d += (double)it[v].p;
    }
    /* a NaN sum makes every probability NaN; the kept sum then fails `sum > 1e-6` (:146-150) */
    if (S != S) {
        free(w);
        free(it);
        return orc_argmax(logits_in, V);
    }
    for (int v = 0; v < V; ++v) it[v].p = it[v].p / S;
    qsort(it, (size_t)V, sizeof(samp_item), samp_cmp);
    double cm = INFINITY;
    /* a cut that rounding could move changes the kept weight by at most mshift and the membership
     * of the items from position win on */
    double mshift = 0.0;
    int win = V;
    /* 4. top-k (:120-125) */
    int n = V;
    const int k = top_k < V ? top_k : V;
    if (k > 0 && k < V) {
        n = k;
        if (samp_dw(w, mx, it, k - 1, k) < 1.0) {
            mshift += (double)it[k - 1].p + (double)it[k].p;
            win = k - 1;
        }
    }
    /* 5. top-p (:127-140) */
    if (top_p > 0.0f && top_p < 1.0f) {
        float cum = 0.0f;
        double cd = 0.0;
        int cut = n, cut_d = n;
        for (int i = 0; i < n; ++i) {
            cum += it[i].p;
            if (cum > top_p) {
                cut = i + 1;
                break;
            }
        }
        for (int i = 0; i < n; ++i) {
            cd += (double)it[i].p;
            if (cd > (double)top_p) {
                cut_d = i + 1;
                break;
            }
        }
        /* the running sums just before and at the cut, in float and in double */
        double before = 0.0;
        float bf = 0.0f;
        for (int i = 0; i + 1 < cut; ++i) {
            before += (double)it[i].p;
            bf += it[i].p;
        }
        const double at = before + (double)it[cut - 1].p;
        const float af = bf + it[cut - 1].p;
        const double err = fmax(fabs((double)bf - before), fabs((double)af - at));
        const double tol = 2.0 * err + (double)top_p * fabs((double)S - S_d) / S_d + 1e-7;
        double mp = ((double)top_p - before) / tol;
        if (cut < n || n < V) mp = fmin(mp, fabs(at - (double)top_p) / tol);
        if (cut < V) mp = fmin(mp, samp_dw(w, mx, it, cut - 1, cut));
        if (cut != cut_d || mp < 1.0) {
            /* the cut may move over the items whose running sum lies within 2 tol of top_p */
            double acc = 0.0;
            int i0 = 0;
            while (i0 < n && acc + (double)it[i0].p < (double)top_p - 2.0 * tol) acc += (double)it[i0++].p;
            win = i0 < win ? i0 : win;
            mshift += 4.0 * tol + (double)it[cut - 1].p + (cut < V ? (double)it[cut].p : 0.0);
        }
        n = cut > 1 ? cut : 1;
    }
    /* 6. renormalisation (:142-150) */
    float sum = -0.0f;
    double sd = 0.0;
    for (int i = 0; i < n; ++i) {
        sum += it[i].p;
        sd += (double)it[i].p;
    }
    if (!(sum > 1e-6f)) {
        free(w);
        free(it);
        return orc_argmax(logits_in, V);
    }
    /* 7. the draw (:152-166) */
    float cum = 0.0f;
    int s = -1;
    for (int i = 0; i < n; ++i) {
        cum += it[i].p / sum;
        if (r <= cum) {
            s = i;
            break;
        }
    }
    /* the normalised running sums in double, and their float error up to the decision */
    double cn = 0.0, err = 0.0;
    float cf = 0.0f;
    int s_d = -1;
    double lo = INFINITY, hi = INFINITY, at = 1.0;
    for (int i = 0; i < n; ++i) {
        const double nx = cn + (double)it[i].p / sd;
        cf += it[i].p / sum;
        err = fmax(err, fabs((double)cf - nx));
        if ((double)r <= nx) {
            s_d = i;
            hi = nx - (double)r;
            if (i > 0) lo = (double)r - cn;
            at = nx;
            break;
        }
        cn = nx;
    }
    if (s_d < 0) lo = (double)r - cn;
    cm = fmin(cm, fmin(lo, hi) / (2.0 * err + 1e-7 + at * mshift / sd));
    if (s != s_d || (s >= 0 ? s : 0) >= win) cm = 0.0;
    const int pos = s >= 0 ? s : 0;
    if (s >= 0) {
        if (pos > 0) cm = fmin(cm, samp_dw(w, mx, it, pos - 1, pos));
        if (pos + 1 < n) cm = fmin(cm, samp_dw(w, mx, it, pos, pos + 1));
    }
    const int tok = it[pos].i;
    if (cond) {
        cond[0] = cm;
        cond[1] = (double)n;
    }
    free(w);
    free(it);
    return tok;
}

/* ------------------------------------------------------------------------- */
/* trait surfaces                                                             */
/* ------------------------------------------------------------------------- */

/* The shader's reduction order: each of 64 lanes sums x[lane], x[lane + 64], ... (or, with
 * contiguous = 1, its own block of d/64 values), then a tree over the lanes with strides
 * 32, 16, ..., 1 (staged_adjoint_picard_clean.wgsl:201-209, 301-309). */
static float lane_tree_sum(const float *x, int d, int contiguous) {
    float lanes[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        if (contiguous) {
            const int per = d / 64;
            for (int k = 0; k < per; ++k) acc = acc + x[l * per + k];
        } else {
            for (int i = l; i < d; i += 64) acc = acc + x[i];
        }
        lanes[l] = acc;
    }
    for (int stride = 32; stride > 0; stride >>= 1)
        for (int l = 0; l < stride; ++l) lanes[l] = lanes[l] + lanes[l + stride];
    return lanes[0];
}

/* one row's RMSNorm VJP terms: inv_rms and coeff_scale (:211-214), with up = beta v */
static void adj_row_terms(int d, const float *pre, const float *v, const float *g, float beta, int contiguous,
                          float *tmp, float *inv_rms, float *coeff_scale) {
    for (int i = 0; i < d; ++i) tmp[i] = pre[i] * pre[i];
    const float sumsq = lane_tree_sum(tmp, d, contiguous);
    for (int i = 0; i < d; ++i) {
        const float up = beta * v[i];
        tmp[i] = up * g[i] * pre[i];
    }
    const float coeff = lane_tree_sum(tmp, d, contiguous);
    const float inv_d = 1.0f / fmaxf(1.0f, (float)d);
    const float rms = sqrtf(sumsq * inv_d + 1.0e-6f);
    *inv_rms = 1.0f / fmaxf(rms, 1.0e-6f);
    *coeff_scale = coeff / fmaxf((float)d * rms * rms * rms, 1.0e-6f);
}

void orc_adjoint(const orc_cfg *c, const float *norm_scale, int ntok, const float *signal, const float *h_star,
                 const float *dl, int iters, float beta, float *v_out, float *src) {
    const int d = c->d, H = c->H, m = c->anderson_m;
    const size_t hd = (size_t)H * d, n = (size_t)ntok * hd;
    float *pre = (float *)malloc(sizeof(float) * n);
    float *v = (float *)malloc(sizeof(float) * n);
    float *vn = (float *)malloc(sizeof(float) * n);
    float *ring = m > 0 ? (float *)malloc(sizeof(float) * n * m) : NULL;
    float *tmp = (float *)malloc(sizeof(float) * d);
    const float rhs_scale = 1.0f / fmaxf(1.0f, (float)H);
    for (size_t e = 0; e < n; ++e) pre[e] = signal[e] + 1.0f * h_star[e];
    for (int t = 0; t < ntok; ++t)
        for (int s = 0; s < H; ++s)
            for (int i = 0; i < d; ++i) v[((size_t)t * H + s) * d + i] = dl[(size_t)t * d + i] * rhs_scale;
    for (int k = 0; k < iters; ++k) {
        for (int t = 0; t < ntok; ++t)
            for (int s = 0; s < H; ++s) {
                const size_t o = ((size_t)t * H + s) * d;
                float inv_rms, cs;
                adj_row_terms(d, pre + o, v + o, norm_scale, beta, 0, tmp, &inv_rms, &cs);
                for (int i = 0; i < d; ++i) {
                    const float vp = v[o + i];
                    const float ng = (norm_scale[i] * inv_rms) * (beta * vp) - pre[o + i] * cs;
                    const float jac = 1.0f * ng + (1.0f - beta) * vp;
                    vn[o + i] = dl[(size_t)t * d + i] * rhs_scale + jac;
                }
            }
        if (m > 0) { /* store, then mix from k >= 2 (gpu_deq.rs:4893-4906; the shader's :1012-1134) */
            memcpy(ring + (size_t)(k % m) * n, vn, sizeof(float) * n);
            const int n_res = k < m - 1 ? k : m - 1;
            if (k >= 2 && n_res >= 2) {
                for (int t = 0; t < ntok; ++t) {
                    float g[16], bt[4];
                    for (int ri = 0; ri < n_res; ++ri)
                        for (int rj = ri; rj < n_res; ++rj) {
                            const float *xi = ring + (size_t)((k + m - ri) % m) * n + (size_t)t * hd;
                            const float *xi1 = ring + (size_t)((k + m - ri - 1) % m) * n + (size_t)t * hd;
                            const float *xj = ring + (size_t)((k + m - rj) % m) * n + (size_t)t * hd;
                            const float *xj1 = ring + (size_t)((k + m - rj - 1) % m) * n + (size_t)t * hd;
                            float acc = 0.0f;
                            for (size_t e = 0; e < hd; ++e) acc += (xi[e] - xi1[e]) * (xj[e] - xj1[e]);
                            g[ri * n_res + rj] = acc;
                            g[rj * n_res + ri] = acc;
                        }
                    orc_anderson_coeffs(n_res, g, bt);
                    for (size_t e = 0; e < hd; ++e) {
                        float acc = 0.0f;
                        for (int i = 0; i < n_res; ++i)
                            acc += bt[i] * ring[(size_t)((k + m - i) % m) * n + (size_t)t * hd + e];
                        vn[(size_t)t * hd + e] = acc;
                    }
                }
            }
        }
        float *sw = v;
        v = vn;
        vn = sw;
    }
    if (v_out) memcpy(v_out, v, sizeof(float) * n);
    if (src) { /* picard_source_grad_reduce_main (:252-336): slots summed in order */
        for (int t = 0; t < ntok; ++t) {
            float *o = src + (size_t)t * d;
            for (int i = 0; i < d; ++i) o[i] = 0.0f;
            for (int s = 0; s < H; ++s) {
                const size_t r = ((size_t)t * H + s) * d;
                float inv_rms, cs;
                /* the shader gives each lane d/64 contiguous dims (d a multiple of 64 there) */
                adj_row_terms(d, pre + r, v + r, norm_scale, beta, d % 64 == 0, tmp, &inv_rms, &cs);
                for (int i = 0; i < d; ++i) o[i] = o[i] + ((norm_scale[i] * inv_rms) * (beta * v[r + i]) - pre[r + i] * cs);
            }
        }
    }
    free(pre); free(v); free(vn); free(ring); free(tmp);
}

/* tokenizer.rs:133-149 embed_context, one window per position (TRAINER:4690-4696).  The reference
 * evaluates result += emb * pos_weight in window order with pos_weight = (pos + 1) as f32 /
 * len as f32 (f32 division), then divides by result.norm() when it exceeds 1e-6.  The norm's
 * summation order (nalgebra) is restated as a sequential sum of squares: ulp-level, unpinned. */
void orc_embed_context(int d, const float *embed, int B, int T, const int32_t *tokens, int ctx, float *out) {
    float *r = (float *)malloc(sizeof(float) * d);
    for (int b = 0; b < B; ++b) {
        for (int i = 0; i < T; ++i) {
            const int start = i + 1 > ctx ? i + 1 - ctx : 0;
            embed_window(d, embed, tokens + (size_t)b * T + start, i + 1 - start, r, out + ((size_t)b * T + i) * d);
        }
    }
    free(r);
}

/* gpu_backend.rs:18-56 CpuBlockBackend::fpm_batch_step (ZOH, h_prev = 0). */
void orc_zoh_step(int d, const float *x, const float *dt, const float *a, const float *b,
                  const float *c, float *y) {
    for (int i = 0; i < d; ++i) {
        const float abar = expf(dt[i] * a[i]);
        const float bbar = fabsf(a[i]) > 1e-8f ? (abar - 1.0f) / a[i] * b[i] : dt[i] * b[i];
        const float hn = bbar * x[i];
        y[i] = c[i] * hn;
    }
}

/* aideen-engine/src/gpu/shaders/ffn_forward.wgsl:22-37: y[row] = sum_i w[i*out + row] x[i]. */
void orc_gemv_colmajor(const float *w, const float *x, int in_dim, int out_dim, float *y) {
    for (int r = 0; r < out_dim; ++r) {
        float acc = 0.0f;
        for (int i = 0; i < in_dim; ++i) acc += w[(size_t)i * out_dim + r] * x[i];
        y[r] = acc;
    }
}

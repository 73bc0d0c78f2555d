/*
 * aideen_oracle.h -- CPU restatement of the AIDEEN DEQ forward (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  Every function cites the reference
 * (SergioAriel/aideen) file:line whose arithmetic it restates.
 *
 * Layout conventions (identical to the product C-ABI, include/aideen_hip.h):
 *   per-slot matrices   W[s][out][in]   row-major, so y = W[s] . x  (FPMR:1314, FPMR:1402-1421)
 *   slot vectors        [H][d]          HSlots row-major [slot][d]   (aideen-core/src/state.rs:85-146)
 *   hidden states       [B][T][H][d]    token-major                  (UWGSL:711-712)
 *   LM head             lm_w [V][d]     row-major                    (lm_head.rs:11-12)
 */
#ifndef AIDEEN_ORACLE_H
#define AIDEEN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Semantic switches; the values equal the ADN_F_* bits of include/aideen_hip.h. */
#define ORC_F_WIN_TRANSPOSED   (1u << 0) /* signal = W_in^T x        (UWGSL:773, PPT:161)            */
#define ORC_F_SCORE_CLAMP4     (1u << 1) /* scores clamped to [-4,4] (PPT:216, ARCHITECTURE.md:128)  */
#define ORC_F_RMS_EXCL_ANCHOR  (1u << 2) /* RMS over o+signal only   (ARCHITECTURE.md:160-170)       */
#define ORC_F_INIT_SIGNAL_RMS  (1u << 3) /* h0 = signal/rms(signal)  (UWGSL:900-943)                 */
#define ORC_F_RESID_L2         (1u << 4) /* L2 residual over [H*d]   (aideen-node/src/inference.rs:214-221) */
#define ORC_F_SCAN_SELECTIVE   (1u << 5) /* input-dependent decay    (gpu_deq.rs:6129-6214)          */
#define ORC_F_MEMORY           (1u << 9) /* memory-coupled forward   (orc_forward_memory; TRAINER:677-720) */
#define ORC_F_TOKEN_CARRY      (1u << 10) /* memory mode: position t starts from h*_{t-1} (UWGSL:898, BRIDGE:167-173) */
#define ORC_F_RESID_RELRMS     (1u << 11) /* largest per-slot relative RMS residual (UWGSL:1654-1695) */
#define ORC_F_HOMEOSTATIC_EXIT (1u << 12) /* plateau exit as well (UWGSL:277-279,1786-1793)         */

typedef struct orc_cfg {
    int32_t d, H, V, N, r;     /* d_r, h_slots, vocab, d_state, write rank (FPMR:290 RETAIN_RANK=32) */
    uint32_t flags;
    int32_t max_iters;
    float eps;                 /* residual tolerance (ArchitectureConfig::deq_epsilon) */
    float beta;                /* Picard damping (FPMR:458, 0.70)                     */
    int32_t anderson_m;        /* 0 = plain Picard                                    */
} orc_cfg;

typedef struct orc_weights {
    const float *w_q, *w_k, *w_v, *w_o, *w_in; /* [H][d][d]                      */
    const float *q_bias, *k_bias;               /* [H][d] or NULL (zero)          */
    const float *anchor;                        /* [H][d] slot_anchor             */
    const float *norm_scale;                    /* [d]                            */
    const float *embed;                         /* [V][d]                         */
    const float *lm_w;                          /* [V][d]                         */
    const float *lm_b;                          /* [V] or NULL (zero)             */
    const float *lm_g;                          /* [d] or NULL (ones)             */
    const float *a_log;                         /* [H][d]                         */
    const float *wx_diag;                       /* [H][d] diagonal of W_x         */
    const float *w_out;                         /* [H][d][d] or NULL (zero)       */
    const float *b_delta;                       /* [H][d] or NULL (zero)          */
    const float *w_kw;                          /* [H][d][r]                      */
    const float *w_vw;                          /* [H][r][d]                      */
    const float *w_b, *w_c;                     /* [H][N][d] or NULL (ones)       */
} orc_weights;

/* --- spectral_norm.rs ---------------------------------------------------- */
float orc_spectral_norm(const float *w, int rows, int cols, int n_iter);
void  orc_normalize(float *w, int rows, int cols, float target, int n_iter);
void  orc_normalize_if_needed(float *w, int rows, int cols, float threshold, int n_iter);

/* --- spectral_renorm.wgsl:83-196 (GpuDeqBackend::renormalize_spectral, gpu_deq.rs:5567-5591;
 *     RustDeqBridge::renormalize_spectral, deq_bridge.rs:1742-1791) ------------------------------
 * sigma of one d x d matrix as the shader estimates it, from the matrix as the shader's buffer
 * holds it, wg[i*d + j]: u = 1/sqrt(d); per iteration v = wg^T u / sqrt(|.|^2 + 1e-12),
 * u' = wg v, sigma = sqrt(|u'|^2 + 1e-12), u = u' / sigma; each dot product summed over j in
 * order, each squared norm as the shader's 256-thread tree. */
float orc_spectral_norm_gpu(const float *wg, int d, int n_iters);
/* The renormalisation of one matrix w (n floats): sigma from orc_spectral_norm_gpu of its buffer
 * form wg; when sigma > threshold every element becomes w * (threshold / sigma).  Returns sigma. */
float orc_renorm_gpu(float *w, long n, const float *wg, int d, float threshold, int n_iters);
void  orc_damped_update(const float *h, const float *f, float beta, int n, float *out);

/* --- FPMR per-token pieces ------------------------------------------------ */
void orc_signal(const orc_cfg *c, const orc_weights *w, const float *x, float *signal);
void orc_init(const orc_cfg *c, const orc_weights *w, const float *x, const float *signal, float *h0);
void orc_picard_step(const orc_cfg *c, const orc_weights *w, const float *h, const float *signal,
                     float *h_next, float *attn /* [H][H] or NULL */);
/* Anderson coefficients for n = 2..4 pseudo-residuals (g is the n x n Gram matrix). */
void orc_anderson_coeffs(int n, const float *g, float *beta);
int  orc_solve_token(const orc_cfg *c, const orc_weights *w, const float *x, float *h_star,
                     float *resid_trace /* [max_iters] or NULL */);

/* --- lm_head.rs ----------------------------------------------------------- */
void orc_lm_head_token(const orc_cfg *c, const orc_weights *w, const float *h_star,
                       float *pooled /* [d] or NULL */, float *logits /* [V] or NULL */);
int  orc_argmax(const float *logits, int V);

/* --- temporal carrier ------------------------------------------------------ */
void orc_scan_seq(const orc_cfg *c, const orc_weights *w, int T, const float *h_star,
                  const float *state_in, float *y, float *state_out);
void orc_scan_recirculate(const orc_cfg *c, const orc_weights *w, int T, const float *h_star,
                          const float *m_in, float *y);

/* --- memory-coupled solve (FPMR:1317-1370, 1454-1485; TRAINER:677-720) ---- */
typedef struct orc_hist_weights {
    const float *w_hist;     /* [d][d] shared W_hist, row-major (u = W_hist m)  */
    const float *slot_scale; /* [H][d] hist_slot_scale                          */
    const float *gate_logit; /* [H]    hist_gate_logit                          */
} orc_hist_weights;
void orc_hist_ctx(const orc_cfg *c, const orc_hist_weights *hw, const float *m_prev /* [H][d] or NULL */,
                  const float *signal /* [H][d] */, float *hist /* [H][d] */);
void orc_temporal_step(const orc_cfg *c, const orc_weights *w, const float *m_prev /* or NULL */,
                       const float *h_star, float *m_next);
void orc_forward_memory(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B,
                        int T, const int32_t *tokens, const float *m_in /* [B][H][d] or NULL */,
                        float *h_star, float *pooled, float *logits, int32_t *iters, int32_t *converged,
                        int32_t *argmax, float *m_seq /* [B][T][H][d] */, int nthreads);

/* --- whole forward and decode ----------------------------------------------- */
/* converged [B][T] (or NULL): 1 = exit on the tolerance or plateau, 0 = stopped at max_iters
 * (a non-finite residual counts as infinite, so a NaN state never converges). */
void orc_forward(const orc_cfg *c, const orc_weights *w, int B, int T, const int32_t *tokens,
                 float *h_star, float *pooled, float *logits, int32_t *iters, int32_t *converged,
                 int32_t *argmax, float *scan_y, float *scan_state, int nthreads);
/* The same forward on a model prepared once (weights transposed for the CPU loops). */
typedef struct orc_model orc_model;
orc_model *orc_model_create(const orc_cfg *c, const orc_weights *w);
void orc_model_forward(orc_model *m, int B, int T, const int32_t *tokens, float *h_star,
                       float *pooled, float *logits, int32_t *iters, int32_t *converged,
                       int32_t *argmax, float *scan_y, float *scan_state, int nthreads);
void orc_model_free(orc_model *m);
/* Trainer::generate's greedy loop (TRAINER:4219-4431): prompt [B][T0], out_tokens [B][n_new];
 * canonical queries are embed_context over the last ctx_len tokens, ORC_F_MEMORY runs the
 * fixed-history form (hw needed); rep_penalty as LmHead::sample (1 = none). */
void orc_decode_greedy(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B, int T0,
                       const int32_t *prompt, int n_new, int ctx_len, float rep_penalty,
                       int32_t *out_tokens, int nthreads);
/* The same loop with LmHead::sample in place of the arg-max: uniforms [B][n_new] the draws, cond
 * [B][n_new] (or NULL) each step's conditioning (orc_lm_sample). */
void orc_decode_sample(const orc_cfg *c, const orc_weights *w, const orc_hist_weights *hw, int B, int T0,
                       const int32_t *prompt, int n_new, int ctx_len, float temperature, float top_p, int top_k,
                       float rep_penalty, const float *uniforms, int32_t *out_tokens, double *cond,
                       int nthreads);

/* LmHead::sample (lm_head.rs:78-168): logits [V], context ctx [L], the draw r (rng.gen::<f32>()
 * in the reference).  cond (or NULL) receives [2]: how far the decision lies from the roundings
 * that could change it (>= 1: a device with its own exp and sum orders takes the same decision;
 * 0: the float running sums already decide otherwise than the same sums in double), and the
 * length of the kept list (0 for greedy or the fallback arg-max). */
int orc_lm_sample(const float *logits_in, int V, const int32_t *ctx, int L, float temperature, float top_p,
                  int top_k, float rep_penalty, float r, double *cond);

/* --- other trait surfaces --------------------------------------------------- */
/* Clean adjoint Picard (staged_adjoint_picard_clean.wgsl:143-337; driver gpu_deq.rs:4736-4975):
 * per (token, slot) row, pre = signal + h*, rhs = dl[t] / H, v_0 = rhs and `iters` steps
 * v_{k+1} = rhs + N^T(beta v_k) + (1 - beta) v_k, N^T the RMSNorm vector-Jacobian product at pre
 * (attention is left out of the adjoint); Anderson(c->anderson_m) over each token's [H][d] iterate
 * after every step (mixing from the third).  src[t] = sum over slots of N^T(beta v*).
 * signal, h_star, v_out [ntok][H][d]; dl, src [ntok][d]; v_out / src may be NULL. */
void orc_adjoint(const orc_cfg *c, const float *norm_scale, int ntok, const float *signal, const float *h_star,
                 const float *dl, int iters, float beta, float *v_out, float *src);
/* tokenizer.rs:133-149 embed_context for the window ending at every position (TRAINER:4690-4696:
 * context = tokens[max(0, i - ctx + 1) ..= i]): out[b][i] = r / |r| (r itself when |r| <= 1e-6),
 * r = sum over the window of E[tok] * ((pos + 1) / len), pos = index in the window. */
void orc_embed_context(int d, const float *embed, int B, int T, const int32_t *tokens, int ctx, float *out);
void orc_zoh_step(int d, const float *x, const float *dt, const float *a, const float *b,
                  const float *c, float *y);
void orc_gemv_colmajor(const float *w, const float *x, int in_dim, int out_dim, float *y);

#ifdef __cplusplus
}
#endif
#endif

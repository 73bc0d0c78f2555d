/*
 * aideen_hip.h -- C ABI of the MI355X (gfx950) DEQ forward path.
 *
 * Drop-in boundary for the reference's wgpu compute block (SergioAriel/aideen):
 * the entry points below replace, one for one, the GPU surfaces the Rust crates bind to.
 * Each declaration cites the reference interface it replaces (file:line).  A thin Rust FFI
 * crate (an `extern "C"` block with one declaration per function here) binds exactly these
 * symbols.
 *
 * Conventions
 *   - Every entry point returns ADN_OK (0) or a negative ADN_E_* code; adn_last_error()
 *     returns the message of the last failure on the calling thread (the reference returns
 *     `&'static str` / `String` errors, gpu_deq.rs:3687-3727, block_backend.rs:22-31).
 *   - Plain pointers and sizes only.  "host" entry points take host memory and block until the
 *     results are back (the reference's map_async + device.poll(Wait), deq_bridge.rs:2017-2038);
 *     "_async" entry points take device memory and only enqueue work on the context's stream
 *     (the reference's *_no_readback / *_from_seq_buf forms, gpu_deq.rs:3855-4078).
 *   - One context per thread (the reference's backends are !Sync).  Contexts own their HIP
 *     stream (default priority) unless adn_set_stream() hands them another.
 *   - Layouts (fp32 everywhere):
 *       per-slot matrices  W[s][out][in]  (ADN_LAYOUT_OUT_IN), so y = W[s] x, or the reference's
 *                          GPU flat layout W[s][in][out] (ADN_LAYOUT_IN_OUT, fixed_point_memory_
 *                          reasoning.rs:516-561 `w_*_gpu_flat`)
 *       slot vectors       [H][d]                 (aideen-core/src/state.rs:85-146 HSlots)
 *       hidden states      [B][T][H][d]           (deq_slot_attn_unified_clean.wgsl:711-712)
 *       inputs S_in        [B][T][d]              (deq_bridge.rs:2672-2720)
 *       pooled             [B][T][d]              (deq_forward_pool.wgsl:32-65)
 *       logits             [B][T][V]              (lm_exact_forward.wgsl:21-47)
 *       carrier state      [B][H][d][N]
 */
#ifndef AIDEEN_HIP_H
#define AIDEEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ADN_ABI_VERSION 3

/* status codes */
#define ADN_OK 0
#define ADN_E_INVALID (-1)    /* bad argument, shape or token id                          */
#define ADN_E_NO_DEVICE (-2)  /* no usable GPU (reference: new_blocking() -> None)         */
#define ADN_E_HIP (-3)        /* HIP runtime failure                                       */
#define ADN_E_NO_WEIGHTS (-4) /* forward before adn_upload_weights                         */
#define ADN_E_CAPACITY (-5)   /* batch*seq beyond the context's capacity                   */

/* semantic switches (adn_config.flags); defaults reproduce the CPU reference forward
 * FixedPointMemoryReasoning::step (fixed_point_memory_reasoning.rs:1372-1424)          */
#define ADN_F_WIN_TRANSPOSED (1u << 0)  /* signal = W_in^T x (deq_slot_attn_unified_clean.wgsl:773) */
#define ADN_F_SCORE_CLAMP4 (1u << 1)    /* clamp slot scores to [-4,4] (picard_pipeline_test.rs:216) */
#define ADN_F_RMS_EXCL_ANCHOR (1u << 2) /* RMS over o+signal only (ARCHITECTURE.md:160-170)          */
#define ADN_F_INIT_SIGNAL_RMS (1u << 3) /* h0 = signal/rms(signal) (deq_slot_attn_unified_clean.wgsl:900-943) */
#define ADN_F_RESID_L2 (1u << 4)        /* L2 exit residual (aideen-node/src/inference.rs:214-221)    */
#define ADN_F_SCAN_SELECTIVE (1u << 5)  /* input-dependent carrier decay (gpu_deq.rs:6129-6214)      */
/* Relative-RMS exit residual (the GPU reference's err_h, deq_slot_attn_unified_clean.wgsl:1654-1695):
 * per slot sqrt(mean_i (h'_i - h_i)^2 + 1e-12) / max(rms, 1e-6), rms the slot's RMSNorm
 * denominator sqrt(mean c^2 + 1e-6); the token's residual is the largest over its slots (the
 * joint-slot analogue of the max-abs default).  Excludes ADN_F_RESID_L2. */
#define ADN_F_RESID_RELRMS (1u << 11)
/* Homeostatic plateau exit as well (deq_slot_attn_unified_clean.wgsl:277-279,1786-1793): a token
 * also stops after update k when k+1 >= 4, r_k <= max(eps, 0.15*0.2) and
 * |r_k - r_{k-1}| <= 0.10 max(r_{k-1}, eps), with r_{-1} = 1 and r the token's residual. */
#define ADN_F_HOMEOSTATIC_EXIT (1u << 12)

/* Memory-coupled forward (the trainer's fixed-history mode, trainer.rs:677-720): per sequence,
 * token t's solve adds the history context fixed_hist_ctx(m_{t-1}, signal_t)
 * (fixed_point_memory_reasoning.rs:1337-1370, weights w_hist / hist_slot_scale /
 * hist_gate_logit) and the carrier advances after each token, m_t = temporal_step(m_{t-1}, h*_t)
 * (fixed_point_memory_reasoning.rs:1454-1485: non-selective decay, m_t = (I + W_out) m_inner).
 * Tokens of a sequence are solved one after another.  Requires d_state == 1 and no
 * ADN_F_SCAN_SELECTIVE; scan_y returns every m_t [B][T][H][d], scan_state the last one
 * [B][H][d], scan_state_in the memory before the first token (NULL = none).  eps = 0 runs
 * exactly max_iters steps per token, as the reference's fixed-history solve does. */
#define ADN_F_MEMORY (1u << 9)
/* With ADN_F_MEMORY: the solve of position t > 0 starts from h* of position t - 1 of the same
 * sequence instead of the init rule (token carry, the GPU reference's default warm start:
 * deq_slot_attn_unified_clean.wgsl:898, deq_bridge.rs:167-173 AIDEEN_DEQ_TOKEN_CARRY). */
#define ADN_F_TOKEN_CARRY (1u << 10)

/* GEMM arithmetic (adn_config.flags; at most one).  Default: fp32 operands carried as fp16
 * hi+lo pairs on the 16-bit MFMA with three products per multiply (hi.hi + hi.lo + lo.hi),
 * fp32 accumulation -- fp32-level accuracy at several times the fp32 MFMA rate. */
#define ADN_F_GEMM_FP32 (1u << 6)   /* plain fp32 MFMA (v_mfma_f32_32x32x2f32)                      */
#define ADN_F_GEMM_BF16X3 (1u << 7) /* bf16 hi+lo pairs, three products (~2^-16 relative)           */
#define ADN_F_GEMM_BF16 (1u << 8)   /* bf16 inputs, fp32 accumulate (one product)                   */

/* weight layouts for adn_upload_weights */
#define ADN_LAYOUT_OUT_IN 0u /* W[s][out][in] row-major                                   */
#define ADN_LAYOUT_IN_OUT 1u /* W[s][in][out]: the reference's GPU flat layout            */

/* Shapes and solver configuration (reference: ArchitectureConfig, aideen-core/src/state.rs:7-58;
 * batch/seq capacities AIDEEN_BATCH_SIZE / AIDEEN_SEQ_CAP, gpu_deq.rs:577-596;
 * Anderson depth AIDEEN_ANDERSON_M, gpu_deq.rs:2093). */
typedef struct adn_config {
    int32_t d_r;        /* slot width d: a multiple of 64 in [64, 2048]          */
    int32_t h_slots;    /* H: 1 .. 16                                            */
    int32_t vocab;      /* V                                                     */
    int32_t d_state;    /* N: carrier states per channel (1..32)                 */
    int32_t rank;       /* write/selective rank r (multiple of 4, <= 64; ref 32) */
    int32_t max_batch;  /* capacity: sequences per call                          */
    int32_t max_seq;    /* capacity: tokens per sequence                         */
    int32_t anderson_m; /* 0 = plain Picard, else ring depth 2..5                */
    uint32_t flags;     /* ADN_F_*                                               */
} adn_config;

/* Model tensors (host memory, fp32).  NULL where noted means the documented default.
 * Reference upload: GpuDeqBackend::upload_weights, gpu_deq.rs:3529-3667 (AllWeights +
 * HistParams), LmHead (lm_head.rs:9-33), Tokenizer::embeddings (tokenizer.rs:22-23). */
typedef struct adn_weights {
    const float *w_q, *w_k, *w_v, *w_o, *w_in; /* [H][d][d]                          */
    const float *q_bias, *k_bias;               /* [H][d], NULL = 0                   */
    const float *anchor;                        /* [H][d] slot_anchor                 */
    const float *norm_scale;                    /* [d]                                */
    const float *embed;                         /* [V][d] token embeddings            */
    const float *lm_w;                          /* [V][d]                             */
    const float *lm_b;                          /* [V], NULL = 0                      */
    const float *lm_g;                          /* [d], NULL = 1                      */
    const float *a_log;                         /* [H][d] carrier decay logits        */
    const float *wx_diag;                       /* [H][d] diagonal of W_x             */
    const float *w_out;                         /* [H][d][d] readout, NULL = 0        */
    const float *b_delta;                       /* [H][d], NULL = 0                   */
    const float *w_kw;                          /* [H][d][r] selective write down     */
    const float *w_vw;                          /* [H][r][d] selective write up       */
    const float *w_b, *w_c;                     /* [H][N][d] carrier B/C, NULL = 1    */
    /* memory-coupled forward (ADN_F_MEMORY; ignored otherwise), fixed_point_memory_reasoning.rs:
     * 279, 312-333 and the export names reasoning.w_hist_shared / hist_slot_scale /
     * hist_gate_logit (:656-671) */
    const float *w_hist;                        /* [d][d] shared, row-major (u = W m)  */
    const float *hist_slot_scale;               /* [H][d]                             */
    const float *hist_gate_logit;               /* [H]                                */
} adn_weights;

/* One forward call (reference: run_forward_deq(batch, seq, max_iters, eps, damping, s_in, ...),
 * gpu_deq.rs:3687-3727).  Exactly one of tokens / s_in is non-NULL. */
typedef struct adn_run {
    int32_t batch, seq;
    int32_t max_iters;            /* >= 1                                              */
    float eps;                    /* exit when the residual is below eps               */
    float damping;                /* Picard beta in (0, 1]                             */
    const int32_t *tokens;        /* [B][T] token ids (embedding gather fused)         */
    const float *s_in;            /* [B][T][d] pre-embedded inputs                     */
    const float *scan_state_in;   /* [B][H][d][N] carried state, NULL = zeros          */
} adn_run;

/* Requested outputs; NULL = not computed.  (read_hnext_seq gpu_deq.rs:5833-5851,
 * read_hpooled_seq gpu_deq.rs:5886-5894, read_exact_logits_from_h gpu_lm_head.rs:1813-1879) */
typedef struct adn_outputs {
    float *h_star;      /* [B][T][H][d] fixed points                            */
    float *pooled;      /* [B][T][d]    mean over slots                         */
    float *logits;      /* [B][T][V]                                            */
    int32_t *argmax;    /* [B][T]       greedy token, last-max tie rule         */
    int32_t *iters;     /* [B][T]       Picard updates applied                  */
    float *scan_y;      /* [B][T][H][d] carrier output Y_t                      */
    float *scan_state;  /* [B][H][d][N] carrier state after the last token      */
    /* [B][T] 1 = the solve exited on the tolerance (or the homeostatic plateau), 0 = it stopped at
     * max_iters unconverged.  A residual that is not finite (the state turned NaN or inf, e.g. from
     * a non-finite input row) counts as infinite, so such a token always runs to max_iters and
     * reports 0 (the reference's finite_or guards, deq_slot_attn_unified_clean.wgsl:99-108; its
     * failure detection, trainer.rs:2931-2995). */
    int32_t *converged;
} adn_outputs;

typedef struct adn_ctx adn_ctx;

/* --- library ------------------------------------------------------------------------ */
int adn_abi_version(void);
const char *adn_last_error(void);
/* Number of visible GPUs (no device is initialised by a count of 0). */
int adn_device_count(int32_t *count);

/* --- context (GpuDeqBackend::new_blocking gpu_deq.rs:3122-3124; RustDeqBridge::new
 *     deq_bridge.rs:159) -------------------------------------------------------------- */
int adn_create(const adn_config *cfg, adn_ctx **out);
void adn_destroy(adn_ctx *ctx);
/* Run on a caller-owned hipStream_t (NULL restores the context's own stream). */
int adn_set_stream(adn_ctx *ctx, void *hip_stream);
int adn_synchronize(adn_ctx *ctx);

/* --- weights (GpuDeqBackend::upload_weights gpu_deq.rs:3529-3667) -------------------- */
int adn_upload_weights(adn_ctx *ctx, const adn_weights *w, uint32_t layout);
/* GpuDeqBackend::reset_state gpu_deq.rs:3127-3164: zero the carried carrier state. */
int adn_reset_state(adn_ctx *ctx);

/* --- forward ------------------------------------------------------------------------ */
/* Host memory, blocking: run_forward_deq / run_forward_deq_pooled + readbacks
 * (gpu_deq.rs:3687-3768, 5833-5894; gpu_lm_head.rs:1813-1879). */
int adn_forward(adn_ctx *ctx, const adn_run *run, const adn_outputs *out);
/* Device memory, enqueue only: run_forward_deq_no_readback / run_forward_from_seq_buf
 * (gpu_deq.rs:3855-4078).  Errors detected on the device (a token id outside [0, V)) are
 * reported by the next adn_synchronize().  It enqueues kernels and device-to-device copies
 * only, so once a first call with the same shapes and outputs has run, a call can be captured
 * into a HIP graph on the context stream and replayed. */
int adn_forward_async(adn_ctx *ctx, const adn_run *run, const adn_outputs *out);

/* Greedy decode, host memory, blocking: Trainer::generate (trainer.rs:4219-4431) with
 * LmHead::sample at temperature <= 0 (lm_head.rs:104-111; a temperature in (0, 1e-4] still
 * divides and samples, see adn_decode_sample).  prompt [B][prompt_len] token ids,
 * out_tokens [B][n_new] the appended tokens.  At step j the context of sequence b is the last
 * ctx_len of its prompt_len + j tokens (trainer.rs:4248-4249) and
 *   - the canonical forward (trainer.rs:4388-4392, 4402-4406): the query is embed_context(context,
 *     ctx_len) (tokenizer.rs:133-149), solved from init(query) with max_iters / eps / damping
 *     (generate runs exactly 10 steps: max_iters = 10, eps = 0);
 *   - with ADN_F_MEMORY, the fixed-history form (trainer.rs:4395-4400, 677-735): the memory is
 *     primed over every prompt token (prime_fixed_history_state, :718-733), then each step solves
 *     the embedding of the last context token with the history context of the memory and advances
 *     it (eps = 0 runs the reference's fixed max_iters); ADN_F_TOKEN_CARRY is refused;
 * then the logits of the LM head (lm_head.rs:50-54), the repetition penalty over the context when
 * |repetition_penalty - 1| > 1e-4 (lm_head.rs:81-99), and the arg-max with the last-max tie rule.
 * Every step runs on the device without host round trips.  Capacity: batch (canonical) or
 * batch * prompt_len (memory) tokens. */
int adn_decode_greedy(adn_ctx *ctx, int32_t batch, int32_t prompt_len, const int32_t *prompt, int32_t n_new,
                      int32_t ctx_len, int32_t max_iters, float eps, float damping, float repetition_penalty,
                      int32_t *out_tokens);

/* LmHead::sample (aideen-backbone/src/lm_head.rs:78-168) on rows of logits, host memory, blocking.
 * logits [rows][vocab]; row i's context is context[i][0, ctx_len[i]) (context [rows][ctx_stride];
 * ctx_stride 0 = no context, context and ctx_len may then be null).  Per row, as the reference:
 *   1. the repetition penalty once per distinct context token when |repetition_penalty - 1| > 1e-4
 *      (a negative logit multiplied by it, any other divided);
 *   2. temperature > 0 with |temperature - 1| > 1e-4 divides every logit by it; a temperature <= 0
 *      returns the arg-max of the penalised row (last maximum, NaN as Iterator::max_by folds it);
 *   3. softmax (exp(l - max) / sum), the list sorted by probability, descending and stable;
 *   4. top_k in (0, vocab) keeps the first top_k (0 = no cut);
 *   5. top_p in (0, 1) keeps the list up to the first item at which the running sum exceeds it;
 *   6. the kept probabilities renormalised (the arg-max of the row as given if their sum is
 *      <= 1e-6 or not a number);
 *   7. the first item at which the running sum reaches uniforms[i] (rng.gen::<f32>() in the
 *      reference, thread_rng: here the caller's draw in [0, 1)), the first item if none does.
 * The decisions are taken on the device's own probabilities; where the kept list has at most 2048
 * items the running sums are the reference's float loops, beyond that exact sums (a token can then
 * differ from the reference only where a running sum lies within its rounding of top_p or the
 * draw).  tokens [rows].  repetition_penalty must be finite and > 0, top_k >= 0, vocab <= 65536. */
int adn_lm_sample(adn_ctx *ctx, int32_t rows, int32_t vocab, const float *logits, const int32_t *context,
                  int32_t ctx_stride, const int32_t *ctx_len, float temperature, float top_p, int32_t top_k,
                  float repetition_penalty, const float *uniforms, int32_t *tokens);

/* Trainer::generate (trainer.rs:4219-4431) with LmHead::sample's temperature, top_p, top_k and
 * repetition penalty (lm_head.rs:78-168, as adn_lm_sample): the steps of adn_decode_greedy, then
 * each step's token drawn from its logits with uniforms[b][j] (uniforms [B][n_new]).  A
 * temperature <= 0 is adn_decode_greedy (uniforms unused).  The model's vocab must be <= 65536. */
int adn_decode_sample(adn_ctx *ctx, int32_t batch, int32_t prompt_len, const int32_t *prompt, int32_t n_new,
                      int32_t ctx_len, int32_t max_iters, float eps, float damping, float temperature, float top_p,
                      int32_t top_k, float repetition_penalty, const float *uniforms, int32_t *out_tokens);

/* --- weight preparation (spectral_norm.rs:25-80; spectral_renorm.wgsl:83-196) ----------- */
/* sigma_max by n_iter power iterations from u0 = 1/sqrt(rows); host memory, blocking. */
int adn_spectral_norm(adn_ctx *ctx, const float *w, int32_t rows, int32_t cols, int32_t n_iter,
                      float *sigma);
/* In place: W *= threshold/sigma when sigma > threshold (normalize_if_needed). */
int adn_normalize_if_needed(adn_ctx *ctx, float *w, int32_t rows, int32_t cols, float threshold,
                            int32_t n_iter);
/* GpuDeqBackend::renormalize_spectral (gpu_deq.rs:5567-5591) -> RustDeqBridge::renormalize_spectral
 * (aideen-block/src/deq_bridge.rs:1742-1791), spectral_renorm.wgsl:83-196: the uploaded block
 * matrices renormalised in place on the device.  Per slot: W_q and W_k against attn_threshold,
 * W_v against wv_threshold, W_o against wo_threshold, W_in against win_threshold, W_x (its
 * diagonal, which is what the carrier keeps) and W_out against fpm_threshold; each matrix's sigma
 * is the shader's n_iters-step power iteration on the matrix as the reference's buffer holds it
 * (W^T for the per-slot [in][out] matrices, W_in as uploaded), and a matrix with sigma > threshold
 * becomes W * (threshold / sigma).  The GEMMs' split copies are rebuilt.  The reference's defaults
 * are 0.10, 0.30, 0.70, 0.50, 0.50 and 12 iterations.  sigmas (or null) receives the 7 * h_slots
 * estimates before rescaling, [role][slot] with roles W_q, W_k, W_v, W_o, W_in, W_x, W_out (0 for
 * W_out when there is none).  Blocking. */
int adn_renormalize_spectral(adn_ctx *ctx, float attn_threshold, float win_threshold, float fpm_threshold,
                             float wv_threshold, float wo_threshold, int32_t n_iters, float *sigmas);

/* --- BlockBackend (aideen-core/src/block_backend.rs:22-31) ------------------------------ */
/* fpm_batch_step: ZOH single step, h_prev = 0 (gpu_backend.rs:18-56, :98-248).  All [d]. */
int adn_block_step(adn_ctx *ctx, int32_t d, const float *x, const float *dt, const float *a,
                   const float *b, const float *c, float *y);

/* --- ComputeBackend (aideen-core/src/compute.rs:11-23; aideen-engine/src/gpu/mod.rs:23-223) */
/* load_tensor: copies n floats to the device and returns a handle. */
int adn_load_tensor(adn_ctx *ctx, const float *data, int64_t n, int32_t *id);
/* ffn_forward: y[row] = sum_i w[i*out_dim + row] * x[i] (column-major, ffn_forward.wgsl:22-37);
 * in_dim = element count of the input tensor; y is host memory [out_dim]. */
int adn_ffn_forward(adn_ctx *ctx, int32_t w_id, int32_t in_id, int32_t out_dim, float *y);

/* --- backward: the clean adjoint Picard (GpuDeqBackend::run_staged_adjoint_picard_no_readback
 *     -> run_clean_adjoint_picard_no_readback, gpu_deq.rs:4080-4920, and
 *     reduce_clean_adjoint_to_source_grad_no_readback, :4922-4975; staged_adjoint_picard_clean.wgsl:
 *     143-337) ----------------------------------------------------------------------------------
 * For the ntok tokens of the most recent forward on this context (its signal; its h* unless
 * h_star is given), per (token, slot) row with pre = signal + h* and rhs = dl[t] / H:
 *   v_0 = rhs,  v_{k+1} = rhs + N^T(damping v_k) + (1 - damping) v_k   (iters steps),
 * N^T the RMSNorm vector-Jacobian product at pre (attention is not part of this adjoint), each step
 * Anderson-mixed per token when the context has anderson_m > 0 (from the third step).  v_out
 * [ntok][H][d] receives v, src [ntok][d] the source gradient sum over slots of N^T(damping v);
 * either may be NULL.  dl [ntok][d] is dL/d(pooled h*).  A forward (or greedy decode) in between
 * replaces the state the adjoint reads.  adn_adjoint: host memory, blocking; adn_adjoint_async:
 * device memory, enqueue only. */
int adn_adjoint(adn_ctx *ctx, int32_t ntok, const float *h_star, const float *dl, int32_t iters, float damping,
                float *v_out, float *src);
int adn_adjoint_async(adn_ctx *ctx, int32_t ntok, const float *h_star, const float *dl, int32_t iters,
                      float damping, float *v_out, float *src);

/* --- input pipeline ------------------------------------------------------------------
 * Tokenizer::embed_context (tokenizer.rs:133-149) for the window ending at every position, as
 * the trainer builds the query of position i (trainer.rs:4690-4696: context =
 * tokens[max(0, i - max_ctx + 1) ..= i]): out[b][i] = r / |r| (r when |r| <= 1e-6),
 * r = sum over the window of E[tok] * (pos + 1) / len.  tokens [B][T], out [B][T][d]; the
 * result is an adn_run.s_in.  Needs uploaded weights (the embedding table); B * T within the
 * context capacity; max_ctx >= 1.  adn_embed_context takes host memory and blocks;
 * adn_embed_context_async takes device memory and only enqueues on the context stream. */
int adn_embed_context(adn_ctx *ctx, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                      float *out);
int adn_embed_context_async(adn_ctx *ctx, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                            float *out);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): adn_embed_context_async
 * with the same arguments, kernels and results, that allocates nothing.  Its per-chunk prefix totals
 * live in a fixed per-device array of ADN_EMBED_NOALLOC_MAX_DOUBLES doubles (32 MiB, held until the
 * process ends) instead of context memory grown on demand; a request needing more than that
 * (2 * batch * ceil(seq / chunk) * d_r doubles, chunk = 32, 16, 8 or 4 positions for d_r up to
 * 256, 512, 1024, 2048) fails with ADN_E_CAPACITY.  Every call on one GPU, from any context, shares
 * that array: calls that overlap on one GPU (other streams, other threads) race.  Such an overlap
 * is detected on the device (a counter of calls in flight beside the array, raised by a call's
 * first kernel and lowered by its last one) and reported by the next blocking call on the context
 * that found the array in use (ADN_E_INVALID, "... overlapped ..."); the raced outputs are not
 * valid.  Callers that use several streams or contexts on one GPU order these calls themselves.
 * The context's uploaded embedding table is read; device memory, enqueue only. */
#define ADN_EMBED_NOALLOC_MAX_DOUBLES 4194304
int adn_embed_context_noalloc(adn_ctx *ctx, int32_t batch, int32_t seq, const int32_t *tokens,
                              int32_t max_ctx, float *out);
/* No counterpart in the reference.  Diagnostics of the overlap detection above: sets the count
 * of adn_embed_context_noalloc calls in flight on the context's GPU (0 when idle), so that tests
 * can force an overlap from the host.  Blocking. */
int adn_noalloc_guard_set(adn_ctx *ctx, uint32_t calls_in_flight);

/* --- byte-level BPE (Tokenizer::encode / decode, tokenizer.rs:94-116, which run the HF
 *     `tokenizers` crate on aideen-backbone/tokenizer.json) --------------------------------------
 * Host-only.  adn_tokenizer_load reads a tokenizer.json with a BPE model, the byte-level
 * pre-tokenizer (no prefix space) and no normalizer; anything else is reported.  encode is
 * encode(text, add_special_tokens = true): text is UTF-8 (len bytes; invalid UTF-8 is
 * ADN_E_INVALID), *n receives the id count, ADN_E_CAPACITY when it exceeds cap.  decode is
 * decode(ids, skip_special_tokens = true): ids without a token are skipped, invalid UTF-8 in the
 * byte stream becomes U+FFFD, *len receives the byte length (not NUL-terminated),
 * ADN_E_CAPACITY when it exceeds cap.  One tokenizer may be used from several threads. */
typedef struct adn_tokenizer adn_tokenizer;
int adn_tokenizer_load(const char *tokenizer_json_path, adn_tokenizer **out);
void adn_tokenizer_free(adn_tokenizer *tok);
int32_t adn_tokenizer_vocab_size(const adn_tokenizer *tok); /* get_vocab_size(true) */
int adn_tokenizer_encode(adn_tokenizer *tok, const char *text, int64_t len, int32_t *ids, int64_t cap, int64_t *n);
int adn_tokenizer_decode(const adn_tokenizer *tok, const int32_t *ids, int64_t count, char *text, int64_t cap,
                         int64_t *len);

/* --- .aidn checkpoints (AidenModel::load, aideen-core/src/model.rs:39-47) ---------------------
 * bincode 1.3 of { config: ArchitectureConfig, weights: name -> [f32], metadata: name -> string }.
 * Host-only: no device is touched.  adn_aidn_weights maps the reference's exported names and
 * layouts (FixedPointMemoryReasoning::export_weights, fixed_point_memory_reasoning.rs:626-784;
 * LmHead::export_weights, lm_head.rs:169-188; Trainer::save_full, trainer.rs:6472-6530) onto
 * adn_weights: the CPU model's shared matrices are replicated per slot, tokenizer.embeddings
 * (nalgebra column-major) is transposed to [V][d], W_x gives its diagonal.  Its arrays stay valid
 * until adn_aidn_close.  It also proposes an adn_config (d_r, h_slots, vocab, d_state = 1,
 * rank = 32, max_seq = ctx_len, the CPU semantics flags = 0) and the run parameters
 * (max_iters = max_deq_iters, eps = deq_epsilon, damping = reasoning.damping). */
typedef struct adn_aidn adn_aidn;
typedef struct adn_aidn_config { /* ArchitectureConfig, aideen-core/src/state.rs:7-35 */
    int64_t d_m, d_r, d_c, d_e, d_sim, h_slots, vocab_size, ctx_len, max_deq_iters;
    float deq_epsilon;
    int64_t adj_iters;
    int32_t train_deq;
    float deq_grad_scale;
    int64_t renorm_every_steps, num_samples;
    float weight_decay;
} adn_aidn_config;
int adn_aidn_open(const char *path, adn_aidn **out);
void adn_aidn_close(adn_aidn *model);
int adn_aidn_config_get(const adn_aidn *model, adn_aidn_config *out);
int adn_aidn_count(const adn_aidn *model, int32_t *n_weights, int32_t *n_metadata);
int adn_aidn_name(const adn_aidn *model, int32_t i, const char **name); /* i-th weight, file order */
/* AidenModel::get_weight (model.rs:55-57): *data = NULL and *count = 0 when absent */
int adn_aidn_tensor(const adn_aidn *model, const char *name, const float **data, int64_t *count);
int adn_aidn_metadata(const adn_aidn *model, const char *key, const char **value); /* NULL if absent */
int adn_aidn_weights(adn_aidn *model, adn_weights *w, adn_config *cfg, adn_run *run);

/* --- measurement (the reference's AIDEEN_DEQ_FORWARD_PROFILE per-pass timing,
 *     deq_bridge.rs:2234-2380, and GPU timestamp queries, gpu_deq.rs:490-570) ------------- */
#define ADN_STAGE_SIGNAL_GEMM 0  /* signal = W_in x (embedding gather fused)          */
#define ADN_STAGE_INIT 1         /* h0 and the first active list                      */
#define ADN_STAGE_QKV_GEMM 2     /* per-slot Q|K|V projections of the active tokens    */
#define ADN_STAGE_ATTN 3         /* slot scores, softmax, mix                          */
#define ADN_STAGE_WO_GEMM 4      /* per-slot W_o projection                            */
#define ADN_STAGE_UPDATE 5       /* RMS norm, damped update, residual partials         */
#define ADN_STAGE_CONVERGE 6     /* exit test, iteration counts, compaction            */
#define ADN_STAGE_ANDERSON 7     /* Anderson store + mix                               */
#define ADN_STAGE_POOL 8         /* slot mean-pool + RMSNorm                           */
#define ADN_STAGE_LMHEAD_GEMM 9  /* logits = W_lm x + b                                */
#define ADN_STAGE_ARGMAX 10      /* greedy arg-max                                     */
#define ADN_STAGE_SCAN_PREP 11   /* carrier prologue (rms, rank-r bottleneck, B/C)     */
#define ADN_STAGE_SCAN 12        /* chunked selective scan                             */
#define ADN_STAGE_READOUT_GEMM 13 /* Y = y + W_out y (memory mode: m_t = m + W_out m)  */
#define ADN_STAGE_HIST_GEMM 14   /* memory mode: u = W_hist m_{t-1}                    */
#define ADN_STAGE_HIST_CTX 15    /* memory mode: history context gate and clamp        */
#define ADN_STAGE_TEMPORAL 16    /* memory mode: m = abar m_{t-1} + (1 - abar) x      */
#define ADN_STAGE_COUNT 17
#define ADN_PROFILE_MAX_ITERS 256

/* A stage done inside another stage's launch (at <= 4 tokens: the attention mix inside the W_o
 * product; with no early exit possible, the previous update inside the Q|K|V product and the
 * pool inside the last update) has no launches of its own: its FLOPs and bytes are counted with
 * the launch that does it. */
typedef struct adn_profile {
    double ms[ADN_STAGE_COUNT];       /* device time summed over the stage's launches   */
    double flops[ADN_STAGE_COUNT];    /* algorithmic FLOPs summed over those launches   */
    double bytes[ADN_STAGE_COUNT];    /* algorithmic (compulsory) HBM bytes             */
    int32_t launches[ADN_STAGE_COUNT];
    int32_t active[ADN_PROFILE_MAX_ITERS]; /* tokens entering Picard iteration k (memory
                                           * mode: summed over the positions)            */
    int32_t n_iters;                  /* iterations enqueued (= max_iters)              */
    double total_ms;                  /* first to last event                            */
} adn_profile;

/* Runs adn_forward_async with a HIP event pair around every kernel launch on the context
 * stream, synchronises, and fills *prof.  Device-memory arguments as adn_forward_async. */
int adn_profile_forward(adn_ctx *ctx, const adn_run *run, const adn_outputs *out, adn_profile *prof);

#ifdef __cplusplus
}
#endif
#endif /* AIDEEN_HIP_H */

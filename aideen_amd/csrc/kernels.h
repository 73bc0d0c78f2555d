// Kernel launch interfaces shared by the runtime (runtime.cpp) and the kernel sources.
#pragma once

#include <type_traits>

#include "common.h"

namespace adn {

// Kernels templated on E = d / 64 values per lane (a lane's share of a d-wide row): d a power of
// two runs the exact instantiation (E = d / 64, PART = false); any other multiple of 64 runs the
// next power of two up with PART = true, where a lane's chunks e >= d / 64 are neither loaded nor
// stored (the rows keep their true width d).  f(std::integral_constant<int, E>, std::bool_constant<PART>).
template <typename F>
void dispatch_width(int d, F &&f) {
    using std::bool_constant;
    using std::integral_constant;
    switch (d) {
        case 64: f(integral_constant<int, 1>{}, bool_constant<false>{}); return;
        case 128: f(integral_constant<int, 2>{}, bool_constant<false>{}); return;
        case 256: f(integral_constant<int, 4>{}, bool_constant<false>{}); return;
        case 512: f(integral_constant<int, 8>{}, bool_constant<false>{}); return;
        case 1024: f(integral_constant<int, 16>{}, bool_constant<false>{}); return;
        case 2048: f(integral_constant<int, 32>{}, bool_constant<false>{}); return;
        default: break;
    }
    const int er = d / 64;
    if (er <= 4)
        f(integral_constant<int, 4>{}, bool_constant<true>{});
    else if (er <= 8)
        f(integral_constant<int, 8>{}, bool_constant<true>{});
    else if (er <= 16)
        f(integral_constant<int, 16>{}, bool_constant<true>{});
    else
        f(integral_constant<int, 32>{}, bool_constant<true>{});
}

enum GemmEpilogue { EPI_NONE = 0, EPI_BIAS = 1, EPI_ADD_A = 2 };
// GemmParams.am_val/am_idx != null: also write each row's (max, last arg-max) over every
// 128-column tile into [ceil(N/128)][M] partials (LM head + greedy decode).
// Each use of the GEMM is a separate kernel symbol so profilers report them apart.
enum GemmRole { ROLE_SIGNAL = 0, ROLE_QKV, ROLE_WO, ROLE_LMHEAD, ROLE_READOUT, ROLE_SCAN_PROJ, ROLE_COUNT };
// GEMM arithmetic: plain fp32 MFMA, or fp32 operands as hi+lo halves on the 16-bit MFMA.
enum GemmPrec { PREC_F16X3 = 0, PREC_FP32 = 1, PREC_BF16X3 = 2, PREC_BF16X1 = 3 };

// C[m][n] = sum_k A(m,s)[k] * B(s)[n][k] (+ epilogue), for m < M (or *m_count), n < N, s < S.
//   A(m,s) = A + row(m)*a_sm + s*a_ss, row(m) = a_idx ? a_idx[m] : m   (a_idx checked < a_idx_max)
//   B(s)   = B + s*b_ss, rows of length K
//   C(m,s) = C + m*c_sm + s*c_ss
struct GemmParams {
    const float *A;
    const int32_t *a_idx;
    long a_sm, a_ss;
    int a_idx_max;
    const float *B;
    long b_ss;
    float *C;
    long c_sm, c_ss;
    const float *bias;
    long bias_ss;
    int bias_n;
    int M, N, K, S;
    const int32_t *m_count;
    unsigned *err;
    int epi;
    int role;
    float *am_val;
    int32_t *am_idx;
    int prec;            // GemmPrec
    const void *Bhi;     // split weights [S][N][K] (prec != PREC_FP32)
    const void *Blo;
    float a_scale;       // A scaled by this power of two before the split
    float out_scale;     // accumulator scaled by this power of two (undoes both scales)
    // Optional data-dependent A scale: with a_absmax set (bit pattern of max |A|, written by
    // launch_absmax), the kernel uses min(a_scale, 2^floor(log2(a_headroom / max|A|))) and
    // adjusts out_scale to match, so caller-supplied rows of any magnitude stay in range.
    const unsigned *a_absmax;
    float a_headroom;
    // A given instead as fp16 hi/lo halves split by its producer with the kernel's own A scale
    // (k_gemm_split's pre-split layout); W_o and the LM head, for the shapes gemm_presplit_ok
    // names; null = none
    const float *a_pre;
    // W_o on at most ATTN_FUSE_ROWS rows (the skinny kernel, split arithmetic): with attn_qkv set
    // the A operand (the attention mix of slot s) is formed in the kernel from the compact
    // [row][S][3K] Q|K|V rows instead of read, so no attention kernel runs; the kernel also does
    // that kernel's bookkeeping (attn_cnt_next = 0, attn_cnt_hist += the active count)
    const float *attn_qkv;
    int attn_clamp;            // ADN_F_SCORE_CLAMP4
    int32_t *attn_cnt_next;
    int32_t *attn_cnt_hist;
    // Q|K|V on at most ATTN_FUSE_ROWS rows (the skinny kernel, split arithmetic) when no token can
    // exit early: with upd_o set the kernel first applies the previous iteration's damped update
    // to its A rows (A = h before it, K = d, S = H; per slot c = o + signal + anchor, h' =
    // g c / rms(c) beta + h (1 - beta), as k_update_tok computes it) and multiplies h'; the
    // slot's first column block writes h' to upd_hout (rows indexed like A).  upd_o is the
    // previous W_o output, compact by active index like the A index list.
    const float *upd_o;
    const float *upd_sig;
    const float *upd_anchor;
    const float *upd_norm;
    float *upd_hout;
    float upd_beta;
    int upd_excl;              // ADN_F_RMS_EXCL_ANCHOR
};
constexpr int ATTN_FUSE_ROWS = 4;
constexpr int GEMM_BN = 128;
void launch_gemm(const GemmParams &p, hipStream_t st);
void launch_gemm_split(const GemmParams &p, hipStream_t st);
// Whether a split GEMM of this shape reads a pre-split A operand (GemmParams::a_pre): fp16
// halves and the 256x256 persistent tiles (M >= 1024, N >= 512).
bool gemm_presplit_ok(int prec, int M, int N);
// Whether W_o on at most M rows runs with the attention formed in its kernel (GemmParams::attn_qkv):
// the skinny split-arithmetic kernel, M <= ATTN_FUSE_ROWS, K a multiple of 64, at most 16 slots.
bool gemm_attn_fusable(int prec, int M, int K, int S);
// Columns per arg-max partial of the LM head over M rows (GEMM_BN, or 64 for the few-row skinny
// LM head): the partial count is ceil(V / this), and the partial buffers hold that many per row.
int gemm_lm_partial_cols(int prec, int M, int K);
// hi = T(w * scale), lo = T(w * scale - hi) with T = fp16 (PREC_F16X3) or bf16, from [S][N][K]
// fp32 weights into the split GEMM's blocked layout (split_weight_elems halves each, N padded to
// a multiple of 32); lo may be null.  The GEMMs' b_ss is then 0 (one matrix for every slot) or
// non-zero (a matrix per slot, N x K).  eye: split w + I (square matrices).
long split_weight_elems(int S, int N, int K);
void launch_split_weights(const float *w, int S, int N, int K, float scale, int prec, void *hi, void *lo,
                          hipStream_t st, bool eye = false);

// ---- DEQ solve kernels (deq.hip) ------------------------------------------------------
struct SolveBuffers {
    float *signal;      // [ntok][H][d]
    float *h;           // [ntok][H][d] iterate (in place)
    float *qkv;         // [ntok][H][3d] compact by active index
    float *mix;         // [ntok][H][d]  compact
    float *o;           // [ntok][H][d]  compact
    int32_t *act[2];    // active token lists
    int32_t *cnt;       // [4]: counts of act[0], act[1]; cnt[2] unused; cnt[3] = total tokens
    int32_t *iters;     // [ntok]
    int32_t *conv;      // [ntok] 1 = exit by the tolerance (or plateau), 0 = stopped unconverged at the cap; or null
    float *rprev;       // [ntok] previous iteration's token residual (homeostatic exit) or null
    int32_t *cnt_hist;  // [ADN_PROFILE_MAX_ITERS] active tokens entering iteration k (summed over positions)
    float *hist;        // Anderson ring [m][ntok][H][d] or null
    unsigned *err;
    // memory-coupled solve: history context of the tokens being solved, [B][H][d] indexed by
    // sequence (token / mem_T), added to the update's sum; null = none
    const float *mem_hist;
    int mem_T;
    // bound on |h| (float bits) for the split GEMMs' A scale: seeded with the update's RMSNorm
    // bound, raised by the init and the Anderson mix; null = not tracked
    unsigned *amax_h;
    // W_o's A written pre-split by the attention instead of mix in fp32 (the same memory; see
    // GemmParams::a_pre), scaled as the split GEMM scales it: its bound word and headroom for mix
    // (a_absmax, a_headroom); mix_pre null = fp32
    float *mix_pre;
    const unsigned *mix_bound;
    float mix_headroom;
    // non-null: the update writes its iterate here (rows indexed like h: the Anderson ring slot
    // of the iteration) instead of into h, and the Anderson pass that follows sets h
    float *h_out;
    // with h_out: write the iterate into h as well (iterations before the first mix)
    int h_both;
    // the last iteration with Anderson mixing (k >= 2): a token that stops at the cap without
    // converging is mixed like a continuing one (the solve mixes after every step that does not
    // exit on the tolerance): the update appends it to the next list as well, and the mixing pass
    // over the update's own list (SolveBuffers::h_out) tells it from a converged one by conv
    // (non-null whenever this is set)
    int cap_mix;
    // a few-token update at which every token exits (the last iteration of a fixed-iteration
    // solve) also forms each token's LM-head prologue from its new rows (pool_finish): pooled
    // rows into pool_out (or null), the normalised rows in fp32 into pool_norm (or null), gain
    // pool_g; pool = 0: none
    int pool;
    float *pool_out;
    float *pool_norm;
    const float *pool_g;
    // [ntok][4] the coefficients of each token's last Anderson mix (launch_update_mix), or null
    float *mix_coef;
};

// h0 per token and the first active list (all tokens, in order).
void launch_init(const Dims &D, const SolveBuffers &b, const float *x_src, const int32_t *tokens,
                 int ntok, const float *anchor, hipStream_t st);
// Slot attention: scores, softmax, mix for each active token; also clears the next list's
// count and records the active count of iteration k.
void launch_attn(const Dims &D, const SolveBuffers &b, int cur, int k, int ntok, hipStream_t st);
// Damped RMS update, token residual, exit test, iteration counts and the next active list.
void launch_update(const Dims &D, const SolveBuffers &b, int cur, int k, int max_iters, float eps, int ntok,
                   const float *anchor, const float *norm_scale, float beta, hipStream_t st);
// Anderson store + mix for the tokens still active after iteration k (at most `rows` of them;
// ntok is the token stride of the ring).
void launch_anderson(const Dims &D, const SolveBuffers &b, int nxt, int ntok, int rows, int k, int m,
                     hipStream_t st);
// Whether launch_anderson_from_slot serves this state width (a thread's share in registers).
bool anderson_from_slot_ok(const Dims &D);
// Anderson after an update that wrote its iterate into ring slot k % m (SolveBuffers::h_out), over
// every token of list cur (the ones the update saw): a token that exited at iteration k gets
// h = its iterate, a continuing one h = the mix (or its iterate while fewer than two residuals
// exist).  The ring slot is not written again.
void launch_anderson_from_slot(const Dims &D, const SolveBuffers &b, int cur, int ntok, int rows, int k, int m,
                               hipStream_t st);
// Whether launch_update_mix serves these rows (up to 16 slots of up to 2048 floats; above 512, a
// token's rows must fit in the device's LDS per workgroup).  Otherwise the update runs with a
// separate mixing pass.
bool update_mix_ok(const Dims &D);
// The update and the Anderson mix of iteration k >= 2 (m >= 3) in one launch over list cur: the
// iterate into ring slot k % m, h = the mix (or the iterate of a token that converged at k), the
// continuing tokens appended to list cur ^ 1.  Every iteration from 2 on must run here: the
// previous iterate is recomputed from the ring and SolveBuffers::mix_coef, not read from h.
void launch_update_mix(const Dims &D, const SolveBuffers &b, int cur, int k, int m, int ntok, int rows,
                       int max_iters, float eps, const float *anchor, const float *norm_scale, float beta,
                       hipStream_t st);

// ---- LM head (head.hip) -----------------------------------------------------------------
// pooled = mean_s h*, pnorm = (pooled/rms(pooled, 1e-5)) * g
// rec: when non-null, also each (token, slot) row's RMS into rec[row * REC] (the carrier record).
// pre_scale > 0: pnorm is written as the split GEMM's pre-split A operand (GemmParams::a_pre) of
// pnorm * pre_scale instead of fp32.
void launch_pool_norm(const Dims &D, const float *h, int ntok, const float *g, float *pooled,
                      float *pnorm, float *rec, int REC, float pre_scale, hipStream_t st);
// A greedy decode step's token append, done by the arg-max kernel that picks the token: row b's
// token also goes to seq[b][len] and out[b][j] (out is [B][n_new]); seq null = none.  bounds,
// when set, gets the next forward's range-guard reset (launch_reset_bounds's work: bounds[0] =
// bound0, the other ADN_BOUNDS words and *absmax zero), so that the next step needs no reset
// launch before its query.
struct TokenAppend {
    int32_t *seq;
    int stride, len;
    int32_t *out;
    int n_new, j;
    unsigned *bounds;
    unsigned bound0;
    unsigned *absmax;
};
// argmax over each row of logits with the last-max tie rule.
void launch_argmax(const float *logits, int ntok, int V, int32_t *out, hipStream_t st,
                   const TokenAppend *app = nullptr);
// final reduction of the per-tile arg-max partials written by the LM-head GEMM
void launch_argmax_reduce(const float *am_val, const int32_t *am_idx, int ntok, int ntiles, int32_t *out,
                          hipStream_t st, const TokenAppend *app = nullptr);
// The init of a forward over B query rows (launch_init's work for the rule h0 = x + anchor), done
// by the kernel that writes the rows: h [B][H][d] = q + anchor[s] per slot, the bound word
// raised to the largest finite |h0|, the first active list (all B rows), iteration counts and
// plateau residuals reset, the list counts and the per-iteration active counts.
struct QueryInit {
    float *h;
    const float *anchor;
    int H;
    int32_t *act0, *iters, *cnt, *cnt_hist;
    float *rprev;      // or null
    unsigned *amax_h;  // or null
};
// Greedy decode.  seq [B][stride] holds each sequence's tokens; step j uses the first len.
// q [B][d] = embed_context of the last ctx of them (d <= 2048).  absmax, when set, is raised
// (atomic max of float bits) to the largest finite |q| written, as launch_absmax would; it must
// have been cleared before the call.  init, when set, also does the forward's init (QueryInit).
void launch_decode_query(const float *E, int d, const int32_t *seq, int stride, int len, int ctx, int B, float *q,
                         hipStream_t st, unsigned *absmax = nullptr, const QueryInit *init = nullptr);
// the repetition penalty over the same context, in place on logits [B][V]
void launch_rep_penalty(float *logits, int V, const int32_t *seq, int stride, int len, int ctx, float pen, int B,
                        hipStream_t st);
// LmHead::sample (lm_head.rs:78-168) on logits [rows][V] with temperature > 0 (or NaN): the
// repetition penalty over each row's context (the last `window` of seq[row][0, len), len from
// lens[row] when lens is set), the temperature, softmax, top-k, top-p, the renormalisation and the
// draw uni[row * uni_stride] (rng.gen::<f32>(), in [0, 1)); with `greedy` (temperature <= 0) the
// arg-max of the penalised row.  ws (sample_workspace_bytes) is workspace; the token is stored as
// the arg-max kernels store theirs.  V <= SAMPLE_VMAX.
constexpr int SAMPLE_VMAX = 65536;
struct SampleParams {
    const int32_t *seq;
    int stride, len;
    const int32_t *lens;
    int window;
    float temperature, top_p, penalty;
    int top_k;
    const float *uni;
    int uni_stride;
    bool greedy;
};
size_t sample_workspace_bytes(int rows, int V);
void launch_sample(const float *logits, int rows, int V, void *ws, const SampleParams &sp, int32_t *out,
                   hipStream_t st, const TokenAppend *app = nullptr);
// last[b] = seq[b][len - 1]
void launch_decode_last(const int32_t *seq, int stride, int len, int32_t *last, int B, hipStream_t st);

// ---- carrier scan (scan.hip) -------------------------------------------------------------
struct ScanBuffers {
    float *rec;        // [ntok][H][REC] per-(token,slot) record: rms, bn[r], B[N], C[N]
    float *y;          // [ntok][H][d] pre-readout output (or final if no W_out)
    float *chunk_s;    // [B][nch][H][d][N]
    float *chunk_p;    // [B][nch][H][d]
    float *mem_mn;     // [max_batch][H][d] memory mode: the state before W_out
    float *mem_hist;   // [max_batch][H][d] memory mode: the history context
};
int scan_rec_len(const Dims &D);
// rec[row*REC] = sqrt(mean(h_row^2) + 1e-6) for every (token, slot) row
void launch_row_rms(const float *h, long rows, int d, float *rec, int REC, hipStream_t st);
// The carrier over B sequences of T steps from h* [B][T][H][d] and the record: y [B][T][H][d],
// state_out [B][H][d][N] (either may be null), state_in [B][H][d][N] or null; nch time chunks
// (chunk_s / chunk_p hold B * nch chunks).
// amax_y (or null): raised to the largest finite |y| (the readout GEMM's A scale).
void launch_scan(const Dims &D, const float *h, const float *rec, int B, int T, int has_bc, const float *a_log,
                 const float *wx_diag, const float *b_delta, const float *w_vw, const float *state_in, float *y,
                 float *state_out, float *chunk_s, float *chunk_p, int nch, unsigned *amax_y, bool ssd,
                 float min_fixed_decay, hipStream_t st);
int scan_chunks(int B, int T, int H, int d, bool ssd);
bool scan_use_ssd(const Dims &D, int B, int T, float min_fixed_decay);

// ---- misc (misc.hip) ----------------------------------------------------------------------
void launch_spectral_norm(const float *w, int rows, int cols, int n_iter, float *sigma,
                          float *work, hipStream_t st);
void launch_scale_if(float *w, long n, const float *sigma, float threshold, hipStream_t st);
// The GPU's spectral renormalisation of uploaded block matrices (spectral_renorm.wgsl:83-196): per
// job, the shader's power iteration on the matrix as the shader's buffer holds it, then
// m *= threshold / sigma when sigma > threshold; sigma goes to sigmas[out].  d <= 2048.
enum RenormKind { RENORM_T = 0, RENORM_N = 1, RENORM_DIAG = 2 };
struct RenormJob {
    float *m;         // [d][d] row-major, or [d] (RENORM_DIAG)
    int kind;         // RenormKind: the shader's buffer is m^T, m, or diag(m)
    float threshold;
    int out;          // index into sigmas
};
void launch_spectral_renorm(const RenormJob *jobs, int njobs, int d, int n_iters, float *sigmas, hipStream_t st);
void launch_zoh(int d, const float *x, const float *dt, const float *a, const float *b,
                const float *c, float *y, hipStream_t st);
void launch_gemv_colmajor(const float *w, const float *x, int in_dim, int out_dim, float *y,
                          hipStream_t st);
void launch_transpose(const float *src, int rows, int cols, long batch, float *dst,
                      hipStream_t st);
void launch_fill_i32(int32_t *p, int32_t v, long n, hipStream_t st);
// Magnitude bounds (float bits) of the split GEMMs' A operands during one forward: [0] |h| (the
// iterate: seeded with the update's RMSNorm bound, raised by the init and the Anderson mix),
// [1] |y| (the carrier output, raised by the scan), [2] |m| (memory mode's carrier state, raised
// by the temporal step and by a caller-supplied start state).  Reset by a kernel (not a memset:
// the forward may be captured in a graph).
constexpr int ADN_BOUNDS = 4;
void launch_reset_bounds(unsigned *words, float h_bound, unsigned *zero, hipStream_t st);  // zero: also cleared, or null
// ---- memory-coupled solve (memory.hip) -----------------------------------------------------
// act[0] = tokens (b, t) = b*T + t for b < B, cnt[0] = B, cnt[1] = 0.
// embed_context of the window ending at every position; tot0/tot1 hold
// B * embed_context_chunks(T) * d doubles each.
long embed_context_chunks(int T);
// doubles each of tot0 / tot1 that launch_embed_context writes for B sequences of T positions
// at width d (B * its chunk count * d; never more than B * embed_context_chunks(T) * d)
long embed_context_total_doubles(int d, int B, int T);
// busy (or null): the overlap guard of a shared tot0/tot1 array (two words, zero when idle)
void launch_embed_context(const float *E, int d, int V, const int32_t *tokens, int B, int T, int ctx, double *tot0,
                          double *tot1, float *out, unsigned *err, unsigned *busy, hipStream_t st);
// Clean adjoint Picard for ntok tokens (rows = ntok * H of d floats); scratch pre, v0, v1 hold
// rows * d floats, terms 2 * rows.  Returns the buffer holding the final iterate (v_out when given).
struct AdjointArgs {
    int ntok, iters, anderson_m;
    float beta;
    const float *signal, *h_star, *dl, *g;  // [ntok][H][d], [ntok][H][d], [ntok][d], [d]
    float *pre, *terms, *v0, *v1;
    float *src;                             // [ntok][d] or null
    float *v_out;                           // [ntok][H][d] or null: receives the final iterate
    SolveBuffers sb;                        // its Anderson ring
    int32_t *act, *cnt;                     // token list and count for the Anderson kernel
};
const float *launch_adjoint(const Dims &D, const AdjointArgs &a, hipStream_t st);
void launch_mem_begin(const SolveBuffers &b, int B, int T, int t, hipStream_t st);
// hist [B][H][d] holds u = W_hist m_prev on entry; becomes the history context.
void launch_hist_ctx(const Dims &D, float *hist, const float *m_prev, long m_sm, const float *signal, int B,
                     int T, int t, const float *slot_scale, const float *gate_logit, hipStream_t st);
// out[b][s] = abar m_prev + (1 - abar) x for the tokens at position t (m_prev null = zeros).
// amax (or null): raised to the largest finite |out|.
void launch_temporal(const Dims &D, const float *h, int B, int T, int t, const float *m_prev, long m_sm,
                     const float *a_log, const float *wx_diag, float *out, long out_sm, unsigned *amax,
                     hipStream_t st);
// *out = bit pattern of max |x[i]| over n floats (atomic max; *out must be zeroed first)
void launch_absmax(const float *x, long n, unsigned *out, hipStream_t st);

}  // namespace adn

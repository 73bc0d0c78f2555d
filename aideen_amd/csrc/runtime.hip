// Runtime and C ABI (include/aideen_hip.h): one context per thread owns a HIP stream, the
// device copies of the weights and the work buffers for its batch*seq capacity.
//
// Replaces the reference's wgpu device/queue runtime for this path: RustDeqBridge
// (deq_bridge.rs:55-2785) and GpuDeqBackend's forward surface (gpu_deq.rs:80-219, 3454-4078).
// The whole Picard loop is enqueued up front: the active-token count lives in device memory,
// so no iteration reads anything back to the host (the reference submits one fused kernel per
// forward and blocks on map_async, deq_bridge.rs:2017-2038).
#include <string.h>

#include <algorithm>
#include <cstring>
#include <cmath>
#include <initializer_list>
#include <utility>
#include <mutex>
#include <vector>

#include "kernels.h"

using namespace adn;

namespace adn {
static thread_local std::string g_last_error;
void set_error(const std::string &msg) { g_last_error = msg; }
}  // namespace adn

// Chunk totals of adn_embed_context_noalloc: a fixed array per device (32 MiB), held until the
// process ends.  Host code never passes the symbol itself to a kernel (on the host it names a
// stand-in, not device memory): the device address is looked up once per device, with that
// device current, when the first context on it is created, and only that address is used.
// After the data, 256 bytes hold the overlap guard (two words, zero when idle: the calls in
// flight and the finished blocks of the current call's last kernel); static device memory starts
// zeroed.
constexpr long NOALLOC_MAX_DOUBLES = 1L << 22;
constexpr long NOALLOC_GUARD_DOUBLES = 32;
static __device__ __align__(256) double scratch[NOALLOC_MAX_DOUBLES + NOALLOC_GUARD_DOUBLES];
static std::mutex g_scratch_mu;
static double *g_scratch_ptr[256];  // by device ordinal; null until looked up

struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
};

struct adn_ctx {
    adn_config cfg{};
    Dims D{};
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    bool has_weights = false;
    long cap_tok = 0;

    // weights (device)
    float *w_qkv = nullptr;  // [H][3d][d]
    float *qk_bias = nullptr;  // [H][2d] or null
    float *w_o = nullptr, *w_in = nullptr;  // [H][d][d]
    float *anchor = nullptr, *norm_scale = nullptr, *embed = nullptr, *lm_w = nullptr;
    float *lm_b = nullptr, *lm_g = nullptr, *a_log = nullptr, *wx_diag = nullptr, *w_out = nullptr;
    float *b_delta = nullptr, *w_kw = nullptr, *w_vw = nullptr, *w_b = nullptr, *w_c = nullptr;
    float *w_cat = nullptr;  // [H][r + 2N][d] = [W_kw^T; W_B; W_C] per slot (carrier projections)
    float *w_hist = nullptr, *hist_scale = nullptr, *hist_gate = nullptr;  // memory-coupled solve
    const float *last_h = nullptr;  // h* of the most recent forward (its signal is sb.signal)
    int last_ntok = 0;
    double *ctx_tot = nullptr;  // embed_context chunk totals (2 x ctx_tot_n doubles)
    long ctx_tot_n = 0;

    // split-precision copies of the GEMM weights (hi/lo halves of w * scale)
    struct Split {
        void *hi = nullptr, *lo = nullptr;
        float scale = 1.0f;
    };
    int prec = PREC_F16X3;
    Split sp_in, sp_qkv, sp_o, sp_out, sp_cat, sp_lm, sp_hist;
    float embed_scale = 1.0f;  // A-side power-of-two scale of the signal GEMM (fp16 split)

    // work buffers (capacity-sized)
    SolveBuffers sb{};
    ScanBuffers scb{};
    int scan_nch_cap = 1;
    float *pnorm = nullptr;
    float *logits_scratch = nullptr;  // lazy [cap_tok][V]
    int32_t *argmax_scratch = nullptr;
    float *am_val = nullptr;      // [cap_tok][ceil(V/128)] LM-head tile arg-max partials
    int32_t *am_idx = nullptr;
    unsigned *absmax = nullptr;   // max |s_in| (float bits) for the signal GEMM's A scale
    // the iterates of a few-row solve with a fixed iteration count (two [ATTN_FUSE_ROWS][H][d]
    // buffers, alternating): there each Q|K|V product applies the previous update itself
    float *fix_h = nullptr;
    // per-token exit flags when the caller asks for none (the mixing pass of the last iteration
    // reads them)
    int32_t *conv_scratch = nullptr;
    // Anderson's update and mix in one pass (launch_update_mix) serve this shape on this device
    bool fuse_mix = false;
    // fp16-split range guard: the A operands' magnitude bounds (ADN_BOUNDS words, reset per forward)
    // and the weight-derived constants they are combined with (set at upload)
    unsigned *bounds = nullptr;
    float h_bound = 0.0f;      // max|norm_scale| (sqrt(d) + 1e3 max|anchor| when the RMS leaves the anchor out)
    float l1_wv = 0.0f;        // largest row L1 norm of W_v: |mix| <= l1_wv |h|
    float l1_wout = 0.0f;      // largest row L1 norm of W_out: |m_t| <= (1 + l1_wout) |m_inner|
    float lm_a_scale = 1.0f;   // LM head A scale: |pnorm| <= max|lm_g| sqrt(d)
    float scan_min_decay = 0.0f;  // min over channels of the fixed carrier decay sigmoid(-a_log)
    unsigned *d_err = nullptr;

    // host-API staging (lazy, capacity-sized)
    std::vector<DevBuf> staging;
    int32_t *tok_dev = nullptr;
    float *sin_dev = nullptr;

    // ComputeBackend tensors
    std::vector<DevBuf> tensors;
    std::vector<void *> allocs;
};

namespace {

void *dmalloc(adn_ctx *c, size_t bytes) {
    void *p = nullptr;
    if (bytes == 0) bytes = 4;
    ADN_HIP(hipMalloc(&p, bytes));
    c->allocs.push_back(p);
    return p;
}

void dfree_all(adn_ctx *c) {
    for (void *p : c->allocs) (void)hipFree(p);
    c->allocs.clear();
    for (auto &t : c->tensors)
        if (t.p) (void)hipFree(t.p);
    c->tensors.clear();
}

int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

int hip_fail(const HipError &e) {
    return fail(ADN_E_HIP, std::string("HIP error ") + hipGetErrorString(e.code) + " in " + e.where);
}

std::string validate_config(const adn_config &c) {
    if (c.d_r < 64 || c.d_r > 2048 || c.d_r % 64) return "d_r must be a multiple of 64 in [64, 2048]";
    if (c.h_slots < 1 || c.h_slots > 16) return "h_slots must be in [1, 16]";
    if (c.vocab < 1) return "vocab must be >= 1";
    if (c.d_state < 1 || c.d_state > 32) return "d_state must be in [1, 32]";
    if (c.rank < 1 || c.rank > 64) return "rank must be in [1, 64]";
    if (c.max_batch < 1 || c.max_seq < 1) return "max_batch and max_seq must be >= 1";
    if ((long)c.max_batch * c.max_seq > (1L << 24)) return "max_batch*max_seq must be <= 2^24";
    if (c.anderson_m < 0 || c.anderson_m > 5) return "anderson_m must be in [0, 5]";
    if (c.flags & ~0x1FFFu) return "unknown flag bits";
    if ((c.flags & ADN_F_RESID_L2) && (c.flags & ADN_F_RESID_RELRMS))
        return "at most one of ADN_F_RESID_L2 and ADN_F_RESID_RELRMS";
    if ((c.flags & ADN_F_TOKEN_CARRY) && !(c.flags & ADN_F_MEMORY))
        return "ADN_F_TOKEN_CARRY needs ADN_F_MEMORY (positions solved in order)";
    if ((c.flags & ADN_F_MEMORY) && c.d_state != 1) return "ADN_F_MEMORY needs d_state == 1";
    if ((c.flags & ADN_F_MEMORY) && (c.flags & ADN_F_SCAN_SELECTIVE))
        return "ADN_F_MEMORY uses the non-selective carrier";
    const uint32_t g = c.flags & (ADN_F_GEMM_FP32 | ADN_F_GEMM_BF16X3 | ADN_F_GEMM_BF16);
    if (g & (g - 1)) return "at most one ADN_F_GEMM_* flag";
    return "";
}

void upload(adn_ctx *c, float **dst, const float *src, size_t n, const char *name, bool required) {
    if (!src) {
        if (required) throw std::string("missing weight tensor: ") + name;
        *dst = nullptr;
        return;
    }
    if (!*dst) *dst = (float *)dmalloc(c, n * sizeof(float));
    ADN_HIP(hipMemcpyAsync(*dst, src, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
}

// Copy a [H][rows][cols] host tensor to the device, transposing each matrix when asked.
void upload_mats(adn_ctx *c, float *dst, const float *src, int H, int rows, int cols, bool transpose,
                 float *tmp) {
    const size_t n = (size_t)H * rows * cols;
    if (!transpose) {
        ADN_HIP(hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
        return;
    }
    ADN_HIP(hipMemcpyAsync(tmp, src, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    launch_transpose(tmp, rows, cols, H, dst, c->stream);
}

float *staging_f(adn_ctx *c, int slot, size_t bytes) {
    if ((int)c->staging.size() <= slot) c->staging.resize(slot + 1);
    DevBuf &b = c->staging[slot];
    if (b.bytes < bytes) {
        if (b.p) (void)hipFree(b.p);
        b.p = nullptr;
        ADN_HIP(hipMalloc(&b.p, bytes));
        b.bytes = bytes;
    }
    return (float *)b.p;
}

// Per-launch event pairs for adn_profile_forward (null when not profiling).
struct Prof {
    struct Rec {
        int stage, k, n;  // n: rows of the launch (-1: every token of the forward)
        hipEvent_t e0, e1;
        int fused;        // PROF_FUSED_* stages done inside this launch
    };
    std::vector<Rec> recs;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    hipEvent_t get() {
        if (used == pool.size()) {
            hipEvent_t e;
            ADN_HIP(hipEventCreate(&e));
            pool.push_back(e);
        }
        return pool[used++];
    }
    ~Prof() {
        for (auto e : pool) (void)hipEventDestroy(e);
    }
};

// work of another stage done inside a launch (its bytes and flops are counted with the launch)
constexpr int PROF_FUSED_ATTN = 1;    // the attention mix, inside the W_o product
constexpr int PROF_FUSED_UPDATE = 2;  // the previous iteration's update, inside the Q|K|V product
constexpr int PROF_FUSED_POOL = 4;    // the LM head's pool, inside the last update
constexpr int PROF_FUSED_ANDERSON = 8;  // the Anderson mix, inside the update

struct Span {
    Prof *p;
    hipStream_t st;
    size_t idx;
    Span(Prof *p_, int stage, int k, hipStream_t st_, int n = -1, int fused = 0) : p(p_), st(st_), idx(0) {
        if (!p) return;
        Prof::Rec r{stage, k, n, p->get(), p->get(), fused};
        ADN_HIP(hipEventRecord(r.e0, st));
        idx = p->recs.size();
        p->recs.push_back(r);
    }
    ~Span() {
        if (p) (void)hipEventRecord(p->recs[idx].e1, st);
    }
};

float host_maxabs(std::initializer_list<std::pair<const float *, size_t>> parts) {
    float m = 0.0f;
    for (const auto &pr : parts)
        if (pr.first)
            for (size_t i = 0; i < pr.second; ++i) m = std::max(m, std::fabs(pr.first[i]));
    return m;
}

// Power-of-two scale putting max|x| in [2^(h-1), 2^h) for fp16 halves (keeps lo out of the
// subnormal range and hi below 65504); 1 for bf16 (same exponent range as fp32).
float split_scale(int prec, float maxabs, int headroom_log2 = 14) {
    if (prec != PREC_F16X3 || !(maxabs > 0.0f) || !std::isfinite(maxabs)) return 1.0f;
    int e = (int)std::floor(std::log2((double)(1 << headroom_log2) / maxabs));
    e = std::max(-24, std::min(24, e));
    return std::ldexp(1.0f, e);
}

// split copies of S matrices [N][K] (the GEMMs' B operand) in the blocked layout
// (eye: of w + I, square matrices; maxabs bounds |w|)
void make_split(adn_ctx *c, adn_ctx::Split &sp, const float *dev_w, int S, int N, int K, float maxabs,
                bool eye = false) {
    if (c->prec == PREC_FP32) return;
    const size_t bytes = (size_t)split_weight_elems(S, N, K) * 2;
    if (!sp.hi) sp.hi = dmalloc(c, bytes);
    if (c->prec != PREC_BF16X1 && !sp.lo) sp.lo = dmalloc(c, bytes);
    sp.scale = split_scale(c->prec, eye ? maxabs + 1.0f : maxabs);
    launch_split_weights(dev_w, S, N, K, sp.scale, c->prec, sp.hi, c->prec == PREC_BF16X1 ? nullptr : sp.lo,
                         c->stream, eye);
}

// The carrier readout y + W_out y (and memory mode's m_inner + W_out m_inner) runs as the plain
// product (I + W_out) y where W_out is split into two halves: the residual then costs the
// epilogue no second read of y, and I + W_out keeps ~22 bits in the hi/lo pair, as every split
// weight does.  With fp32 GEMMs, or the single bf16 half (8 bits would round y itself), the
// epilogue adds y.
bool readout_eye(const adn_ctx *c) { return c->prec == PREC_F16X3 || c->prec == PREC_BF16X3; }

void set_split(const adn_ctx *c, GemmParams &g, const adn_ctx::Split &sp, float a_scale = 1.0f) {
    g.prec = c->prec;
    if (c->prec == PREC_FP32) return;
    g.Bhi = sp.hi;
    g.Blo = sp.lo ? sp.lo : sp.hi;
    g.a_scale = a_scale;
    g.out_scale = 1.0f / (sp.scale * a_scale);
}

// The fp16 halves hold values below 65504: an A operand whose bound (bound word w, times 1/gain)
// reaches 2^14 is scaled down by a power of two inside the GEMM (results are unchanged in the
// ordinary range, where the scale stays 1).  bf16 halves have fp32's exponent range.
void set_range(const adn_ctx *c, GemmParams &g, int w, float gain = 1.0f) {
    if (c->prec != PREC_F16X3) return;
    g.a_absmax = c->bounds + w;
    g.a_headroom = gain > 0.0f ? 16384.0f / gain : INFINITY;
}

// Largest L1 norm of an output row of H [d][d] matrices (host, either upload layout).
float max_row_l1(const float *w, int H, int d, bool in_out) {
    float best = 0.0f;
    std::vector<double> acc((size_t)d);
    for (int s = 0; s < H; ++s) {
        const float *m = w + (size_t)s * d * d;
        std::fill(acc.begin(), acc.end(), 0.0);
        for (int i = 0; i < d; ++i)
            for (int j = 0; j < d; ++j) acc[in_out ? j : i] += std::fabs(m[(size_t)i * d + j]);
        for (int i = 0; i < d; ++i) best = std::max(best, (float)acc[i]);
    }
    return best;
}

// ---------------------------------------------------------------------------------------
// the forward pipeline (device pointers; enqueue only)
// ---------------------------------------------------------------------------------------
// signal[t][s] = W_in[s] x_t for every token, h0 and the first active list (all tokens).
// s_in_ready: the bounds were reset and max |s_in| accumulated into c->absmax by the caller's
// kernels (a decode step: the previous step's arg-max and this step's query); init_done: so was
// the init (the query kernel, QueryInit).
void enqueue_signal_init(adn_ctx *c, const adn_run &r, const SolveBuffers &b, int ntok, Prof *prof,
                         bool s_in_ready = false, bool init_done = false) {
    const Dims &D = c->D;
    const int d = D.d, H = D.H;
    hipStream_t st = c->stream;
    // caller-supplied rows on the fp16 split: the signal GEMM's A scale also honours their actual
    // magnitude (max |s_in|, accumulated into c->absmax, which the reset clears)
    const bool dyn_scale = r.s_in && c->prec == PREC_F16X3;
    if (!s_in_ready) launch_reset_bounds(c->bounds, c->h_bound, dyn_scale ? c->absmax : nullptr, st);
    // x gathered from the embedding when tokens are given
    {
        GemmParams g{};
        g.role = ROLE_SIGNAL;
        g.A = r.tokens ? c->embed : r.s_in;
        g.a_idx = r.tokens;
        g.a_idx_max = D.V;
        g.a_sm = d;
        g.a_ss = 0;
        g.B = c->w_in;
        g.b_ss = (long)d * d;
        g.C = b.signal;
        g.c_sm = (long)H * d;
        g.c_ss = d;
        g.M = ntok;
        g.N = d;
        g.K = d;
        g.S = H;
        g.err = b.err;
        g.epi = EPI_NONE;
        set_split(c, g, c->sp_in, c->embed_scale);
        Span sp(prof, ADN_STAGE_SIGNAL_GEMM, -1, st);
        if (dyn_scale) {
            // rows of any size stay inside the fp16 range (rows no larger than the embedding
            // table's entries keep the embedding's scale, and match the token path bit for bit)
            if (!s_in_ready) launch_absmax(r.s_in, (long)ntok * d, c->absmax, st);
            g.a_absmax = c->absmax;
            g.a_headroom = 1024.0f;
        }
        launch_gemm(g, st);
    }
    if (!init_done) {
        Span sp(prof, ADN_STAGE_INIT, -1, st);
        launch_init(D, b, r.tokens ? c->embed : r.s_in, r.tokens, ntok, c->anchor, st);
    }
}

// max_iters Picard steps over the active list b.act[0] / b.cnt[0]: at most `rows` tokens are
// active, token indices are < ntok (the row stride of h, signal and the Anderson ring).
// pool: the head's pool outputs (SolveBuffers::pool_*), formed by the last update where it can
// (a fixed-iteration solve whose rows fit in LDS); returns whether it did.
bool enqueue_iterations(adn_ctx *c, const adn_run &r, const SolveBuffers &b, int rows, int ntok, Prof *prof,
                        const SolveBuffers *pool = nullptr) {
    const Dims &D = c->D;
    const int d = D.d, H = D.H;
    hipStream_t st = c->stream;
    // Anderson depths 1 and 2 never mix (n_res = min(k, m - 1) < 2), so they run as plain Picard
    // (no ring of iterates)
    const int m = c->cfg.anderson_m >= 3 ? c->cfg.anderson_m : 0;
    // W_o on the 256x256 fp16-split tiles reads its A (mix) pre-split: the attention writes the
    // halves, in mix's memory, with the scale the GEMM derives from the h bound (set_range below)
    const bool wo_pre = gemm_presplit_ok(c->prec, rows, d);
    SolveBuffers ba = b;
    if (wo_pre) {
        ba.mix_pre = b.mix;
        ba.mix_bound = c->bounds;
        ba.mix_headroom = c->l1_wv > 0.0f ? 16384.0f / c->l1_wv : INFINITY;
    }
    // A few rows where no token can exit before the last iteration (a tolerance of zero or less,
    // no plateau exit, no Anderson mixing, no history term): each Q|K|V product applies the
    // previous iteration's update to its rows itself (GemmParams::upd_o), so the update runs only
    // at the last iteration, where it records the iteration counts.  The iterates alternate
    // between two small buffers (a product's column blocks read h_{k-1} while the slot's first
    // block writes h_k), and the active list stays list 0.
    const bool fixed = gemm_attn_fusable(c->prec, rows, d, H) && rows == ntok && !(r.eps > 0.0f) &&
                       !b.rprev && m == 0 && !b.mem_hist && r.max_iters >= 2;
    const long fix_stride = (long)std::min<long>(c->cap_tok, ATTN_FUSE_ROWS) * H * d;
    const bool pool_here = fixed && pool && (long)H * d <= 16384;  // the update's LDS holds a token's rows
    auto iterate = [&](int j) { return j == 0 ? b.h : c->fix_h + (long)(j & 1) * fix_stride; };
    for (int k = 0; k < r.max_iters; ++k) {
        const int cur = fixed ? 0 : k & 1;
        {  // Q|K|V for every slot of every active token
            GemmParams g{};
            g.role = ROLE_QKV;
            g.A = fixed ? iterate(k > 0 ? k - 1 : 0) : b.h;
            if (fixed && k > 0) {
                g.upd_o = b.o;
                g.upd_sig = b.signal;
                g.upd_anchor = c->anchor;
                g.upd_norm = c->norm_scale;
                g.upd_hout = iterate(k);
                g.upd_beta = r.damping;
                g.upd_excl = (D.flags & ADN_F_RMS_EXCL_ANCHOR) != 0;
            }
            g.a_idx = b.act[cur];
            g.a_idx_max = ntok;
            g.a_sm = (long)H * d;
            g.a_ss = d;
            g.B = c->w_qkv;
            g.b_ss = 3L * d * d;
            g.C = b.qkv;
            g.c_sm = 3L * H * d;
            g.c_ss = 3L * d;
            g.bias = c->qk_bias;
            g.bias_ss = 2L * d;
            g.bias_n = 2 * d;
            g.M = rows;
            g.N = 3 * d;
            g.K = d;
            g.S = H;
            g.m_count = b.cnt + cur;
            g.err = b.err;
            g.epi = c->qk_bias ? EPI_BIAS : EPI_NONE;
            set_split(c, g, c->sp_qkv);
            set_range(c, g, 0);
            Span sp(prof, ADN_STAGE_QKV_GEMM, k, st, -1, g.upd_o ? PROF_FUSED_UPDATE : 0);
            launch_gemm(g, st);
        }
        // At a few rows the attention is formed inside the W_o product (one launch less per
        // iteration; the attention stage then reads zero)
        const bool attn_in_wo = gemm_attn_fusable(c->prec, rows, d, H);
        if (!attn_in_wo) {
            Span sp(prof, ADN_STAGE_ATTN, k, st);
            launch_attn(D, ba, cur, k, rows, st);
        }
        {  // o = W_o mix
            GemmParams g{};
            g.role = ROLE_WO;
            g.A = b.mix;
            g.a_sm = (long)H * d;
            g.a_ss = d;
            g.B = c->w_o;
            g.b_ss = (long)d * d;
            g.C = b.o;
            g.c_sm = (long)H * d;
            g.c_ss = d;
            g.M = rows;
            g.N = d;
            g.K = d;
            g.S = H;
            g.m_count = b.cnt + cur;
            g.err = b.err;
            g.epi = EPI_NONE;
            set_split(c, g, c->sp_o);
            set_range(c, g, 0, c->l1_wv);  // mix is a convex combination of V = W_v h rows
            if (wo_pre) g.a_pre = b.mix;
            if (attn_in_wo) {
                g.attn_qkv = b.qkv;
                g.attn_clamp = (D.flags & ADN_F_SCORE_CLAMP4) != 0;
                g.attn_cnt_next = b.cnt + (cur ^ 1);
                g.attn_cnt_hist = b.cnt_hist + k;
            }
            Span sp(prof, ADN_STAGE_WO_GEMM, k, st, -1, attn_in_wo ? PROF_FUSED_ATTN : 0);
            launch_gemm(g, st);
        }
        // With Anderson mixing after this update, the update writes its iterate straight into the
        // iteration's ring slot and the mixing pass, over every token the update saw, sets h (the
        // mix, or the iterate of a token that exited): the iterate is written once instead of to h
        // and then again to the slot.
        // Before the first mix (k < 2) the update writes the iterate into both, and no mixing pass
        // runs.
        // Anderson mixes after every step that a token does not exit on the tolerance, the last
        // one included (a token stopped at the cap unconverged ends with the mix)
        const bool mix = m > 0;
        const bool from_slot = mix && anderson_from_slot_ok(D);
        const int cap_mix = mix && k + 1 == r.max_iters && k >= 2;
        if (m >= 3 && k >= 2 && b.mix_coef && c->fuse_mix) {
            // from the first mix on, the update and the mix in one pass (the previous iterate
            // rebuilt from the ring, so h is not read)
            SolveBuffers bu = b;
            bu.cap_mix = cap_mix;
            Span sp(prof, ADN_STAGE_UPDATE, k, st, -1, PROF_FUSED_ANDERSON);
            launch_update_mix(D, bu, cur, k, m, ntok, rows, r.max_iters, r.eps, c->anchor, c->norm_scale, r.damping,
                              st);
            continue;
        }
        if (!fixed || k + 1 == r.max_iters) {
            SolveBuffers bu = b;
            bu.cap_mix = cap_mix;
            if (from_slot) {
                bu.h_out = b.hist + (long)(k % m) * ntok * H * d;
                bu.h_both = k < 2;
            }
            if (fixed) {  // from the last small buffer into h
                bu.h = iterate(k);
                bu.h_out = b.h;
                if (pool_here) {
                    bu.pool = 1;
                    bu.pool_out = pool->pool_out;
                    bu.pool_norm = pool->pool_norm;
                    bu.pool_g = pool->pool_g;
                }
            }
            Span sp(prof, ADN_STAGE_UPDATE, k, st, -1, bu.pool ? PROF_FUSED_POOL : 0);
            launch_update(D, bu, cur, k, r.max_iters, r.eps, rows, c->anchor, c->norm_scale, r.damping, st);
        }
        if (mix && !(from_slot && k < 2)) {
            Span sp(prof, ADN_STAGE_ANDERSON, k, st);
            SolveBuffers ba2 = b;
            ba2.cap_mix = cap_mix;
            if (from_slot)
                launch_anderson_from_slot(D, ba2, cur, ntok, rows, k, m, st);
            else
                launch_anderson(D, ba2, cur ^ 1, ntok, rows, k, m, st);
        }
    }
    return pool_here;
}

// The carrier's per-row record: rms (unless the pooling pass wrote it: rms_done) and the
// projections P[t][s] = W_cat[s] h[t][s] into rec[1 .. REC).
void enqueue_scan_prep(adn_ctx *c, int ntok, const SolveBuffers &b, Prof *prof, bool rms_done) {
    const Dims &D = c->D;
    const int d = D.d, H = D.H;
    const int REC = scan_rec_len(D);
    hipStream_t st = c->stream;
    Span sp(prof, ADN_STAGE_SCAN_PREP, -1, st);
    if (!rms_done) launch_row_rms(b.h, (long)ntok * H, d, c->scb.rec, REC, st);
    GemmParams g{};
    g.role = ROLE_SCAN_PROJ;
    g.A = b.h;
    g.a_sm = (long)H * d;
    g.a_ss = d;
    g.B = c->w_cat;
    g.b_ss = (long)(REC - 1) * d;
    g.C = c->scb.rec + 1;
    g.c_sm = (long)H * REC;
    g.c_ss = REC;
    g.M = ntok;
    g.N = REC - 1;
    g.K = d;
    g.S = H;
    g.err = b.err;
    g.epi = EPI_NONE;
    set_split(c, g, c->sp_cat);
    set_range(c, g, 0);
    launch_gemm(g, st);
}

// pooled rows, logits and arg-max of the solved h of all ntok tokens.  scan_rms: the pooling
// pass also writes every row's RMS into the carrier record, and the carrier's projections
// follow it at once, before the LM head, while h* is still in the caches (the LM head's logits
// stream would evict it).  Returns whether it did (the scan then skips its preparation).
// app: a decode step's token append, done by the arg-max kernel.
bool enqueue_head(adn_ctx *c, const adn_outputs &o, const SolveBuffers &b, int ntok, Prof *prof,
                  bool scan_rms = false, const TokenAppend *app = nullptr, bool pool_done = false) {
    const Dims &D = c->D;
    const int d = D.d;
    hipStream_t st = c->stream;
    const bool want_logits = o.logits || o.argmax;
    const bool pool = o.pooled || want_logits;
    // the LM head on the 256x256 fp16-split tiles reads its A pre-split, written so by the pool
    // kernel with the head's A scale
    const bool lm_pre = want_logits && gemm_presplit_ok(c->prec, ntok, D.V);
    if (pool && !pool_done) {
        Span sp(prof, ADN_STAGE_POOL, -1, st);
        launch_pool_norm(D, b.h, ntok, c->lm_g, o.pooled, want_logits ? c->pnorm : nullptr,
                         scan_rms ? c->scb.rec : nullptr, scan_rec_len(D), lm_pre ? c->lm_a_scale : 0.0f, st);
    }
    if (pool && scan_rms) enqueue_scan_prep(c, ntok, b, prof, true);
    if (want_logits) {
        float *logits = o.logits;
        if (!logits) {
            if (!c->logits_scratch)
                c->logits_scratch = (float *)dmalloc(c, (size_t)c->cap_tok * D.V * sizeof(float));
            logits = c->logits_scratch;
        }
        GemmParams g{};
        g.role = ROLE_LMHEAD;
        g.A = c->pnorm;
        g.a_sm = d;
        g.B = c->lm_w;
        g.C = logits;
        g.c_sm = D.V;
        g.bias = c->lm_b;
        g.bias_n = D.V;
        g.M = ntok;
        g.N = D.V;
        g.K = d;
        g.S = 1;
        g.err = b.err;
        g.epi = c->lm_b ? EPI_BIAS : EPI_NONE;
        set_split(c, g, c->sp_lm, c->lm_a_scale);
        if (lm_pre) g.a_pre = c->pnorm;
        const int pcols = gemm_lm_partial_cols(c->prec, ntok, d);
        const int ntiles = (D.V + pcols - 1) / pcols;
        if (o.argmax) {
            g.am_val = c->am_val;
            g.am_idx = c->am_idx;
        }
        {
            Span sp(prof, ADN_STAGE_LMHEAD_GEMM, -1, st);
            launch_gemm(g, st);
        }
        if (o.argmax) {
            Span sp(prof, ADN_STAGE_ARGMAX, -1, st);
            launch_argmax_reduce(c->am_val, c->am_idx, ntok, ntiles, o.argmax, st, app);
        }
    }
    return pool && scan_rms;
}

// canonical carrier over each sequence's solved h (the readout scan).
void enqueue_scan(adn_ctx *c, const adn_run &r, const adn_outputs &o, const SolveBuffers &b, Prof *prof,
                  bool prep_done = false) {
    const Dims &D = c->D;
    const int ntok = r.batch * r.seq;
    const int d = D.d, H = D.H;
    hipStream_t st = c->stream;
    if (o.scan_y || o.scan_state) {
        if (!prep_done) enqueue_scan_prep(c, ntok, b, prof, false);
        // chunk buffers hold max_batch * scan_nch_cap sequence-chunks
        const int nch_fit = std::max(1, (c->cfg.max_batch * c->scan_nch_cap) / r.batch);
        const bool ssd = scan_use_ssd(D, r.batch, r.seq, c->scan_min_decay);
        const int nch = std::min(std::min(scan_chunks(r.batch, r.seq, H, d, ssd), c->scan_nch_cap), nch_fit);
        float *y = (o.scan_y && !c->w_out) ? o.scan_y : c->scb.y;
        {
            Span sp(prof, ADN_STAGE_SCAN, nch, st);
            launch_scan(D, b.h, c->scb.rec, r.batch, r.seq, c->w_b != nullptr, c->a_log, c->wx_diag, c->b_delta,
                        c->w_vw, r.scan_state_in, y, o.scan_state, c->scb.chunk_s, c->scb.chunk_p, nch,
                        c->bounds + 1, ssd, c->scan_min_decay, st);
        }
        if (o.scan_y && c->w_out) {
            GemmParams g{};
            g.role = ROLE_READOUT;
            g.A = y;
            g.a_sm = (long)H * d;
            g.a_ss = d;
            g.B = c->w_out;
            g.b_ss = (long)d * d;
            g.C = o.scan_y;
            g.c_sm = (long)H * d;
            g.c_ss = d;
            g.M = ntok;
            g.N = d;
            g.K = d;
            g.S = H;
            g.err = b.err;
            g.epi = readout_eye(c) ? EPI_NONE : EPI_ADD_A;
            set_split(c, g, c->sp_out);
            set_range(c, g, 1);
            Span sp(prof, ADN_STAGE_READOUT_GEMM, -1, st);
            launch_gemm(g, st);
        }
    }
}

// A greedy decode step's extras: the query kernel has reset the range guard's bounds and
// accumulated max |s_in| (s_in_ready), and the arg-max kernel appends the token (app).
struct DecodeStep {
    bool s_in_ready;
    bool init_done;
    const TokenAppend *app;
};

void enqueue_forward(adn_ctx *c, const adn_run &r, const adn_outputs &o, Prof *prof = nullptr,
                     const DecodeStep *ds = nullptr) {
    const int ntok = r.batch * r.seq;
    SolveBuffers b = c->sb;
    if (o.h_star) b.h = o.h_star;
    if (o.iters) b.iters = o.iters;
    b.conv = o.converged ? o.converged : c->conv_scratch;
    b.mem_hist = nullptr;
    b.amax_h = c->bounds;
    c->last_h = b.h;  // the adjoint reads this forward's h* and signal
    c->last_ntok = ntok;
    enqueue_signal_init(c, r, b, ntok, prof, ds && ds->s_in_ready, ds && ds->init_done);
    // the pool may be formed by the last update (fixed-iteration solves): not where the head's
    // pool also feeds the carrier or writes the LM head's A pre-split
    const bool want_logits = o.logits || o.argmax;
    const bool scan = o.scan_y || o.scan_state;
    SolveBuffers pr{};
    pr.pool_out = o.pooled;
    pr.pool_norm = want_logits ? c->pnorm : nullptr;
    pr.pool_g = c->lm_g;
    const bool pool_ok = (want_logits || o.pooled) && !scan && !(want_logits && gemm_presplit_ok(c->prec, ntok, c->D.V));
    const bool pooled = enqueue_iterations(c, r, b, ntok, ntok, prof, pool_ok ? &pr : nullptr);
    const bool prep_done = enqueue_head(c, o, b, ntok, prof, scan, ds ? ds->app : nullptr, pooled);
    enqueue_scan(c, r, o, b, prof, prep_done);
}

// Memory-coupled forward (fixed-history mode, trainer.rs:677-720): position t of every sequence
// is solved with the history context of m_{t-1} added to the update, then m_t = temporal_step(
// m_{t-1}, h*_t) (fixed_point_memory_reasoning.rs:1317-1370, 1454-1485).  The B tokens of one
// position form the active list; positions run in order.  m_t of every token lands in scan_y
// (or scratch), the last one in scan_state; scan_state_in is m_{-1} (null = zero state, no
// history context at t = 0).
void enqueue_forward_memory(adn_ctx *c, const adn_run &r, const adn_outputs &o, Prof *prof = nullptr,
                            const TokenAppend *app = nullptr) {
    const Dims &D = c->D;
    const int B = r.batch, T = r.seq, ntok = B * T;
    const int d = D.d, H = D.H;
    const long hd = (long)H * d;
    hipStream_t st = c->stream;
    SolveBuffers b = c->sb;
    if (o.h_star) b.h = o.h_star;
    if (o.iters) b.iters = o.iters;
    b.conv = o.converged ? o.converged : c->conv_scratch;
    b.mem_hist = nullptr;
    b.amax_h = c->bounds;
    b.mem_T = T;
    c->last_h = b.h;
    c->last_ntok = ntok;
    enqueue_signal_init(c, r, b, ntok, prof);
    if (r.scan_state_in && c->prec == PREC_F16X3)  // a caller-supplied memory bounds m as well
        launch_absmax(r.scan_state_in, hd * B, c->bounds + 2, st);
    float *mseq = o.scan_y ? o.scan_y : c->scb.y;  // [B][T][H][d]
    float *hist = c->scb.mem_hist;                   // [B][H][d]
    float *mn = c->scb.mem_mn;                       // [B][H][d] state before W_out
    for (int t = 0; t < T; ++t) {
        {
            Span sp(prof, ADN_STAGE_CONVERGE, -1, st, B);
            launch_mem_begin(b, B, T, t, st);
        }
        const float *mprev = t > 0 ? mseq + (long)(t - 1) * hd : r.scan_state_in;
        const long msm = t > 0 ? (long)T * hd : hd;
        b.mem_hist = nullptr;
        if (t > 0 && (c->cfg.flags & ADN_F_TOKEN_CARRY))  // warm start from h*_{t-1}
            ADN_HIP(hipMemcpy2DAsync(b.h + (long)t * hd, (size_t)T * hd * sizeof(float), b.h + (long)(t - 1) * hd,
                                     (size_t)T * hd * sizeof(float), hd * sizeof(float), B, hipMemcpyDeviceToDevice,
                                     st));
        if (mprev) {
            GemmParams g{};  // u[b][s] = W_hist m_prev[b][s]  (one W_hist for every slot)
            g.role = ROLE_WO;
            g.A = mprev;
            g.a_sm = msm;
            g.a_ss = d;
            g.B = c->w_hist;
            g.b_ss = 0;
            g.C = hist;
            g.c_sm = hd;
            g.c_ss = d;
            g.M = B;
            g.N = d;
            g.K = d;
            g.S = H;
            g.err = b.err;
            g.epi = EPI_NONE;
            set_split(c, g, c->sp_hist);
            set_range(c, g, 2, 1.0f + (c->w_out ? c->l1_wout : 0.0f));  // m_{t-1} = (I + W_out) m_inner
            {
                Span sp(prof, ADN_STAGE_HIST_GEMM, -1, st, B);
                launch_gemm(g, st);
            }
            Span sp(prof, ADN_STAGE_HIST_CTX, -1, st, B);
            launch_hist_ctx(D, hist, mprev, msm, b.signal, B, T, t, c->hist_scale, c->hist_gate, st);
            b.mem_hist = hist;
        }
        enqueue_iterations(c, r, b, B, ntok, prof);
        float *mt = mseq + (long)t * hd;
        if (c->w_out) {
            {
                Span sp(prof, ADN_STAGE_TEMPORAL, -1, st, B);
                launch_temporal(D, b.h, B, T, t, mprev, msm, c->a_log, c->wx_diag, mn, hd, c->bounds + 2, st);
            }
            GemmParams g{};  // m_t = m_inner + W_out m_inner
            g.role = ROLE_READOUT;
            g.A = mn;
            g.a_sm = hd;
            g.a_ss = d;
            g.B = c->w_out;
            g.b_ss = (long)d * d;
            g.C = mt;
            g.c_sm = (long)T * hd;
            g.c_ss = d;
            g.M = B;
            g.N = d;
            g.K = d;
            g.S = H;
            g.err = b.err;
            g.epi = readout_eye(c) ? EPI_NONE : EPI_ADD_A;
            set_split(c, g, c->sp_out);
            set_range(c, g, 2);
            Span sp(prof, ADN_STAGE_READOUT_GEMM, -1, st, B);
            launch_gemm(g, st);
        } else {
            Span sp(prof, ADN_STAGE_TEMPORAL, -1, st, B);
            launch_temporal(D, b.h, B, T, t, mprev, msm, c->a_log, c->wx_diag, mt, (long)T * hd, c->bounds + 2, st);
        }
    }
    if (o.scan_state)
        ADN_HIP(hipMemcpy2DAsync(o.scan_state, hd * sizeof(float), mseq + (long)(T - 1) * hd,
                                 (size_t)T * hd * sizeof(float), hd * sizeof(float), B, hipMemcpyDeviceToDevice,
                                 st));
    enqueue_head(c, o, b, ntok, prof, false, app);
}

void enqueue_run(adn_ctx *c, const adn_run &r, const adn_outputs &o, Prof *prof = nullptr) {
    if (c->cfg.flags & ADN_F_MEMORY)
        enqueue_forward_memory(c, r, o, prof);
    else
        enqueue_forward(c, r, o, prof);
}

int check_run(adn_ctx *c, const adn_run *r) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    if (!r) return fail(ADN_E_INVALID, "null run");
    if (!c->has_weights) return fail(ADN_E_NO_WEIGHTS, "forward before adn_upload_weights");
    if (r->batch < 1 || r->seq < 1) return fail(ADN_E_INVALID, "batch and seq must be >= 1");
    if ((long)r->batch * r->seq > c->cap_tok)
        return fail(ADN_E_CAPACITY, "batch*seq exceeds the context capacity");
    if (r->max_iters < 1 || r->max_iters > ADN_PROFILE_MAX_ITERS)
        return fail(ADN_E_INVALID, "max_iters must be in [1, 256]");
    if (!(r->damping > 0.0f && r->damping <= 1.0f)) return fail(ADN_E_INVALID, "damping must be in (0, 1]");
    if (!(r->eps >= 0.0f)) return fail(ADN_E_INVALID, "eps must be >= 0");
    if ((r->tokens == nullptr) == (r->s_in == nullptr))
        return fail(ADN_E_INVALID, "exactly one of tokens / s_in must be given");
    return ADN_OK;
}

int check_device_error(adn_ctx *c) {
    unsigned err = 0;
    ADN_HIP(hipMemcpyAsync(&err, c->d_err, sizeof(unsigned), hipMemcpyDeviceToHost, c->stream));
    ADN_HIP(hipStreamSynchronize(c->stream));
    if (err) {
        ADN_HIP(hipMemsetAsync(c->d_err, 0, sizeof(unsigned), c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
        if (err & ADN_DEVERR_TOKEN) return fail(ADN_E_INVALID, "token id outside [0, vocab)");
        if (err & ADN_DEVERR_OVERLAP)
            return fail(ADN_E_INVALID, "adn_embed_context_noalloc calls overlapped on one GPU (other streams or "
                                       "threads): the shared device array they use was raced, their outputs are "
                                       "not valid");
        return fail(ADN_E_INVALID, "device-side error");
    }
    return ADN_OK;
}

}  // namespace

// =========================================================================================
// C ABI
// =========================================================================================
extern "C" {

int adn_abi_version(void) { return ADN_ABI_VERSION; }

const char *adn_last_error(void) { return g_last_error.c_str(); }

int adn_device_count(int32_t *count) {
    if (!count) return fail(ADN_E_INVALID, "null count");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return ADN_OK;
}

int adn_create(const adn_config *cfg, adn_ctx **out) {
    if (!cfg || !out) return fail(ADN_E_INVALID, "null argument");
    *out = nullptr;
    const std::string msg = validate_config(*cfg);
    if (!msg.empty()) return fail(ADN_E_INVALID, msg);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(ADN_E_NO_DEVICE, "no HIP device");
    adn_ctx *c = new adn_ctx();
    try {
        c->cfg = *cfg;
        c->D = Dims{cfg->d_r, cfg->h_slots, cfg->vocab, cfg->d_state, cfg->rank, cfg->flags};
        c->prec = (cfg->flags & ADN_F_GEMM_FP32)     ? PREC_FP32
                  : (cfg->flags & ADN_F_GEMM_BF16X3) ? PREC_BF16X3
                  : (cfg->flags & ADN_F_GEMM_BF16)   ? PREC_BF16X1
                                                     : PREC_F16X3;
        ADN_HIP(hipGetDevice(&c->device));
        if (c->device < 0 || c->device >= 256) throw HipError{hipErrorInvalidDevice, "adn_create: device ordinal"};
        c->fuse_mix = cfg->anderson_m >= 3 && update_mix_ok(c->D);
        {  // the allocation-free entry point's per-device array (once per device)
            std::lock_guard<std::mutex> lk(g_scratch_mu);
            if (!g_scratch_ptr[c->device]) {
                void *p = nullptr;
                ADN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
                g_scratch_ptr[c->device] = (double *)p;
            }
        }
        ADN_HIP(hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking));
        c->stream = c->own_stream;
        const long T = (long)cfg->max_batch * cfg->max_seq;
        c->cap_tok = T;
        const long d = cfg->d_r, H = cfg->h_slots;
        const size_t hd = (size_t)T * H * d * sizeof(float);
        SolveBuffers &b = c->sb;
        b.signal = (float *)dmalloc(c, hd);
        b.h = (float *)dmalloc(c, hd);
        b.qkv = (float *)dmalloc(c, 3 * hd);
        b.mix = (float *)dmalloc(c, hd);
        b.o = (float *)dmalloc(c, hd);
        b.act[0] = (int32_t *)dmalloc(c, (size_t)T * sizeof(int32_t));
        b.act[1] = (int32_t *)dmalloc(c, (size_t)T * sizeof(int32_t));
        b.cnt = (int32_t *)dmalloc(c, 4 * sizeof(int32_t));
        b.iters = (int32_t *)dmalloc(c, (size_t)T * sizeof(int32_t));
        b.rprev = (cfg->flags & ADN_F_HOMEOSTATIC_EXIT) ? (float *)dmalloc(c, (size_t)T * sizeof(float)) : nullptr;
        b.cnt_hist = (int32_t *)dmalloc(c, ADN_PROFILE_MAX_ITERS * sizeof(int32_t));
        b.hist = cfg->anderson_m > 0 ? (float *)dmalloc(c, hd * cfg->anderson_m) : nullptr;
        b.mix_coef = cfg->anderson_m >= 3 ? (float *)dmalloc(c, (size_t)T * 4 * sizeof(float)) : nullptr;
        c->d_err = (unsigned *)dmalloc(c, sizeof(unsigned));
        c->absmax = (unsigned *)dmalloc(c, sizeof(unsigned));
        c->fix_h = (float *)dmalloc(c, 2 * (size_t)std::min<long>(T, ATTN_FUSE_ROWS) * H * d * sizeof(float));
        c->conv_scratch = (int32_t *)dmalloc(c, (size_t)T * sizeof(int32_t));
        c->bounds = (unsigned *)dmalloc(c, ADN_BOUNDS * sizeof(unsigned));
        b.err = c->d_err;
        ADN_HIP(hipMemsetAsync(c->d_err, 0, sizeof(unsigned), c->stream));
        c->pnorm = (float *)dmalloc(c, (size_t)T * d * sizeof(float));
        c->argmax_scratch = (int32_t *)dmalloc(c, (size_t)T * sizeof(int32_t));
        // arg-max partials: per 128 columns, or per 64 at up to ATTN_FUSE_ROWS rows
        const size_t ntiles = ((size_t)cfg->vocab + GEMM_BN - 1) / GEMM_BN;
        const size_t am_n = std::max((size_t)T * ntiles, (size_t)std::min<long>(T, ATTN_FUSE_ROWS) * ((cfg->vocab + 63) / 64));
        c->am_val = (float *)dmalloc(c, am_n * sizeof(float));
        c->am_idx = (int32_t *)dmalloc(c, am_n * sizeof(int32_t));
        c->scb.rec = (float *)dmalloc(c, (size_t)T * H * scan_rec_len(c->D) * sizeof(float));
        c->scb.y = (float *)dmalloc(c, hd);
        if (cfg->flags & ADN_F_MEMORY) {
            // [batch][H][d] per position; a memory forward may run any batch with batch * seq <=
            // cap_tok (e.g. max_batch = 1, max_seq = 8 admits batch 2 x seq 4), so size for cap_tok rows
            c->scb.mem_mn = (float *)dmalloc(c, hd);
            c->scb.mem_hist = (float *)dmalloc(c, hd);
        }
        c->scan_nch_cap = 16;
        const size_t chunk_states = (size_t)cfg->max_batch * c->scan_nch_cap * H * d;
        c->scb.chunk_s = (float *)dmalloc(c, chunk_states * cfg->d_state * sizeof(float));
        c->scb.chunk_p = (float *)dmalloc(c, chunk_states * sizeof(float));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        int rc = hip_fail(e);
        dfree_all(c);
        if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
        delete c;
        return rc;
    }
    *out = c;
    return ADN_OK;
}

void adn_destroy(adn_ctx *c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    dfree_all(c);
    for (auto &b : c->staging)
        if (b.p) (void)hipFree(b.p);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

int adn_set_stream(adn_ctx *c, void *s) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    try {
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    c->stream = s ? (hipStream_t)s : c->own_stream;
    return ADN_OK;
}

int adn_synchronize(adn_ctx *c) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    try {
        ADN_HIP(hipStreamSynchronize(c->stream));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

int adn_upload_weights(adn_ctx *c, const adn_weights *w, uint32_t layout) {
    if (!c || !w) return fail(ADN_E_INVALID, "null argument");
    if (layout != ADN_LAYOUT_OUT_IN && layout != ADN_LAYOUT_IN_OUT) return fail(ADN_E_INVALID, "unknown layout");
    const adn_config &cf = c->cfg;
    const int d = cf.d_r, H = cf.h_slots, V = cf.vocab, N = cf.d_state, r = cf.rank;
    const size_t mat = (size_t)d * d;
    try {
        for (const float *p : {w->w_q, w->w_k, w->w_v, w->w_o, w->w_in, w->anchor, w->norm_scale, w->embed,
                               w->lm_w, w->a_log, w->wx_diag})
            if (!p) return fail(ADN_E_INVALID, "missing required weight tensor");
        if ((cf.flags & ADN_F_SCAN_SELECTIVE) && (!w->w_kw || !w->w_vw))
            return fail(ADN_E_INVALID, "selective carrier needs w_kw and w_vw");
        if ((w->w_b == nullptr) != (w->w_c == nullptr)) return fail(ADN_E_INVALID, "w_b and w_c go together");
        float *tmp = staging_f(c, 15, (size_t)H * mat * sizeof(float));
        const bool in_out = layout == ADN_LAYOUT_IN_OUT;
        if (!c->w_qkv) c->w_qkv = (float *)dmalloc(c, 3 * H * mat * sizeof(float));
        if (!c->w_o) c->w_o = (float *)dmalloc(c, H * mat * sizeof(float));
        if (!c->w_in) c->w_in = (float *)dmalloc(c, H * mat * sizeof(float));
        // W_qkv[s] = [W_q[s]; W_k[s]; W_v[s]] as rows [3d][d]: one strided transpose/copy per part.
        const float *parts[3] = {w->w_q, w->w_k, w->w_v};
        float *qkv_tmp = staging_f(c, 14, H * mat * sizeof(float));
        for (int p = 0; p < 3; ++p) {
            upload_mats(c, qkv_tmp, parts[p], H, d, d, in_out, tmp);
            ADN_HIP(hipMemcpy2DAsync(c->w_qkv + p * mat, 3 * mat * sizeof(float), qkv_tmp, mat * sizeof(float),
                                     mat * sizeof(float), H, hipMemcpyDeviceToDevice, c->stream));
        }
        upload_mats(c, c->w_o, w->w_o, H, d, d, in_out, tmp);
        // signal = W_in x, or W_in^T x under ADN_F_WIN_TRANSPOSED: the GEMM wants rows = outputs.
        const bool win_t = (cf.flags & ADN_F_WIN_TRANSPOSED) != 0;
        upload_mats(c, c->w_in, w->w_in, H, d, d, in_out != win_t, tmp);
        if (w->q_bias || w->k_bias) {
            if (!c->qk_bias) c->qk_bias = (float *)dmalloc(c, 2 * (size_t)H * d * sizeof(float));
            ADN_HIP(hipMemsetAsync(c->qk_bias, 0, 2 * (size_t)H * d * sizeof(float), c->stream));
            if (w->q_bias)
                ADN_HIP(hipMemcpy2DAsync(c->qk_bias, 2 * d * sizeof(float), w->q_bias, d * sizeof(float),
                                         d * sizeof(float), H, hipMemcpyHostToDevice, c->stream));
            if (w->k_bias)
                ADN_HIP(hipMemcpy2DAsync(c->qk_bias + d, 2 * d * sizeof(float), w->k_bias, d * sizeof(float),
                                         d * sizeof(float), H, hipMemcpyHostToDevice, c->stream));
        } else {
            c->qk_bias = nullptr;
        }
        upload(c, &c->anchor, w->anchor, (size_t)H * d, "anchor", true);
        upload(c, &c->norm_scale, w->norm_scale, d, "norm_scale", true);
        upload(c, &c->embed, w->embed, (size_t)V * d, "embed", true);
        upload(c, &c->lm_w, w->lm_w, (size_t)V * d, "lm_w", true);
        upload(c, &c->lm_b, w->lm_b, V, "lm_b", false);
        upload(c, &c->lm_g, w->lm_g, d, "lm_g", false);
        upload(c, &c->a_log, w->a_log, (size_t)H * d, "a_log", true);
        {
            float mn = 1.0f;
            for (size_t i = 0; i < (size_t)H * d; ++i) mn = std::min(mn, 1.0f / (1.0f + std::exp(w->a_log[i])));
            c->scan_min_decay = mn;  // NaN a_log compares false: a NaN decay leaves mn as it was
        }
        upload(c, &c->wx_diag, w->wx_diag, (size_t)H * d, "wx_diag", true);
        if (w->w_out) {
            if (!c->w_out) c->w_out = (float *)dmalloc(c, H * mat * sizeof(float));
            upload_mats(c, c->w_out, w->w_out, H, d, d, in_out, tmp);
        } else {
            c->w_out = nullptr;
        }
        if (cf.flags & ADN_F_MEMORY) {
            // u = W_hist m with W_hist [out][in] row-major in either layout (the reference exports
            // reasoning.w_hist_shared row-major, FPMR:656-659)
            upload(c, &c->w_hist, w->w_hist, mat, "w_hist", true);
            upload(c, &c->hist_scale, w->hist_slot_scale, (size_t)H * d, "hist_slot_scale", true);
            upload(c, &c->hist_gate, w->hist_gate_logit, H, "hist_gate_logit", true);
        }
        upload(c, &c->b_delta, w->b_delta, (size_t)H * d, "b_delta", false);
        upload(c, &c->w_kw, w->w_kw, (size_t)H * d * r, "w_kw", false);
        upload(c, &c->w_vw, w->w_vw, (size_t)H * r * d, "w_vw", false);
        upload(c, &c->w_b, w->w_b, (size_t)H * N * d, "w_b", false);
        upload(c, &c->w_c, w->w_c, (size_t)H * N * d, "w_c", false);
        {  // W_cat[s] = [W_kw[s]^T (r rows); W_B[s] (N rows); W_C[s] (N rows)], zeros where absent
            const size_t rows = (size_t)r + 2 * N;
            if (!c->w_cat) c->w_cat = (float *)dmalloc(c, (size_t)H * rows * d * sizeof(float));
            ADN_HIP(hipMemsetAsync(c->w_cat, 0, (size_t)H * rows * d * sizeof(float), c->stream));
            if (c->w_kw) {
                float *t2 = staging_f(c, 18, (size_t)H * r * d * sizeof(float));
                launch_transpose(c->w_kw, d, r, H, t2, c->stream);
                ADN_HIP(hipMemcpy2DAsync(c->w_cat, rows * d * sizeof(float), t2, (size_t)r * d * sizeof(float),
                                         (size_t)r * d * sizeof(float), H, hipMemcpyDeviceToDevice, c->stream));
            }
            if (c->w_b) {
                ADN_HIP(hipMemcpy2DAsync(c->w_cat + (size_t)r * d, rows * d * sizeof(float), c->w_b,
                                         (size_t)N * d * sizeof(float), (size_t)N * d * sizeof(float), H,
                                         hipMemcpyDeviceToDevice, c->stream));
                ADN_HIP(hipMemcpy2DAsync(c->w_cat + (size_t)(r + N) * d, rows * d * sizeof(float), c->w_c,
                                         (size_t)N * d * sizeof(float), (size_t)N * d * sizeof(float), H,
                                         hipMemcpyDeviceToDevice, c->stream));
            }
        }
        // split-precision copies of every GEMM weight (device-side, from the fp32 copies)
        const size_t nmat = (size_t)H * mat;
        make_split(c, c->sp_qkv, c->w_qkv, H, 3 * d, d,
                   host_maxabs({{w->w_q, nmat}, {w->w_k, nmat}, {w->w_v, nmat}}));
        make_split(c, c->sp_o, c->w_o, H, d, d, host_maxabs({{w->w_o, nmat}}));
        make_split(c, c->sp_in, c->w_in, H, d, d, host_maxabs({{w->w_in, nmat}}));
        if (c->w_out) make_split(c, c->sp_out, c->w_out, H, d, d, host_maxabs({{w->w_out, nmat}}), readout_eye(c));
        make_split(c, c->sp_cat, c->w_cat, H, r + 2 * N, d,
                   host_maxabs({{w->w_kw, (size_t)H * d * r}, {w->w_b, (size_t)H * N * d},
                                {w->w_c, (size_t)H * N * d}}));
        make_split(c, c->sp_lm, c->lm_w, 1, V, d, host_maxabs({{w->lm_w, (size_t)V * d}}));
        if (c->w_hist) make_split(c, c->sp_hist, c->w_hist, 1, d, d, host_maxabs({{w->w_hist, mat}}));
        {  // the fp16-split range guard's weight-derived bounds (see set_range)
            const float sq = std::sqrt((float)d);
            const float gmax = host_maxabs({{w->norm_scale, (size_t)d}});
            const float anmax = host_maxabs({{w->anchor, (size_t)H * d}});
            c->h_bound = gmax * (sq + ((cf.flags & ADN_F_RMS_EXCL_ANCHOR) ? 1e3f * anmax : 0.0f));
            c->l1_wv = max_row_l1(w->w_v, H, d, in_out);
            c->l1_wout = w->w_out ? max_row_l1(w->w_out, H, d, in_out) : 0.0f;
            const float lg = w->lm_g ? host_maxabs({{w->lm_g, (size_t)d}}) : 1.0f;
            c->lm_a_scale = std::min(1.0f, split_scale(c->prec, lg * sq));
        }
        // The signal GEMM's A operand (gathered embedding rows, or s_in rows of the same
        // scale) is scaled up too, with 6 bits of headroom: inputs up to 64x the table's
        // maximum magnitude stay inside the fp16 range.
        c->embed_scale = split_scale(c->prec, host_maxabs({{w->embed, (size_t)V * d}}), 10);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    } catch (const std::string &s) {
        return fail(ADN_E_INVALID, s);
    }
    c->has_weights = true;
    return ADN_OK;
}

int adn_reset_state(adn_ctx *c) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    // The carried carrier state is caller-owned (adn_run.scan_state_in); the context keeps no
    // state between calls besides the device error flag, which is cleared here.
    try {
        ADN_HIP(hipMemsetAsync(c->d_err, 0, sizeof(unsigned), c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_forward_async(adn_ctx *c, const adn_run *r, const adn_outputs *o) {
    int rc = check_run(c, r);
    if (rc) return rc;
    if (!o) return fail(ADN_E_INVALID, "null outputs");
    try {
        enqueue_run(c, *r, *o);
        ADN_HIP(hipGetLastError());
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_forward(adn_ctx *c, const adn_run *r, const adn_outputs *o) {
    int rc = check_run(c, r);
    if (rc) return rc;
    if (!o) return fail(ADN_E_INVALID, "null outputs");
    const long ntok = (long)r->batch * r->seq;
    const Dims &D = c->D;
    if (r->tokens) {
        for (long i = 0; i < ntok; ++i)
            if (r->tokens[i] < 0 || r->tokens[i] >= D.V)
                return fail(ADN_E_INVALID, "token id outside [0, vocab)");
    }
    try {
        adn_run dr = *r;
        if (r->tokens) {
            if (!c->tok_dev) c->tok_dev = (int32_t *)dmalloc(c, (size_t)c->cap_tok * sizeof(int32_t));
            ADN_HIP(hipMemcpyAsync(c->tok_dev, r->tokens, ntok * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
            dr.tokens = c->tok_dev;
        } else {
            float *sd = staging_f(c, 8, (size_t)ntok * D.d * sizeof(float));
            ADN_HIP(hipMemcpyAsync(sd, r->s_in, (size_t)ntok * D.d * sizeof(float), hipMemcpyHostToDevice, c->stream));
            dr.s_in = sd;
        }
        const size_t hsz = (size_t)ntok * D.H * D.d, stsz = (size_t)r->batch * D.H * D.d * D.N;
        if (r->scan_state_in) {
            float *si = staging_f(c, 9, stsz * sizeof(float));
            ADN_HIP(hipMemcpyAsync(si, r->scan_state_in, stsz * sizeof(float), hipMemcpyHostToDevice, c->stream));
            dr.scan_state_in = si;
        }
        adn_outputs dout{};
        if (o->h_star) dout.h_star = staging_f(c, 0, hsz * sizeof(float));
        if (o->pooled) dout.pooled = staging_f(c, 1, (size_t)ntok * D.d * sizeof(float));
        if (o->logits) dout.logits = staging_f(c, 2, (size_t)ntok * D.V * sizeof(float));
        if (o->argmax) dout.argmax = (int32_t *)staging_f(c, 3, (size_t)ntok * sizeof(int32_t));
        if (o->iters) dout.iters = (int32_t *)staging_f(c, 4, (size_t)ntok * sizeof(int32_t));
        if (o->scan_y) dout.scan_y = staging_f(c, 5, hsz * sizeof(float));
        if (o->scan_state) dout.scan_state = staging_f(c, 6, stsz * sizeof(float));
        if (o->converged) dout.converged = (int32_t *)staging_f(c, 7, (size_t)ntok * sizeof(int32_t));
        enqueue_run(c, dr, dout);
        ADN_HIP(hipGetLastError());
        auto d2h = [&](void *dst, const void *src, size_t bytes) {
            if (dst) ADN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
        };
        d2h(o->h_star, dout.h_star, hsz * sizeof(float));
        d2h(o->pooled, dout.pooled, (size_t)ntok * D.d * sizeof(float));
        d2h(o->logits, dout.logits, (size_t)ntok * D.V * sizeof(float));
        d2h(o->argmax, dout.argmax, (size_t)ntok * sizeof(int32_t));
        d2h(o->iters, dout.iters, (size_t)ntok * sizeof(int32_t));
        d2h(o->scan_y, dout.scan_y, hsz * sizeof(float));
        d2h(o->scan_state, dout.scan_state, stsz * sizeof(float));
        d2h(o->converged, dout.converged, (size_t)ntok * sizeof(int32_t));
        ADN_HIP(hipStreamSynchronize(c->stream));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

namespace {

// LmHead::sample's arguments beyond greedy; uniforms [batch][n_new] host memory
struct SampleCfg {
    float temperature, top_p;
    int top_k;
    const float *uniforms;
};

// Trainer::generate's loop; smp null = greedy (LmHead::sample at temperature <= 0)
int decode_run(adn_ctx *c, int32_t batch, int32_t prompt_len, const int32_t *prompt, int32_t n_new, int32_t ctx_len,
               int32_t max_iters, float eps, float damping, float repetition_penalty, const SampleCfg *smp,
               int32_t *out_tokens) {
    if (!c || !prompt || !out_tokens) return fail(ADN_E_INVALID, "null argument");
    if (!c->has_weights) return fail(ADN_E_NO_WEIGHTS, "decode before adn_upload_weights");
    if (batch < 1 || prompt_len < 1 || n_new < 0 || ctx_len < 1)
        return fail(ADN_E_INVALID, "batch, prompt_len and ctx_len must be >= 1, n_new >= 0");
    if (!(repetition_penalty > 0.0f) || !std::isfinite(repetition_penalty))
        return fail(ADN_E_INVALID, "repetition_penalty must be finite and > 0");
    const bool memory = (c->cfg.flags & ADN_F_MEMORY) != 0;
    if (memory && (c->cfg.flags & ADN_F_TOKEN_CARRY))
        return fail(ADN_E_INVALID, "the fixed-history decode solves every query from the init rule "
                                   "(solve_query_with_fixed_history); ADN_F_TOKEN_CARRY is not available here");
    if ((long)batch * (memory ? prompt_len : 1) > c->cap_tok)
        return fail(ADN_E_CAPACITY, memory ? "batch*prompt_len exceeds the context capacity"
                                           : "batch exceeds the context capacity");
    for (long i = 0; i < (long)batch * prompt_len; ++i)
        if (prompt[i] < 0 || prompt[i] >= c->D.V) return fail(ADN_E_INVALID, "token id outside [0, vocab)");
    adn_run r{};
    r.batch = batch;
    r.seq = 1;
    r.max_iters = max_iters;
    r.eps = eps;
    r.damping = damping;
    r.tokens = prompt;  // placeholder for the checks; the device inputs are set per step
    int rc = check_run(c, &r);
    if (rc) return rc;
    if (n_new == 0) return ADN_OK;
    // LmHead::sample applies the penalty only when |penalty - 1| > 1e-4 (lm_head.rs:81)
    const bool penalise = std::fabs(repetition_penalty - 1.0f) > 1e-4f;
    const Dims &D = c->D;
    const int stride = prompt_len + n_new;
    hipStream_t st = c->stream;
    try {
        int32_t *seq = (int32_t *)staging_f(c, 10, (size_t)batch * stride * sizeof(int32_t));
        int32_t *outd = (int32_t *)staging_f(c, 11, (size_t)batch * n_new * sizeof(int32_t));
        ADN_HIP(hipMemcpy2DAsync(seq, (size_t)stride * sizeof(int32_t), prompt, (size_t)prompt_len * sizeof(int32_t),
                                 (size_t)prompt_len * sizeof(int32_t), batch, hipMemcpyHostToDevice, st));
        // sampling reads the logits rows (and applies the penalty in its own workspace)
        const bool rows_out = penalise || smp;
        float *lg = rows_out ? staging_f(c, 24, (size_t)batch * D.V * sizeof(float)) : nullptr;
        int32_t *am = c->argmax_scratch;
        unsigned *sws = nullptr;
        float *uni = nullptr;
        if (smp) {
            sws = (unsigned *)staging_f(c, 31, sample_workspace_bytes(batch, D.V));
            uni = staging_f(c, 32, (size_t)batch * n_new * sizeof(float));
            ADN_HIP(hipMemcpyAsync(uni, smp->uniforms, (size_t)batch * n_new * sizeof(float), hipMemcpyHostToDevice,
                                   st));
        }
        float *q = nullptr, *m_cur = nullptr, *m_nxt = nullptr;
        int32_t *last = nullptr;
        if (memory) {
            // prime_fixed_history_state (trainer.rs:718-733): the memory after every prompt token
            const size_t msz = (size_t)batch * D.H * D.d;
            m_cur = staging_f(c, 25, msz * sizeof(float));
            m_nxt = staging_f(c, 26, msz * sizeof(float));
            last = (int32_t *)staging_f(c, 27, (size_t)batch * prompt_len * sizeof(int32_t));
            ADN_HIP(hipMemcpyAsync(last, prompt, (size_t)batch * prompt_len * sizeof(int32_t), hipMemcpyHostToDevice,
                                   st));
            adn_run rp = r;
            rp.seq = prompt_len;
            rp.tokens = last;
            adn_outputs op{};
            op.scan_state = m_cur;
            enqueue_forward_memory(c, rp, op);
        } else {
            q = staging_f(c, 28, (size_t)batch * D.d * sizeof(float));
            // the first step's range-guard reset; each step's arg-max kernel then does the next one's
            launch_reset_bounds(c->bounds, c->h_bound, c->absmax, st);
        }
        // The token is appended to seq and out by the arg-max kernel that picks it; on the
        // canonical path that kernel also resets the range guard's bounds and max |s_in| for the
        // next step, whose query kernel accumulates max |q|, so the step's forward launches neither
        // (the same values as launch_reset_bounds and launch_absmax).
        unsigned hb;
        std::memcpy(&hb, &c->h_bound, sizeof hb);
        for (int j = 0; j < n_new; ++j) {
            const int len = prompt_len + j;
            adn_outputs o{};
            if (rows_out)
                o.logits = lg;
            else
                o.argmax = am;
            TokenAppend app{seq, stride, len, outd, n_new, j, memory ? nullptr : c->bounds, hb,
                            memory ? nullptr : c->absmax};
            if (memory) {
                // query = embed(last context token) with the history of m (trainer.rs:4395-4400)
                launch_decode_last(seq, stride, len, last, batch, st);
                r.tokens = last;
                r.s_in = nullptr;
                r.scan_state_in = m_cur;
                o.scan_state = m_nxt;
                enqueue_forward_memory(c, r, o, nullptr, rows_out ? nullptr : &app);
                std::swap(m_cur, m_nxt);
            } else {
                // query = embed_context(context, ctx_len) (trainer.rs:4388-4392); the query
                // kernel also does the init where it is h0 = query + anchor
                const bool init_q = !(D.flags & ADN_F_INIT_SIGNAL_RMS);
                const SolveBuffers &sb = c->sb;
                const QueryInit qi{sb.h, c->anchor, D.H, sb.act[0], sb.iters, sb.cnt, sb.cnt_hist, sb.rprev, c->bounds};
                launch_decode_query(c->embed, D.d, seq, stride, len, ctx_len, batch, q, st,
                                    c->prec == PREC_F16X3 ? c->absmax : nullptr, init_q ? &qi : nullptr);
                r.tokens = nullptr;
                r.s_in = q;
                const DecodeStep ds{true, init_q, rows_out ? nullptr : &app};
                enqueue_forward(c, r, o, nullptr, &ds);
            }
            if (smp) {
                const SampleParams sp{seq, stride, len, nullptr, ctx_len, smp->temperature, smp->top_p,
                                      repetition_penalty, smp->top_k, uni + j, n_new, false};
                launch_sample(lg, batch, D.V, sws, sp, am, st, &app);
            } else if (penalise) {
                launch_rep_penalty(lg, D.V, seq, stride, len, ctx_len, repetition_penalty, batch, st);
                launch_argmax(lg, batch, D.V, am, st, &app);
            }
        }
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(out_tokens, outd, (size_t)batch * n_new * sizeof(int32_t), hipMemcpyDeviceToHost, st));
        ADN_HIP(hipStreamSynchronize(st));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

}  // namespace

int adn_decode_greedy(adn_ctx *c, int32_t batch, int32_t prompt_len, const int32_t *prompt, int32_t n_new,
                      int32_t ctx_len, int32_t max_iters, float eps, float damping, float repetition_penalty,
                      int32_t *out_tokens) {
    return decode_run(c, batch, prompt_len, prompt, n_new, ctx_len, max_iters, eps, damping, repetition_penalty,
                      nullptr, out_tokens);
}

// LmHead::sample's argument checks shared by the sampling entry points
static int check_sample_args(float temperature, float top_p, int32_t top_k, float repetition_penalty) {
    (void)temperature;
    (void)top_p;  // any value: outside (0, 1) (NaN included) there is no top-p cut, as in the reference
    if (top_k < 0) return fail(ADN_E_INVALID, "top_k must be >= 0 (0 = no top-k cut)");
    if (!(repetition_penalty > 0.0f) || !std::isfinite(repetition_penalty))
        return fail(ADN_E_INVALID, "repetition_penalty must be finite and > 0");
    return ADN_OK;
}

int adn_decode_sample(adn_ctx *c, int32_t batch, int32_t prompt_len, const int32_t *prompt, int32_t n_new,
                      int32_t ctx_len, int32_t max_iters, float eps, float damping, float temperature, float top_p,
                      int32_t top_k, float repetition_penalty, const float *uniforms, int32_t *out_tokens) {
    int rc = check_sample_args(temperature, top_p, top_k, repetition_penalty);
    if (rc) return rc;
    // lm_head.rs:104-111: a temperature <= 0 is the arg-max of the penalised logits
    if (!(temperature > 0.0f) && temperature <= 1e-4f)
        return decode_run(c, batch, prompt_len, prompt, n_new, ctx_len, max_iters, eps, damping, repetition_penalty,
                          nullptr, out_tokens);
    if (!uniforms && n_new > 0) return fail(ADN_E_INVALID, "null uniforms");
    if (c && c->D.V > SAMPLE_VMAX) return fail(ADN_E_INVALID, "sampling supports vocabularies up to 65536");
    const SampleCfg smp{temperature, top_p, top_k, uniforms};
    return decode_run(c, batch, prompt_len, prompt, n_new, ctx_len, max_iters, eps, damping, repetition_penalty, &smp,
                      out_tokens);
}

int adn_lm_sample(adn_ctx *c, int32_t rows, int32_t vocab, const float *logits, const int32_t *context,
                  int32_t ctx_stride, const int32_t *ctx_len, float temperature, float top_p, int32_t top_k,
                  float repetition_penalty, const float *uniforms, int32_t *tokens) {
    if (!c || !logits || !tokens || !uniforms) return fail(ADN_E_INVALID, "null argument");
    if (rows < 0 || vocab < 1 || vocab > SAMPLE_VMAX)
        return fail(ADN_E_INVALID, "rows must be >= 0 and vocab in [1, 65536]");
    if (ctx_stride < 0 || (ctx_stride > 0 && (!context || !ctx_len)))
        return fail(ADN_E_INVALID, "a context needs its tokens and lengths");
    int rc = check_sample_args(temperature, top_p, top_k, repetition_penalty);
    if (rc) return rc;
    for (int i = 0; ctx_stride > 0 && i < rows; ++i)
        if (ctx_len[i] < 0 || ctx_len[i] > ctx_stride) return fail(ADN_E_INVALID, "ctx_len outside [0, ctx_stride]");
    if (rows == 0) return ADN_OK;
    const bool greedy = !(temperature > 0.0f) && temperature <= 1e-4f;
    hipStream_t st = c->stream;
    try {
        const size_t n = (size_t)rows * vocab;
        float *lg = staging_f(c, 33, n * sizeof(float));
        int32_t *out = (int32_t *)staging_f(c, 34, (size_t)rows * sizeof(int32_t));
        const int cs = ctx_stride > 0 ? ctx_stride : 1;
        int32_t *ctx = (int32_t *)staging_f(c, 35, (size_t)rows * cs * sizeof(int32_t));
        int32_t *lens = (int32_t *)staging_f(c, 36, (size_t)rows * sizeof(int32_t));
        ADN_HIP(hipMemcpyAsync(lg, logits, n * sizeof(float), hipMemcpyHostToDevice, st));
        if (ctx_stride > 0) {
            ADN_HIP(hipMemcpyAsync(ctx, context, (size_t)rows * cs * sizeof(int32_t), hipMemcpyHostToDevice, st));
            ADN_HIP(hipMemcpyAsync(lens, ctx_len, (size_t)rows * sizeof(int32_t), hipMemcpyHostToDevice, st));
        } else {
            ADN_HIP(hipMemsetAsync(lens, 0, (size_t)rows * sizeof(int32_t), st));
        }
        unsigned *ws = (unsigned *)staging_f(c, 31, sample_workspace_bytes(rows, vocab));
        float *uni = staging_f(c, 32, (size_t)rows * sizeof(float));
        ADN_HIP(hipMemcpyAsync(uni, uniforms, (size_t)rows * sizeof(float), hipMemcpyHostToDevice, st));
        // lm_head.rs:104-111: a temperature <= 0 is the arg-max of the penalised row
        const SampleParams sp{ctx, cs, 0, lens, cs, temperature, top_p, repetition_penalty, top_k, uni, 1, greedy};
        launch_sample(lg, rows, vocab, ws, sp, out, st);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(tokens, out, (size_t)rows * sizeof(int32_t), hipMemcpyDeviceToHost, st));
        ADN_HIP(hipStreamSynchronize(st));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

int adn_spectral_norm(adn_ctx *c, const float *w, int32_t rows, int32_t cols, int32_t n_iter, float *sigma) {
    if (!c || !w || !sigma) return fail(ADN_E_INVALID, "null argument");
    if (rows < 0 || cols < 0 || n_iter < 0) return fail(ADN_E_INVALID, "negative size");
    if (rows == 0 || cols == 0) {
        *sigma = 1.0f;
        return ADN_OK;
    }
    try {
        const size_t n = (size_t)rows * cols;
        float *dw = staging_f(c, 12, n * sizeof(float));
        float *work = staging_f(c, 13, ((size_t)rows + 2 * cols + 1) * sizeof(float));
        ADN_HIP(hipMemcpyAsync(dw, w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
        float *ds = work + rows + 2 * cols;
        launch_spectral_norm(dw, rows, cols, n_iter, ds, work, c->stream);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(sigma, ds, sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_normalize_if_needed(adn_ctx *c, float *w, int32_t rows, int32_t cols, float threshold, int32_t n_iter) {
    if (!c || !w) return fail(ADN_E_INVALID, "null argument");
    if (rows < 0 || cols < 0 || n_iter < 0) return fail(ADN_E_INVALID, "negative size");
    if (rows == 0 || cols == 0) return ADN_OK;  // sigma = 1 (spectral_norm.rs:28-30)
    try {
        const size_t n = (size_t)rows * cols;
        float *dw = staging_f(c, 12, n * sizeof(float));
        float *work = staging_f(c, 13, ((size_t)rows + 2 * cols + 1) * sizeof(float));
        ADN_HIP(hipMemcpyAsync(dw, w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
        float *ds = work + rows + 2 * cols;
        launch_spectral_norm(dw, rows, cols, n_iter, ds, work, c->stream);
        launch_scale_if(dw, (long)n, ds, threshold, c->stream);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(w, dw, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_renormalize_spectral(adn_ctx *c, float attn_threshold, float win_threshold, float fpm_threshold,
                             float wv_threshold, float wo_threshold, int32_t n_iters, float *sigmas) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    if (!c->has_weights) return fail(ADN_E_NO_WEIGHTS, "renormalize_spectral before adn_upload_weights");
    if (n_iters < 1 || n_iters > 1000) return fail(ADN_E_INVALID, "n_iters must be in [1, 1000]");
    for (float t : {attn_threshold, win_threshold, fpm_threshold, wv_threshold, wo_threshold})
        if (!(t > 0.0f) || !std::isfinite(t)) return fail(ADN_E_INVALID, "thresholds must be finite and > 0");
    const int d = c->D.d, H = c->D.H;
    const size_t mat = (size_t)d * d;
    try {
        // jobs in the shader's matrix order per slot role: W_q, W_k (attention threshold), W_v, W_o,
        // W_in, W_x, W_out (the carrier's threshold); sigmas[role * H + s]
        std::vector<RenormJob> jobs;
        const bool win_t = (c->cfg.flags & ADN_F_WIN_TRANSPOSED) != 0;
        for (int s = 0; s < H; ++s) {
            float *qkv = c->w_qkv + (size_t)s * 3 * mat;
            jobs.push_back({qkv, RENORM_T, attn_threshold, 0 * H + s});
            jobs.push_back({qkv + mat, RENORM_T, attn_threshold, 1 * H + s});
            jobs.push_back({qkv + 2 * mat, RENORM_T, wv_threshold, 2 * H + s});
            jobs.push_back({c->w_o + (size_t)s * mat, RENORM_T, wo_threshold, 3 * H + s});
            // the reference's W_in buffer is the CPU matrix; the GEMM copy here holds it (or its
            // transpose under ADN_F_WIN_TRANSPOSED, whose product is W_in^T x)
            jobs.push_back({c->w_in + (size_t)s * mat, win_t ? RENORM_T : RENORM_N, win_threshold, 4 * H + s});
            jobs.push_back({c->wx_diag + (size_t)s * d, RENORM_DIAG, fpm_threshold, 5 * H + s});
            if (c->w_out) jobs.push_back({c->w_out + (size_t)s * mat, RENORM_T, fpm_threshold, 6 * H + s});
        }
        const int nj = (int)jobs.size();
        auto *djobs = (RenormJob *)staging_f(c, 29, jobs.size() * sizeof(RenormJob));
        float *dsig = staging_f(c, 30, (7 * (size_t)H + 8) * sizeof(float));
        unsigned *words = reinterpret_cast<unsigned *>(dsig + 7 * H);  // 4 absmax words
        ADN_HIP(hipMemsetAsync(dsig, 0, (7 * (size_t)H + 8) * sizeof(float), c->stream));
        ADN_HIP(hipMemcpyAsync(djobs, jobs.data(), jobs.size() * sizeof(RenormJob), hipMemcpyHostToDevice,
                               c->stream));
        launch_spectral_renorm(djobs, nj, d, n_iters, dsig, c->stream);
        // the split copies from the rescaled matrices, with scales from their new magnitudes
        launch_absmax(c->w_qkv, (long)(3 * H * mat), words + 0, c->stream);
        launch_absmax(c->w_o, (long)(H * mat), words + 1, c->stream);
        launch_absmax(c->w_in, (long)(H * mat), words + 2, c->stream);
        if (c->w_out) launch_absmax(c->w_out, (long)(H * mat), words + 3, c->stream);
        std::vector<float> hs(7 * (size_t)H + 8);
        ADN_HIP(hipMemcpyAsync(hs.data(), dsig, hs.size() * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
        float mx[4];
        std::memcpy(mx, hs.data() + 7 * H, sizeof(mx));
        make_split(c, c->sp_qkv, c->w_qkv, H, 3 * d, d, mx[0]);
        make_split(c, c->sp_o, c->w_o, H, d, d, mx[1]);
        make_split(c, c->sp_in, c->w_in, H, d, d, mx[2]);
        if (c->w_out) make_split(c, c->sp_out, c->w_out, H, d, d, mx[3], readout_eye(c));
        // row-L1 bounds of W_v and W_out (the range guard's): a slot scaled by f has f times its
        // rows' L1 norms, so the largest factor keeps the bound valid
        auto factor = [&](int role, float thr) {
            float f = 0.0f;
            for (int s = 0; s < H; ++s) {
                const float sg = hs[(size_t)role * H + s];
                f = std::max(f, sg > thr ? thr / sg : 1.0f);
            }
            return f;
        };
        c->l1_wv *= factor(2, wv_threshold);
        if (c->w_out) c->l1_wout *= factor(6, fpm_threshold);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipStreamSynchronize(c->stream));
        if (sigmas) {
            std::memcpy(sigmas, hs.data(), 7 * (size_t)H * sizeof(float));
            if (!c->w_out)
                for (int s = 0; s < H; ++s) sigmas[6 * H + s] = 0.0f;
        }
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_block_step(adn_ctx *c, int32_t d, const float *x, const float *dt, const float *a, const float *b,
                   const float *cc, float *y) {
    if (!c || !x || !dt || !a || !b || !cc || !y) return fail(ADN_E_INVALID, "null argument");
    if (d <= 0) return fail(ADN_E_INVALID, "d_model=0");
    try {
        float *buf = staging_f(c, 16, 6 * (size_t)d * sizeof(float));
        const float *src[5] = {x, dt, a, b, cc};
        for (int i = 0; i < 5; ++i)
            ADN_HIP(hipMemcpyAsync(buf + (size_t)i * d, src[i], d * sizeof(float), hipMemcpyHostToDevice, c->stream));
        launch_zoh(d, buf, buf + d, buf + 2 * (size_t)d, buf + 3 * (size_t)d, buf + 4 * (size_t)d,
                   buf + 5 * (size_t)d, c->stream);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(y, buf + 5 * (size_t)d, d * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_load_tensor(adn_ctx *c, const float *data, int64_t n, int32_t *id) {
    if (!c || !data || !id) return fail(ADN_E_INVALID, "null argument");
    if (n <= 0) return fail(ADN_E_INVALID, "empty tensor");
    try {
        DevBuf t;
        t.bytes = (size_t)n * sizeof(float);
        ADN_HIP(hipMalloc(&t.p, t.bytes));
        ADN_HIP(hipMemcpyAsync(t.p, data, t.bytes, hipMemcpyHostToDevice, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
        c->tensors.push_back(t);
        *id = (int32_t)c->tensors.size() - 1;
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_ffn_forward(adn_ctx *c, int32_t w_id, int32_t in_id, int32_t out_dim, float *y) {
    if (!c || !y) return fail(ADN_E_INVALID, "null argument");
    if (w_id < 0 || w_id >= (int)c->tensors.size() || in_id < 0 || in_id >= (int)c->tensors.size())
        return fail(ADN_E_INVALID, "unknown tensor id");
    if (out_dim <= 0) return fail(ADN_E_INVALID, "out_dim must be >= 1");
    const DevBuf &w = c->tensors[w_id];
    const DevBuf &x = c->tensors[in_id];
    const long in_dim = (long)(x.bytes / sizeof(float));
    if ((long)(w.bytes / sizeof(float)) != in_dim * out_dim)
        return fail(ADN_E_INVALID, "weight size != in_dim * out_dim");
    try {
        float *dy = staging_f(c, 17, (size_t)out_dim * sizeof(float));
        launch_gemv_colmajor((const float *)w.p, (const float *)x.p, (int)in_dim, out_dim, dy, c->stream);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(y, dy, out_dim * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

}  // extern "C"

namespace {

int check_embed_context(adn_ctx *c, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                        const float *out) {
    if (!c || !tokens || !out) return fail(ADN_E_INVALID, "null argument");
    if (!c->has_weights) return fail(ADN_E_NO_WEIGHTS, "embed_context before adn_upload_weights");
    if (batch < 1 || seq < 1) return fail(ADN_E_INVALID, "batch and seq must be >= 1");
    if ((long)batch * seq > c->cap_tok) return fail(ADN_E_CAPACITY, "batch*seq exceeds the context capacity");
    if (max_ctx < 1) return fail(ADN_E_INVALID, "max_ctx must be >= 1");
    return ADN_OK;
}

void enqueue_embed_context(adn_ctx *c, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                           float *out) {
    const long need = (long)batch * embed_context_chunks(seq) * c->D.d;
    if (need > c->ctx_tot_n) {  // grows to the largest request (the old block is freed with the context)
        c->ctx_tot = (double *)dmalloc(c, 2 * (size_t)need * sizeof(double));
        c->ctx_tot_n = need;
    }
    launch_embed_context(c->embed, c->D.d, c->D.V, tokens, batch, seq, max_ctx, c->ctx_tot, c->ctx_tot + need, out,
                         c->d_err, nullptr, c->stream);
}

}  // namespace

extern "C" {

int adn_embed_context_async(adn_ctx *c, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                            float *out) {
    int rc = check_embed_context(c, batch, seq, tokens, max_ctx, out);
    if (rc) return rc;
    try {
        enqueue_embed_context(c, batch, seq, tokens, max_ctx, out);
        ADN_HIP(hipGetLastError());
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_embed_context_noalloc(adn_ctx *c, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx,
                              float *out) {
    int rc = check_embed_context(c, batch, seq, tokens, max_ctx, out);
    if (rc) return rc;
    const long half = embed_context_total_doubles(c->D.d, batch, seq);
    if (2 * half > NOALLOC_MAX_DOUBLES)
        return fail(ADN_E_CAPACITY, "adn_embed_context_noalloc: 2 * batch * chunks * d_r exceeds the fixed "
                                    "buffer of 4194304 doubles");
    double *p = g_scratch_ptr[c->device];
    if (!p) return fail(ADN_E_HIP, "adn_embed_context_noalloc: no device buffer for this device");
    try {
        // every total the window kernel reads is written by the chunk kernel of this call first,
        // so the buffer needs no clearing
        launch_embed_context(c->embed, c->D.d, c->D.V, tokens, batch, seq, max_ctx, p, p + half, out, c->d_err,
                             reinterpret_cast<unsigned *>(p + NOALLOC_MAX_DOUBLES), c->stream);
        ADN_HIP(hipGetLastError());
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_noalloc_guard_set(adn_ctx *c, uint32_t calls_in_flight) {
    if (!c) return fail(ADN_E_INVALID, "null context");
    double *p = g_scratch_ptr[c->device];
    if (!p) return fail(ADN_E_HIP, "adn_noalloc_guard_set: no device buffer for this device");
    try {
        const uint32_t words[2] = {calls_in_flight, 0u};
        ADN_HIP(hipMemcpyAsync(p + NOALLOC_MAX_DOUBLES, words, sizeof(words), hipMemcpyHostToDevice, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_embed_context(adn_ctx *c, int32_t batch, int32_t seq, const int32_t *tokens, int32_t max_ctx, float *out) {
    int rc = check_embed_context(c, batch, seq, tokens, max_ctx, out);
    if (rc) return rc;
    const long n = (long)batch * seq;
    for (long i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c->D.V) return fail(ADN_E_INVALID, "token id outside [0, vocab)");
    try {
        if (!c->tok_dev) c->tok_dev = (int32_t *)dmalloc(c, (size_t)c->cap_tok * sizeof(int32_t));
        ADN_HIP(hipMemcpyAsync(c->tok_dev, tokens, n * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
        float *dout = staging_f(c, 19, (size_t)n * c->D.d * sizeof(float));
        enqueue_embed_context(c, batch, seq, c->tok_dev, max_ctx, dout);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipMemcpyAsync(out, dout, (size_t)n * c->D.d * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

}  // extern "C"

namespace {

int check_adjoint(adn_ctx *c, int32_t ntok, const float *dl, int32_t iters, float damping) {
    if (!c || !dl) return fail(ADN_E_INVALID, "null argument");
    if (!c->last_h || c->last_ntok < 1) return fail(ADN_E_INVALID, "adjoint before a forward on this context");
    if (ntok != c->last_ntok) return fail(ADN_E_INVALID, "ntok differs from the most recent forward's token count");
    if (iters < 0 || iters > ADN_PROFILE_MAX_ITERS) return fail(ADN_E_INVALID, "iters must be in [0, 256]");
    if (!(damping > 0.0f && damping <= 1.0f)) return fail(ADN_E_INVALID, "damping must be in (0, 1]");
    return ADN_OK;
}

void enqueue_adjoint(adn_ctx *c, int32_t ntok, const float *h_star, const float *dl, int32_t iters, float damping,
                     float *v_out, float *src) {
    const size_t n = (size_t)ntok * c->D.H * c->D.d;
    AdjointArgs a{};
    a.ntok = ntok;
    a.iters = iters;
    a.anderson_m = c->cfg.anderson_m;
    a.beta = damping;
    a.signal = c->sb.signal;
    a.h_star = h_star ? h_star : c->last_h;
    a.dl = dl;
    a.g = c->norm_scale;
    a.pre = c->sb.qkv;  // Q|K|V scratch is 3 * n floats: pre and the two iterates
    a.v0 = c->sb.qkv + n;
    a.v1 = c->sb.qkv + 2 * n;
    a.terms = c->sb.mix;
    a.src = src;
    a.v_out = v_out;
    a.sb = c->sb;
    a.act = c->sb.act[0];
    a.cnt = c->sb.cnt;
    const float *v = launch_adjoint(c->D, a, c->stream);
    if (v_out && v && v != v_out)
        ADN_HIP(hipMemcpyAsync(v_out, v, n * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
}

}  // namespace

extern "C" {

int adn_adjoint_async(adn_ctx *c, int32_t ntok, const float *h_star, const float *dl, int32_t iters, float damping,
                      float *v_out, float *src) {
    int rc = check_adjoint(c, ntok, dl, iters, damping);
    if (rc) return rc;
    try {
        enqueue_adjoint(c, ntok, h_star, dl, iters, damping, v_out, src);
        ADN_HIP(hipGetLastError());
    } catch (const HipError &e) {
        return hip_fail(e);
    }
    return ADN_OK;
}

int adn_adjoint(adn_ctx *c, int32_t ntok, const float *h_star, const float *dl, int32_t iters, float damping,
                float *v_out, float *src) {
    int rc = check_adjoint(c, ntok, dl, iters, damping);
    if (rc) return rc;
    try {
        const size_t hd = (size_t)c->D.H * c->D.d, d = c->D.d;
        const float *dh = nullptr;
        if (h_star) {
            float *t = staging_f(c, 20, (size_t)ntok * hd * sizeof(float));
            ADN_HIP(hipMemcpyAsync(t, h_star, (size_t)ntok * hd * sizeof(float), hipMemcpyHostToDevice, c->stream));
            dh = t;
        }
        float *ddl = staging_f(c, 21, (size_t)ntok * d * sizeof(float));
        ADN_HIP(hipMemcpyAsync(ddl, dl, (size_t)ntok * d * sizeof(float), hipMemcpyHostToDevice, c->stream));
        float *dv = v_out ? staging_f(c, 22, (size_t)ntok * hd * sizeof(float)) : nullptr;
        float *ds = src ? staging_f(c, 23, (size_t)ntok * d * sizeof(float)) : nullptr;
        enqueue_adjoint(c, ntok, dh, ddl, iters, damping, dv, ds);
        ADN_HIP(hipGetLastError());
        if (v_out) ADN_HIP(hipMemcpyAsync(v_out, dv, (size_t)ntok * hd * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        if (src) ADN_HIP(hipMemcpyAsync(src, ds, (size_t)ntok * d * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        ADN_HIP(hipStreamSynchronize(c->stream));
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

int adn_profile_forward(adn_ctx *c, const adn_run *r, const adn_outputs *o, adn_profile *prof) {
    int rc = check_run(c, r);
    if (rc) return rc;
    if (!o || !prof) return fail(ADN_E_INVALID, "null argument");
    try {
        Prof P;
        enqueue_run(c, *r, *o, &P);
        ADN_HIP(hipGetLastError());
        ADN_HIP(hipStreamSynchronize(c->stream));
        int32_t hist[ADN_PROFILE_MAX_ITERS] = {0};
        ADN_HIP(hipMemcpy(hist, c->sb.cnt_hist, r->max_iters * sizeof(int32_t), hipMemcpyDeviceToHost));
        memset(prof, 0, sizeof(*prof));
        prof->n_iters = r->max_iters;
        for (int k = 0; k < r->max_iters; ++k) prof->active[k] = hist[k];
        const double d = c->D.d, H = c->D.H, V = c->D.V, N = c->D.N, R = c->D.r;
        const double ntok = (double)r->batch * r->seq, REC = 1 + R + 2 * N, f = 4.0;
        const int m = c->cfg.anderson_m;
        // hist[k] sums the active tokens of iteration k over every launch of it (one per
        // position in memory mode): a launch's share is hist[k] / (launches of its stage at k)
        std::vector<int> per_k((size_t)ADN_STAGE_COUNT * ADN_PROFILE_MAX_ITERS, 0);
        for (const auto &rec : P.recs)
            if (rec.k >= 0 && rec.k < ADN_PROFILE_MAX_ITERS) ++per_k[(size_t)rec.stage * ADN_PROFILE_MAX_ITERS + rec.k];
        auto act = [&](int st, int k, int kk) {  // active tokens of launch (st, k) entering iteration kk
            const int cnt = per_k[(size_t)st * ADN_PROFILE_MAX_ITERS + k];
            return (kk < r->max_iters && cnt > 0) ? (double)hist[kk] / cnt : 0.0;
        };
        for (const auto &rec : P.recs) {
            float ms = 0.0f;
            ADN_HIP(hipEventElapsedTime(&ms, rec.e0, rec.e1));
            const int st = rec.stage;
            const bool per_iter = rec.k >= 0 && st >= ADN_STAGE_QKV_GEMM && st <= ADN_STAGE_CONVERGE;
            const double n = per_iter ? act(st, rec.k, rec.k) : (rec.n >= 0 ? rec.n : ntok);
            double fl = 0, by = 0;
            switch (st) {
                case ADN_STAGE_SIGNAL_GEMM: fl = 2 * ntok * H * d * d; by = f * (ntok * d + H * d * d + ntok * H * d); break;
                case ADN_STAGE_INIT: by = f * (ntok * d + ntok * H * d); break;
                case ADN_STAGE_QKV_GEMM:
                    fl = 6 * n * H * d * d;
                    by = n > 0 ? f * (n * H * d + 3 * H * d * d + 3 * n * H * d) : 0;
                    if (rec.fused & PROF_FUSED_UPDATE) {  // reads o, the signal and h_{k-1}; writes h_k
                        fl += 10 * n * H * d;
                        by += f * 3 * n * H * d;
                    }
                    break;
                case ADN_STAGE_ATTN: fl = 4 * n * H * H * d; by = f * 4 * n * H * d; break;
                case ADN_STAGE_WO_GEMM:
                    fl = 2 * n * H * d * d;
                    by = n > 0 ? f * (2 * n * H * d + H * d * d) : 0;
                    if (rec.fused & PROF_FUSED_ATTN) {  // A from the Q|K|V rows instead of the mix
                        fl += 4 * n * H * H * d;
                        by += f * 2 * n * H * d;
                    }
                    break;
                case ADN_STAGE_UPDATE:
                    fl = 10 * n * H * d;
                    by = f * (4 * n * H * d + 3 * n);
                    if (rec.fused & PROF_FUSED_POOL) {  // the pooled and normalised rows written
                        fl += n * H * d;
                        by += f * 2 * n * d;
                    }
                    if (rec.fused & PROF_FUSED_ANDERSON) {  // reads n_res ring slots instead of h, writes the slot too
                        const int k = rec.k, nr = k < m - 1 ? k : m - 1;
                        fl += n * H * d * (nr * (nr + 1) + 2 * nr);
                        by += f * (n * H * d * nr + 4 * n);
                    }
                    break;
                case ADN_STAGE_CONVERGE: by = f * (n * (rec.k >= 0 ? H + 3 : 1) + 2); break;
                case ADN_STAGE_ANDERSON: {
                    // the tokens continuing past iteration k; at the last one the tokens that entered
                    // it (those stopped at the cap are mixed; an upper bound)
                    const double nn = rec.k + 1 < r->max_iters ? act(st, rec.k, rec.k + 1) : act(st, rec.k, rec.k);
                    const int k = rec.k, n_res = k < m - 1 ? k : m - 1;
                    const double nr = (k >= 2 && n_res >= 2) ? n_res : 0;
                    fl = nn * H * d * (nr * (nr + 1) + 2 * nr);
                    by = f * nn * H * d * (2 + (nr > 0 ? 2 * nr + 2 : 0));
                    break;
                }
                case ADN_STAGE_POOL: fl = ntok * H * d; by = f * (ntok * H * d + 2 * ntok * d); break;
                case ADN_STAGE_LMHEAD_GEMM: fl = 2 * ntok * V * d; by = f * (ntok * d + V * d + ntok * V); break;
                case ADN_STAGE_ARGMAX:  // tile partials
                    by = f * (2 * ntok * std::ceil(V / gemm_lm_partial_cols(c->prec, (int)ntok, (int)d)) + ntok);
                    break;
                case ADN_STAGE_SCAN_PREP: fl = 2 * ntok * H * d * (R + 2 * N); by = f * (ntok * H * d + ntok * H * REC + H * d * (R + 2 * N)); break;
                case ADN_STAGE_SCAN:  // compulsory: read h*, the record; write y
                    fl = ntok * H * d * (2 * R + 4 * N + 10);
                    by = f * (ntok * H * d + ntok * H * REC + ntok * H * d); break;
                case ADN_STAGE_READOUT_GEMM: fl = 2 * n * H * d * d; by = f * (2 * n * H * d + H * d * d); break;
                case ADN_STAGE_HIST_GEMM: fl = 2 * n * H * d * d; by = f * (2 * n * H * d + d * d); break;
                case ADN_STAGE_HIST_CTX: fl = 9 * n * H * d; by = f * (4 * n * H * d + H * d + H); break;
                case ADN_STAGE_TEMPORAL: fl = 10 * n * H * d; by = f * (3 * n * H * d + 2 * H * d); break;
                default: break;
            }
            prof->ms[st] += ms;
            prof->flops[st] += fl;
            prof->bytes[st] += by;
            prof->launches[st] += 1;
        }
        if (!P.recs.empty()) {
            float tot = 0.0f;
            ADN_HIP(hipEventElapsedTime(&tot, P.recs.front().e0, P.recs.back().e1));
            prof->total_ms = tot;
        }
        return check_device_error(c);
    } catch (const HipError &e) {
        return hip_fail(e);
    }
}

}  // extern "C"

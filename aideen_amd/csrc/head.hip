// LM-head prologue (slot mean-pool + RMSNorm) and greedy arg-max.
//
// Reference: LmHead::{pool_h_star, rmsnorm, forward, argmax} (lm_head.rs:35-69);
// deq_forward_pool.wgsl:32-65 (pool).  The projection itself is the MFMA GEMM (gemm.hip).
#include "kernels.h"

namespace adn {

namespace {

constexpr int WPB = 4;

// pooled = fold(0, acc + h_s)/H (slot order kept); pnorm = (pooled/rms) * g, eps 1e-5.  One wave
// per token; each lane keeps its E = d/64 pooled values in registers between the two passes.
template <int E, bool PART>
__global__ __launch_bounds__(256) void k_pool_norm(Dims D, const float *h, int ntok, const float *g,
                                                   float *pooled, float *pnorm, float *rec, int REC, float pre) {
    const int t = blockIdx.x * WPB + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= ntok) return;
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const int H = D.H;
    const float *ht = h + (long)t * H * d;
    // slot by slot: the pooled sums add the slots in order; with `rec` each slot row's RMS
    // sqrt(mean h^2 + 1e-6) (the carrier's record, summed as k_row_rms does) is formed from the
    // same loads, lane s keeping slot s's, and stored after the loop
    float pv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) pv[e] = 0.0f;
    float my_rms = 0.0f;
    for (int s = 0; s < H; ++s) {
        float x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = (!PART || e < er) ? ht[(long)s * d + lane + 64 * e] : 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) pv[e] = pv[e] + x[e];
        if (rec) {
            float sr = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) sr += x[e] * x[e];
            sr = wave_sum(sr);
            const float rr = sqrtf(sr / (float)d + 1e-6f);
            if (lane == s) my_rms = rr;
        }
    }
    if (rec && lane < H) rec[((long)t * H + lane) * REC] = my_rms;
    pool_finish<E>(pv, H, d, er, lane, t, g, pooled, pnorm, pre);
}

// Arg-max of one logits row; ties go to the LAST maximal index, as Iterator::max_by does
// (lm_head.rs:62-69).  256 threads, strided scan, then a (value, index) tree reduction whose
// combine keeps the larger value and, on equal values, the larger index.
constexpr int AM_NT = 256;

__device__ __forceinline__ void am_combine(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 > i)) {
        v = v2;
        i = i2;
    }
}

// the chosen token of row `row` (see TokenAppend)
__device__ __forceinline__ void am_store(int32_t *out, int row, int tok, const TokenAppend &app) {
    out[row] = tok;
    if (app.seq) {
        app.seq[(long)row * app.stride + app.len] = tok;
        app.out[(long)row * app.n_new + app.j] = tok;
    }
    if (app.bounds && row == 0) {
        for (int i = 0; i < ADN_BOUNDS; ++i) app.bounds[i] = i == 0 ? app.bound0 : 0u;
        if (app.absmax) *app.absmax = 0u;
    }
}

__global__ __launch_bounds__(AM_NT) void k_argmax(const float *logits, int V, int32_t *out, TokenAppend app) {
    __shared__ float sv[AM_NT / 64];
    __shared__ int si[AM_NT / 64];
    const long row = blockIdx.x;
    const float *x = logits + row * (long)V;
    float bv = -INFINITY;
    int bi = -1;
    for (int v = threadIdx.x; v < V; v += AM_NT) {
        const float xv = x[v];
        if (!(xv < bv)) {  // keep later index on ties
            bv = xv;
            bi = v;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(bv, off, 64);
        const int i2 = __shfl_xor(bi, off, 64);
        am_combine(bv, bi, v2, i2);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sv[0];
        int i = si[0];
        for (int w = 1; w < AM_NT / 64; ++w) am_combine(v, i, sv[w], si[w]);
        am_store(out, (int)row, i < 0 ? 0 : i, app);
    }
}

// Reduce the LM-head tile partials of one row (one wave per row), same tie rule.
// A block takes 64 rows (one per lane: the [tile][row] partials are read coalesced) and its
// AR_W waves split the tiles; the waves' candidates are combined through LDS (the combination is
// a maximum with ties to the larger index, so its order does not change the result).
constexpr int AR_W = 16;

__global__ __launch_bounds__(64 * AR_W) void k_argmax_reduce(const float *am_val, const int32_t *am_idx,
                                                            int ntok, int ntiles, int32_t *out,
                                                            TokenAppend app) {
    // 32 rows per block: half-wave hw of wave w takes tiles 2w + hw, 2w + hw + 2 AR_W, ... (the
    // combination is a maximum with ties to the larger index, so its order does not matter), four
    // tiles' loads in flight at a time
    __shared__ float sv[2 * AR_W][32];
    __shared__ int si[2 * AR_W][32];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hw = lane >> 5, rl = lane & 31;
    const int row = blockIdx.x * 32 + rl;
    const int q0 = 2 * w + hw;
    constexpr int QS = 2 * AR_W;
    float bv = -INFINITY;
    int bi = -1;
    if (row < ntok) {
        int t = q0;
        for (; t + 3 * QS < ntiles; t += 4 * QS) {
            float v[4];
            int ix[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v[u] = am_val[(long)(t + u * QS) * ntok + row];
                ix[u] = am_idx[(long)(t + u * QS) * ntok + row];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) am_combine(bv, bi, v[u], ix[u]);
        }
        for (; t < ntiles; t += QS) am_combine(bv, bi, am_val[(long)t * ntok + row], am_idx[(long)t * ntok + row]);
    }
    sv[q0][rl] = bv;
    si[q0][rl] = bi;
    __syncthreads();
    if (threadIdx.x < 32 && row < ntok) {
        for (int q = 1; q < QS; ++q) am_combine(bv, bi, sv[q][rl], si[q][rl]);
        am_store(out, row, bi < 0 ? 0 : bi, app);
    }
}

// The same reduction for a few rows (a decode step): one block per row, its threads over the
// row's tiles (a block of 32 rows would leave 31 of every 32 lanes idle and walk the tiles in
// dependent rounds), the candidates combined by wave shuffles and then across the waves.
constexpr int ARR_NT = 256;
__global__ __launch_bounds__(ARR_NT) void k_argmax_reduce_rows(const float *am_val, const int32_t *am_idx,
                                                             int ntok, int ntiles, int32_t *out,
                                                             TokenAppend app) {
    __shared__ float sv[ARR_NT / 64];
    __shared__ int si[ARR_NT / 64];
    const int row = blockIdx.x;
    float bv = -INFINITY;
    int bi = -1;
    for (int t = threadIdx.x; t < ntiles; t += ARR_NT)
        am_combine(bv, bi, am_val[(long)t * ntok + row], am_idx[(long)t * ntok + row]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        am_combine(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < ARR_NT / 64; ++w) am_combine(bv, bi, sv[w], si[w]);
        am_store(out, row, bi < 0 ? 0 : bi, app);
    }
}

// ---------------------------------------------------------------------------------------
// Greedy decode (Trainer::generate, trainer.rs:4219-4431).  seq [B][stride] holds each
// sequence's tokens so far (the prompt, then the appended arg-maxes); step j works on the first
// len = T0 + j of them, its context being the last ctx of those (trainer.rs:4248-4249).
// ---------------------------------------------------------------------------------------
// The context query embed_context(context, ctx) (tokenizer.rs:133-149) of every sequence, one
// block per sequence: v = sum_{p < L} (p + 1) E[tok_p] over the window in fp64, q = v / |v| --
// r = v / L itself when |r| <= 1e-6, as embed_context keeps a near-zero sum unnormalised.  The
// same quantity as k_ctx_window's at the last position, formed directly for one window per
// sequence.  Wave w sums the positions p = w mod W over whole rows (lane l holds columns
// l + 64 e, so each load is 256 contiguous bytes), four rows in flight; the W partial rows are
// then added in wave order (deterministic).  W waves x the padded row in fp64 stay within 64 KB
// of LDS: W = 16 up to d = 512, 8 at 1024, 4 at 2048.
constexpr int dq_waves(int E) { return E <= 8 ? 16 : (E <= 16 ? 8 : 4); }

template <int E, bool PART>
__global__ __launch_bounds__(64 * dq_waves(E)) void k_decode_query(const float *Emb, int d, const int32_t *seq,
                                                                   int stride, int len, int ctx, float *q,
                                                                   unsigned *absmax, QueryInit qi) {
    constexpr int W = dq_waves(E);
    __shared__ double part[W][64 * E];
    __shared__ double red[W];
    const int b = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int er = PART ? d / 64 : E;
    const int start = len > ctx ? len - ctx : 0, L = len - start;
    const int32_t *tk = seq + (long)b * stride + start;
    double acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0;
    int p = wave;
    for (; p + 3 * W < L; p += 4 * W) {
        float x[4][E];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float *row = Emb + (long)tk[p + u * W] * d + lane;
#pragma unroll
            for (int e = 0; e < E; ++e) x[u][e] = e < er ? row[64 * e] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] += (double)(p + u * W + 1) * (double)x[u][e];
    }
    for (; p < L; p += W) {
        const float *row = Emb + (long)tk[p] * d + lane;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (e < er) acc[e] += (double)(p + 1) * (double)row[64 * e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e) part[wave][lane + 64 * e] = acc[e];
    __syncthreads();
    // column sums in wave order, then |v|^2
    double ss = 0.0;
    for (int j = threadIdx.x; j < d; j += 64 * W) {
        double v = 0.0;
#pragma unroll
        for (int w = 0; w < W; ++w) v += part[w][j];
        part[0][j] = v;  // column j is read and written by this thread only
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double n2 = 0.0;
#pragma unroll
    for (int w = 0; w < W; ++w) n2 += red[w];
    const double nv = sqrt(n2);
    const double inv = 1.0 / (nv > 1e-6 * (double)L ? nv : (double)L);
    unsigned mb = 0;  // largest finite |q| of this lane, as float bits
    float hmax = 0.0f;  // largest finite |h0| of this lane
    for (int j = threadIdx.x; j < d; j += 64 * W) {
        const float v = (float)(part[0][j] * inv);
        q[(long)b * d + j] = v;
        const float a = fabsf(v);
        if (a < INFINITY) mb = max(mb, __float_as_uint(a));
        if (qi.h) {  // h0 = x + anchor, as k_init forms it
            for (int s = 0; s < qi.H; ++s) {
                const float hv = v + qi.anchor[(long)s * d + j];
                qi.h[((long)b * qi.H + s) * d + j] = hv;
                hmax = fmaxf(hmax, fabsf(hv) < INFINITY ? fabsf(hv) : 0.0f);
            }
        }
    }
    if (absmax) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mb = max(mb, (unsigned)__shfl_xor((int)mb, off, 64));
        if (lane == 0 && mb) atomicMax(absmax, mb);
    }
    if (qi.h) {
        if (qi.amax_h) track_absmax(qi.amax_h, hmax);
        if (threadIdx.x == 0) {
            qi.act0[b] = b;
            qi.iters[b] = 0;
            if (qi.rprev) qi.rprev[b] = 1.0f;
        }
        if (b == 0) {
            if (threadIdx.x == 0) {
                qi.cnt[0] = (int)gridDim.x;
                qi.cnt[1] = 0;
            }
            for (int k = threadIdx.x; k < ADN_PROFILE_MAX_ITERS; k += 64 * W) qi.cnt_hist[k] = 0;
        }
    }
}

// LmHead::sample's repetition penalty (lm_head.rs:81-99) on each sequence's logits row: every
// distinct token of the context (the thread holding its first occurrence) has its logit
// multiplied by pen when negative, divided by it otherwise.
__global__ __launch_bounds__(256) void k_rep_penalty(float *logits, int V, const int32_t *seq, int stride, int len,
                                                     int ctx, float pen) {
    const int b = blockIdx.x;
    const int start = len > ctx ? len - ctx : 0, L = len - start;
    const int32_t *tk = seq + (long)b * stride + start;
    float *lg = logits + (long)b * V;
    for (int p = threadIdx.x; p < L; p += blockDim.x) {
        const int tok = tk[p];
        bool seen = false;
        for (int u = 0; u < p && !seen; ++u) seen = tk[u] == tok;
        if (seen || tok < 0 || tok >= V) continue;
        const float sc = lg[tok];
        lg[tok] = sc < 0.0f ? sc * pen : sc / pen;
    }
}

// last[b] = seq[b][len - 1]
__global__ void k_decode_last(const int32_t *seq, int stride, int len, int32_t *last, int B) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) last[b] = seq[(long)b * stride + len - 1];
}

// ---- LmHead::sample (lm_head.rs:78-168) ------------------------------------------------------
// The per-element work runs over many workgroups per row (SP_EPB elements each), through a
// workspace row ws[V]: k_samp_scale writes the penalised and scaled logits and each block's
// maximum; k_samp_exp writes e = exp(l - max) and each block's sum; k_samp_keys writes the bit
// pattern ("key") of p = e / S and each block's histogram of count and weight over SP_NBIN bins
// of key below the largest (bins of 2^sh keys: the narrowest power of two, at most 1/128 octave,
// at which the bins span the row's positive probabilities; a flat row gets fine bins).  p lies in [0, 1] (the maximum contributes exp(0) = 1 to S),
// so keys order as p does, and the reference's sorted list (p descending by a stable sort: ties
// keep index order) is the order "key descending, index ascending".  A probability weighs
// floor(p * 2^60) in exact integer sums (the sum over a row stays below 2^61).
//
// k_sample (one workgroup per row) takes the cut points of the list (the top_k-th item, the
// first item past which the running sum exceeds top_p, the item at which it reaches the draw)
// without sorting the row: the row's bin histogram names the bin of the crossing, passes counting
// the items inside it above eight thresholds (in registers) narrow it further where it holds more
// than SP_CAP items, and an interval of at most SP_CAP items is gathered, sorted in LDS and
// scanned.  When the kept list has at most SP_CAP items (top_k <=
// SP_CAP, or a top_p cut within that many items, or a vocabulary that small) it is gathered,
// sorted, and one thread runs the reference's loops on it in float arithmetic; otherwise the cuts
// are taken on the exact sums.
constexpr int SP_NT = 1024;          // k_sample's threads
constexpr int SP_CAP = 2048;         // lists sorted in LDS
constexpr int SP_PT = 256;           // threads of the per-element kernels
constexpr int SP_EPB = SP_PT * 8;    // elements per block of the per-element kernels
constexpr int SP_NBIN = 1024;        // bins of p below the largest (the last takes all below): a bin
constexpr int SP_BSH = 16;           // spans 2^sh key values, sh <= SP_BSH (1/128 octave) chosen so
                                     // that the bins span the row's keys where they fit
static_assert(SP_NBIN == SP_NT, "k_sample's thread t takes bin t");
typedef unsigned long long u64;

struct SampleSmem {
    unsigned hc[SP_NT];  // sub-interval bins / wave partials
    u64 hm[SP_NT];
    u64 list[SP_CAP];  // (~key << 32) | index: ascending = key descending, index ascending
    unsigned oc[SP_NBIN];  // the row's bins (sums of the blocks' histograms)
    u64 om[SP_NBIN];
    u64 wc[SP_NT / 64], wm[SP_NT / 64];
    float wf[SP_NT / 64];
    int wi[SP_NT / 64];
    float wf2[SP_NT];  // the blocks' partial sums
    u64 bc, bm, bn;
    unsigned boff[SAMPLE_VMAX / SP_EPB + 1];  // the blocks' offsets in a gathered prefix
    unsigned cnt, blo, bhi;
    int tok, need_exact, bsel;
};

struct SpCut {  // keeps the items up to and including (key, idx) in the list order; `on` false keeps all
    bool on;
    unsigned key;
    int idx;
};

struct SpSel {  // an item and the count and weight of the list up to and including it
    unsigned key;
    int idx;
    u64 cnt, mass;
    bool found;
};

// f(i, value, u) over this thread's elements i = tid + u * SP_NT of ws, in index order, the
// loads of each batch of 8 issued together; every lane takes every step (value 0 for i >= V,
// which f must skip), so f may use wave-wide operations
template <int KPT, typename F>
__device__ __forceinline__ void sp_each(const unsigned *ws, int V, F &&f) {
    constexpr int BT = KPT < 8 ? KPT : 8;
#pragma unroll 1
    for (int b0 = 0; b0 < KPT; b0 += BT) {
        unsigned kb[BT];
#pragma unroll
        for (int v = 0; v < BT; ++v) {
            const int i = threadIdx.x + (b0 + v) * SP_NT;
            kb[v] = i < V ? ws[i] : 0u;
        }
#pragma unroll
        for (int v = 0; v < BT; ++v) f(threadIdx.x + (b0 + v) * SP_NT, kb[v], b0 + v);
    }
}

// Gather of the elements pred(i, k) selects into sm.list as (~key << 32) | index, in index order of
// threads (the caller sorts): a count pass, a block scan of the counts, a write pass.  At most
// SP_CAP are written; returns how many there are.
template <int KPT, typename P>
__device__ unsigned sp_gather(const unsigned *ws, int V, P &&pred, struct SampleSmem &sm);

// floor(p * 2^60) from p's bit pattern: p = m 2^(max(e, 1) - 150)
__device__ __forceinline__ u64 sp_mass(unsigned k) {
    const int e = (int)(k >> 23);
    const u64 m = (k & 0x7fffffu) | (e ? 0x800000u : 0u);
    const int sh = (e ? e : 1) - 90;
    return sh >= 0 ? (m << sh) : (sh > -64 ? (m >> -sh) : 0ull);
}

__device__ __forceinline__ bool sp_in(const SpCut &c, unsigned k, int i) {
    return !c.on || k > c.key || (k == c.key && i <= c.idx);
}

// the bin of key k below the largest key khi (k <= khi)
__device__ __forceinline__ int sp_bin(unsigned khi, unsigned k, int sh) { return min(SP_NBIN - 1, (int)((khi - k) >> sh)); }

// the bin width for keys from kmin to khi: the narrowest power of two at which SP_NBIN bins span
// them, at most 2^SP_BSH
__device__ __forceinline__ int sp_bin_shift(unsigned khi, unsigned kmin) {
    const unsigned span = khi - kmin;  // the bins must hold span + 1 key values
    int sh = 0;
    while (sh < SP_BSH && (span >> sh) >= (unsigned)SP_NBIN) ++sh;
    return sh;
}

template <int NT>
__device__ float sp_bmax(float v, float *red) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
    for (int u = 1; u < NT / 64; ++u) v = fmaxf(v, red[u]);
    __syncthreads();
    return v;
}

// the block's sum in a fixed order (wave butterflies, then the waves in order)
template <int NT>
__device__ float sp_bsum(float v, float *red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
    for (int u = 1; u < NT / 64; ++u) v += red[u];
    __syncthreads();
    return v;
}

// inclusive scan of (c, m) over the threads in thread order
__device__ void sp_scan(u64 &c, u64 &m, SampleSmem &sm) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int off = 1; off < 64; off <<= 1) {
        const u64 c2 = __shfl_up(c, off, 64), m2 = __shfl_up(m, off, 64);
        if (lane >= off) {
            c += c2;
            m += m2;
        }
    }
    if (lane == 63) {
        sm.wc[w] = c;
        sm.wm[w] = m;
    }
    __syncthreads();
    u64 pc = 0, pm = 0;
    for (int u = 0; u < w; ++u) {
        pc += sm.wc[u];
        pm += sm.wm[u];
    }
    c += pc;
    m += pm;
    __syncthreads();
}

// 1. the repetition penalty (lm_head.rs:81-99: the context's distinct tokens, here a bit set of
// the block's range), 2. the temperature (:103-111; none with `greedy`), the block's maximum as
// f32::max folds it (NaN skipped); the row's bin histogram cleared
__global__ __launch_bounds__(SP_PT) void k_samp_scale(const float *logits, int V, float *w, float *pmax,
                                                      unsigned *gc, u64 *gm, SampleParams a) {
    __shared__ unsigned bits[SP_EPB / 32];
    __shared__ float red[SP_PT / 64];
    const int NB = gridDim.x, b = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    // the row's bin histogram starts at zero (k_samp_keys adds to it)
    for (int q = b * SP_PT + tid; q < SP_NBIN; q += NB * SP_PT) {
        gc[(long)row * SP_NBIN + q] = 0u;
        gm[(long)row * SP_NBIN + q] = 0ull;
    }
    const int i0 = b * SP_EPB;
    const float *lg = logits + (long)row * V;
    float *wr = w + (long)row * V;
    const int len = a.lens ? a.lens[row] : a.len;
    const int start = len > a.window ? len - a.window : 0, L = len - start;
    const bool pen = fabsf(a.penalty - 1.0f) > 1e-4f && L > 0;
    if (pen) {
        for (int q = tid; q < SP_EPB / 32; q += SP_PT) bits[q] = 0u;
        __syncthreads();
        const int32_t *tk = a.seq + (long)row * a.stride + start;
        for (int p = tid; p < L; p += SP_PT) {
            const int t = tk[p] - i0;
            if (t >= 0 && t < SP_EPB && t + i0 < V) atomicOr(&bits[t >> 5], 1u << (t & 31));
        }
        __syncthreads();
    }
    const float Tm = a.temperature;
    const bool scale = !a.greedy && Tm > 0.0f && fabsf(Tm - 1.0f) > 1e-4f;
    float v[SP_EPB / SP_PT];
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        v[e] = i < V ? lg[i] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int o = tid + e * SP_PT, i = i0 + o;
        if (i < V) {
            float x = v[e];
            if (pen && ((bits[o >> 5] >> (o & 31)) & 1u)) x = x < 0.0f ? x * a.penalty : x / a.penalty;
            if (scale) x = x / Tm;
            wr[i] = x;
            mx = fmaxf(mx, x);
        }
    }
    mx = sp_bmax<SP_PT>(mx, red);
    if (tid == 0) pmax[(long)row * NB + b] = mx;
}

// e = exp(l - max), the block's sum (softmax, lm_head.rs:71-76) and its smallest positive e
__global__ __launch_bounds__(SP_PT) void k_samp_exp(int V, float *w, const float *pmax, float *psum, float *pmin) {
    __shared__ float red[SP_PT / 64];
    __shared__ float part[SP_PT];
    const int NB = gridDim.x, b = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int i0 = b * SP_EPB;
    float *wr = w + (long)row * V;
    for (int q = tid; q < NB; q += SP_PT) part[q] = pmax[(long)row * NB + q];
    __syncthreads();
    float mx = -INFINITY;
    for (int q = 0; q < NB; ++q) mx = fmaxf(mx, part[q]);
    float v[SP_EPB / SP_PT];
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        v[e] = i < V ? wr[i] : 0.0f;
    }
    float s = 0.0f, mn = INFINITY;
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        if (i < V) {
            const float x = expf(v[e] - mx);
            wr[i] = x;
            s += x;
            if (x > 0.0f) mn = fminf(mn, x);
        }
    }
    s = sp_bsum<SP_PT>(s, red);
    mn = -sp_bmax<SP_PT>(-mn, red);
    if (tid == 0) {
        psum[(long)row * NB + b] = s;
        pmin[(long)row * NB + b] = mn;
    }
}

// S = the blocks' sums in block order; the keys, and their histogram by bin added into the row's
// (integer sums: their order does not matter)
__global__ __launch_bounds__(SP_PT) void k_samp_keys(int V, unsigned *w, const float *psum, const float *pmin,
                                                     unsigned *gc, u64 *gm, u64 *bucket, unsigned *bcum) {
    __shared__ unsigned c[SP_NBIN];
    __shared__ u64 m[SP_NBIN];
    __shared__ unsigned cur[SP_NBIN];
    __shared__ unsigned wsum[SP_PT / 64];
    __shared__ float part[SP_PT], partm[SP_PT];
    const int NB = gridDim.x, b = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int i0 = b * SP_EPB;
    unsigned *wr = w + (long)row * V;
    for (int q = tid; q < NB; q += SP_PT) {
        part[q] = psum[(long)row * NB + q];
        partm[q] = pmin[(long)row * NB + q];
    }
    __syncthreads();
    float S = 0.0f, emin = INFINITY;
    for (int q = 0; q < NB; ++q) {
        S += part[q];
        emin = fminf(emin, partm[q]);
    }
    if (!(S == S)) return;  // k_sample takes the arg-max of the row as given
    const unsigned khi = __float_as_uint(1.0f / S);
    const int sh = sp_bin_shift(khi, __float_as_uint(emin / S));
    for (int q = tid; q < SP_NBIN; q += SP_PT) {
        c[q] = 0u;
        m[q] = 0ull;
    }
    __syncthreads();
    unsigned v[SP_EPB / SP_PT];
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        v[e] = i < V ? wr[i] : 0u;
    }
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        if (i < V) {
            const unsigned k = __float_as_uint(__uint_as_float(v[e]) / S);
            wr[i] = k;
            const int d = sp_bin(khi, k, sh);
            atomicAdd(&c[d], 1u);
            atomicAdd(&m[d], sp_mass(k));
        }
    }
    __syncthreads();
    for (int q = tid; q < SP_NBIN; q += SP_PT)
        if (c[q]) {
            atomicAdd(&gc[(long)row * SP_NBIN + q], c[q]);
            atomicAdd(&gm[(long)row * SP_NBIN + q], m[q]);
        }
    // the block's items bucketed by bin (bin 0, the largest keys, first) as (~key << 32) | index,
    // and the running count through each bin: the items of bins 0..d are the first bcum[d]
    constexpr int BPT = SP_NBIN / SP_PT;  // bins per thread
    unsigned run = 0;
#pragma unroll
    for (int x = 0; x < BPT; ++x) run += c[tid * BPT + x];
    unsigned inc = run;  // inclusive scan over the threads
    const int lane = tid & 63, wv = tid >> 6;
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned o = __shfl_up(inc, off, 64);
        if (lane >= off) inc += o;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    for (int x = 0; x < wv; ++x) inc += wsum[x];
    unsigned st = inc - run;
    const long hb = ((long)row * NB + b) * SP_NBIN;
#pragma unroll
    for (int x = 0; x < BPT; ++x) {
        const int q = tid * BPT + x;
        cur[q] = st;
        st += c[q];
        bcum[hb + q] = st;
    }
    __syncthreads();
    u64 *bk = bucket + ((long)row * NB + b) * SP_EPB;
#pragma unroll
    for (int e = 0; e < SP_EPB / SP_PT; ++e) {
        const int i = i0 + tid + e * SP_PT;
        if (i < V) {
            const unsigned k = __float_as_uint(__uint_as_float(v[e]) / S);
            const unsigned slot = atomicAdd(&cur[sp_bin(khi, k, sh)], 1u);
            bk[slot] = ((u64)(~k) << 32) | (unsigned)i;
        }
    }
}

// The first item of the list that `cut` keeps at which the running count (by_mass false) or the
// running weight (true) exceeds T.  Not found: cnt and mass are the kept list's totals.  The
// row's bin histogram (sm.oc, sm.om) names the bin of the crossing (with a cut, the cut item's bin
// is recounted and the bins below it are empty); passes that count and weigh the interval's items
// above eight thresholds narrow it until it holds at most SP_CAP items, which are gathered, sorted
// and scanned; one key value held by more (equal probabilities) is searched in index order.
template <int KPT>
__device__ __noinline__ SpSel sp_select(const unsigned *ws, int V, bool by_mass, u64 T, const SpCut &cut, unsigned khi,
                                        int bsh, SampleSmem &sm) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int dcut = cut.on ? sp_bin(khi, cut.key, bsh) : SP_NBIN - 1;
    u64 cp = 0, mp = 0;  // the kept items of the cut item's bin
    if (cut.on) {
        sp_each<KPT>(ws, V, [&](int i, unsigned k, int) {
            if (i < V && sp_bin(khi, k, bsh) == dcut && sp_in(cut, k, i)) {
                cp += 1;
                mp += sp_mass(k);
            }
        });
        sp_scan(cp, mp, sm);
        if (tid == SP_NT - 1) {
            sm.bc = cp;
            sm.bm = mp;
        }
        __syncthreads();
        cp = sm.bc;
        mp = sm.bm;
        __syncthreads();
    }
    // bin tid (SP_NT == SP_NBIN) as the cut keeps it; the running sums over the bins in order
    const u64 cd = tid < dcut ? sm.oc[tid] : (tid == dcut ? (cut.on ? cp : sm.oc[tid]) : 0ull);
    const u64 md = tid < dcut ? sm.om[tid] : (tid == dcut ? (cut.on ? mp : sm.om[tid]) : 0ull);
    u64 ic = cd, im = md;
    sp_scan(ic, im, sm);
    const int dd0 = __syncthreads_count(!((by_mass ? im : ic) > T));  // the bins before the crossing
    if (dd0 == SP_NBIN && tid == SP_NT - 1) {  // no crossing: the totals
        sm.bc = ic;
        sm.bm = im;
    }
    if (dd0 < SP_NBIN && tid == dd0) {
        sm.bc = ic - cd;
        sm.bm = im - md;
        sm.bn = cd;
        // bin dd0: keys in [khi + 1 - (dd0 + 1) 2^bsh, khi + 1 - dd0 2^bsh) (the last bin down to 0)
        const u64 top = (u64)khi + 1;
        const u64 lo = dd0 == SP_NBIN - 1 ? 0 : (top > ((u64)(dd0 + 1) << bsh) ? top - ((u64)(dd0 + 1) << bsh) : 0);
        sm.blo = (unsigned)lo;
        sm.bhi = (unsigned)(top - ((u64)dd0 << bsh));
    }
    __syncthreads();
    const int dd = dd0 < SP_NBIN ? dd0 : -1;
    u64 cb = sm.bc, mb = sm.bm, n_int = sm.bn;
    unsigned lo = sm.blo, hi = sm.bhi;
    __syncthreads();
    if (dd < 0) return SpSel{0u, -1, cb, mb, false};
    if (n_int > (u64)SP_CAP) {
        // the interval narrowed to its smallest and largest key (a tie holding most of the row
        // then needs no narrowing passes)
        unsigned kmn = 0xffffffffu, kmx = 0u;
        sp_each<KPT>(ws, V, [&](int i, unsigned k, int) {
            if (i < V && k >= lo && k < hi && sp_in(cut, k, i)) {
                kmn = min(kmn, k);
                kmx = max(kmx, k);
            }
        });
        if (tid == 0) {
            sm.blo = 0xffffffffu;
            sm.bhi = 0u;
        }
        __syncthreads();
        atomicMin(&sm.blo, kmn);
        atomicMax(&sm.bhi, kmx);
        __syncthreads();
        lo = sm.blo;
        hi = sm.bhi + 1u;
        __syncthreads();
    }
    for (int pass = 0; pass < 12 && n_int > (u64)SP_CAP && hi - lo > 1u; ++pass) {
        // eight thresholds over [lo, hi): each thread counts and weighs its items above them in
        // registers (no atomics: a crowded interval holds tens of thousands of items)
        const unsigned wd = hi - lo;
        unsigned t[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) t[q] = lo + (unsigned)(((u64)wd * (unsigned)q) >> 3);
        unsigned c8[8];
        u64 m8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            c8[q] = 0u;
            m8[q] = 0ull;
        }
        sp_each<KPT>(ws, V, [&](int i, unsigned k, int) {
            if (i < V && k >= lo && k < hi && sp_in(cut, k, i)) {
                const u64 mk = sp_mass(k);
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (k >= t[q]) {
                        c8[q] += 1u;
                        m8[q] += mk;
                    }
            }
        });
        // block totals: wave butterflies, the waves' partials through LDS, summed by one thread
#pragma unroll
        for (int q = 0; q < 8; ++q)
            for (int off = 32; off > 0; off >>= 1) {
                c8[q] += __shfl_xor(c8[q], off, 64);
                m8[q] += __shfl_xor(m8[q], off, 64);
            }
        if (lane == 0)
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                sm.hc[w * 8 + q] = c8[q];
                sm.hm[w * 8 + q] = m8[q];
            }
        __syncthreads();
        if (tid < 8) {  // threshold tid's totals over the waves
            unsigned ct = 0u;
            u64 mt = 0ull;
            for (int x = 0; x < SP_NT / 64; ++x) {
                ct += sm.hc[x * 8 + tid];
                mt += sm.hm[x * 8 + tid];
            }
            sm.hc[SP_NT / 8 + tid] = ct;
            sm.hm[SP_NT / 8 + tid] = mt;
        }
        __syncthreads();
        if (tid == 0) {
            // the last threshold whose items above it (and the items above the interval) pass T;
            // the sums fall with q
            unsigned nlo = lo, nhi = hi;
            u64 ca = 0, ma = 0, cn = sm.hc[SP_NT / 8];
            for (int q = 0; q < 8; ++q) {
                const u64 cq = sm.hc[SP_NT / 8 + q], mq = sm.hm[SP_NT / 8 + q];
                if ((by_mass ? mb + mq : cb + cq) > T) {
                    nlo = t[q];
                    nhi = q < 7 ? t[q < 7 ? q + 1 : 7] : hi;
                    ca = q < 7 ? (u64)sm.hc[SP_NT / 8 + q + 1] : 0ull;
                    ma = q < 7 ? sm.hm[SP_NT / 8 + q + 1] : 0ull;
                    cn = cq - ca;
                }
            }
            sm.bc = cb + ca;
            sm.bm = mb + ma;
            sm.bn = cn;
            sm.blo = nlo;
            sm.bhi = nhi;
        }
        __syncthreads();
        cb = sm.bc;
        mb = sm.bm;
        n_int = sm.bn;
        lo = sm.blo;
        hi = sm.bhi;
        __syncthreads();
    }
    if (n_int <= (u64)SP_CAP) {
        // the interval's items, sorted; the running sums from (cb, mb) find the crossing
        sp_gather<KPT>(ws, V, [&](int i, unsigned k) { return k >= lo && k < hi && sp_in(cut, k, i); }, sm);
        const int n = (int)n_int;
        int n2 = 2;
        while (n2 < n) n2 <<= 1;
        for (int k = 2; k <= n2; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1) {
                if (tid < n2 / 2) {
                    const int i = 2 * tid - (tid & (j - 1)), l = i + j;
                    const u64 xa = sm.list[i], ya = sm.list[l];
                    if ((xa > ya) == ((i & k) == 0)) {
                        sm.list[i] = ya;
                        sm.list[l] = xa;
                    }
                }
                __syncthreads();
            }
        // entries 2 tid and 2 tid + 1: inclusive running sums, then the first past T
        const int e0 = 2 * tid, e1 = 2 * tid + 1;
        const u64 m0 = e0 < n ? sp_mass(~(unsigned)(sm.list[e0] >> 32)) : 0ull;
        const u64 m1 = e1 < n ? sp_mass(~(unsigned)(sm.list[e1] >> 32)) : 0ull;
        u64 ic = (u64)(e0 < n) + (u64)(e1 < n), im = m0 + m1;
        sp_scan(ic, im, sm);
        const u64 v0 = by_mass ? mb + im - m1 : cb + ic - (u64)(e1 < n);
        const u64 v1 = by_mass ? mb + im : cb + ic;
        const bool p0 = e0 < n && v0 > T, p1 = e1 < n && v1 > T;
        const int before = __syncthreads_count(e0 < n && !p0) + __syncthreads_count(e1 < n && !p1);
        if (tid == 0) sm.tok = -1;
        __syncthreads();
        if (before < n && (e0 == before || e1 == before)) {
            sm.tok = (int)(unsigned)(sm.list[before] & 0xffffffffull);
            sm.bm = mb + (e0 == before ? im - m1 : im);
            sm.bc = ~(unsigned)(sm.list[before] >> 32);
        }
        __syncthreads();
        const SpSel r{(unsigned)sm.bc, sm.tok, cb + (u64)before + 1, sm.bm, sm.tok >= 0};
        __syncthreads();
        return r;
    }
    // one key value (lo) held by more than SP_CAP items, each weighing mu: the j-th in index order
    // (slot u first, then thread), from this thread's matches as a bit per slot
    const unsigned kk = lo;
    const u64 mu = sp_mass(kk);
    const u64 j = by_mass ? (mu ? (T - mb) / mu : 0) : T - cb;
    u64 mine = 0;
    sp_each<KPT>(ws, V, [&](int i, unsigned k, int u) {
        if (i < V && k == kk && sp_in(cut, k, i)) mine |= 1ull << u;
    });
    // the matches per slot u (index order is u first): one ballot per slot and wave, summed in LDS
    for (int u = tid; u < KPT; u += SP_NT) sm.hc[u] = 0u;
    if (tid == 0) sm.tok = -1;
    __syncthreads();
    for (int u = 0; u < KPT; ++u) {
        const u64 bal = __ballot((mine >> u) & 1ull);
        if (lane == 0 && bal) atomicAdd(&sm.hc[u], (unsigned)__popcll(bal));
    }
    __syncthreads();
    if (tid == 0) {
        u64 run = 0;
        int us = KPT;
        for (int u = 0; u < KPT; ++u) {
            if (run + sm.hc[u] > j) {
                us = u;
                break;
            }
            run += sm.hc[u];
        }
        sm.bsel = us;
        sm.bn = j - run;  // the rank within slot us
    }
    __syncthreads();
    const int us = sm.bsel;
    if (us < KPT) {
        // the rank-th match of slot us in thread order
        const bool pr = (mine >> us) & 1ull;
        const u64 bal = __ballot(pr);
        if (lane == 0) sm.wi[w] = __popcll(bal);
        __syncthreads();
        int bw = 0;
        for (int x = 0; x < w; ++x) bw += sm.wi[x];
        const int rank = bw + __popcll(bal & ((1ull << lane) - 1ull));
        if (pr && (u64)rank == sm.bn) sm.tok = tid + us * SP_NT;
    }
    __syncthreads();
    const SpSel r{kk, sm.tok, cb + j + 1, mb + (j + 1) * mu, sm.tok >= 0};
    __syncthreads();
    return r;
}

template <int KPT, typename P>
__device__ unsigned sp_gather(const unsigned *ws, int V, P &&pred, SampleSmem &sm) {
    u64 n = 0, unused = 0;
    sp_each<KPT>(ws, V, [&](int i, unsigned k, int) {
        if (i < V && pred(i, k)) ++n;
    });
    const u64 mine = n;
    sp_scan(n, unused, sm);  // inclusive
    if (threadIdx.x == SP_NT - 1) sm.cnt = (unsigned)n;
    u64 q = n - mine;
    for (int u = threadIdx.x; u < SP_CAP; u += SP_NT) sm.list[u] = ~0ull;
    __syncthreads();
    sp_each<KPT>(ws, V, [&](int i, unsigned k, int) {
        if (i < V && pred(i, k)) {
            if (q < (u64)SP_CAP) sm.list[q] = ((u64)(~k) << 32) | (unsigned)i;
            ++q;
        }
    });
    __syncthreads();
    return sm.cnt;
}

// LmHead::argmax (lm_head.rs:62-69) as Iterator::max_by folds over x[0, V): NaN compares Equal,
// so the fold restarts after the last NaN and returns the last maximum after it (the NaN itself
// when last).
template <int KPT>
__device__ int sp_argmax(const float *x, int V, SampleSmem &sm) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const unsigned *xb = reinterpret_cast<const unsigned *>(x);
    int jn = -1;
    sp_each<KPT>(xb, V, [&](int i, unsigned b, int) {
        const float v = __uint_as_float(b);
        if (i < V && v != v) jn = i;
    });
    for (int off = 32; off > 0; off >>= 1) jn = max(jn, __shfl_xor(jn, off, 64));
    if (lane == 0) sm.wi[w] = jn;
    __syncthreads();
    jn = sm.wi[0];
    for (int u = 1; u < SP_NT / 64; ++u) jn = max(jn, sm.wi[u]);
    __syncthreads();
    float bv = -INFINITY;
    int bi = -1;
    sp_each<KPT>(xb, V, [&](int i, unsigned b, int) {
        const float v = __uint_as_float(b);
        if (i < V && i > jn && !(v < bv)) {
            bv = v;
            bi = i;
        }
    });
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(bv, off, 64);
        const int i2 = __shfl_xor(bi, off, 64);
        am_combine(bv, bi, v2, i2);
    }
    if (lane == 0) {
        sm.wf[w] = bv;
        sm.wi[w] = bi;
    }
    __syncthreads();
    bv = sm.wf[0];
    bi = sm.wi[0];
    for (int u = 1; u < SP_NT / 64; ++u) am_combine(bv, bi, sm.wf[u], sm.wi[u]);
    __syncthreads();
    return bi >= 0 ? bi : (jn >= 0 ? jn : 0);
}

template <int KPT>
__global__ __launch_bounds__(SP_NT) void k_sample(const float *logits, int V, int NB, unsigned *ws, const float *psum,
                                                  const float *pmin, const unsigned *gc, const u64 *gm,
                                                  const u64 *bucket, const unsigned *bcum, SampleParams a,
                                                  int32_t *out, TokenAppend app) {
    __shared__ SampleSmem sm;
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *lg = logits + (long)row * V;
    unsigned *wk = ws + (long)row * V;
    if (a.greedy) {  // lm_head.rs:104-111: the arg-max of the penalised row
        const int g = sp_argmax<KPT>(reinterpret_cast<const float *>(wk), V, sm);
        if (tid == 0) am_store(out, row, g, app);
        return;
    }
    // the blocks' partials staged through LDS (one load per thread, not a chain of loads)
    for (int q = tid; q < NB; q += SP_NT) {
        sm.wf2[q] = psum[(long)row * NB + q];
        sm.wf2[SP_NT / 2 + q] = pmin[(long)row * NB + q];
    }
    __syncthreads();
    float S = 0.0f, emin = INFINITY;
    for (int q = 0; q < NB; ++q) {
        S += sm.wf2[q];
        emin = fminf(emin, sm.wf2[SP_NT / 2 + q]);
    }
    const float r = a.uni[(long)row * a.uni_stride];
    int tok = -2;  // -2: LmHead::argmax of the row as given (lm_head.rs:148-150)
    // a NaN S (a NaN or infinite logit, or no finite one) makes every p NaN: the reference's kept
    // sum then fails `sum > 1e-6`
    if (S == S) {
        const unsigned khi = __float_as_uint(1.0f / S);  // the largest key: exp(0) / S
        const int bsh = sp_bin_shift(khi, __float_as_uint(emin / S));  // as k_samp_keys binned
        // the row's bins (thread t, bin t) and their running sums from the largest keys down
        const unsigned c_t = gc[(long)row * SP_NBIN + tid];
        const u64 m_t = gm[(long)row * SP_NBIN + tid];
        sm.oc[tid] = c_t;
        sm.om[tid] = m_t;
        u64 ic_t = c_t, im_t = m_t;
        sp_scan(ic_t, im_t, sm);
        if (tid == SP_NT - 1) sm.bm = im_t;
        __syncthreads();
        const u64 total = sm.bm;
        __syncthreads();
        const bool kon = a.top_k > 0 && a.top_k < V, pon = a.top_p > 0.0f && a.top_p < 1.0f;
        const SpCut none{false, 0u, 0};
        // The common case: the list up to the decision lies in a prefix of bins of at most SP_CAP
        // items: the bins through the top_k-th item; without top-k, the bins whose weight exceeds
        // top_p by 2^-10 of slack, or (no cut at all) reaches the draw's share of the total by it.
        // That prefix is gathered, sorted, and the reference's loops run on it.
        bool done = false;
        if (!kon || a.top_k <= SP_CAP) {
            const u64 slack = 1ull << 50;
            bool past;
            if (kon)
                past = ic_t >= (u64)a.top_k;
            else if (pon)
                past = im_t > (u64)((double)a.top_p * 1152921504606846976.0) + slack;
            else
                past = (double)im_t >= (double)r * (double)total + (double)slack;
            const int db = min(SP_NBIN - 1, __syncthreads_count(!past));  // the bins before the deciding one
            if (tid == db) {
                sm.bn = ic_t;  // the prefix's items
                const u64 top = (u64)khi + 1;
                sm.blo = db == SP_NBIN - 1 ? 0u
                                           : (unsigned)(top > ((u64)(db + 1) << bsh) ? top - ((u64)(db + 1) << bsh) : 0);
            }
            __syncthreads();
            const u64 P = sm.bn;
            const unsigned plo = sm.blo;
            __syncthreads();
            if (P <= (u64)SP_CAP) {
                // the prefix's items: block q's first bcum[q][db] bucketed items
                if (tid < NB) sm.boff[tid + 1] = bcum[((long)row * NB + tid) * SP_NBIN + db];
                if (tid == 0) sm.boff[0] = 0u;
                __syncthreads();
                if (tid == 0)
                    for (int q = 0; q < NB; ++q) sm.boff[q + 1] += sm.boff[q];
                __syncthreads();
                for (int e = tid; e < SP_CAP; e += SP_NT) {
                    u64 v = ~0ull;
                    if (e < (int)P) {
                        int q = 0;
                        while (q + 1 < NB && sm.boff[q + 1] <= (unsigned)e) ++q;
                        v = bucket[((long)row * NB + q) * SP_EPB + (e - (int)sm.boff[q])];
                    }
                    sm.list[e] = v;
                }
                __syncthreads();
                int n2 = 2;
                while (n2 < (int)P) n2 <<= 1;
                for (int k = 2; k <= n2; k <<= 1)
                    for (int j = k >> 1; j > 0; j >>= 1) {
                        if (tid < n2 / 2) {
                            const int i = 2 * tid - (tid & (j - 1)), l = i + j;
                            const u64 xa = sm.list[i], ya = sm.list[l];
                            if ((xa > ya) == ((i & k) == 0)) {
                                sm.list[i] = ya;
                                sm.list[l] = xa;
                            }
                        }
                        __syncthreads();
                    }
                if (tid == 0) {
                    // the reference's loops (:120-166) over the sorted prefix; `full`: the prefix
                    // is the whole row
                    auto pk = [&](int i) { return __uint_as_float(~(unsigned)(sm.list[i] >> 32)); };
                    auto ix = [&](int i) { return (int)(unsigned)(sm.list[i] & 0xffffffffull); };
                    const bool full = P == (u64)V;
                    int n = kon ? a.top_k : (int)P;
                    bool ok = true;
                    if (pon) {
                        float cum = 0.0f;
                        int cut = -1;
                        for (int i = 0; i < n; ++i) {
                            cum += pk(i);
                            if (cum > a.top_p) {
                                cut = i + 1;
                                break;
                            }
                        }
                        if (cut < 0) {
                            if (kon || full)
                                cut = n;
                            else
                                ok = false;  // the float sum crossed later than the slack allowed for
                        }
                        n = cut < 1 ? 1 : cut;
                    }
                    int t = -1;
                    if (ok) {
                        // the kept list is in the prefix unless no cut applies to a partial prefix:
                        // then its sum is the row's exact weight
                        const bool whole = kon || pon || full;
                        float sum = -0.0f;
                        if (whole)
                            for (int i = 0; i < n; ++i) sum += pk(i);
                        else
                            sum = (float)((double)total * (1.0 / 1152921504606846976.0));
                        if (!(sum > 1e-6f)) {
                            t = -2;
                        } else {
                            float cum = 0.0f;
                            for (int i = 0; i < n; ++i) {
                                cum += pk(i) / sum;
                                if (r <= cum) {
                                    t = ix(i);
                                    break;
                                }
                            }
                            if (t < 0 && whole) t = ix(0);
                        }
                    }
                    sm.tok = t;  // -1: decide on the exact sums below
                }
                __syncthreads();
                tok = sm.tok;
                done = tok != -1;
                __syncthreads();
            }
        }
        if (!done) {
        // 3. top-k (:121-125): the list ends at its top_k-th item
        SpCut ck = none;
        u64 nk = (u64)V, mk = total;
        if (kon) {
            const SpSel sk = sp_select<KPT>(wk, V, false, (u64)(a.top_k - 1), none, khi, bsh, sm);
            ck = SpCut{true, sk.key, sk.idx};
            nk = sk.cnt;
            mk = sk.mass;
        }
        // 4. the short list: past top_p by 2^-10 of slack (the float running sum of <= SP_CAP items
        // stays within 2^-12 of the exact one), or the whole kept list
        SpCut cl = ck;
        u64 M = nk;
        bool full = true;
        if (!(kon && a.top_k <= SP_CAP) && pon) {
            const SpSel sp = sp_select<KPT>(wk, V, true, (u64)((double)a.top_p * 1152921504606846976.0) + (1ull << 50),
                                            ck, khi, bsh, sm);
            if (sp.found) {
                cl = SpCut{true, sp.key, sp.idx};
                M = sp.cnt;
                full = M == nk;
            }
        }
        bool exact = M > (u64)SP_CAP;
        if (!exact) {
            sp_gather<KPT>(wk, V, [&](int i, unsigned k) { return sp_in(cl, k, i); }, sm);
            if (tid == 0) {
                sm.tok = -1;
                sm.need_exact = 0;
            }
            int n2 = 2;
            while (n2 < (int)M) n2 <<= 1;
            for (int k = 2; k <= n2; k <<= 1)
                for (int j = k >> 1; j > 0; j >>= 1) {
                    if (tid < n2 / 2) {
                        const int i = 2 * tid - (tid & (j - 1)), l = i + j;
                        const u64 xa = sm.list[i], ya = sm.list[l];
                        if ((xa > ya) == ((i & k) == 0)) {
                            sm.list[i] = ya;
                            sm.list[l] = xa;
                        }
                    }
                    __syncthreads();
                }
            if (tid == 0) {
                // the reference's loops (:127-166) over the sorted list
                auto pk = [&](int i) { return __uint_as_float(~(unsigned)(sm.list[i] >> 32)); };
                auto ix = [&](int i) { return (int)(unsigned)(sm.list[i] & 0xffffffffull); };
                int n = (int)M;
                bool ok = true;
                if (pon) {
                    float cum = 0.0f;
                    int cut = -1;
                    for (int i = 0; i < n; ++i) {
                        cum += pk(i);
                        if (cum > a.top_p) {
                            cut = i + 1;
                            break;
                        }
                    }
                    if (cut < 0) {
                        if (full)
                            cut = n;
                        else
                            ok = false;  // the float sum crossed later than the slack allowed for
                    }
                    n = cut < 1 ? 1 : cut;
                }
                if (!ok) {
                    sm.need_exact = 1;
                } else {
                    float sum = -0.0f;
                    for (int i = 0; i < n; ++i) sum += pk(i);
                    if (sum > 1e-6f) {
                        float cum = 0.0f;
                        int t = ix(0);
                        for (int i = 0; i < n; ++i) {
                            cum += pk(i) / sum;
                            if (r <= cum) {
                                t = ix(i);
                                break;
                            }
                        }
                        sm.tok = t;
                    } else {
                        sm.tok = -2;
                    }
                }
            }
            __syncthreads();
            tok = sm.tok;
            exact = sm.need_exact != 0;
            __syncthreads();
        }
        if (exact) {
            // 5. top-p (:127-140), the renormalisation (:142-150) and the draw (:152-166) on the
            // exact sums: the first item past which the weight exceeds top_p; then the first at
            // which it reaches r times the kept weight (the first item when r <= 0 or NaN)
            SpCut cf = ck;
            u64 mkept = mk;
            if (pon) {
                const SpSel sp = sp_select<KPT>(wk, V, true, (u64)((double)a.top_p * 1152921504606846976.0), ck, khi, bsh, sm);
                if (sp.found) {
                    cf = SpCut{true, sp.key, sp.idx};
                    mkept = sp.mass;
                }
            }
            if ((double)mkept > 1e-6 * 1152921504606846976.0) {
                SpSel sd{};
                bool first = !(r > 0.0f);
                if (!first) {
                    const u64 Tt = (u64)ceil((double)r * (double)mkept);  // >= 1
                    sd = sp_select<KPT>(wk, V, true, Tt - 1, cf, khi, bsh, sm);
                    first = !sd.found;
                }
                if (first) sd = sp_select<KPT>(wk, V, false, 0, cf, khi, bsh, sm);
                tok = sd.idx;
            } else {
                tok = -2;
            }
        }
        }  // !done
    }
    if (tok == -2) tok = sp_argmax<KPT>(lg, V, sm);
    if (tid == 0) am_store(out, row, tok < 0 ? 0 : tok, app);
}

}  // namespace

void launch_pool_norm(const Dims &D, const float *h, int ntok, const float *g, float *pooled,
                      float *pnorm, float *rec, int REC, float pre_scale, hipStream_t st) {
    const dim3 grid((unsigned)((ntok + WPB - 1) / WPB)), blk(64 * WPB);
    dispatch_width(D.d, [&](auto Ec, auto Pc) {
        hipLaunchKernelGGL((k_pool_norm<decltype(Ec)::value, decltype(Pc)::value>), grid, blk, 0, st, D, h, ntok, g,
                           pooled, pnorm, rec, REC, pre_scale);
    });
}

void launch_argmax(const float *logits, int ntok, int V, int32_t *out, hipStream_t st, const TokenAppend *app) {
    const TokenAppend a = app ? *app : TokenAppend{};
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)ntok), dim3(AM_NT), 0, st, logits, V, out, a);
}

void launch_argmax_reduce(const float *am_val, const int32_t *am_idx, int ntok, int ntiles, int32_t *out,
                          hipStream_t st, const TokenAppend *app) {
    const TokenAppend a = app ? *app : TokenAppend{};
    if (ntok <= 4) {
        hipLaunchKernelGGL(k_argmax_reduce_rows, dim3((unsigned)ntok), dim3(ARR_NT), 0, st, am_val, am_idx, ntok,
                           ntiles, out, a);
        return;
    }
    hipLaunchKernelGGL(k_argmax_reduce, dim3((unsigned)((ntok + 31) / 32)), dim3(64 * AR_W), 0, st, am_val, am_idx, ntok,
                       ntiles, out, a);
}

void launch_decode_query(const float *E, int d, const int32_t *seq, int stride, int len, int ctx, int B, float *q,
                         hipStream_t st, unsigned *absmax, const QueryInit *init) {
    const QueryInit qi = init ? *init : QueryInit{};
    dispatch_width(d, [&](auto Ec, auto Pc) {
        constexpr int EC = decltype(Ec)::value;
        hipLaunchKernelGGL((k_decode_query<EC, decltype(Pc)::value>), dim3((unsigned)B), dim3(64 * dq_waves(EC)), 0, st,
                           E, d, seq, stride, len, ctx, q, absmax, qi);
    });
}

void launch_rep_penalty(float *logits, int V, const int32_t *seq, int stride, int len, int ctx, float pen, int B,
                        hipStream_t st) {
    hipLaunchKernelGGL(k_rep_penalty, dim3((unsigned)B), dim3(256), 0, st, logits, V, seq, stride, len, ctx, pen);
}

size_t sample_workspace_bytes(int rows, int V) {
    const size_t NB = (size_t)(V + SP_EPB - 1) / SP_EPB, R = (size_t)rows;
    return R * SP_NBIN * (sizeof(u64) + sizeof(unsigned)) + R * NB * SP_EPB * sizeof(u64) +
           R * NB * SP_NBIN * sizeof(unsigned) + 3 * R * NB * sizeof(float) + R * (size_t)V * 4;
}

void launch_sample(const float *logits, int rows, int V, void *ws, const SampleParams &sp, int32_t *out,
                   hipStream_t st, const TokenAppend *app) {
    const TokenAppend a = app ? *app : TokenAppend{};
    const int NB = (V + SP_EPB - 1) / SP_EPB;
    const size_t R = (size_t)rows;
    u64 *gm = (u64 *)ws;
    u64 *bucket = gm + R * SP_NBIN;
    unsigned *gc = (unsigned *)(bucket + R * NB * SP_EPB);
    unsigned *bcum = gc + R * SP_NBIN;
    float *pmax = (float *)(bcum + R * NB * SP_NBIN), *psum = pmax + R * NB, *pmin = psum + R * NB;
    unsigned *wk = (unsigned *)(pmin + R * NB);
    const dim3 ge((unsigned)NB, (unsigned)rows);
    hipLaunchKernelGGL(k_samp_scale, ge, dim3(SP_PT), 0, st, logits, V, (float *)wk, pmax, gc, gm, sp);
    if (!sp.greedy) {
        hipLaunchKernelGGL(k_samp_exp, ge, dim3(SP_PT), 0, st, V, (float *)wk, pmax, psum, pmin);
        hipLaunchKernelGGL(k_samp_keys, ge, dim3(SP_PT), 0, st, V, wk, psum, pmin, gc, gm, bucket, bcum);
    }
    const dim3 g((unsigned)rows), b(SP_NT);
    const int kpt = (V + SP_NT - 1) / SP_NT;
    if (kpt <= 4)
        hipLaunchKernelGGL(k_sample<4>, g, b, 0, st, logits, V, NB, wk, psum, pmin, gc, gm, bucket, bcum, sp, out, a);
    else if (kpt <= 16)
        hipLaunchKernelGGL(k_sample<16>, g, b, 0, st, logits, V, NB, wk, psum, pmin, gc, gm, bucket, bcum, sp, out, a);
    else if (kpt <= 32)
        hipLaunchKernelGGL(k_sample<32>, g, b, 0, st, logits, V, NB, wk, psum, pmin, gc, gm, bucket, bcum, sp, out, a);
    else
        hipLaunchKernelGGL(k_sample<64>, g, b, 0, st, logits, V, NB, wk, psum, pmin, gc, gm, bucket, bcum, sp, out, a);
}

void launch_decode_last(const int32_t *seq, int stride, int len, int32_t *last, int B, hipStream_t st) {
    hipLaunchKernelGGL(k_decode_last, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, seq, stride, len, last, B);
}

}  // namespace adn

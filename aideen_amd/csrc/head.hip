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

void launch_decode_last(const int32_t *seq, int stride, int len, int32_t *last, int B, hipStream_t st) {
    hipLaunchKernelGGL(k_decode_last, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, seq, stride, len, last, B);
}

}  // namespace adn

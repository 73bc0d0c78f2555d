// embed_context for the window ending at every position (tokenizer.rs:133-149, with the
// windows the trainer's evaluation builds, trainer.rs:4690-4696):
//   out[b][i] = r / |r|   (r itself when |r| <= 1e-6),
//   r = sum_{p=s..i} E[tok_p] (p - s + 1) / L,   s = max(0, i - ctx + 1),   L = i - s + 1.
// As a prefix scan: with P0_i = sum_{p<=i} E_p and P1_i = sum_{p<=i} (p + 1) E_p,
//   L r = (P1_i - P1_{i-ctx}) - s (P0_i - P0_{i-ctx}),
// so every position costs O(d) instead of O(ctx d).  The prefixes are carried in fp64, which
// makes the differences exact to far below the fp32 rounding of the reference's own
// sequential sum.  The 1/L factor cancels in the normalisation and is applied only on the
// small-norm branch.
//   k_ctx_chunks: per (sequence, chunk of positions): chunk totals of E_p and (p + 1) E_p.
//   k_ctx_scan:   per (sequence, dim): the totals become exclusive prefixes over the chunks.
//   k_ctx_window: per (sequence, chunk): prefixes from the earlier chunks' totals; the chunk's
//                 rows and the rows leaving the window (ctx positions behind) are loaded into
//                 registers up front, every window value of the chunk is formed, and one block
//                 barrier gives all of the chunk's norms.
#include "kernels.h"

namespace adn {

namespace {

constexpr int ENT = 256;  // threads per block
// positions per chunk: CHK * DPT = 32 values of each row set per thread
template <int DPT>
constexpr int chunk_len() {
    return 32 / DPT;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// this thread's DPT values of the rows of positions [p0, p0 + CHK) (zero outside [0, pend)).
// Branch-free, so that all CHK id loads and then all row loads are in flight together.
template <int DPT, int CHK>
__device__ __forceinline__ void load_rows(float (&x)[CHK][DPT], const float *E, int d, int V,
                                          const int32_t *tokens, long sb, int p0, int pend, unsigned *err) {
    long row[CHK];
    bool bad = false;
#pragma unroll
    for (int p = 0; p < CHK; ++p) {
        const bool ok = p0 + p >= 0 && p0 + p < pend;
        const long t = ok ? (long)tokens[sb + p0 + p] : 0;
        const bool out = t < 0 || t >= V;
        bad |= out;
        row[p] = out ? 0 : t;
    }
#pragma unroll
    for (int p = 0; p < CHK; ++p) {
        const bool ok = p0 + p >= 0 && p0 + p < pend;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            const float v = E[row[p] * d + (j < d ? j : 0)];
            x[p][q] = (ok && j < d) ? v : 0.0f;
        }
    }
    if (bad && threadIdx.x == 0) atomicOr(err, ADN_DEVERR_TOKEN);
}

template <int DPT>
// busy (or null): the overlap guard of a shared chunk-total array, [0] the calls in flight, [1] the
// window kernel's finished blocks.  The chunk kernel raises [0] (a call that finds it raised
// overlaps another: ADN_DEVERR_OVERLAP), the last block of the window kernel lowers it.
__global__ __launch_bounds__(ENT) void k_ctx_chunks(const float *E, int d, int V, const int32_t *tokens, int T,
                                                     int nch, double *tot0, double *tot1, unsigned *err,
                                                     unsigned *busy) {
    constexpr int CHK = chunk_len<DPT>();
    if (busy && blockIdx.x == 0 && threadIdx.x == 0 && atomicAdd(busy, 1u) != 0u) atomicOr(err, ADN_DEVERR_OVERLAP);
    const int b = blockIdx.x / nch, c = blockIdx.x - b * nch;
    const int p0 = c * CHK;
    float x[CHK][DPT];
    load_rows<DPT, CHK>(x, E, d, V, tokens, (long)b * T, p0, T, err);
    double s0[DPT], s1[DPT];
#pragma unroll
    for (int q = 0; q < DPT; ++q) s0[q] = s1[q] = 0.0;
#pragma unroll
    for (int p = 0; p < CHK; ++p)
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            s0[q] += (double)x[p][q];
            s1[q] += (double)(p0 + p + 1) * (double)x[p][q];
        }
    const long o = ((long)b * nch + c) * d;
#pragma unroll
    for (int q = 0; q < DPT; ++q) {
        const int j = threadIdx.x + q * ENT;
        if (j < d) {
            tot0[o + j] = s0[q];
            tot1[o + j] = s1[q];
        }
    }
}

// chunk totals -> exclusive prefixes over the chunks, in place, per (sequence, dim)
__global__ __launch_bounds__(ENT) void k_ctx_scan(int d, int nch, int B, double *tot0, double *tot1) {
    const long g = (long)blockIdx.x * ENT + threadIdx.x;
    if (g >= (long)B * d) return;
    const int b = (int)(g / d), j = (int)(g - (long)b * d);
    double *t0 = tot0 + (long)b * nch * d + j, *t1 = tot1 + (long)b * nch * d + j;
    double r0 = 0.0, r1 = 0.0;
#pragma unroll 8
    for (int c = 0; c < nch; ++c) {
        const double a0 = t0[(long)c * d], a1 = t1[(long)c * d];
        t0[(long)c * d] = r0;
        t1[(long)c * d] = r1;
        r0 += a0;
        r1 += a1;
    }
}

template <int DPT>
__global__ __launch_bounds__(ENT) void k_ctx_window(const float *E, int d, int V, const int32_t *tokens, int T,
                                                     int nch, int ctx, const double *tot0, const double *tot1,
                                                     float *out, unsigned *err, unsigned *busy) {
    constexpr int CHK = chunk_len<DPT>();
    __shared__ double red[CHK][ENT / 64];
    const int b = blockIdx.x / nch, c = blockIdx.x - b * nch;
    const int i0 = c * CHK;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long tb = (long)b * nch * d;
    const long sb = (long)b * T;
    // the chunk's rows, and the rows that leave the window after each of its positions
    float xe[CHK][DPT], xl[CHK][DPT];
    load_rows<DPT, CHK>(xe, E, d, V, tokens, sb, i0, T, err);
    load_rows<DPT, CHK>(xl, E, d, V, tokens, sb, i0 + 1 - ctx, T, err);
    double P0[DPT], P1[DPT], L0[DPT], L1[DPT];
#pragma unroll
    for (int q = 0; q < DPT; ++q) P0[q] = P1[q] = L0[q] = L1[q] = 0.0;
    // P: prefix through i0 - 1 (tot0/tot1 hold the chunks' exclusive prefixes)
#pragma unroll
    for (int q = 0; q < DPT; ++q) {
        const int j = threadIdx.x + q * ENT;
        if (j < d) {
            P0[q] = tot0[tb + (long)c * d + j];
            P1[q] = tot1[tb + (long)c * d + j];
        }
    }
    // L: prefix through q0 = i0 - ctx (empty while q0 < 0)
    const int q0 = i0 - ctx;
    if (q0 >= 0) {
        const int cq = q0 / CHK;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            if (j < d) {
                L0[q] = tot0[tb + (long)cq * d + j];
                L1[q] = tot1[tb + (long)cq * d + j];
            }
        }
        // then the positions cq*CHK ..= q0 of that chunk, loaded together (zero past q0)
        float xw[CHK][DPT];
        load_rows<DPT, CHK>(xw, E, d, V, tokens, sb, cq * CHK, q0 + 1, err);
#pragma unroll
        for (int p = 0; p < CHK; ++p)
#pragma unroll
            for (int q = 0; q < DPT; ++q) {
                const double x = xw[p][q];
                L0[q] += x;
                L1[q] += (double)(cq * CHK + p + 1) * x;
            }
    }
    double v[CHK][DPT];
#pragma unroll
    for (int p = 0; p < CHK; ++p) {
        const int i = i0 + p;
        const int s = i - ctx + 1 > 0 ? i - ctx + 1 : 0;
        double ss = 0.0;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const double x = xe[p][q];
            P0[q] += x;
            P1[q] += (double)(i + 1) * x;
            v[p][q] = (P1[q] - L1[q]) - (double)s * (P0[q] - L0[q]);
            ss += v[p][q] * v[p][q];
            // position i + 1 - ctx leaves the next window (its row is zero while < 0)
            const double xo = xl[p][q];
            L0[q] += xo;
            L1[q] += (double)(i + 2 - ctx) * xo;
        }
        ss = wave_sum_d(ss);
        if (lane == 0) red[p][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < CHK; ++p) {
        const int i = i0 + p;
        if (i >= T) break;
        double n2 = 0.0;
#pragma unroll
        for (int w = 0; w < ENT / 64; ++w) n2 += red[p][w];
        const double nv = sqrt(n2);
        const int s = i - ctx + 1 > 0 ? i - ctx + 1 : 0;
        const double len = (double)(i - s + 1);
        const double inv = 1.0 / (nv > 1e-6 * len ? nv : len);  // r/|r| = v/|v|; r = v/len
        float *o = out + (sb + i) * d;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            if (j < d) o[j] = (float)(v[p][q] * inv);
        }
    }
    if (busy) {  // the call's last block (every block has read its totals) lowers the guard
        __syncthreads();
        if (threadIdx.x == 0) {
            __threadfence();
            if (atomicAdd(busy + 1, 1u) == gridDim.x - 1) {
                atomicExch(busy + 1, 0u);
                atomicSub(busy, 1u);
            }
        }
    }
}

template <int DPT>
void launch_ctx(const float *E, int d, int V, const int32_t *tokens, int B, int T, int ctx, double *tot0,
                double *tot1, float *out, unsigned *err, unsigned *busy, hipStream_t st) {
    constexpr int CHK = chunk_len<DPT>();
    const int nch = (T + CHK - 1) / CHK;
    const dim3 grid((unsigned)(B * nch)), blk(ENT);
    hipLaunchKernelGGL(k_ctx_chunks<DPT>, grid, blk, 0, st, E, d, V, tokens, T, nch, tot0, tot1, err, busy);
    hipLaunchKernelGGL(k_ctx_scan, dim3((unsigned)(((long)B * d + ENT - 1) / ENT)), blk, 0, st, d, nch, B, tot0, tot1);
    hipLaunchKernelGGL(k_ctx_window<DPT>, grid, blk, 0, st, E, d, V, tokens, T, nch, ctx, tot0, tot1, out, err,
                       busy);
}

}  // namespace

// chunk count for the smallest chunk (d > 1024: 4 positions)
long embed_context_chunks(int T) { return (T + 3) / 4; }

// values per thread of a row: the launch's template bucket for d
static int ctx_dpt(int d) {
    const int dpt = (d + ENT - 1) / ENT;
    return dpt <= 1 ? 1 : dpt <= 2 ? 2 : dpt <= 4 ? 4 : 8;
}

long embed_context_total_doubles(int d, int B, int T) {
    const int chk = 32 / ctx_dpt(d);
    return (long)B * ((T + chk - 1) / chk) * d;
}

void launch_embed_context(const float *E, int d, int V, const int32_t *tokens, int B, int T, int ctx, double *tot0,
                          double *tot1, float *out, unsigned *err, unsigned *busy, hipStream_t st) {
    const int dpt = ctx_dpt(d);
    if (dpt <= 1)
        launch_ctx<1>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, busy, st);
    else if (dpt <= 2)
        launch_ctx<2>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, busy, st);
    else if (dpt <= 4)
        launch_ctx<4>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, busy, st);
    else
        launch_ctx<8>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, busy, st);
}

}  // namespace adn

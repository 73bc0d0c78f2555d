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
//   k_ctx_chunks: per (sequence, chunk of CH positions): chunk totals of E_p and (p + 1) E_p.
//   k_ctx_window: per (sequence, chunk): prefixes from the earlier chunks' totals; walks its
//                 chunk and, ctx positions behind, the positions that leave the window; one
//                 block-wide norm per position.
#include "kernels.h"

namespace adn {

namespace {

constexpr int CH = 32;    // positions per chunk
constexpr int ENT = 256;  // threads per block

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// embedding row of token idx; an id outside [0, V) is reported (by thread 0) and reads row 0
__device__ __forceinline__ const float *erow(const float *E, int d, int V, const int32_t *tokens, long idx,
                                             unsigned *err) {
    long t = tokens[idx];
    if (t < 0 || t >= V) {
        if (threadIdx.x == 0) atomicOr(err, ADN_DEVERR_TOKEN);
        t = 0;
    }
    return E + t * d;
}

template <int DPT>
__global__ __launch_bounds__(ENT) void k_ctx_chunks(const float *E, int d, int V, const int32_t *tokens, int T,
                                                     int nch, double *tot0, double *tot1, unsigned *err) {
    const int b = blockIdx.x / nch, c = blockIdx.x - b * nch;
    const int p0 = c * CH, p1 = min(T, p0 + CH);
    double s0[DPT], s1[DPT];
#pragma unroll
    for (int q = 0; q < DPT; ++q) s0[q] = s1[q] = 0.0;
    for (int p = p0; p < p1; ++p) {
        const float *e = erow(E, d, V, tokens, (long)b * T + p, err);
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            if (j < d) {
                const double x = e[j];
                s0[q] += x;
                s1[q] += (double)(p + 1) * x;
            }
        }
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

template <int DPT>
__global__ __launch_bounds__(ENT) void k_ctx_window(const float *E, int d, int V, const int32_t *tokens, int T,
                                                     int nch, int ctx, const double *tot0, const double *tot1,
                                                     float *out, unsigned *err) {
    __shared__ double red[ENT / 64];
    __shared__ double nrm2_s;
    const int b = blockIdx.x / nch, c = blockIdx.x - b * nch;
    const int i0 = c * CH, i1 = min(T, i0 + CH);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long tb = (long)b * nch * d;
    const long sb = (long)b * T;
    double P0[DPT], P1[DPT], L0[DPT], L1[DPT];
    // P = prefix through i0 - 1 (the earlier chunks' totals)
#pragma unroll
    for (int q = 0; q < DPT; ++q) P0[q] = P1[q] = L0[q] = L1[q] = 0.0;
    for (int cc = 0; cc < c; ++cc)
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            if (j < d) {
                P0[q] += tot0[tb + (long)cc * d + j];
                P1[q] += tot1[tb + (long)cc * d + j];
            }
        }
    // lagged prefix through q0 = i0 - ctx (empty while q0 < 0)
    const int q0 = i0 - ctx;
    if (q0 >= 0) {
        const int cq = q0 / CH;
        for (int cc = 0; cc < cq; ++cc)
#pragma unroll
            for (int q = 0; q < DPT; ++q) {
                const int j = threadIdx.x + q * ENT;
                if (j < d) {
                    L0[q] += tot0[tb + (long)cc * d + j];
                    L1[q] += tot1[tb + (long)cc * d + j];
                }
            }
        for (int p = cq * CH; p <= q0; ++p) {
            const float *e = erow(E, d, V, tokens, sb + p, err);
#pragma unroll
            for (int q = 0; q < DPT; ++q) {
                const int j = threadIdx.x + q * ENT;
                if (j < d) {
                    const double x = e[j];
                    L0[q] += x;
                    L1[q] += (double)(p + 1) * x;
                }
            }
        }
    }
    for (int i = i0; i < i1; ++i) {
        const float *e = erow(E, d, V, tokens, sb + i, err);
        const int s = i - ctx + 1 > 0 ? i - ctx + 1 : 0;
        double v[DPT];
        double ss = 0.0;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            v[q] = 0.0;
            if (j < d) {
                const double x = e[j];
                P0[q] += x;
                P1[q] += (double)(i + 1) * x;
                v[q] = (P1[q] - L1[q]) - (double)s * (P0[q] - L0[q]);
                ss += v[q] * v[q];
            }
        }
        ss = wave_sum_d(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        if (threadIdx.x == 0) {
            double t = 0.0;
            for (int w = 0; w < ENT / 64; ++w) t += red[w];
            nrm2_s = t;
        }
        __syncthreads();
        const double nv = sqrt(nrm2_s);
        const double len = (double)(i - s + 1);
        const bool unit = nv / len > 1e-6;
        float *o = out + (sb + i) * d;
#pragma unroll
        for (int q = 0; q < DPT; ++q) {
            const int j = threadIdx.x + q * ENT;
            if (j < d) o[j] = (float)(unit ? v[q] / nv : v[q] / len);
        }
        // position i + 1 - ctx leaves the next window: it joins the lagged prefix
        const int ql = i + 1 - ctx;
        if (ql >= 0) {
            const float *el = erow(E, d, V, tokens, sb + ql, err);
#pragma unroll
            for (int q = 0; q < DPT; ++q) {
                const int j = threadIdx.x + q * ENT;
                if (j < d) {
                    const double x = el[j];
                    L0[q] += x;
                    L1[q] += (double)(ql + 1) * x;
                }
            }
        }
    }
}

template <int DPT>
void launch_ctx(const float *E, int d, int V, const int32_t *tokens, int B, int T, int ctx, double *tot0,
                double *tot1, float *out, unsigned *err, hipStream_t st) {
    const int nch = (T + CH - 1) / CH;
    const dim3 grid((unsigned)(B * nch)), blk(ENT);
    hipLaunchKernelGGL(k_ctx_chunks<DPT>, grid, blk, 0, st, E, d, V, tokens, T, nch, tot0, tot1, err);
    hipLaunchKernelGGL(k_ctx_window<DPT>, grid, blk, 0, st, E, d, V, tokens, T, nch, ctx, tot0, tot1, out, err);
}

}  // namespace

long embed_context_chunks(int T) { return (T + CH - 1) / CH; }

void launch_embed_context(const float *E, int d, int V, const int32_t *tokens, int B, int T, int ctx, double *tot0,
                          double *tot1, float *out, unsigned *err, hipStream_t st) {
    const int dpt = (d + ENT - 1) / ENT;
    if (dpt <= 1)
        launch_ctx<1>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, st);
    else if (dpt <= 2)
        launch_ctx<2>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, st);
    else if (dpt <= 4)
        launch_ctx<4>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, st);
    else
        launch_ctx<8>(E, d, V, tokens, B, T, ctx, tot0, tot1, out, err, st);
}

}  // namespace adn

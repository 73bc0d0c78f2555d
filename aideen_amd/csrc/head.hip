// LM-head prologue (slot mean-pool + RMSNorm) and greedy arg-max.
//
// Reference: LmHead::{pool_h_star, rmsnorm, forward, argmax} (lm_head.rs:35-69);
// deq_forward_pool.wgsl:32-65 (pool).  The projection itself is the MFMA GEMM (gemm.hip).
#include "kernels.h"

namespace adn {

namespace {

constexpr int WPB = 4;

// pooled = fold(0, acc + h_s)/H (slot order kept); pnorm = (pooled/rms) * g, eps 1e-5.
__global__ __launch_bounds__(256) void k_pool_norm(Dims D, const float *h, int ntok, const float *g,
                                                   float *pooled, float *pnorm) {
    const int t = blockIdx.x * WPB + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= ntok) return;
    const int d = D.d, H = D.H;
    const float *ht = h + (long)t * H * d;
    float ss = 0.0f;
    for (int i = lane; i < d; i += 64) {
        float acc = 0.0f;
        for (int s = 0; s < H; ++s) acc = acc + ht[(long)s * d + i];
        const float p = acc / (float)H;
        if (pooled) pooled[(long)t * d + i] = p;
        ss += p * p;
    }
    if (!pnorm) return;
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-5f);
    for (int i = lane; i < d; i += 64) {
        float acc = 0.0f;
        for (int s = 0; s < H; ++s) acc = acc + ht[(long)s * d + i];
        const float p = acc / (float)H;
        pnorm[(long)t * d + i] = (p / rms) * (g ? g[i] : 1.0f);
    }
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

__global__ __launch_bounds__(AM_NT) void k_argmax(const float *logits, int V, int32_t *out) {
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
        out[row] = i < 0 ? 0 : i;
    }
}

// Reduce the LM-head tile partials of one row (one wave per row), same tie rule.
__global__ __launch_bounds__(256) void k_argmax_reduce(const float *am_val, const int32_t *am_idx, int ntok,
                                                       int ntiles, int32_t *out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= ntok) return;
    float bv = -INFINITY;
    int bi = -1;
    for (int t = lane; t < ntiles; t += 64) {
        const float v = am_val[(long)t * ntok + row];
        const int i = am_idx[(long)t * ntok + row];
        am_combine(bv, bi, v, i);
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(bv, off, 64);
        const int i2 = __shfl_xor(bi, off, 64);
        am_combine(bv, bi, v2, i2);
    }
    if (lane == 0) out[row] = bi < 0 ? 0 : bi;
}

// Greedy decode bookkeeping: tokens[b] = argmax[b]; out_seq[b][j] = argmax[b].
__global__ void k_decode_step(const int32_t *argmax, int32_t *tokens, int32_t *out_seq, int B,
                              int n_new, int j) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int32_t v = argmax[b];
    tokens[b] = v;
    out_seq[(long)b * n_new + j] = v;
}

}  // namespace

void launch_pool_norm(const Dims &D, const float *h, int ntok, const float *g, float *pooled,
                      float *pnorm, hipStream_t st) {
    hipLaunchKernelGGL(k_pool_norm, dim3((unsigned)((ntok + WPB - 1) / WPB)), dim3(64 * WPB), 0, st, D,
                       h, ntok, g, pooled, pnorm);
}

void launch_argmax(const float *logits, int ntok, int V, int32_t *out, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)ntok), dim3(AM_NT), 0, st, logits, V, out);
}

void launch_argmax_reduce(const float *am_val, const int32_t *am_idx, int ntok, int ntiles, int32_t *out,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_reduce, dim3((unsigned)((ntok + 3) / 4)), dim3(256), 0, st, am_val, am_idx, ntok,
                       ntiles, out);
}

void launch_copy_tokens_from_argmax(const int32_t *argmax, int32_t *tokens, int32_t *out_seq,
                                    int B, int n_new, int j, hipStream_t st) {
    hipLaunchKernelGGL(k_decode_step, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, argmax,
                       tokens, out_seq, B, n_new, j);
}

}  // namespace adn

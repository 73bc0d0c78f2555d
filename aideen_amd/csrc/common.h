// Shared definitions for the gfx950 kernels and the runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "aideen_hip.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

#define ADN_WAVE 64

// Device error flags (set by kernels, read back by adn_synchronize).
#define ADN_DEVERR_TOKEN 1u
#define ADN_DEVERR_OVERLAP 2u  // adn_embed_context_noalloc calls overlapped on one GPU

namespace adn {

// Error state of the calling thread (adn_last_error).
void set_error(const std::string &msg);

struct HipError {
    hipError_t code;
    std::string where;
};

#define ADN_HIP(call)                                                  \
    do {                                                               \
        hipError_t e_ = (call);                                        \
        if (e_ != hipSuccess) throw ::adn::HipError{e_, #call};        \
    } while (0)

// Fixed parameters of a forward pass shared by the kernels.
struct Dims {
    int d, H, V, N, r;
    uint32_t flags;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Raise *word, the bit pattern of a non-negative float bound on an array's magnitude, to the
// wave's largest finite |v| (a > 0 float orders like its bits).  NaN and inf are left out: they
// stay in their own rows and must not turn the split GEMMs' scale of every row into 0 or NaN.
// One atomic per wave, issued only when the wave's value exceeds the word as read (a stale read
// costs at most an extra atomic).  Every lane of the wave calls it.
__device__ __forceinline__ void track_absmax(unsigned *word, float v) {
    float a = fabsf(v);
    a = a < INFINITY ? a : 0.0f;
    a = wave_max(a);
    if ((threadIdx.x & 63) == 0 && a > __uint_as_float(*word)) atomicMax(word, __float_as_uint(a));
}

// The LM head's prologue after the slot sum (lm_head.rs:35-54): pv[e] holds the sum over the
// slots, in slot order, of element lane + 64e of one token's rows (zeros past the row for e >=
// er).  pooled = pv / H (stored when `pooled` is set), pnorm = (pooled / rms) * g with eps 1e-5
// (g null = 1), stored in fp32, or (pre > 0) as the split GEMM's pre-split A operand of pnorm *
// pre: fp16 halves hi = f16(x), lo = f16(x - hi), each 8 consecutive elements as 8 hi halves then
// 8 lo halves.  One wave per token; every kernel that pools calls this, so that they agree bit
// for bit.
template <int E>
__device__ __forceinline__ void pool_finish(float (&pv)[E], int H, int d, int er, int lane, long t, const float *g,
                                            float *pooled, float *pnorm, float pre) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        pv[e] = pv[e] / (float)H;
        if (pooled && e < er) pooled[t * d + i] = pv[e];
        ss += pv[e] * pv[e];
    }
    if (!pnorm) return;
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-5f);
    if (pre > 0.0f) {
        _Float16 *row = reinterpret_cast<_Float16 *>(pnorm + t * d);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = lane + 64 * e;
            if (e < er) {
                const float x = ((pv[e] / rms) * (g ? g[i] : 1.0f)) * pre;
                const _Float16 hv = (_Float16)x;
                row[(i >> 3) * 16 + (i & 7)] = hv;
                row[(i >> 3) * 16 + 8 + (i & 7)] = (_Float16)(x - (float)hv);
            }
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        if (e < er) pnorm[t * d + i] = (pv[e] / rms) * (g ? g[i] : 1.0f);
    }
}

// Sequential-in-slot order of the reference is kept where it matters (pooling); wave
// reductions are tree-ordered (fp32 reassociation within the parity tolerance).

}  // namespace adn

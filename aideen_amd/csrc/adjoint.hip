// Clean adjoint Picard, the reference's backward for the DEQ solve
// (staged_adjoint_picard_clean.wgsl:143-337; driver gpu_deq.rs:4736-4975).  Per (token, slot) row,
// with pre = signal + h* (the forward's stored signal and fixed point) and rhs = dl[t] / H
// (dl = dL/d pooled h*):
//   v_0 = rhs,   v_{k+1} = rhs + N^T(beta v_k) + (1 - beta) v_k,
//   N^T(u)_i = (g_i / rms) u_i - pre_i (sum_j u_j g_j pre_j) / (d rms^3),  rms = sqrt(mean pre^2 + 1e-6)
// (the RMSNorm vector-Jacobian product; attention is left out of this adjoint, as in the
// reference), optionally Anderson-mixed per token after every step (the forward's mixing kernel);
// then the source gradient src[t] = sum over slots of N^T(beta v*).
//   k_adj_first:  pre, the row's 1/rms and 1/(d rms^3), and the first step from v_0 = rhs
//   k_adj_prep:   the same preparation with v_0 stored, when no step is asked for
//   k_adj_step:   one Picard step (one wave per row; pre is reused, only the coefficient reduces)
// The last step writes the caller's v_out directly.
//   k_adj_source: per token, the slots' N^T(beta v*) summed in slot order
#include "kernels.h"

namespace adn {

namespace {

constexpr int AW = 4;  // waves per block

template <int E, bool PART>
__global__ __launch_bounds__(64 * AW) void k_adj_prep(int H, int dd, const float *signal, const float *h_star,
                                                       const float *dl, int rows, float *pre, float *terms,
                                                       float *v0) {
    const int d = PART ? dd : 64 * E, er = PART ? dd / 64 : E;  // chunks e >= er are outside the row
    const int row = blockIdx.x * AW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int t = row / H;
    const long o = (long)row * d;
    const float rhs_scale = 1.0f / fmaxf(1.0f, (float)H);
    // every load before the first store (a load issued after stores is waited for behind them)
    float pv[E], rv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        pv[e] = on ? signal[o + i] + 1.0f * h_star[o + i] : 0.0f;
        rv[e] = on ? dl[(long)t * d + i] : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        if (!PART || e < er) {
            pre[o + i] = pv[e];
            v0[o + i] = rv[e] * rhs_scale;
        }
        ss += pv[e] * pv[e];
    }
    ss = wave_sum(ss);
    if (lane == 0) {
        const float rms = sqrtf(ss * (1.0f / (float)d) + 1.0e-6f);
        terms[2 * row] = 1.0f / fmaxf(rms, 1.0e-6f);
        terms[2 * row + 1] = 1.0f / fmaxf((float)d * rms * rms * rms, 1.0e-6f);
    }
}

// the first step fused with the preparation: v_0 = rhs is formed in registers (never stored)
template <int E, bool PART>
__global__ __launch_bounds__(64 * AW) void k_adj_first(int H, int dd, const float *signal, const float *h_star,
                                                        const float *g, const float *dl, int rows, float beta,
                                                        float *pre, float *terms, float *vn) {
    const int d = PART ? dd : 64 * E, er = PART ? dd / 64 : E;  // chunks e >= er are outside the row
    const int row = blockIdx.x * AW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int t = row / H;
    const long o = (long)row * d;
    const float rhs_scale = 1.0f / fmaxf(1.0f, (float)H);
    float pv[E], rv[E], gv[E];
    // every load before the first store (a load issued after stores is waited for behind them)
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        pv[e] = on ? signal[o + i] + 1.0f * h_star[o + i] : 0.0f;
        rv[e] = on ? dl[(long)t * d + i] * rhs_scale : 0.0f;
        gv[e] = on ? g[i] : 0.0f;
    }
    float ss = 0.0f, cf = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (!PART || e < er) pre[o + lane + 64 * e] = pv[e];
        ss += pv[e] * pv[e];
        cf += beta * rv[e] * gv[e] * pv[e];
    }
    ss = wave_sum(ss);
    cf = wave_sum(cf);
    const float rms = sqrtf(ss * (1.0f / (float)d) + 1.0e-6f);
    const float inv_rms = 1.0f / fmaxf(rms, 1.0e-6f);
    const float cden = 1.0f / fmaxf((float)d * rms * rms * rms, 1.0e-6f);
    if (lane == 0) {
        terms[2 * row] = inv_rms;
        terms[2 * row + 1] = cden;
    }
    const float cs = cf * cden;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float ng = (gv[e] * inv_rms) * (beta * rv[e]) - pv[e] * cs;
        if (!PART || e < er) vn[o + lane + 64 * e] = rv[e] + (1.0f * ng + (1.0f - beta) * rv[e]);
    }
}

template <int E, bool PART>
__global__ __launch_bounds__(64 * AW) void k_adj_step(int H, int dd, const float *pre, const float *terms,
                                                       const float *g, const float *dl, int rows, float beta,
                                                       const float *v, float *vn) {
    const int d = PART ? dd : 64 * E, er = PART ? dd / 64 : E;  // chunks e >= er are outside the row
    const int row = blockIdx.x * AW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int t = row / H;
    const long o = (long)row * d;
    const float rhs_scale = 1.0f / fmaxf(1.0f, (float)H);
    float pv[E], vv[E], gv[E], rv[E];
    float cf = 0.0f;
    // every load (dl too) before the first store: a load issued after stores is waited for
    // behind them
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        pv[e] = on ? pre[o + i] : 0.0f;
        vv[e] = on ? v[o + i] : 0.0f;
        gv[e] = on ? g[i] : 0.0f;
        rv[e] = on ? dl[(long)t * d + i] : 0.0f;
        cf += beta * vv[e] * gv[e] * pv[e];
    }
    const float inv_rms = terms[2 * row];
    const float cs = wave_sum(cf) * terms[2 * row + 1];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const float ng = (gv[e] * inv_rms) * (beta * vv[e]) - pv[e] * cs;
        if (!PART || e < er) vn[o + i] = rv[e] * rhs_scale + (1.0f * ng + (1.0f - beta) * vv[e]);
    }
}

template <int E, bool PART>
__global__ __launch_bounds__(64 * AW) void k_adj_source(int H, int dd, const float *pre, const float *terms,
                                                         const float *g, int ntok, float beta, const float *v,
                                                         float *src) {
    const int d = PART ? dd : 64 * E, er = PART ? dd / 64 : E;  // chunks e >= er are outside the row
    const int t = blockIdx.x * AW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= ntok) return;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    for (int s = 0; s < H; ++s) {
        const int row = t * H + s;
        const long o = (long)row * d;
        float pv[E], up[E];
        float cf = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = lane + 64 * e;
            const bool on = !PART || e < er;  // zeros outside the row add nothing below
            pv[e] = on ? pre[o + i] : 0.0f;
            up[e] = on ? beta * v[o + i] : 0.0f;
            cf += up[e] * (on ? g[i] : 0.0f) * pv[e];
        }
        const float inv_rms = terms[2 * row];
        const float cs = wave_sum(cf) * terms[2 * row + 1];
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (!PART || e < er) acc[e] = acc[e] + ((g[lane + 64 * e] * inv_rms) * up[e] - pv[e] * cs);
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (!PART || e < er) src[(long)t * d + lane + 64 * e] = acc[e];
}

__global__ void k_iota(int32_t *a, int n, int32_t *cnt) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = i;
    if (i == 0) cnt[0] = n;
}

template <int E, bool PART>
const float *adj_run(const Dims &D, const AdjointArgs &a, hipStream_t st) {
    const int rows = a.ntok * D.H;
    const dim3 rg((unsigned)((rows + AW - 1) / AW)), blk(64 * AW);
    // step k writes dst(k); the last one writes v_out directly when the caller asked for it
    auto dst = [&](int k) { return (k == a.iters - 1 && a.v_out) ? a.v_out : ((k & 1) ? a.v1 : a.v0); };
    float *v;
    if (a.iters == 0) {
        v = a.v_out ? a.v_out : a.v0;
        hipLaunchKernelGGL((k_adj_prep<E, PART>), rg, blk, 0, st, D.H, D.d, a.signal, a.h_star, a.dl, rows, a.pre, a.terms, v);
    } else {
        v = dst(0);
        hipLaunchKernelGGL((k_adj_first<E, PART>), rg, blk, 0, st, D.H, D.d, a.signal, a.h_star, a.g, a.dl, rows, a.beta, a.pre,
                           a.terms, v);
    }
    SolveBuffers b = a.sb;
    if (a.anderson_m > 0) {
        b.act[0] = a.act;
        b.cnt = a.cnt;
        hipLaunchKernelGGL(k_iota, dim3((unsigned)((a.ntok + 255) / 256)), dim3(256), 0, st, a.act, a.ntok, a.cnt);
    }
    for (int k = 0; k < a.iters; ++k) {
        float *vn = dst(k);
        if (k > 0)
            hipLaunchKernelGGL((k_adj_step<E, PART>), rg, blk, 0, st, D.H, D.d, a.pre, a.terms, a.g, a.dl, rows, a.beta, v, vn);
        if (a.anderson_m > 0) {  // store the new iterate, mix from the third step (per token)
            b.h = vn;
            launch_anderson(D, b, 0, a.ntok, a.ntok, k, a.anderson_m, st);
        }
        v = vn;
    }
    if (a.src)
        hipLaunchKernelGGL((k_adj_source<E, PART>), dim3((unsigned)((a.ntok + AW - 1) / AW)), blk, 0, st, D.H, D.d, a.pre,
                           a.terms, a.g, a.ntok, a.beta, v, a.src);
    return v;
}

}  // namespace

const float *launch_adjoint(const Dims &D, const AdjointArgs &a, hipStream_t st) {
    const float *v = nullptr;
    dispatch_width(D.d, [&](auto Ec, auto Pc) { v = adj_run<decltype(Ec)::value, decltype(Pc)::value>(D, a, st); });
    return v;
}

}  // namespace adn

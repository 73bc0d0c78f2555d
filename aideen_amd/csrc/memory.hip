// Memory-coupled solve (the trainer's fixed-history mode, trainer.rs:677-720): tokens of a
// sequence are solved one position at a time, all sequences of the batch together.  Per
// position t:
//   k_mem_begin   active list = the B tokens (b, t)
//   GEMM          u = W_hist m_{t-1}                      (shared W_hist, rows = (b, slot))
//   k_hist_ctx    hist = u' * alpha * min(1, rms(signal)/rms(u')),  u' = u + scale * m/rms(m)
//                 (fixed_point_memory_reasoning.rs:1337-1370)
//   Picard iterations over the B tokens with hist added to the update
//   k_temporal    m_inner = abar m_{t-1} + (1 - abar) x,  x = u(1 + 0.5 tanh wx),  u = h*/rms(h*)
//   GEMM          m_t = m_inner + W_out m_inner           (fixed_point_memory_reasoning.rs:1454-1485)
// One wave per (sequence, slot) row in the elementwise kernels; the rows are d floats wide.
#include "kernels.h"

namespace adn {

namespace {

constexpr int MW = 4;  // waves per block

__global__ void k_mem_begin(SolveBuffers b, int B, int T, int t) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) b.act[0][i] = i * T + t;
    if (i == 0) {
        b.cnt[0] = B;
        b.cnt[1] = 0;
    }
}

// hist holds u = W_hist m_prev on entry ([B][H][d]); m_prev rows are m_prev + b*m_sm + s*d.
// E = d/64 values per lane, held in registers: every load of the row is issued before the
// first store (a load issued after stores is waited for behind them), and u is not re-read.
template <int E, bool PART>
__global__ __launch_bounds__(64 * MW) void k_hist_ctx(Dims D, float *hist, const float *m_prev, long m_sm,
                                                      const float *signal, int B, int T, int t,
                                                      const float *slot_scale, const float *gate_logit) {
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const int row = blockIdx.x * MW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int H = D.H;
    if (row >= B * H) return;
    const int bb = row / H, s = row - bb * H;
    float *u = hist + (long)row * d;
    const float *pm = m_prev + (long)bb * m_sm + (long)s * d;
    const float *sg = signal + ((long)(bb * T + t) * H + s) * d;
    const float *sc = slot_scale + (long)s * d;
    float vs[E], vp[E], vu[E], vc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        vs[e] = on ? sg[i] : 0.0f;
        vp[e] = on ? pm[i] : 0.0f;
        vu[e] = on ? u[i] : 0.0f;
        vc[e] = on ? sc[i] : 0.0f;
    }
    float ssg = 0.0f, spm = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        ssg += vs[e] * vs[e];
        spm += vp[e] * vp[e];
    }
    const float inj_rms = sqrtf(wave_sum(ssg) / (float)d + 1e-6f);
    const float prev_rms = sqrtf(wave_sum(spm) / (float)d + 1e-6f);
    float su = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        vu[e] = vu[e] + vc[e] * (vp[e] / prev_rms);
        su += vu[e] * vu[e];
    }
    const float u_rms = sqrtf(wave_sum(su) / (float)d + 1e-6f);
    const float scale = u_rms > 1e-6f ? fminf(inj_rms / u_rms, 1.0f) : 1.0f;
    const float sigma = 1.0f / (1.0f + expf(-gate_logit[s]));
    const float g = (0.070f + (0.20f - 0.070f) * sigma) * scale;
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (!PART || e < er) u[lane + 64 * e] = vu[e] * g;
}

// m_inner for the tokens at position t; m_prev == nullptr is the zero state.  E = d/64 values
// per lane in registers, all loads before the stores.
template <int E, bool PART>
__global__ __launch_bounds__(64 * MW) void k_temporal(Dims D, const float *h, int B, int T, int t,
                                                      const float *m_prev, long m_sm, const float *a_log,
                                                      const float *wx_diag, float *out, long out_sm,
                                                      unsigned *amax) {
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const int row = blockIdx.x * MW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int H = D.H;
    if (row >= B * H) return;
    const int bb = row / H, s = row - bb * H;
    const float *hs = h + ((long)(bb * T + t) * H + s) * d;
    const float *pm = m_prev ? m_prev + (long)bb * m_sm + (long)s * d : nullptr;
    float vh[E], vw[E], va[E], vp[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        vh[e] = on ? hs[i] : 0.0f;
        vw[e] = on ? wx_diag[(long)s * d + i] : 0.0f;
        va[e] = on ? a_log[(long)s * d + i] : 0.0f;
        vp[e] = (on && pm) ? pm[i] : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += vh[e] * vh[e];
    const float rms = sqrtf(wave_sum(ss) / (float)d + 1e-6f);
    float *o = out + (long)bb * out_sm + (long)s * d;
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float u = vh[e] / rms;
        const float wx = 0.5f * tanhf(vw[e]);
        const float x = u + wx * u;
        const float ab = 1.0f / (1.0f + expf(va[e]));
        const float v = ab * vp[e] + (1.0f - ab) * x;
        if (!PART || e < er) {
            o[lane + 64 * e] = v;
            mx = fmaxf(mx, fabsf(v) < INFINITY ? fabsf(v) : 0.0f);
        }
    }
    if (amax) track_absmax(amax, mx);  // the bound the next GEMMs scale this state by
}

}  // namespace

void launch_mem_begin(const SolveBuffers &b, int B, int T, int t, hipStream_t st) {
    hipLaunchKernelGGL(k_mem_begin, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, b, B, T, t);
}

void launch_hist_ctx(const Dims &D, float *hist, const float *m_prev, long m_sm, const float *signal, int B,
                     int T, int t, const float *slot_scale, const float *gate_logit, hipStream_t st) {
    const int rows = B * D.H;
    const dim3 grid((unsigned)((rows + MW - 1) / MW)), blk(64 * MW);
dispatch_width(D.d, [&](auto Ec, auto Pc) {
        hipLaunchKernelGGL((k_hist_ctx<decltype(Ec)::value, decltype(Pc)::value>), grid, blk, 0, st, D, hist, m_prev,
                           m_sm, signal, B, T, t, slot_scale, gate_logit);
    });
}

void launch_temporal(const Dims &D, const float *h, int B, int T, int t, const float *m_prev, long m_sm,
                     const float *a_log, const float *wx_diag, float *out, long out_sm, unsigned *amax,
                     hipStream_t st) {
    const int rows = B * D.H;
    const dim3 grid((unsigned)((rows + MW - 1) / MW)), blk(64 * MW);
dispatch_width(D.d, [&](auto Ec, auto Pc) {
        hipLaunchKernelGGL((k_temporal<decltype(Ec)::value, decltype(Pc)::value>), grid, blk, 0, st, D, h, B, T, t,
                           m_prev, m_sm, a_log, wx_diag, out, out_sm, amax);
    });
}

}  // namespace adn

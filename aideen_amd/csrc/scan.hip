// Temporal carrier after the solve: chunked parallel selective scan over time.
//
// Reference: FixedPointMemoryReasoning::temporal_step (fixed_point_memory_reasoning.rs:1455-1486)
// with the selective decay of gpu_deq.rs:6129-6214 and the diagonal readout carrier of
// deq_slot_attn_unified_clean.wgsl:2109-2140, generalised to N states per channel:
//   u = h*/rms(h*), x = u + 0.5 tanh(wx) u,
//   delta = softplus(b_delta + W_vw^T (W_kw^T u)),  abar = 0.1 + 0.9 sigmoid(-a_log)^delta
//   (non-selective: abar = sigmoid(-a_log)),
//   m_t[n] = abar m_{t-1}[n] + (1-abar) B_t[n] x,   y_t = sum_n C_t[n] m_t[n],
//   Y_t = y_t + W_out y_t (readout GEMM, gemm.hip).
//
// k_scan_prep: one wave per (token, slot) computes the per-row record
//   [rms, bn[0..r), B[0..N), C[0..N)]  (the rank-r bottleneck and the B/C projections).
// k_scan: one thread per (sequence, slot, channel) carries the N states in registers; the
//   record of each step is read with uniform (scalar) loads.  Long sequences are split into
//   chunks: pass A (zero start) produces each chunk's end state and decay product, pass B
//   carries the chunk starts sequentially, pass C re-runs every chunk from its start.
#include "kernels.h"

namespace adn {

namespace {

constexpr int WPB = 4;

__global__ __launch_bounds__(256) void k_scan_prep(Dims D, const float *h, int ntok,
                                                   const float *w_kw, const float *w_b,
                                                   const float *w_c, float *rec) {
    const int row = blockIdx.x * WPB + (threadIdx.x >> 6);  // (t, s)
    const int lane = threadIdx.x & 63;
    if (row >= ntok * D.H) return;
    const int s = row % D.H;
    const int d = D.d, r = D.r, N = D.N;
    const int REC = 1 + r + 2 * N;
    const float *hr = h + (long)row * d;
    float ss = 0.0f;
    for (int i = lane; i < d; i += 64) ss += hr[i] * hr[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-6f);
    float *out = rec + (long)row * REC;
    if (lane == 0) out[0] = rms;
    if (D.flags & ADN_F_SCAN_SELECTIVE) {
        const float *wk = w_kw + (long)s * d * r;
        for (int j = 0; j < r; ++j) {
            float p = 0.0f;
            for (int i = lane; i < d; i += 64) p += wk[(long)i * r + j] * (hr[i] / rms);
            p = wave_sum(p);
            if (lane == 0) out[1 + j] = p;
        }
    }
    for (int n = 0; n < N; ++n) {
        float pb = 1.0f, pc = 1.0f;
        if (w_b) {
            const float *wb = w_b + ((long)s * N + n) * d;
            const float *wc = w_c + ((long)s * N + n) * d;
            pb = 0.0f;
            pc = 0.0f;
            for (int i = lane; i < d; i += 64) {
                const float u = hr[i] / rms;
                pb += wb[i] * u;
                pc += wc[i] * u;
            }
            pb = wave_sum(pb);
            pc = wave_sum(pc);
        }
        if (lane == 0) {
            out[1 + r + n] = pb;
            out[1 + r + N + n] = pc;
        }
    }
}

// MODE 0: full scan from state_in, emit y and state_out (single chunk).
// MODE 1: chunk pass A, zero start, emit chunk end state and decay product.
// MODE 2: chunk pass C, start from chunk_s (carried), emit y; last chunk writes state_out.
template <int NS, int RK, int MODE>
__global__ __launch_bounds__(256) void k_scan(Dims D, const float *h, const float *rec, int T,
                                              int nch, const float *a_log, const float *wx_diag,
                                              const float *b_delta, const float *w_vw,
                                              const float *state_in, float *y, float *state_out,
                                              float *chunk_s, float *chunk_p) {
    const int d = D.d, H = D.H, N = D.N, r = D.r;
    const int dim = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    const int bc = blockIdx.z;
    const int b = bc / nch, c = bc - (bc / nch) * nch;
    if (dim >= d) return;
    const int REC = 1 + r + 2 * N;
    const int Tc = (T + nch - 1) / nch;
    const int t0 = c * Tc, t1 = min(T, t0 + Tc);
    const bool selective = (D.flags & ADN_F_SCAN_SELECTIVE) != 0;

    const float al = a_log[(long)s * d + dim];
    const float abase = 1.0f / (1.0f + expf(al));
    const float ln_ab = logf(fmaxf(abase, 1.0e-6f));
    const float wx = 0.5f * tanhf(wx_diag[(long)s * d + dim]);
    const float bd = b_delta ? b_delta[(long)s * d + dim] : 0.0f;
    float wv[RK];
    if (selective) {
#pragma unroll
        for (int j = 0; j < RK; ++j) wv[j] = j < r ? w_vw[((long)s * r + j) * d + dim] : 0.0f;
    }
    float m[NS];
    const long st_off = (((long)b * H + s) * d + dim) * N;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        m[n] = 0.0f;
        if (n < N) {
            if (MODE == 0 && state_in) m[n] = state_in[st_off + n];
            if (MODE == 2) m[n] = chunk_s[((((long)b * nch + c) * H + s) * d + dim) * N + n];
        }
    }
    float prod = 1.0f;
    for (int t = t0; t < t1; ++t) {
        const long row = ((long)b * T + t) * H + s;
        const float *rc = rec + row * REC;
        const float u = h[row * d + dim] / rc[0];
        const float x = u + wx * u;
        float abar;
        if (selective) {
            float pre = bd;
#pragma unroll
            for (int j = 0; j < RK; ++j)
                if (j < r) pre += wv[j] * rc[1 + j];
            const float delta = logf(1.0f + expf(pre));
            const float acore = expf(delta * ln_ab);
            abar = 0.10f + (1.0f - 0.10f) * acore;
        } else {
            abar = abase;
        }
        const float bb = 1.0f - abar;
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < NS; ++n) {
            if (n < N) {
                m[n] = abar * m[n] + bb * (rc[1 + r + n] * x);
                acc += rc[1 + r + N + n] * m[n];
            }
        }
        if (MODE == 1)
            prod *= abar;
        else
            y[row * d + dim] = acc;
    }
    if (MODE == 1) {
        const long co = (((long)b * nch + c) * H + s) * d + dim;
        chunk_p[co] = prod;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) chunk_s[co * N + n] = m[n];
    } else if (state_out && (MODE == 0 || c == nch - 1)) {
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) state_out[st_off + n] = m[n];
    }
}

// Pass B: chunk starts.  One thread per (b, s, dim, n): carry_0 = state_in; the start of
// chunk c replaces its end state in chunk_s; carry_{c+1} = P_c carry_c + S_c.
__global__ void k_scan_carry(Dims D, int B, int nch, const float *state_in, float *chunk_s,
                             const float *chunk_p) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int d = D.d, H = D.H, N = D.N;
    const long total = (long)B * H * d * N;
    if (idx >= total) return;
    const int n = idx % N;
    const long bsd = idx / N;  // ((b*H + s)*d + dim)
    const int dim = bsd % d;
    const long bs = bsd / d;
    const int s = bs % H;
    const int b = (int)(bs / H);
    float carry = state_in ? state_in[idx] : 0.0f;
    for (int c = 0; c < nch; ++c) {
        const long co = (((long)b * nch + c) * H + s) * d + dim;
        const float sc = chunk_s[co * N + n];
        chunk_s[co * N + n] = carry;
        carry = chunk_p[co] * carry + sc;
    }
}

template <int NS, int RK>
void scan_modes(const Dims &D, const float *h, const float *rec, int B, int T, const float *a_log,
                const float *wx_diag, const float *b_delta, const float *w_vw,
                const float *state_in, float *y, float *state_out, float *chunk_s, float *chunk_p,
                int nch, hipStream_t st) {
    const int bx = D.d < 256 ? D.d : 256;
    const dim3 grid((unsigned)((D.d + bx - 1) / bx), (unsigned)D.H, (unsigned)(B * nch));
    if (nch <= 1) {
        hipLaunchKernelGGL((k_scan<NS, RK, 0>), grid, dim3(bx), 0, st, D, h, rec, T, 1, a_log, wx_diag,
                           b_delta, w_vw, state_in, y, state_out, chunk_s, chunk_p);
        return;
    }
    hipLaunchKernelGGL((k_scan<NS, RK, 1>), grid, dim3(bx), 0, st, D, h, rec, T, nch, a_log, wx_diag,
                       b_delta, w_vw, state_in, y, state_out, chunk_s, chunk_p);
    const long total = (long)B * D.H * D.d * D.N;
    hipLaunchKernelGGL(k_scan_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, D, B, nch,
                       state_in, chunk_s, chunk_p);
    hipLaunchKernelGGL((k_scan<NS, RK, 2>), grid, dim3(bx), 0, st, D, h, rec, T, nch, a_log, wx_diag,
                       b_delta, w_vw, state_in, y, state_out, chunk_s, chunk_p);
}

}  // namespace

int scan_rec_len(const Dims &D) { return 1 + D.r + 2 * D.N; }

int scan_chunks(int B, int T, int H, int d) {
    const long waves = (long)B * H * ((d + 63) / 64);
    int nch = 1;
    while (waves * nch < 4096 && T / (nch * 2) >= 64) nch *= 2;
    return nch;
}

void launch_scan_prep(const Dims &D, const float *h, int ntok, const float *w_kw, const float *w_b,
                      const float *w_c, float *rec, hipStream_t st) {
    const long rows = (long)ntok * D.H;
    hipLaunchKernelGGL(k_scan_prep, dim3((unsigned)((rows + WPB - 1) / WPB)), dim3(64 * WPB), 0, st, D, h,
                       ntok, w_kw, w_b, w_c, rec);
}

void launch_scan(const Dims &D, const float *h, const float *rec, int B, int T, const float *a_log,
                 const float *wx_diag, const float *b_delta, const float *w_vw, const float *state_in,
                 float *y, float *state_out, float *chunk_s, float *chunk_p, int nch, hipStream_t st) {
    // register budget: NS >= N states, RK >= r rank entries
    if (D.N <= 16) {
        if (D.r <= 32)
            scan_modes<16, 32>(D, h, rec, B, T, a_log, wx_diag, b_delta, w_vw, state_in, y, state_out,
                               chunk_s, chunk_p, nch, st);
        else
            scan_modes<16, 64>(D, h, rec, B, T, a_log, wx_diag, b_delta, w_vw, state_in, y, state_out,
                               chunk_s, chunk_p, nch, st);
    } else {
        if (D.r <= 32)
            scan_modes<32, 32>(D, h, rec, B, T, a_log, wx_diag, b_delta, w_vw, state_in, y, state_out,
                               chunk_s, chunk_p, nch, st);
        else
            scan_modes<32, 64>(D, h, rec, B, T, a_log, wx_diag, b_delta, w_vw, state_in, y, state_out,
                               chunk_s, chunk_p, nch, st);
    }
}

}  // namespace adn

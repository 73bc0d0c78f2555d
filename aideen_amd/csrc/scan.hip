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
// Pipeline: k_row_rms (rms of every (token, slot) row) and one MFMA GEMM against the per-slot
//   W_cat[s] = [W_kw[s]^T; W_B[s]; W_C[s]]  (r + 2N rows of length d)
// fill the per-row record [rms, P_bn[0..r), P_B[0..N), P_C[0..N)] with un-normalised
// projections P = W_cat h; the scan divides them by rms as it stages them.
// k_scan_gate: the per-element decay and input (all transcendental and rank-r work), fully
//   parallel over (token, slot, channel).
// k_scan: one thread per (sequence, slot, channel) carries the N states in registers; per chunk
//   of TC steps the B/C values are staged in LDS and the gate values prefetched into registers.
//   Long sequences are split into time chunks: pass A (zero start) produces each chunk's end
//   state and decay product, pass B carries the chunk starts, pass C re-runs every chunk.
#include "kernels.h"

namespace adn {

namespace {

constexpr int WPB = 4;

// E = d/64 values per lane, all loaded before the sum (in the same order as a strided loop)
template <int E>
__global__ __launch_bounds__(256) void k_row_rms(const float *h, long rows, float *rec, int REC) {
    constexpr int d = 64 * E;
    const long row = (long)blockIdx.x * WPB + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *hr = h + row * d;
    float x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = hr[lane + 64 * e];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[e] * x[e];
    ss = wave_sum(ss);
    if (lane == 0) rec[row * REC] = sqrtf(ss / (float)d + 1e-6f);
}

constexpr int SCAN_NT = 256;
constexpr int TC = 16;
constexpr int GATE_ROWS = 16;

// Gate: for every (token, slot, channel) the decay abar and the carrier input (1-abar) x,
// fully parallel (the rank-r bottleneck comes from the record; W_vw's column for the channel
// is held in registers across GATE_ROWS tokens of one slot).  The block's GATE_ROWS records
// (rms and the r projections) are staged in LDS, and a thread loads all of its h values before
// its first store: a load issued after stores would be waited for behind them (the
// vector-memory counter retires in issue order).
template <int RK, bool SEL>
__global__ __launch_bounds__(SCAN_NT) void k_scan_gate(Dims D, const float *__restrict__ h,
                                                       const float *__restrict__ rec, int ntok,
                                                       const float *__restrict__ a_log,
                                                       const float *__restrict__ wx_diag,
                                                       const float *__restrict__ b_delta,
                                                       const float *__restrict__ w_vw,
                                                       float *__restrict__ gate_a, float *__restrict__ gate_x) {
    constexpr int RKA = RK > 0 ? RK : 1;
    constexpr int RS = 4 + RKA;  // [0] rms, [4 + q] projection q (16-byte aligned for broadcast reads)
    __shared__ __attribute__((aligned(16))) float srec[GATE_ROWS][RS];
    const int d = D.d, H = D.H, r = D.r;
    const int dim = blockIdx.x * SCAN_NT + threadIdx.x;
    const int s = blockIdx.y;
    const int t0 = blockIdx.z * GATE_ROWS;
    const int REC = 1 + D.r + 2 * D.N;
    const int nrow = min(ntok - t0, GATE_ROWS);
    for (int idx = threadIdx.x; idx < GATE_ROWS * RS; idx += SCAN_NT) {
        const int j = idx / RS, q = idx - j * RS;
        float v = 0.0f;
        if (j < nrow) {
            const float *rc = rec + ((long)(t0 + j) * H + s) * REC;
            if (q == 0)
                v = rc[0];
            else if (SEL && q >= 4 && q - 4 < r)
                v = rc[1 + (q - 4)];
        }
        srec[j][q] = v;
    }
    __syncthreads();
    if (dim >= d) return;
    // h* is not read again after the gate: non-temporal loads keep it from displacing cached data
    float hv[GATE_ROWS];
#pragma unroll
    for (int j = 0; j < GATE_ROWS; ++j) hv[j] = j < nrow ? __builtin_nontemporal_load(h + ((long)(t0 + j) * H + s) * d + dim) : 0.0f;
    const float al = a_log[(long)s * d + dim];
    const float abase = 1.0f / (1.0f + expf(al));
    const float ln_ab = logf(fmaxf(abase, 1.0e-6f));
    const float wx = 0.5f * tanhf(wx_diag[(long)s * d + dim]);
    const float bd = b_delta ? b_delta[(long)s * d + dim] : 0.0f;
    float wv[RKA];
#pragma unroll
    for (int q = 0; q < RKA; ++q) wv[q] = (SEL && q < r) ? w_vw[((long)s * r + q) * d + dim] : 0.0f;
#pragma unroll
    for (int j = 0; j < GATE_ROWS; ++j) {
        if (j >= nrow) continue;
        const long row = (long)(t0 + j) * H + s;
        const float rms = srec[j][0];
        const float u = hv[j] / rms;
        const float x = u + wx * u;
        float abar;
        if (SEL) {
            // W_vw^T (W_kw^T u) with u = h/rms: the record holds W_kw^T h, so divide once (the
            // weights and the staged projections past r are zero)
            float dot = 0.0f;
#pragma unroll
            for (int q = 0; q < RKA; ++q) dot += wv[q] * srec[j][4 + q];
            const float pre = bd + dot / rms;
            const float delta = logf(1.0f + expf(pre));
            const float acore = expf(delta * ln_ab);
            abar = 0.10f + (1.0f - 0.10f) * acore;
        } else {
            abar = abase;
        }
        gate_a[row * d + dim] = abar;
        gate_x[row * d + dim] = (1.0f - abar) * x;
    }
}

// Recurrence over time for one (sequence, slot, channel) per thread, N states in registers:
//   m[n] = abar m[n] + B[n] ((1-abar) x),  y = sum_n C[n] m[n].
// MODE 0: full scan from state_in, emit y and state_out (single chunk).
// MODE 1: chunk pass A, zero start, emit chunk end state and decay product.
// MODE 2: chunk pass C, start from chunk_s (carried), emit y; last chunk writes state_out.
// Per TC steps the B/C values (projection / rms) are staged in LDS and the gate values are
// loaded into registers up front.  EXACT: NS == N (branch-free inner loops).
template <int NS, int MODE, bool EXACT>
__global__ __launch_bounds__(SCAN_NT) void k_scan(Dims D, const float *__restrict__ gate_a,
                                                  const float *__restrict__ gate_x,
                                                  const float *__restrict__ rec, int T, int nch, int has_bc,
                                                  const float *__restrict__ state_in, float *__restrict__ y,
                                                  float *__restrict__ state_out, float *__restrict__ chunk_s,
                                                  float *__restrict__ chunk_p) {
    __shared__ float sbc[TC][2 * NS];
    const int d = D.d, H = D.H;
    const int N = EXACT ? NS : D.N;
    const int tid = threadIdx.x;
    const int dim = blockIdx.x * SCAN_NT + tid;
    const int s = blockIdx.y;
    const int bc = blockIdx.z;
    const int b = bc / nch, c = bc - (bc / nch) * nch;
    const bool active = dim < d;
    const int REC = 1 + D.r + 2 * D.N;
    const int boff = 1 + D.r;
    const int Tc = (T + nch - 1) / nch;
    const int t0 = c * Tc, t1 = min(T, t0 + Tc);
    const int dd = active ? dim : 0;
    float m[NS];
    const long st_off = (((long)b * H + s) * d + dd) * D.N;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        m[n] = 0.0f;
        if (n < N && active) {
            if (MODE == 0 && state_in) m[n] = state_in[st_off + n];
            if (MODE == 2) m[n] = chunk_s[((((long)b * nch + c) * H + s) * d + dd) * D.N + n];
        }
    }
    float prod = 1.0f;
    // Per chunk of TC steps the B/C values (projection / rms) are staged in LDS and the gate
    // values held in registers.  Where y is stored (passes 0 and C) two register sets alternate
    // (the chunk loop is unrolled by two)
    // so that the next chunk's loads are issued before this chunk's y stores: a load issued
    // after stores is waited for behind them (the vector-memory counter retires in issue order).
    // The loads are unconditional, at addresses clamped into the chunk (steps past its end are
    // not used), so that the compiler can count them exactly.
    constexpr int BCP = (TC * 2 * NS + SCAN_NT - 1) / SCAN_NT;  // staged B/C values per thread
    struct Chunk {
        float a[TC], x[TC], bv[BCP], rv[BCP];
    };
    const long tstride = (long)H * d;                          // one time step of (b, s, dim)
    const long gbase = (long)b * T * tstride + (long)s * d + dd;  // (b, t = 0, s, dd)
    const int last = t1 - 1;
    // pass C is the gate values' last use: loaded non-temporally there
    auto fetch = [&](Chunk &k, int tb) {
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const long off = gbase + (long)min(tb + j, last) * tstride;
            k.a[j] = MODE == 2 ? __builtin_nontemporal_load(gate_a + off) : gate_a[off];
            k.x[j] = MODE == 2 ? __builtin_nontemporal_load(gate_x + off) : gate_x[off];
        }
        if (has_bc) {
#pragma unroll
            for (int q2 = 0; q2 < BCP; ++q2) {
                const int idx = min(tid + q2 * SCAN_NT, TC * 2 * N - 1);
                const int j = idx / (2 * N), q = idx - j * 2 * N;
                const float *rc = rec + (((long)b * T + min(tb + j, last)) * H + s) * REC;
                k.bv[q2] = rc[boff + q];
                k.rv[q2] = rc[0];
            }
        }
    };
    auto process = [&](const Chunk &k, int tb) {
        const int nt = min(TC, t1 - tb);
        if (has_bc) {
#pragma unroll
            for (int q2 = 0; q2 < BCP; ++q2) {
                const int idx = tid + q2 * SCAN_NT;
                if (idx < nt * 2 * N) {
                    const int j = idx / (2 * N), q = idx - j * 2 * N;
                    sbc[j][q] = k.bv[q2] / k.rv[q2];
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            if (j < nt) {
                float acc = 0.0f;
#pragma unroll
                for (int n = 0; n < NS; ++n) {
                    if (EXACT || n < N) {
                        const float Bn = has_bc ? sbc[j][n] : 1.0f;
                        const float Cn = has_bc ? sbc[j][N + n] : 1.0f;
                        m[n] = k.a[j] * m[n] + Bn * k.x[j];
                        acc += Cn * m[n];
                    }
                }
                if (MODE == 1)
                    prod *= k.a[j];
                else if (active)
                    y[gbase + (long)(tb + j) * tstride] = acc;
            }
        }
        __syncthreads();
    };
    // (the fetches are unconditional too: past the end they re-read the last step, unused).
    // Pass A stores nothing in the loop, so there one register set serves.
    Chunk ca;
    if constexpr (MODE == 1) {
        for (int tb = t0; tb < t1; tb += TC) {
            fetch(ca, tb);
            process(ca, tb);
        }
    } else {
        Chunk cb;
        if (t0 < t1) fetch(ca, t0);
        for (int tb = t0; tb < t1; tb += 2 * TC) {
            fetch(cb, tb + TC);
            process(ca, tb);
            if (tb + TC >= t1) break;
            fetch(ca, tb + 2 * TC);
            process(cb, tb + TC);
        }
    }
    if (!active) return;
    if (MODE == 1) {
        const long co = (((long)b * nch + c) * H + s) * d + dd;
        chunk_p[co] = prod;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) chunk_s[co * D.N + n] = m[n];
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

template <int NS, bool EXACT>
void scan_modes(const Dims &D, const float *ga, const float *gx, const float *rec, int B, int T, int has_bc,
                const float *state_in, float *y, float *state_out, float *chunk_s, float *chunk_p, int nch,
                hipStream_t st) {
    const dim3 grid((unsigned)((D.d + SCAN_NT - 1) / SCAN_NT), (unsigned)D.H, (unsigned)(B * nch));
    if (nch <= 1) {
        hipLaunchKernelGGL((k_scan<NS, 0, EXACT>), grid, dim3(SCAN_NT), 0, st, D, ga, gx, rec, T, 1, has_bc,
                           state_in, y, state_out, chunk_s, chunk_p);
        return;
    }
    hipLaunchKernelGGL((k_scan<NS, 1, EXACT>), grid, dim3(SCAN_NT), 0, st, D, ga, gx, rec, T, nch, has_bc,
                       state_in, y, state_out, chunk_s, chunk_p);
    const long total = (long)B * D.H * D.d * D.N;
    hipLaunchKernelGGL(k_scan_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, D, B, nch,
                       state_in, chunk_s, chunk_p);
    hipLaunchKernelGGL((k_scan<NS, 2, EXACT>), grid, dim3(SCAN_NT), 0, st, D, ga, gx, rec, T, nch, has_bc,
                       state_in, y, state_out, chunk_s, chunk_p);
}

}  // namespace

int scan_rec_len(const Dims &D) { return 1 + D.r + 2 * D.N; }

int scan_chunks(int B, int T, int H, int d) {
    const long wgs = (long)B * H * ((d + SCAN_NT - 1) / SCAN_NT);
    int nch = 1;
    while (wgs * nch < 2048 && T / (nch * 2) >= 4 * TC) nch *= 2;
    return nch;
}

void launch_row_rms(const float *h, long rows, int d, float *rec, int REC, hipStream_t st) {
    const dim3 grid((unsigned)((rows + WPB - 1) / WPB)), blk(64 * WPB);
    switch (d) {
        case 64: hipLaunchKernelGGL(k_row_rms<1>, grid, blk, 0, st, h, rows, rec, REC); break;
        case 128: hipLaunchKernelGGL(k_row_rms<2>, grid, blk, 0, st, h, rows, rec, REC); break;
        case 256: hipLaunchKernelGGL(k_row_rms<4>, grid, blk, 0, st, h, rows, rec, REC); break;
        case 512: hipLaunchKernelGGL(k_row_rms<8>, grid, blk, 0, st, h, rows, rec, REC); break;
        case 1024: hipLaunchKernelGGL(k_row_rms<16>, grid, blk, 0, st, h, rows, rec, REC); break;
        case 2048: hipLaunchKernelGGL(k_row_rms<32>, grid, blk, 0, st, h, rows, rec, REC); break;
        default: break;  // rejected at context creation
    }
}

void launch_scan_gate(const Dims &D, const float *h, const float *rec, int ntok, const float *a_log,
                      const float *wx_diag, const float *b_delta, const float *w_vw, float *gate_a, float *gate_x,
                      hipStream_t st) {
    const dim3 grid((unsigned)((D.d + SCAN_NT - 1) / SCAN_NT), (unsigned)D.H,
                    (unsigned)((ntok + GATE_ROWS - 1) / GATE_ROWS));
    const bool sel = (D.flags & ADN_F_SCAN_SELECTIVE) != 0;
#define ADN_GATE_ARGS D, h, rec, ntok, a_log, wx_diag, b_delta, w_vw, gate_a, gate_x
    if (!sel)
        hipLaunchKernelGGL((k_scan_gate<0, false>), grid, dim3(SCAN_NT), 0, st, ADN_GATE_ARGS);
    else if (D.r <= 32)
        hipLaunchKernelGGL((k_scan_gate<32, true>), grid, dim3(SCAN_NT), 0, st, ADN_GATE_ARGS);
    else
        hipLaunchKernelGGL((k_scan_gate<64, true>), grid, dim3(SCAN_NT), 0, st, ADN_GATE_ARGS);
#undef ADN_GATE_ARGS
}

void launch_scan(const Dims &D, const float *gate_a, const float *gate_x, const float *rec, int B, int T,
                 int has_bc, const float *state_in, float *y, float *state_out, float *chunk_s, float *chunk_p,
                 int nch, hipStream_t st) {
#define ADN_SCAN_ARGS D, gate_a, gate_x, rec, B, T, has_bc, state_in, y, state_out, chunk_s, chunk_p, nch, st
    if (D.N == 16)
        scan_modes<16, true>(ADN_SCAN_ARGS);
    else if (D.N == 1)
        scan_modes<1, true>(ADN_SCAN_ARGS);
    else if (D.N == 32)
        scan_modes<32, true>(ADN_SCAN_ARGS);
    else if (D.N <= 8)
        scan_modes<8, false>(ADN_SCAN_ARGS);
    else
        scan_modes<32, false>(ADN_SCAN_ARGS);
#undef ADN_SCAN_ARGS
}

}  // namespace adn

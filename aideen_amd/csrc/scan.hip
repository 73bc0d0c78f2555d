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
// Pipeline: the row RMS of every (token, slot) row (k_row_rms, or the pooling kernel from the same
// loads) and one MFMA GEMM against the per-slot
//   W_cat[s] = [W_kw[s]^T; W_B[s]; W_C[s]]  (r + 2N rows of length d)
// fill the per-row record [rms, P_bn[0..r), P_B[0..N), P_C[0..N)] with un-normalised
// projections P = W_cat h.  k_scan_fused then forms each element's decay and input from h* and
// the record and carries the recurrence in the same pass: nothing per element is written but y.
// Sequences too few to fill the GPU are split into time chunks: pass A (zero start) produces
// each chunk's end state and decay product, k_scan_carry the chunk starts, and pass C re-runs
// every chunk from its start.
#include "kernels.h"

namespace adn {

namespace {

constexpr int WPB = 4;
#ifndef SCAN_MIN_WGS
#define SCAN_MIN_WGS 512
#endif

// E = d/64 values per lane, all loaded before the sum (in the same order as a strided loop)
template <int E, bool PART>
__global__ __launch_bounds__(256) void k_row_rms(const float *h, long rows, int dd, float *rec, int REC) {
    const int d = PART ? dd : 64 * E, er = PART ? dd / 64 : E;  // chunks e >= er are outside the row
    const long row = (long)blockIdx.x * WPB + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *hr = h + row * d;
    float x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = (!PART || e < er) ? hr[lane + 64 * e] : 0.0f;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[e] * x[e];
    ss = wave_sum(ss);
    if (lane == 0) rec[row * REC] = sqrtf(ss / (float)d + 1e-6f);
}

constexpr int SCAN_NT = 256;
constexpr int TC = 16;

// Fused gate and recurrence over time, one thread per (sequence, slot, channel) with the N states
// in registers.  Per step the thread forms the gate from h* and the row's record itself
// (selective: u = h / rms, x = u + 0.5 tanh(w_x) u, pre = b + W_vw^T (W_kw^T u),
// abar = 0.1 + 0.9 sigmoid(-a_log)^softplus(pre); otherwise abar = sigmoid(-a_log)), so no
// per-element gate tensor is written or read back:
//   m[n] = abar m[n] + B[n] ((1 - abar) x),   y = sum_n C[n] m[n].
// softplus and the power use the hardware base-2 exponential and logarithm:
//   sigmoid(-a_log)^softplus(pre) = 2^(log2(1 + 2^(pre log2 e)) ln(sigmoid(-a_log))).
// MODE 0: whole sequence from state_in, emit y and state_out.
// MODE 1: chunk pass A, zero start, emit the chunk's end state and decay product.
// MODE 2: chunk pass C, start from chunk_s (carried), emit y; the last chunk writes state_out.
// Per TC steps the record values a step needs (1/rms, the rank-r projections, B and C) are staged
// raw in LDS and the 1/rms scales applied where they are used; h and the next TC steps' record
// values are fetched into a second register set before the current steps are processed (a load
// issued after stores would wait behind them: the vector-memory counter retires in issue order).
// NORM: within a block of TC steps the states are carried divided by the block's running decay
// product P (m = P mh): mh[n] += B[n] (xin / P), y = P sum_n C[n] mh[n], one FMA per state and
// step instead of two; m = P mh at the block's end.  It needs every TC-step decay product to stay
// a normal fp32 number (the selective decay is at least 0.1; a fixed one is checked at upload).
// RK: rank bucket (0 = not selective); EXACT: NS == N.
template <int NS, int RK, int MODE, bool EXACT, bool NORM>
__global__ __launch_bounds__(SCAN_NT) void k_scan_fused(Dims D, const float *__restrict__ h,
                                                        const float *__restrict__ rec, int T, int nch, int has_bc,
                                                        const float *__restrict__ a_log,
                                                        const float *__restrict__ wx_diag,
                                                        const float *__restrict__ b_delta,
                                                        const float *__restrict__ w_vw,
                                                        const float *__restrict__ state_in, float *__restrict__ y,
                                                        float *__restrict__ state_out, float *__restrict__ chunk_s,
                                                        float *__restrict__ chunk_p, unsigned *amax_y) {
    constexpr bool SEL = RK > 0;
    constexpr int RKA = SEL ? RK : 0;
    constexpr int BC0 = 4 + RKA;         // staged step: [0] 1/rms, [4 + q] projection q,
    constexpr int SW = BC0 + 2 * NS;     // [BC0 + n] B[n], [BC0 + NS + n] C[n] (un-normalised)
    constexpr int QMAX = 1 + RKA + 2 * NS;
    constexpr int RPT = (TC * QMAX + SCAN_NT - 1) / SCAN_NT;  // staged values per thread
    __shared__ __attribute__((aligned(16))) float sr[TC][SW];
    float *srf = &sr[0][0];
    // the rank-r term of every step of every channel, [channel][step] (row stride TC + 4: the
    // b128 writes and reads of eight consecutive rows hit distinct banks)
    __shared__ __attribute__((aligned(16))) float sp[SEL ? SCAN_NT : 1][TC + 4];
    const int d = D.d, H = D.H, r = D.r;
    const int N = EXACT ? NS : D.N;
    const int tid = threadIdx.x;
    const int dim = blockIdx.x * SCAN_NT + tid;
    const int s = blockIdx.y;
    const int bc = blockIdx.z;
    const int b = bc / nch, c = bc - (bc / nch) * nch;
    // d is a multiple of 64: a wave's channels are all inside d or all outside (wave-uniform)
    const bool active = __builtin_amdgcn_readfirstlane(dim < d ? 1 : 0) != 0;
    const int REC = 1 + r + 2 * D.N;
    const int Tc = (T + nch - 1) / nch;
    const int t0 = c * Tc, t1 = min(T, t0 + Tc);
    const int dd = active ? dim : 0;
    const int nq = 1 + RKA + 2 * N;  // staged values per step (bucket-padded rank; B = C = 1 without has_bc)
    // this thread's staged values (fixed over the blocks): LDS offset, step, record field; the
    // value staged is 1 / x for the rms, else x * s_mul + s_add (threads without a value write the
    // unused column 1 of step 0)
    int s_off[RPT], s_j[RPT], s_f[RPT];
    bool s_inv[RPT];
    float s_mul[RPT], s_add[RPT];
#pragma unroll
    for (int q2 = 0; q2 < RPT; ++q2) {
        const int idx = tid + q2 * SCAN_NT;
        s_off[q2] = 1;
        s_j[q2] = 0;
        s_f[q2] = 0;
        s_inv[q2] = false;
        s_mul[q2] = 0.0f;
        s_add[q2] = 0.0f;
        if (idx < TC * nq) {
            const int j = idx / nq, q = idx - j * nq;
            const int qb = q - 1 - RKA;  // B[0..N) then C[0..N) in the record; C staged at BC0 + NS
            const int slot = q == 0 ? 0 : (q <= RKA ? 4 + (q - 1) : BC0 + (qb < N ? qb : NS + qb - N));
            const int f = q == 0 ? 0 : (q <= RKA ? (q - 1 < r ? q : -1) : 1 + r + qb);
            const int kind = q == 0 ? 0 : (q <= RKA ? (f >= 0 ? 1 : 3) : (has_bc ? 1 : 2));
            s_off[q2] = j * SW + slot;
            s_j[q2] = j;
            s_f[q2] = f < 0 ? 0 : f;
            s_inv[q2] = kind == 0;
            s_mul[q2] = kind == 1 ? 1.0f : 0.0f;
            s_add[q2] = kind == 2 ? 1.0f : 0.0f;
        }
    }

    // per-channel constants
    const float al = a_log[(long)s * d + dd];
    const float abase = 1.0f / (1.0f + expf(al));
    const float ln_ab = logf(fmaxf(abase, 1.0e-6f));
    const float wxh = 0.5f * tanhf(wx_diag[(long)s * d + dd]);
    const float bd = (SEL && b_delta) ? b_delta[(long)s * d + dd] : 0.0f;
    // W_vw as the B operand of v_mfma_f32_16x16x4f32: per 16-channel tile t of this wave and rank
    // block kb, lane l holds W_vw[s][4 kb + l / 16][channel of tile t, l % 16]
    const int lane = tid & 63, wave = tid >> 6;
    constexpr int KB = SEL ? RKA / 4 : 1;
    float wb[4][KB];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int ch = blockIdx.x * SCAN_NT + wave * 64 + t * 16 + (lane & 15);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const int q = 4 * kb + (lane >> 4);
            wb[t][kb] = (SEL && q < r && ch < d) ? w_vw[((long)s * r + q) * d + ch] : 0.0f;
        }
    }

    float m[NS];
    const long st_off = (((long)b * H + s) * d + dd) * D.N;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        m[n] = 0.0f;
        if ((EXACT || n < N) && active) {
            if (MODE == 0 && state_in) m[n] = state_in[st_off + n];
            if (MODE == 2) m[n] = chunk_s[((((long)b * nch + c) * H + s) * d + dd) * D.N + n];
        }
    }
    float prod = 1.0f;
    float ymax = 0.0f;  // largest finite |y| this thread stores

    struct Chunk {
        float hv[TC], rv[RPT];
    };
    const long tstride = (long)H * d;                          // one time step of (b, s, dim)
    const long gbase = (long)b * T * tstride + (long)s * d + dd;  // (b, t = 0, s, dd)
    const long rstride = (long)H * REC;                        // one time step of the records
    const int last = t1 - 1;
    const float *recb = rec + ((long)b * T * H + s) * REC;
    // h is read again by pass C after pass A (through the caches where it fits): non-temporal
    // only where this is its last read
    auto fetch = [&](Chunk &k, int tb) {
        if (tb + TC <= t1) {  // a whole block of steps: no clamping
            const float *hp = h + gbase + (long)tb * tstride;
#pragma unroll
            for (int j = 0; j < TC; ++j)
                k.hv[j] = MODE == 1 ? hp[(long)j * tstride] : __builtin_nontemporal_load(hp + (long)j * tstride);
        } else {
#pragma unroll
            for (int j = 0; j < TC; ++j) {
                const long off = gbase + (long)min(tb + j, last) * tstride;
                k.hv[j] = MODE == 1 ? h[off] : __builtin_nontemporal_load(h + off);
            }
        }
#pragma unroll
        for (int q2 = 0; q2 < RPT; ++q2) k.rv[q2] = recb[(long)min(tb + s_j[q2], last) * rstride + s_f[q2]];
    };
    auto process = [&](const Chunk &k, int tb) {
        const int nt = min(TC, t1 - tb);
#pragma unroll
        for (int q2 = 0; q2 < RPT; ++q2) {
            const float x = k.rv[q2];
            srf[s_off[q2]] = s_inv[q2] ? __builtin_amdgcn_rcpf(x) : x * s_mul[q2] + s_add[q2];
        }
        __syncthreads();
        // the rank-r dot of every step, W_vw^T (W_kw^T u), on the matrix cores: per rank block of
        // four, one MFMA per 16-channel tile (A: the staged projections of the 16 steps), then
        // through LDS so that each thread holds its own channel's 16 values
        float pj[TC];
        if constexpr (SEL) {
            floatx4 acc[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const float a = sr[lane & 15][4 + 4 * kb + (lane >> 4)];
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, wb[t][kb], acc[t], 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
                *reinterpret_cast<floatx4 *>(&sp[wave * 64 + t * 16 + (lane & 15)][4 * (lane >> 4)]) = acc[t];
            // the rows a thread reads were written by lanes of its own wave
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int q = 0; q < TC / 4; ++q) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(&sp[tid][4 * q]);
                pj[4 * q] = v[0];
                pj[4 * q + 1] = v[1];
                pj[4 * q + 2] = v[2];
                pj[4 * q + 3] = v[3];
            }
        }
        float P = 1.0f;  // NORM: the block's running decay product (m = P mh)
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            if (j < nt) {
                const float inv = sr[j][0];
                const float cs = has_bc ? inv : 1.0f;  // B and C are projections of u = h / rms
                const float u = k.hv[j] * inv;
                const float x = u + wxh * u;
                float abar = abase;
                if constexpr (SEL) {
                    const float pre = bd + pj[j] * inv;
                    const float l2 = __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(pre * 1.44269504088896341f));
                    abar = 0.10f + (1.0f - 0.10f) * __builtin_amdgcn_exp2f(l2 * ln_ab);
                }
                const float xin = (1.0f - abar) * x * cs;
                float a2[2] = {0.0f, 0.0f};
                if constexpr (NORM) {
                    P *= abar;
                    const float z = xin * __builtin_amdgcn_rcpf(P);
#pragma unroll
                    for (int n = 0; n < NS; ++n) {
                        if (EXACT || n < N) {
                            m[n] += sr[j][BC0 + n] * z;
                            a2[n & 1] += sr[j][BC0 + NS + n] * m[n];
                        }
                    }
                } else {
#pragma unroll
                    for (int n = 0; n < NS; ++n) {
                        if (EXACT || n < N) {
                            m[n] = abar * m[n] + sr[j][BC0 + n] * xin;
                            a2[n & 1] += sr[j][BC0 + NS + n] * m[n];
                        }
                    }
                }
                if (MODE == 1) {
                    prod *= abar;
                } else if (active) {
                    const float yv = (NORM ? P : 1.0f) * cs * (a2[0] + a2[1]);
                    y[gbase + (long)(tb + j) * tstride] = yv;
                    ymax = fmaxf(ymax, fabsf(yv) < INFINITY ? fabsf(yv) : 0.0f);
                }
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int n = 0; n < NS; ++n) m[n] *= P;
        }
        __syncthreads();
    };
    // two register sets alternate so that the next TC steps' loads are issued before this TC's
    // y stores; loads are unconditional, at addresses clamped into the chunk (unused past it)
    Chunk ca, cb;
    if (t0 < t1) fetch(ca, t0);
    for (int tb = t0; tb < t1; tb += 2 * TC) {
        fetch(cb, tb + TC);
        process(ca, tb);
        if (tb + TC >= t1) break;
        fetch(ca, tb + 2 * TC);
        process(cb, tb + TC);
    }
    if (MODE != 1 && amax_y) track_absmax(amax_y, ymax);  // the readout GEMM's A bound
    if (!active) return;
    if (MODE == 1) {
        const long co = (((long)b * nch + c) * H + s) * d + dd;
        chunk_p[co] = prod;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (EXACT || n < N) chunk_s[co * D.N + n] = m[n];
    } else if (state_out && (MODE == 0 || c == nch - 1)) {
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (EXACT || n < N) state_out[st_off + n] = m[n];
    }
}

// Chunked matrix form of the same recurrence (the state-space-duality form of a selective scan),
// for carriers whose decay products over 16 steps stay normal fp32 numbers (the selective decay
// is at least 0.1; a fixed decay is checked at upload).  Over a chunk of L = 16 steps with start
// state M0 (N states per channel), decays a_t, inputs xt_t = (1 - a_t) x_t, chunk-local prefix
// products P_t = a_0 ... a_t and z_t = xt_t / P_t:
//   m_t = P_t (M0 + sum_{tau <= t} B_tau z_tau),   y_t = P_t (C_t . M0 + sum_{tau <= t} G[t][tau] z_tau)
// with G[t][tau] = C_t . B_tau shared by all channels of the slot; the next chunk starts from m_15.
// Per wave (16 channels) and chunk these are 16x16 fp32 MFMA tiles (v_mfma_f32_16x16x4f32):
//   G^T = B C^T,  Y = G_masked Z + C M0,  M = P_15 (M0 + B^T Z),
// so the N-state update costs no vector instructions per element.  The element work (gate,
// prefix products, y = P Y) runs in the MFMA output layout, lane (g, c) holding steps 4g + v
// (v = 0..3) of channel c; each product's contraction index is ordered to match that layout
// (steps tau = 4g + kb, states n = 16 nt + 4g + kb), so the output registers of one product are
// the operand registers of the next and nothing is transposed.  The chunk's prefix product is
// formed within a lane over v and across the four lane groups with lane permutes.
// The chunk's records are staged raw (only 1/rms is formed at staging); the 1/rms row scales are
// applied as the operands are read.  MODE as in k_scan_fused; the gate arithmetic is the same.
constexpr int SSD_WAVES = 8;
constexpr int SSD_NT = 64 * SSD_WAVES;
constexpr int SSD_CH = 16 * SSD_WAVES;  // channels per block
constexpr int SSD_L = 16;               // steps per chunk
constexpr int SSD_PF = 4;               // chunks whose loads are in flight

__device__ __forceinline__ float lane_from(int src, float v) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}
__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int NS, int RK, int MODE>
__global__ __launch_bounds__(SSD_NT) void k_scan_ssd(Dims D, const float *__restrict__ h,
                                                     const float *__restrict__ rec, int T, int nch, int has_bc,
                                                     const float *__restrict__ a_log,
                                                     const float *__restrict__ wx_diag,
                                                     const float *__restrict__ b_delta,
                                                     const float *__restrict__ w_vw,
                                                     const float *__restrict__ state_in, float *__restrict__ y,
                                                     float *__restrict__ state_out, float *__restrict__ chunk_s,
                                                     float *__restrict__ chunk_p, unsigned *amax_y) {
    static_assert(NS % 16 == 0, "states in tiles of 16");
    constexpr bool SEL = RK > 0;
    constexpr int RKA = SEL ? RK : 0;
    constexpr int BC0 = 4 + RKA;      // staged step: [0] 1/rms, [4 + q] projection q,
    constexpr int SW = BC0 + 2 * NS;  // [BC0 + n] B[n], [BC0 + NS + n] C[n] (un-normalised)
    constexpr int QMAX = 1 + RKA + 2 * NS;
    constexpr int RPT = (SSD_L * QMAX + SSD_NT - 1) / SSD_NT;  // staged values per thread
    constexpr int NT = NS / 16;
    constexpr int KB = SEL ? RKA / 4 : 1;  // rank values per lane: q = KB g + kb
    constexpr int GB = NS / 4;             // states per lane in G^T: n = GB g + kb
    // SW % 64 is 4 or 36: the scalar operand reads sr[4g + kb][.. + c] hit 64 banks
    __shared__ __attribute__((aligned(16))) float sr[SSD_L][SW];
    float *srf = &sr[0][0];
    const int d = D.d, H = D.H, r = D.r, N = D.N;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, cl = lane & 15;
    const int ch = blockIdx.x * SSD_CH + wave * 16 + cl;
    // d is a multiple of 16: a wave's channels are all inside d or all outside (wave-uniform)
    const bool active = __builtin_amdgcn_readfirstlane(blockIdx.x * SSD_CH + wave * 16 < d ? 1 : 0) != 0;
    const int cc = active ? ch : 0;
    const int s = blockIdx.y, bc = blockIdx.z;
    const int b = bc / nch, c = bc - (bc / nch) * nch;
    const int REC = 1 + r + 2 * N;
    const int Tc = (T + nch - 1) / nch;
    const int t0 = c * Tc, t1 = min(T, t0 + Tc);
    const int nq = 1 + RKA + 2 * N;  // staged values per step

    // the staging writes B and C for n < N only: the state padding reads zeros
    for (int i = tid; i < SSD_L * 2 * NS; i += SSD_NT) {
        const int j = i / (2 * NS), q = i - j * (2 * NS);
        if ((q < NS ? q : q - NS) >= N) sr[j][BC0 + q] = 0.0f;
    }
    // this thread's staged values (fixed over the chunks): LDS offset, step, record field, kind
    // (0: 1/rms, 1: the field, 2: one (B = C = 1 without B/C projections), 3: zero (rank padding))
    // Staged value = kind 0 ? 1 / x : x * s_mul + s_add; threads without a value write the unused
    // column 1 of step 0.
    int s_off[RPT], s_j[RPT], s_f[RPT];
    bool s_inv[RPT];
    float s_mul[RPT], s_add[RPT];
#pragma unroll
    for (int q2 = 0; q2 < RPT; ++q2) {
        const int idx = tid + q2 * SSD_NT;
        s_off[q2] = 1;
        s_j[q2] = 0;
        s_f[q2] = 0;
        s_inv[q2] = false;
        s_mul[q2] = 0.0f;
        s_add[q2] = 0.0f;
        if (idx < SSD_L * nq) {
            const int j = idx / nq, q = idx - j * nq;
            const int qb = q - 1 - RKA;  // B[0..N) then C[0..N) in the record; C staged at BC0 + NS
            const int slot = q == 0 ? 0 : (q <= RKA ? 4 + (q - 1) : BC0 + (qb < N ? qb : NS + qb - N));
            const int f = q == 0 ? 0 : (q <= RKA ? (q - 1 < r ? q : -1) : 1 + r + qb);
            const int kind = q == 0 ? 0 : (q <= RKA ? (f >= 0 ? 1 : 3) : (has_bc ? 1 : 2));
            s_off[q2] = j * SW + slot;
            s_j[q2] = j;
            s_f[q2] = f < 0 ? 0 : f;
            s_inv[q2] = kind == 0;
            s_mul[q2] = kind == 1 ? 1.0f : 0.0f;
            s_add[q2] = kind == 2 ? 1.0f : 0.0f;
        }
    }

    // per-channel constants
    const float al = a_log[(long)s * d + cc];
    const float abase = 1.0f / (1.0f + expf(al));
    const float ln_ab = logf(fmaxf(abase, 1.0e-6f));
    const float wxh = 0.5f * tanhf(wx_diag[(long)s * d + cc]);
    const float bd = (SEL && b_delta) ? b_delta[(long)s * d + cc] : 0.0f;
    // W_vw as the B operand of the rank-r product: lane (g, c), value kb: W_vw[s][KB g + kb][ch]
    float wb[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const int q = KB * g + kb;
        wb[kb] = (SEL && q < r) ? w_vw[((long)s * r + q) * d + cc] : 0.0f;
    }

    // state: lane (g, c), tile nt, register v holds state n = 16 nt + 4 g + v of channel ch
    floatx4 M[NT];
    const long st_off = (((long)b * H + s) * d + cc) * N;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = 16 * nt + 4 * g + v;
            float m0 = 0.0f;
            if (n < N && active) {
                if (MODE == 0 && state_in) m0 = state_in[st_off + n];
                if (MODE == 2) m0 = chunk_s[((((long)b * nch + c) * H + s) * d + cc) * N + n];
            }
            M[nt][v] = m0;
        }
    float prod = 1.0f;
    float ymax = 0.0f;  // largest finite |y| this thread stores

    struct Chunk {
        float hv[4], rv[RPT];
    };
    const long tstride = (long)H * d;                          // one time step of (b, s, ch)
    const long gbase = (long)b * T * tstride + (long)s * d + cc;  // (b, t = 0, s, ch)
    const long rstride = (long)H * REC;                        // one time step of the records
    const int last = t1 - 1;
    const float *recb = rec + ((long)b * T * H + s) * REC;
    // Loads go through pointers advanced by one chunk per fetch (fetches run in step order);
    // only a chunk reaching past the range's last step takes the clamped addresses.
    const long ylane = gbase + (long)(4 * g) * tstride;          // step 4g of this lane
    const float *hp = h + ylane + (long)t0 * tstride;            // step t0 + 4g of this lane
    const float *rp[RPT];
#pragma unroll
    for (int q2 = 0; q2 < RPT; ++q2) rp[q2] = recb + (long)(t0 + s_j[q2]) * rstride + s_f[q2];
    auto fetch = [&](Chunk &k, int tb) {
        if (tb + SSD_L <= t1) {
            if (active) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    k.hv[v] = MODE == 1 ? hp[v * tstride] : __builtin_nontemporal_load(hp + v * tstride);
            }
#pragma unroll
            for (int q2 = 0; q2 < RPT; ++q2) k.rv[q2] = *rp[q2];
        } else {
            if (active) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const long off = gbase + (long)min(tb + 4 * g + v, last) * tstride;
                    k.hv[v] = MODE == 1 ? h[off] : __builtin_nontemporal_load(h + off);
                }
            }
#pragma unroll
            for (int q2 = 0; q2 < RPT; ++q2) k.rv[q2] = recb[(long)min(tb + s_j[q2], last) * rstride + s_f[q2]];
        }
        hp += SSD_L * tstride;
#pragma unroll
        for (int q2 = 0; q2 < RPT; ++q2) rp[q2] += SSD_L * rstride;
    };
    auto process = [&](const Chunk &k, int tb) {
        const int nt_ = min(SSD_L, t1 - tb);
#pragma unroll
        for (int q2 = 0; q2 < RPT; ++q2) {
            const float x = k.rv[q2];
            srf[s_off[q2]] = s_inv[q2] ? __builtin_amdgcn_rcpf(x) : x * s_mul[q2] + s_add[q2];
        }
        __syncthreads();
        // Operands straight from the staged (un-normalised) record; the row scales are applied to
        // the products instead: pj and Y by the scale of their step row t = 4g + v, and z (the
        // step-contracted operand) by that of its step tau = 4g + v before it meets B or G.
        float invr[4], bs[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            invr[v] = sr[4 * g + v][0];
            bs[v] = has_bc ? invr[v] : 1.0f;  // B and C are projections of u = h / rms
        }
        float ra[KB], gbv[GB], gcv[GB], cm[NT][4], bm[NT][4];
        if constexpr (SEL) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) ra[kb] = sr[cl][4 + KB * g + kb];
        }
#pragma unroll
        for (int kb = 0; kb < GB; ++kb) {
            gbv[kb] = sr[cl][BC0 + GB * g + kb];
            gcv[kb] = sr[cl][BC0 + NS + GB * g + kb];
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                cm[nt][kb] = sr[cl][BC0 + NS + 16 * nt + 4 * g + kb];
                bm[nt][kb] = sr[4 * g + kb][BC0 + 16 * nt + cl];
            }
        // gate: the rank-r dot W_vw^T (W_kw^T h) of the chunk's steps (pj[v]: step 4g + v), and the
        // raw G^T = B C^T (lane (g, c) register v = G[t = c][tau = 4g + v]): independent chains
        floatx4 pj = {0.0f, 0.0f, 0.0f, 0.0f}, gt = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < (KB > GB ? KB : GB); ++kb) {
            if (SEL && kb < KB) pj = mfma4(ra[kb < KB ? kb : 0], wb[kb < KB ? kb : 0], pj);
            if (kb < GB) gt = mfma4(gbv[kb < GB ? kb : 0], gcv[kb < GB ? kb : 0], gt);
        }
        float xt[4], p[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int j = 4 * g + v;
            const float u = k.hv[v] * invr[v];
            const float x = u + wxh * u;
            float abar = abase;
            if constexpr (SEL) {
                const float pre = bd + pj[v] * invr[v];
                const float l2 = __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(pre * 1.44269504088896341f));
                abar = 0.10f + (1.0f - 0.10f) * __builtin_amdgcn_exp2f(l2 * ln_ab);
            }
            const bool on = j < nt_;  // steps past the chunk end: decay 1, input 0
            xt[v] = on ? (1.0f - abar) * x : 0.0f;
            p[v] = on ? abar : 1.0f;
        }
        // prefix products: within the lane over v, then over the lane groups g (lanes c, 16 + c,
        // 32 + c, 48 + c), whose four totals every lane fetches at once
        p[1] *= p[0];
        p[2] *= p[1];
        p[3] *= p[2];
        const float T0 = lane_from(cl, p[3]), T1 = lane_from(16 + cl, p[3]);
        const float T2 = lane_from(32 + cl, p[3]), T3 = lane_from(48 + cl, p[3]);
        const float ex = (g >= 1 ? T0 : 1.0f) * (g >= 2 ? T1 : 1.0f) * (g >= 3 ? T2 : 1.0f);  // groups before g
        const float plast = ((T0 * T1) * T2) * T3;  // the whole chunk
        float P[4];
        floatx4 z;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            P[v] = ex * p[v];
            z[v] = xt[v] * __builtin_amdgcn_rcpf(P[v]) * bs[v];
        }
        // A non-finite input (NaN / inf h*, record or decay at step tau) makes z non-finite from tau
        // on.  The causal mask is a select on G, so in the product below a masked entry would still
        // add 0 * z[tau] = NaN to the earlier steps t < tau, which the sequential recurrence keeps
        // finite: the masked product takes such z as 0, and the steps from the channel's first
        // non-finite one on are written as NaN after it (the state update below keeps the raw z,
        // so the state turns non-finite as the recurrence's does).
        bool bad[4], anybad = false;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            bad[v] = !(fabsf(z[v]) < INFINITY);
            anybad |= bad[v];
        }
        // Y = G_masked Z + C M0 (the old state) before the row scale of C: register v = step 4g + v
        floatx4 Y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) Y = mfma4(4 * g + kb <= cl ? gt[kb] : 0.0f, bad[kb] ? 0.0f : z[kb], Y);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) Y = mfma4(cm[nt][kb], M[nt][kb], Y);
        // M = P_15 (M0 + B^T Z)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            floatx4 acc = M[nt];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) acc = mfma4(bm[nt][kb], z[kb], acc);
#pragma unroll
            for (int v = 0; v < 4; ++v) M[nt][v] = plast * acc[v];
        }
        if (MODE == 1) {
            prod *= plast;
        } else if (active) {
            float *yp = y + ylane + (long)tb * tstride;
            float yv[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) yv[v] = P[v] * bs[v] * Y[v];
            if (__builtin_amdgcn_ballot_w64(anybad)) {  // wave-uniform: rare
                // the channel's first non-finite step over its four lane groups (16 = none)
                int fb = 16;
#pragma unroll
                for (int v = 3; v >= 0; --v) fb = bad[v] ? 4 * g + v : fb;
                const int f0 = __builtin_amdgcn_ds_bpermute(cl << 2, fb);
                const int f1 = __builtin_amdgcn_ds_bpermute((16 + cl) << 2, fb);
                const int f2 = __builtin_amdgcn_ds_bpermute((32 + cl) << 2, fb);
                const int f3 = __builtin_amdgcn_ds_bpermute((48 + cl) << 2, fb);
                const int first = min(min(f0, f1), min(f2, f3));
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (4 * g + v >= first) yv[v] = __builtin_nanf("");
            }
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ymax = fmaxf(ymax, (4 * g + v < nt_ && fabsf(yv[v]) < INFINITY) ? fabsf(yv[v]) : 0.0f);
            if (nt_ == SSD_L) {
#pragma unroll
                for (int v = 0; v < 4; ++v) yp[v * tstride] = yv[v];
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (4 * g + v < nt_) yp[v * tstride] = yv[v];
            }
        }
        __syncthreads();
    };
    // SSD_PF chunks in flight: a chunk's loads are issued SSD_PF - 1 chunks before it is processed
    // (a wave's chunk is 1 KB of h; one chunk ahead leaves the loads' latency exposed).  The ring
    // of register sets is indexed at compile time (the loop is unrolled by SSD_PF); loads past the
    // range are clamped to its last step and not used.
    Chunk ring[SSD_PF];
#pragma unroll
    for (int u = 0; u + 1 < SSD_PF; ++u) fetch(ring[u], t0 + u * SSD_L);
    for (int tb = t0; tb < t1; tb += SSD_PF * SSD_L) {
#pragma unroll
        for (int u = 0; u < SSD_PF; ++u) {
            const int tbu = tb + u * SSD_L;
            if (tbu >= t1) break;
            fetch(ring[(u + SSD_PF - 1) % SSD_PF], tbu + (SSD_PF - 1) * SSD_L);
            process(ring[u], tbu);
        }
    }
    if (MODE != 1 && amax_y) track_absmax(amax_y, ymax);  // the readout GEMM's A bound
    if (!active) return;
    if (MODE == 1) {
        const long co = (((long)b * nch + c) * H + s) * d + ch;
        if (g == 0) chunk_p[co] = prod;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = 16 * nt + 4 * g + v;
                if (n < N) chunk_s[co * N + n] = M[nt][v];
            }
    } else if (state_out && (MODE == 0 || c == nch - 1)) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = 16 * nt + 4 * g + v;
                if (n < N) state_out[st_off + n] = M[nt][v];
            }
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

struct ScanArgs {
    const float *h, *rec;
    int B, T, has_bc;
    const float *a_log, *wx_diag, *b_delta, *w_vw, *state_in;
    float *y, *state_out, *chunk_s, *chunk_p;
    int nch;
    unsigned *amax_y;
};

template <int NS, int RK, bool EXACT, bool NORM>
void scan_modes(const Dims &D, const ScanArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((D.d + SCAN_NT - 1) / SCAN_NT), (unsigned)D.H, (unsigned)(a.B * a.nch));
#define ADN_SCAN_K(MODE)                                                                                          \
    hipLaunchKernelGGL((k_scan_fused<NS, RK, MODE, EXACT, NORM>), grid, dim3(SCAN_NT), 0, st, D, a.h, a.rec, a.T,  \
                       a.nch,                                                                                     \
                       a.has_bc, a.a_log, a.wx_diag, a.b_delta, a.w_vw, a.state_in, a.y, a.state_out, a.chunk_s,   \
                       a.chunk_p, a.amax_y)
    if (a.nch <= 1) {
        ADN_SCAN_K(0);
        return;
    }
    ADN_SCAN_K(1);
    const long total = (long)a.B * D.H * D.d * D.N;
    hipLaunchKernelGGL(k_scan_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, D, a.B, a.nch,
                       a.state_in, a.chunk_s, a.chunk_p);
    ADN_SCAN_K(2);
#undef ADN_SCAN_K
}

template <int NS, int RK>
void scan_modes_ssd(const Dims &D, const ScanArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((D.d + SSD_CH - 1) / SSD_CH), (unsigned)D.H, (unsigned)(a.B * a.nch));
#define ADN_SSD_K(MODE)                                                                                         \
    hipLaunchKernelGGL((k_scan_ssd<NS, RK, MODE>), grid, dim3(SSD_NT), 0, st, D, a.h, a.rec, a.T, a.nch, a.has_bc, \
                       a.a_log, a.wx_diag, a.b_delta, a.w_vw, a.state_in, a.y, a.state_out, a.chunk_s, a.chunk_p, \
                       a.amax_y)
    if (a.nch <= 1) {
        ADN_SSD_K(0);
        return;
    }
    ADN_SSD_K(1);
    const long total = (long)a.B * D.H * D.d * D.N;
    hipLaunchKernelGGL(k_scan_carry, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, D, a.B, a.nch,
                       a.state_in, a.chunk_s, a.chunk_p);
    ADN_SSD_K(2);
#undef ADN_SSD_K
}

template <int RK>
void scan_ssd_n(const Dims &D, const ScanArgs &a, hipStream_t st) {
    if (D.N <= 16)
        scan_modes_ssd<16, RK>(D, a, st);
    else
        scan_modes_ssd<32, RK>(D, a, st);
}

template <int RK, bool NORM>
void scan_n(const Dims &D, const ScanArgs &a, hipStream_t st) {
    if (D.N == 16)
        scan_modes<16, RK, true, NORM>(D, a, st);
    else if (D.N == 1)
        scan_modes<1, RK, true, NORM>(D, a, st);
    else if (D.N == 32)
        scan_modes<32, RK, true, NORM>(D, a, st);
    else if (D.N <= 8)
        scan_modes<8, RK, false, NORM>(D, a, st);
    else
        scan_modes<32, RK, false, NORM>(D, a, st);
}

}  // namespace

int scan_rec_len(const Dims &D) { return 1 + D.r + 2 * D.N; }

// The chunked matrix form needs every 16-step decay product to stay a normal fp32 number: the
// selective decay is at least 0.1 (0.1^16 = 1e-16); a fixed decay sigmoid(-a_log) must be at
// least 0.02 everywhere (0.02^16 = 6.6e-28, so 1 / P and the inputs scaled by it stay far from
// the fp32 limits).  Up to 32 states and a rank up to 64.
static bool scan_ssd_ok(const Dims &D, float min_fixed_decay) {
    return D.N >= 1 && D.N <= 32 && D.r <= 64 && D.d % 16 == 0 &&
           ((D.flags & ADN_F_SCAN_SELECTIVE) || min_fixed_decay >= 0.02f);
}

// The matrix form where the per-step recurrence would be split into time chunks (too few
// sequences to fill the GPU: the chunked recurrence runs twice): per element the two forms cost
// about the same, so the single pass wins there and the per-step form elsewhere.
bool scan_use_ssd(const Dims &D, int B, int T, float min_fixed_decay) {
    return scan_ssd_ok(D, min_fixed_decay) && scan_chunks(B, T, D.H, D.d, false) > 1;
}

// Time chunks only where the sequences alone leave the GPU short of about two waves per SIMD
// (the matrix form: 16 channels a wave) or two workgroups per CU: a chunked scan runs the
// recurrence twice (pass A, then pass C from the carried start).
int scan_chunks(int B, int T, int H, int d, bool ssd) {
    int nch = 1;
    if (ssd) {
        const long waves = (long)B * H * (d / 16);
        while (waves * nch < 2048 && T / (nch * 2) >= 4 * SSD_L) nch *= 2;
        return nch;
    }
    const long wgs = (long)B * H * ((d + SCAN_NT - 1) / SCAN_NT);
    while (wgs * nch < SCAN_MIN_WGS && T / (nch * 2) >= 4 * TC) nch *= 2;
    return nch;
}

void launch_row_rms(const float *h, long rows, int d, float *rec, int REC, hipStream_t st) {
    const dim3 grid((unsigned)((rows + WPB - 1) / WPB)), blk(64 * WPB);
    dispatch_width(d, [&](auto Ec, auto Pc) {
        hipLaunchKernelGGL((k_row_rms<decltype(Ec)::value, decltype(Pc)::value>), grid, blk, 0, st, h, rows, d, rec,
                           REC);
    });
}

void launch_scan(const Dims &D, const float *h, const float *rec, int B, int T, int has_bc, const float *a_log,
                 const float *wx_diag, const float *b_delta, const float *w_vw, const float *state_in, float *y,
                 float *state_out, float *chunk_s, float *chunk_p, int nch, unsigned *amax_y, bool ssd,
                 float min_fixed_decay, hipStream_t st) {
    const ScanArgs a{h,     rec, B,       T,       has_bc,  a_log, wx_diag, b_delta, w_vw, state_in,
                     y,     state_out, chunk_s, chunk_p, nch, amax_y};
    if (ssd) {
        if (!(D.flags & ADN_F_SCAN_SELECTIVE))
            scan_ssd_n<0>(D, a, st);
        else if (D.r <= 32)
            scan_ssd_n<32>(D, a, st);
        else
            scan_ssd_n<64>(D, a, st);
        return;
    }
    // the per-step form carries the states divided by the block's decay product where every
    // 16-step product stays normal (the same condition as the matrix form's)
    if (!(D.flags & ADN_F_SCAN_SELECTIVE)) {
        if (min_fixed_decay >= 0.02f)
            scan_n<0, true>(D, a, st);
        else
            scan_n<0, false>(D, a, st);
    } else if (D.r <= 32) {
        scan_n<32, true>(D, a, st);
    } else {
        scan_n<64, true>(D, a, st);
    }
}

}  // namespace adn

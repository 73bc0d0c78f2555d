// Pieces shared by the fp32 and the split-precision MFMA GEMMs: block ordering and the
// epilogue (bias / residual add / per-row arg-max partials) of a 2x2 grid of 32x32 MFMA tiles
// per wave, 64x64 per wave, 128x128 per workgroup.
#pragma once

#include "kernels.h"

namespace adn {
namespace gemm {

constexpr int BM = 128, BN = 128, NT = 256, GROUP_M = 8, NXCD = 8;

// Workgroup barrier without the memory fence of __syncthreads (which would drain every
// outstanding global load and store, LDS DMA included): this wave's LDS operations are completed
// first (through the builtin, so that the compiler's own wait-count tracking sees it), the memory
// clobber keeps the compiler from moving LDS accesses across the barrier.  For exchanges through
// LDS only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ void map_block(int bid, int total, int nM, int nN, int &s, int &mt,
                                          int &nt) {
    // XCD-contiguous remap: hardware sends workgroup i to XCD i % 8.
    const int q = total / NXCD, rem = total % NXCD;
    const int x = bid % NXCD, j = bid / NXCD;
    const int logical = x * q + (x < rem ? x : rem) + j;
    const int per_slot = nM * nN;
    s = logical / per_slot;
    const int l = logical - s * per_slot;
    const int group = l / (GROUP_M * nN);
    const int first_m = group * GROUP_M;
    const int gsz = min(nM - first_m, GROUP_M);
    const int within = l - group * GROUP_M * nN;
    mt = first_m + within % gsz;
    nt = within / gsz;
}

// Epilogue for one wave's 2x2 accumulators.  `scratch` is >= 2*BM floats of LDS no longer
// needed by the main loop (ints are stored through the same space, second half).
__device__ __forceinline__ void epilogue(const GemmParams &p, floatx16 (&acc)[2][2], int M, int s, int m0,
                                         int n0, int nt, int nN, float *scratch_v, int *scratch_i) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, hh = lane >> 5;
    // Epilogue.  Output layout of a 32x32 MFMA tile: lane holds column lane%32, register e holds
    // row 8*(e/4) + 4*(lane/32) + e%4.  Each value is formed once (acc + bias[n], or A[m][n] +
    // acc) and feeds both the store and the optional per-row arg-max.
    float bj[2] = {0.0f, 0.0f};
    bool nv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + r;
        nv[j] = n < p.N;
        if (p.epi == EPI_BIAS && nv[j] && n < p.bias_n) bj[j] = p.bias[(long)s * p.bias_ss + n];
    }
    const bool want_am = p.am_val != nullptr;
    float *am_v = scratch_v;
    int *am_i = scratch_i;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int ml = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
            const int m = m0 + ml;
            const bool mv = m < M;
            float *crow = p.C + (long)m * p.c_sm + (long)s * p.c_ss;
            const float *res_row = p.A + (long)m * p.a_sm + (long)s * p.a_ss;
            float bv = -INFINITY;
            int bi = -1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 64 + j * 32 + r;
                float v = acc[i][j][e];
                if (p.epi == EPI_BIAS)
                    v += bj[j];
                else if (p.epi == EPI_ADD_A && mv && nv[j])
                    v = res_row[n] + v;
                if (mv && nv[j]) {
                    crow[n] = v;
                    if (v > bv || (v == bv && n > bi)) {
                        bv = v;
                        bi = n;
                    }
                }
            }
            if (want_am) {
#pragma unroll
                for (int off = 16; off > 0; off >>= 1) {
                    const float v2 = __shfl_xor(bv, off, 64);
                    const int i2 = __shfl_xor(bi, off, 64);
                    if (v2 > bv || (v2 == bv && i2 > bi)) {
                        bv = v2;
                        bi = i2;
                    }
                }
                if (r == 0) {
                    am_v[wn * BM + ml] = bv;
                    am_i[wn * BM + ml] = bi;
                }
            }
        }
    }
    if (want_am) {
        __syncthreads();
        if (tid < BM) {
            const int m = m0 + tid;
            if (m < M) {
                float v = am_v[tid];
                int ix = am_i[tid];
                const float v2 = am_v[BM + tid];
                const int i2 = am_i[BM + tid];
                if (v2 > v || (v2 == v && i2 > ix)) {
                    v = v2;
                    ix = i2;
                }
                p.am_val[(long)nt * p.M + m] = v;  // [tile][row]: coalesced across rows
                p.am_idx[(long)nt * p.M + m] = ix;
            }
        }
    }
}


// Generic epilogue: each wave holds WTM x WTN tiles of 32x32 (acc[i][j]); the workgroup is a
// WGM x WGN grid of waves, block tile (WGM*WTM*32) x (WGN*WTN*32).  Per-row arg-max partials go
// through `scratch_v/scratch_i` (>= WGN * block-rows entries of LDS free after the k loop).
// The epilogue mode (EPI), the arg-max (AM) and the bounds checks (CHECK: only edge tiles need
// them) are compile-time, so an interior tile's epilogue is straight-line code: scale, bias,
// store.  The tile rows are walked by template recursion (I = 0..WTM-1) so that every
// accumulator index is a compile-time constant: a runtime row loop leaves the accumulator
// array in scratch memory.
struct EpiCtx {
    int M, s, m0, n0, wm, wn, r, hh;
    float osc;  // accumulator scale (undoes the power-of-two operand scaling)
    float *scratch_v;
    int *scratch_i;
};

// One transposing step of the arg-max butterfly at lane offset OFF (< 32, within a half-wave):
// of the 2 OFF candidates held in cv/ci[0 .. 2 OFF), a lane keeps the upper half if bit OFF of
// its lane index is set and the lower half otherwise, combined with its partner's candidates for
// the same rows, into cv/ci[0 .. OFF).
template <int OFF, typename F>
__device__ __forceinline__ void butterfly_step(float (&cv)[16], int (&ci)[16], int r, F better) {
    const bool up = (r & OFF) != 0;
#pragma unroll
    for (int j = 0; j < OFF; ++j) {
        const float sv = up ? cv[j] : cv[j + OFF];
        const int si = up ? ci[j] : ci[j + OFF];
        float kv = up ? cv[j + OFF] : cv[j];
        int ki = up ? ci[j + OFF] : ci[j];
        better(__int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(sv), (OFF << 10) | 0x1F)),
               __builtin_amdgcn_ds_swizzle(si, (OFF << 10) | 0x1F), kv, ki);
        cv[j] = kv;
        ci[j] = ki;
    }
}

template <int I, int WTM, int WTN, int WGM, int EPI, bool AM, bool CHECK, bool STREAM>
__device__ __forceinline__ void epi_rows(const GemmParams &p, floatx16 (&acc)[WTM][WTN], const EpiCtx &c,
                                         const float (&bj)[WTN], const bool (&nv)[WTN]) {
    constexpr int BMt = WGM * WTM * 32;
    const int ncol0 = c.n0 + c.wn * WTN * 32 + c.r;  // column of j = 0
    float cv[16];  // per row e: this lane's (max, last arg-max) over its WTN columns
    int ci[16];
    // The residual operand is loaded EB rows at a time before their stores: a load issued after
    // stores is waited for behind them (the vector-memory counter retires in issue order).
    constexpr int EB = EPI == EPI_ADD_A ? 8 : 16;
    float av[EPI == EPI_ADD_A ? EB : 1][EPI == EPI_ADD_A ? WTN : 1];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        if constexpr (EPI == EPI_ADD_A) {
            if (e % EB == 0) {
#pragma unroll
                for (int q = 0; q < EB; ++q) {
                    const int m = c.m0 + (c.wm * WTM + I) * 32 + 8 * ((e + q) >> 2) + 4 * c.hh + ((e + q) & 3);
                    const bool mv = !CHECK || m < c.M;
#pragma unroll
                    for (int j = 0; j < WTN; ++j)
                        av[q][j] = (!CHECK || (mv && nv[j]))
                                       ? p.A[(long)m * p.a_sm + (long)c.s * p.a_ss + ncol0 + 32 * j]
                                       : 0.0f;
                }
            }
        }
        const int ml = (c.wm * WTM + I) * 32 + 8 * (e >> 2) + 4 * c.hh + (e & 3);
        const int m = c.m0 + ml;
        const bool mv = !CHECK || m < c.M;
        float *crow = p.C + (long)m * p.c_sm + (long)c.s * p.c_ss + ncol0;
        float bv = -INFINITY;
        int bi = -1;
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const bool ok = !CHECK || (mv && nv[j]);
            float v = acc[I][j][e] * c.osc;
            if constexpr (EPI == EPI_BIAS) v += bj[j];
            if constexpr (EPI == EPI_ADD_A) v = av[e % EB][j] + v;
            if (ok) {
                if constexpr (STREAM)
                    __builtin_nontemporal_store(v, crow + 32 * j);
                else
                    crow[32 * j] = v;
                if constexpr (AM) {
                    // this lane's columns grow with j, so "larger, or equal at a larger index"
                    // is v >= bv here (false for NaN either way)
                    if (v >= bv) {
                        bv = v;
                        bi = ncol0 + 32 * j;
                    }
                }
            }
        }
        if constexpr (AM) {
            cv[e] = bv;
            ci[e] = bi;
        }
    }
    if constexpr (AM) {
        // (max, last arg-max) of each of the 16 rows over the 32 lanes of a half-wave, by a
        // transposing butterfly: offset 16 combines all 16 candidates with the partner's, then at
        // offsets 8, 4, 2, 1 each lane keeps half of the rows it still holds (the upper half if
        // that offset bit is set) and combines its partner's candidates for them.  Lane r ends
        // with row e = r % 16.  The combination is a maximum with ties to the larger index, so
        // the order of combination does not change the result.
        auto better = [](float v2, int i2, float &v, int &i) {
            if (v2 > v || (v2 == v && i2 > i)) {
                v = v2;
                i = i2;
            }
        };
#pragma unroll
        for (int e = 0; e < 16; ++e)
            better(__int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(cv[e]), (16 << 10) | 0x1F)),
                   __builtin_amdgcn_ds_swizzle(ci[e], (16 << 10) | 0x1F), cv[e], ci[e]);
        butterfly_step<8>(cv, ci, c.r, better);
        butterfly_step<4>(cv, ci, c.r, better);
        butterfly_step<2>(cv, ci, c.r, better);
        butterfly_step<1>(cv, ci, c.r, better);
        if (c.r < 16) {
            const int e = c.r;
            const int ml = (c.wm * WTM + I) * 32 + 8 * (e >> 2) + 4 * c.hh + (e & 3);
            c.scratch_v[c.wn * BMt + ml] = cv[0];
            c.scratch_i[c.wn * BMt + ml] = ci[0];
        }
    }
    if constexpr (I + 1 < WTM) epi_rows<I + 1, WTM, WTN, WGM, EPI, AM, CHECK, STREAM>(p, acc, c, bj, nv);
}

// PW: columns per arg-max partial (128; 64 for the few-row LM head's one-wave 64-column blocks)
template <int WTM, int WTN, int WGM, int WGN, int EPI, bool AM, bool CHECK, bool STREAM = false, int PW = 128>
__device__ __forceinline__ void epi_tile(const GemmParams &p, floatx16 (&acc)[WTM][WTN], const EpiCtx &c) {
    constexpr int BMt = WGM * WTM * 32;
    float bj[WTN];
    bool nv[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
        const int n = c.n0 + (c.wn * WTN + j) * 32 + c.r;
        nv[j] = !CHECK || n < p.N;
        bj[j] = 0.0f;
        if constexpr (EPI == EPI_BIAS) {
            if (nv[j] && n < p.bias_n)
                bj[j] = p.bias[(long)c.s * p.bias_ss + n];
        }
    }
    epi_rows<0, WTM, WTN, WGM, EPI, AM, CHECK, STREAM>(p, acc, c, bj, nv);
    if constexpr (AM) {
        // partials are per PW columns: waves covering fewer columns are combined
        constexpr int CPW = WTN * 32;
        static_assert((CPW == 64 || CPW == 128) && PW >= CPW, "arg-max partials need whole waves per partial");
        constexpr int TPW = PW / CPW;
        constexpr int QT = WGN * CPW / PW;  // partial tiles per block (the LM head's blocks hold whole ones)
        // the partials are exchanged through LDS; the logits stores need not wait.  A one-wave
        // block reads back its own writes (a wave's LDS operations complete in order).
        if constexpr (WGM * WGN > 1) lds_barrier();
        const int tid = threadIdx.x;
        for (int idx = tid; idx < BMt * QT; idx += 64 * WGM * WGN) {
            const int ml = idx % BMt, q = idx / BMt;
            const int m = c.m0 + ml;
            const int tile = c.n0 / PW + q;
            if (m < c.M && tile * PW < p.N) {
                float v = c.scratch_v[q * TPW * BMt + ml];
                int ix = c.scratch_i[q * TPW * BMt + ml];
#pragma unroll
                for (int w = 1; w < TPW; ++w) {
                    const float v2 = c.scratch_v[(q * TPW + w) * BMt + ml];
                    const int i2 = c.scratch_i[(q * TPW + w) * BMt + ml];
                    if (v2 > v || (v2 == v && i2 > ix)) {
                        v = v2;
                        ix = i2;
                    }
                }
                p.am_val[(long)tile * p.M + m] = v;  // [tile][row]: coalesced across rows
                p.am_idx[(long)tile * p.M + m] = ix;
            }
        }
    }
}

// Epilogue dispatch for one GEMM role: the modes a role can use are compiled for it, each in a
// checked (edge tile) and an unchecked (interior tile) form.
template <int ROLE, int WTM, int WTN, int WGM, int WGN>
__device__ __forceinline__ void epilogue_t(const GemmParams &p, floatx16 (&acc)[WTM][WTN], int M, int s,
                                           int m0, int n0, float osc, float *scratch_v, int *scratch_i) {
    constexpr int BMt = WGM * WTM * 32, BNt = WGN * WTN * 32;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const EpiCtx c{M, s, m0, n0, wave / WGN, wave % WGN, lane & 31, lane >> 5, osc, scratch_v, scratch_i};
    const bool interior = m0 + BMt <= M && n0 + BNt <= p.N;
    if constexpr (ROLE == ROLE_READOUT) {
        // y + W y: the residual added here, or already in the weights (I + W, EPI_NONE)
        if (p.epi == EPI_ADD_A) {
            if (interior)
                epi_tile<WTM, WTN, WGM, WGN, EPI_ADD_A, false, false>(p, acc, c);
            else
                epi_tile<WTM, WTN, WGM, WGN, EPI_ADD_A, false, true>(p, acc, c);
        } else {
            if (interior)
                epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, false>(p, acc, c);
            else
                epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, true>(p, acc, c);
        }
    } else if constexpr (ROLE == ROLE_LMHEAD) {
        // the arg-max branch and the bias branch are uniform over the grid; the logits (nothing in
        // the forward reads them back) are stored non-temporally, which keeps the A rows and weights
        // of the tiles still being multiplied in L2
        constexpr bool LM_ST = true;
        constexpr int PW = (WGM * WGN == 1 && WTN == 2) ? 64 : 128;  // gemm_lm_partial_cols
        if (p.am_val) {
            if (p.epi == EPI_BIAS) {
                if (interior)
                    epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, true, false, LM_ST, PW>(p, acc, c);
                else
                    epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, true, true, LM_ST, PW>(p, acc, c);
            } else {
                if (interior)
                    epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, true, false, LM_ST, PW>(p, acc, c);
                else
                    epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, true, true, LM_ST, PW>(p, acc, c);
            }
        } else {
            if (p.epi == EPI_BIAS) {
                if (interior)
                    epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, false, false, LM_ST>(p, acc, c);
                else
                    epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, false, true, LM_ST>(p, acc, c);
            } else {
                if (interior)
                    epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, false, LM_ST>(p, acc, c);
                else
                    epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, true, LM_ST>(p, acc, c);
            }
        }
    } else {
        // Q|K|V and W_o outputs are read by the very next kernel (attention, update): stored
        // non-temporally they stream past L2, which keeps the operands of the tiles still being
        // multiplied in L2 and leaves the outputs to the consumer in the memory-side cache.  The
        // one-wave blocks of the few-row products store normally: their outputs are a few
        // kilobytes that the next kernel reads straight from L2.
        constexpr bool ST = (ROLE == ROLE_QKV || ROLE == ROLE_WO) && WGM * WGN > 1;
        if (p.epi == EPI_BIAS) {
            if (interior)
                epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, false, false, ST>(p, acc, c);
            else
                epi_tile<WTM, WTN, WGM, WGN, EPI_BIAS, false, true, ST>(p, acc, c);
        } else {
            if (interior)
                epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, false, ST>(p, acc, c);
            else
                epi_tile<WTM, WTN, WGM, WGN, EPI_NONE, false, true, ST>(p, acc, c);
        }
    }
}

}  // namespace gemm
}  // namespace adn

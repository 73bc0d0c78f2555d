// fp32 MFMA GEMM for the slot projections, the input projection, the carrier readout and the
// LM head:  C[m][n] = sum_k A[row(m)][k] * B[n][k]  (+ epilogue), batched over slots.
//
// A and B are both k-contiguous ("NT"): A rows are token/slot state vectors, B rows are weight
// rows W[s][out][:] (the y = W x orientation), so neither operand needs a transpose.
//
// Tiling for gfx950 (64-wide waves, v_mfma_f32_32x32x2f32, 64 FLOP/clk/SIMD fp32 peak):
//   workgroup 256 threads = 4 waves in 2x2, block tile 128x128, k-step 32, double-buffered LDS
//   (2 x (128+128) x 36 floats = 73.7 KB, 2 workgroups per CU); each wave owns 64x64 = 2x2
//   MFMA 32x32 tiles (64 accumulators per lane).  A lane feeds 4 consecutive MFMAs from one
//   ds_read_b128 of A and one of B: the k-pair of MFMA q on lane-half hh is {q, 4+q}, so the
//   k order is a fixed permutation shared by A and B.
//   Block order: slot-major, then groups of 8 m-tiles with n fastest inside a group, spread so
//   each XCD (own L2) gets a contiguous range -> one slot's weights stay resident in one L2.
#include "gemm_common.h"

namespace adn {

namespace {

using namespace gemm;
constexpr int BK = 32, LDK = BK + 4;

template <int ROLE>
__global__ __launch_bounds__(NT, 2) void k_gemm_nt(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float As[2][BM][LDK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN][LDK];

    const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
    int s, mt, nt;
    map_block(blockIdx.x, nM * nN * p.S, nM, nN, s, mt, nt);
    const int M = p.m_count ? min(*p.m_count, p.M) : p.M;
    const int m0 = mt * BM, n0 = nt * BN;
    if (m0 >= M) return;

    const int tid = threadIdx.x;
    const int lrow = tid >> 3;       // 0..31
    const int lk = (tid & 7) * 4;    // 0..28
    const float *arow[4];
    const float *brow[4];
    bool aval[4], bval[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m0 + lrow + 32 * j;
        aval[j] = m < M;
        long r = 0;
        if (aval[j]) {
            r = p.a_idx ? (long)p.a_idx[m] : (long)m;
            if (p.a_idx && (r < 0 || r >= p.a_idx_max)) {
                if (p.err) atomicOr(p.err, ADN_DEVERR_TOKEN);
                r = 0;
            }
        }
        arow[j] = p.A + r * p.a_sm + (long)s * p.a_ss;
        const int n = n0 + lrow + 32 * j;
        bval[j] = n < p.N;
        brow[j] = p.B + (long)s * p.b_ss + (long)(bval[j] ? n : 0) * p.K;
    }

    floatx4 ga[4], gb[4];
    auto gload = [&](int kt) {
        const int k = kt * BK + lk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ga[j] = aval[j] ? *reinterpret_cast<const floatx4 *>(arow[j] + k) : floatx4{0, 0, 0, 0};
            gb[j] = bval[j] ? *reinterpret_cast<const floatx4 *>(brow[j] + k) : floatx4{0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            *reinterpret_cast<floatx4 *>(&As[buf][lrow + 32 * j][lk]) = ga[j];
            *reinterpret_cast<floatx4 *>(&Bs[buf][lrow + 32 * j][lk]) = gb[j];
        }
    };

    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, hh = lane >> 5;
    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int nk = p.K / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 8) {
            floatx4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const floatx4 *>(&As[buf][wm * 64 + i * 32 + r][kk + hh * 4]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const floatx4 *>(&Bs[buf][wn * 64 + j * 32 + r][kk + hh * 4]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][q], b[j][q], acc[i][j],
                                                                          0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // the main loop ended with a barrier: its LDS is free for the arg-max partials
    epilogue(p, acc, M, s, m0, n0, nt, nN, &As[0][0][0], reinterpret_cast<int *>(&Bs[0][0][0]));
}

}  // namespace

void launch_gemm(const GemmParams &p, hipStream_t st) {
    if (p.prec != PREC_FP32) {
        launch_gemm_split(p, st);
        return;
    }
    const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
    const int total = nM * nN * p.S;
    if (total <= 0) return;
    switch (p.role) {
        case ROLE_QKV: hipLaunchKernelGGL(k_gemm_nt<ROLE_QKV>, dim3(total), dim3(NT), 0, st, p); break;
        case ROLE_WO: hipLaunchKernelGGL(k_gemm_nt<ROLE_WO>, dim3(total), dim3(NT), 0, st, p); break;
        case ROLE_LMHEAD: hipLaunchKernelGGL(k_gemm_nt<ROLE_LMHEAD>, dim3(total), dim3(NT), 0, st, p); break;
        case ROLE_READOUT: hipLaunchKernelGGL(k_gemm_nt<ROLE_READOUT>, dim3(total), dim3(NT), 0, st, p); break;
        case ROLE_SCAN_PROJ: hipLaunchKernelGGL(k_gemm_nt<ROLE_SCAN_PROJ>, dim3(total), dim3(NT), 0, st, p); break;
        default: hipLaunchKernelGGL(k_gemm_nt<ROLE_SIGNAL>, dim3(total), dim3(NT), 0, st, p); break;
    }
}

}  // namespace adn

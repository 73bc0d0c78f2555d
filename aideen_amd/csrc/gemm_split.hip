// Split-precision MFMA GEMM: fp32 operands carried as hi + lo halves on the 16-bit MFMA
// (v_mfma_f32_32x32x16_{f16,bf16}, 2.5 PFLOP/s dense on gfx950, 16x the fp32 MFMA rate).
//
//   x = hi + lo,  hi = T(x),  lo = T(x - hi)                (T = fp16 or bf16, RNE)
//   a.b ~= hi_a.hi_b + hi_a.lo_b + lo_a.hi_b                (TERMS = 3; fp32 accumulate)
//
// With fp16 halves the dropped lo_a.lo_b term and the representation error are ~2^-22 of the
// product, i.e. fp32-level accuracy; the weights carry a power-of-two scale so their lo halves
// stay out of the fp16 subnormal range (the accumulator is unscaled exactly in the epilogue).
// With bf16 halves (no range issue) the error is ~2^-16; TERMS = 1 is the plain bf16-input,
// fp32-accumulate product.
//
// Weights (B) are split once at upload ([S][N][K] hi and lo arrays); activations (A, fp32 in
// HBM) are split while the tile is staged into LDS.  Tiling as the fp32 kernel: 256 threads,
// 128x128 block tile, k-step 32, each wave 64x64 = 2x2 tiles of 32x32.  LDS rows are 64 bytes
// (32 halves) with the 16-byte chunks XOR-swizzled by (row & 3), so the ds_read_b128 operand
// fetches of 32 consecutive rows are bank-conflict free without padding.
#include "gemm_common.h"

namespace adn {

namespace {

using namespace gemm;
constexpr int BK = 32;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

template <typename T>
struct Vec8;
template <>
struct Vec8<_Float16> {
    typedef half8 type;
};
template <>
struct Vec8<__bf16> {
    typedef bf8 type;
};

__device__ __forceinline__ floatx16 mfma16(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma16(bf8 a, bf8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <int ROLE, typename T, int TERMS>
__global__ __launch_bounds__(NT, 2) void k_gemm_split(GemmParams p) {
    typedef typename Vec8<T>::type V8;
    constexpr int PARTS = TERMS == 3 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) T As[2][PARTS][BM][BK];
    __shared__ __attribute__((aligned(16))) T Bs[2][PARTS][BN][BK];

    const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
    int s, mt, nt;
    map_block(blockIdx.x, nM * nN * p.S, nM, nN, s, mt, nt);
    const int M = p.m_count ? min(*p.m_count, p.M) : p.M;
    const int m0 = mt * BM, n0 = nt * BN;
    if (m0 >= M) return;

    const int tid = threadIdx.x;
    const int lrow = tid >> 2;  // 0..63, and lrow + 64
    const int lc = tid & 3;     // 16-byte chunk (8 k values) within the 32-wide k step
    const float *arow[2];
    const T *bhi[2];
    const T *blo[2];
    bool aval[2], bval[2];
    const T *Bh = reinterpret_cast<const T *>(p.Bhi);
    const T *Bl = reinterpret_cast<const T *>(p.Blo);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int m = m0 + lrow + 64 * j;
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
        const int n = n0 + lrow + 64 * j;
        bval[j] = n < p.N;
        const long boff = (long)s * p.b_ss + (long)(bval[j] ? n : 0) * p.K;
        bhi[j] = Bh + boff;
        blo[j] = Bl + boff;
    }

    floatx4 ga[2][2];
    V8 gbh[2], gbl[2];
    auto gload = [&](int kt) {
        const int k = kt * BK + lc * 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (aval[j]) {
                ga[j][0] = *reinterpret_cast<const floatx4 *>(arow[j] + k);
                ga[j][1] = *reinterpret_cast<const floatx4 *>(arow[j] + k + 4);
            } else {
                ga[j][0] = floatx4{0, 0, 0, 0};
                ga[j][1] = floatx4{0, 0, 0, 0};
            }
            if (bval[j]) {
                gbh[j] = *reinterpret_cast<const V8 *>(bhi[j] + k);
                if (TERMS == 3) gbl[j] = *reinterpret_cast<const V8 *>(blo[j] + k);
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    gbh[j][q] = (T)0.0f;
                    gbl[j][q] = (T)0.0f;
                }
            }
        }
    };
    const float asc = p.a_scale;
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = lrow + 64 * j;
            const int pc = (lc ^ (row & 3)) * 8;
            V8 h8, l8;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float x = ga[j][q >> 2][q & 3] * asc;
                const T hv = (T)x;
                h8[q] = hv;
                if (TERMS == 3) l8[q] = (T)(x - (float)hv);
            }
            *reinterpret_cast<V8 *>(&As[buf][0][row][pc]) = h8;
            *reinterpret_cast<V8 *>(&Bs[buf][0][row][pc]) = gbh[j];
            if constexpr (TERMS == 3) {
                *reinterpret_cast<V8 *>(&As[buf][1][row][pc]) = l8;
                *reinterpret_cast<V8 *>(&Bs[buf][1][row][pc]) = gbl[j];
            }
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
        for (int kk = 0; kk < 2; ++kk) {
            // lane half hh takes chunk 2*kk + hh of each row (8 consecutive k); the physical
            // chunk is swizzled by row & 3 == r & 3 (tile row bases are multiples of 32)
            const int pc = ((2 * kk + hh) ^ (r & 3)) * 8;
            V8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ah[i] = *reinterpret_cast<const V8 *>(&As[buf][0][wm * 64 + i * 32 + r][pc]);
                if constexpr (TERMS == 3) al[i] = *reinterpret_cast<const V8 *>(&As[buf][1][wm * 64 + i * 32 + r][pc]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                bh[j] = *reinterpret_cast<const V8 *>(&Bs[buf][0][wn * 64 + j * 32 + r][pc]);
                if constexpr (TERMS == 3) bl[j] = *reinterpret_cast<const V8 *>(&Bs[buf][1][wn * 64 + j * 32 + r][pc]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if constexpr (TERMS == 3) {
                        acc[i][j] = mfma16(al[i], bh[j], acc[i][j]);
                        acc[i][j] = mfma16(ah[i], bl[j], acc[i][j]);
                    }
                    acc[i][j] = mfma16(ah[i], bh[j], acc[i][j]);
                }
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    const float osc = p.out_scale;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] *= osc;
    epilogue(p, acc, M, s, m0, n0, nt, nN, reinterpret_cast<float *>(&As[0][0][0][0]),
             reinterpret_cast<int *>(&Bs[0][0][0][0]));
}

// Weight split at upload: hi = T(w * scale), lo = T(w * scale - hi).
template <typename T>
__global__ void k_split(const float *w, long n, float scale, T *hi, T *lo) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
        const float x = w[i] * scale;
        const T h = (T)x;
        hi[i] = h;
        if (lo) lo[i] = (T)(x - (float)h);
    }
}

template <typename T, int TERMS>
void launch_role(const GemmParams &p, int total, hipStream_t st) {
    const dim3 g(total), b(NT);
    switch (p.role) {
        case ROLE_QKV: hipLaunchKernelGGL((k_gemm_split<ROLE_QKV, T, TERMS>), g, b, 0, st, p); break;
        case ROLE_WO: hipLaunchKernelGGL((k_gemm_split<ROLE_WO, T, TERMS>), g, b, 0, st, p); break;
        case ROLE_LMHEAD: hipLaunchKernelGGL((k_gemm_split<ROLE_LMHEAD, T, TERMS>), g, b, 0, st, p); break;
        case ROLE_READOUT: hipLaunchKernelGGL((k_gemm_split<ROLE_READOUT, T, TERMS>), g, b, 0, st, p); break;
        case ROLE_SCAN_PROJ: hipLaunchKernelGGL((k_gemm_split<ROLE_SCAN_PROJ, T, TERMS>), g, b, 0, st, p); break;
        default: hipLaunchKernelGGL((k_gemm_split<ROLE_SIGNAL, T, TERMS>), g, b, 0, st, p); break;
    }
}

}  // namespace

void launch_gemm_split(const GemmParams &p, hipStream_t st) {
    const int nM = (p.M + BM - 1) / BM, nN = (p.N + BN - 1) / BN;
    const int total = nM * nN * p.S;
    if (total <= 0) return;
    switch (p.prec) {
        case PREC_BF16X3: launch_role<__bf16, 3>(p, total, st); break;
        case PREC_BF16X1: launch_role<__bf16, 1>(p, total, st); break;
        default: launch_role<_Float16, 3>(p, total, st); break;
    }
}

void launch_split_weights(const float *w, long n, float scale, int prec, void *hi, void *lo, hipStream_t st) {
    const long blocks = std::min<long>((n + 255) / 256, 8192);
    if (prec == PREC_F16X3)
        hipLaunchKernelGGL(k_split<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st, w, n, scale,
                           (_Float16 *)hi, (_Float16 *)lo);
    else
        hipLaunchKernelGGL(k_split<__bf16>, dim3((unsigned)blocks), dim3(256), 0, st, w, n, scale,
                           (__bf16 *)hi, (__bf16 *)lo);
}

}  // namespace adn

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
// Weights (B) are split once at upload into hi and lo arrays in a blocked layout (k_split: each
// 32-row x 16-K block one contiguous kilobyte).  Activations (A) stay fp32 in HBM and in LDS and
// are split when a wave reads its MFMA fragments.
//
// Data movement is gfx950's direct global->LDS load (global_load_lds_dwordx4: lane L of a wave
// writes LDS bytes [16L, 16L+16) of a 1 KB block at the wave-uniform address in M0), so no
// staging registers are needed and the k loop runs a STAGES-deep LDS ring of BK = 16 slices:
// the loads for slice kt + STAGES - 1 are issued while slice kt is multiplied, which hides the
// HBM latency of the A rows that miss in L2.  One barrier per slice; each wave waits only for
// its own loads of the slice about to be read (s_waitcnt vmcnt(n) with n = loads still allowed
// in flight), then the barrier makes every wave's part visible and frees the slot that the next
// loads overwrite.  The fragments of the next slice are read from LDS while the current one is
// multiplied (A one step ahead, B one 32-column tile ahead).
//
// LDS rows: A is 16 fp32 = 64 bytes (4 chunks of 16 B), B is 16 halves = 32 bytes (2 chunks).
// The chunks are XOR-swizzled so that the ds_read_b128 fragment reads (32 consecutive rows, one
// chunk each) are conflict-free for 32 and for 64 four-byte banks:
//   A: chunk ^ (((row >> 1) ^ (row >> 2)) & 3)        B: chunk ^ (((row >> 2) ^ (row >> 3)) & 1)
// The DMA writes an LDS block linearly, so the swizzle is applied on the global side: lane L
// fetches the chunk that belongs at its LDS position.
//
// Each wave owns WTM x WTN MFMA tiles of 32x32 (v_mfma_f32_32x32x16), the workgroup a WGM x WGN
// grid of waves.  Wide GEMMs use 256x256 blocks of 8 waves (64x128 each, 2 waves per SIMD; the
// Q|K|V product 32x256 each, so that every A row block is split by one wave), run persistent: a
// resident workgroup per CU walks its share of the tiles, loading the next tile's first slices
// while the current tile's results are stored.
#include "gemm_common.h"

namespace adn {

namespace {

using namespace gemm;
constexpr int BK = 16;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

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

__device__ __forceinline__ int swz_a(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }
__device__ __forceinline__ int swz_b(int row) { return ((row >> 2) ^ (row >> 3)) & 1; }

// Slot stride of the split weights (blocked layout, rows padded to a multiple of 32); b_ss only
// says whether the slots have matrices of their own (non-zero) or share one (zero).
__device__ __forceinline__ long split_slot_stride(const GemmParams &p) {
    return p.b_ss ? (long)((p.N + 31) / 32 * 32) * p.K : 0;
}

__device__ __forceinline__ floatx16 mfma16(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma16(bf8 a, bf8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}


template <int ROLE, typename T, int TERMS, int WTM, int WTN, int WGM, int WGN, int STAGES, bool PRE = false>
__global__ __launch_bounds__(64 * WGM * WGN, (WGM * WGN >= 8) ? 1 : 2) void k_gemm_split(GemmParams p) {
    typedef typename Vec8<T>::type V8;
    constexpr int NW = WGM * WGN;
    constexpr int BMt = WGM * WTM * 32, BNt = WGN * WTN * 32;
    constexpr int PARTS = TERMS == 3 ? 2 : 1;
    constexpr int A_BLK = BMt / 16;  // 1 KB DMA blocks per A slice (16 rows of 64 B)
    constexpr int B_BLK = BNt / 32;  // 1 KB DMA blocks per B slice and part (32 rows of 32 B)
    static_assert(A_BLK % NW == 0 && B_BLK % NW == 0, "DMA blocks must split evenly over waves");
    constexpr int A_PW = A_BLK / NW, B_PW = B_BLK / NW;
    constexpr int LOADS = A_PW + PARTS * B_PW;  // DMA instructions per wave per slice
    static_assert(STAGES >= 3 && (STAGES - 2) * LOADS < 64, "pipeline depth");
    __shared__ __attribute__((aligned(1024))) float As[STAGES][BMt][BK];
    __shared__ __attribute__((aligned(1024))) T Bs[STAGES][PARTS][BNt][BK];

    const int nM = (p.M + BMt - 1) / BMt, nN = (p.N + BNt - 1) / BNt;
    const int total = nM * nN * p.S;
    const int M = p.m_count ? min(*p.m_count, p.M) : p.M;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;

    // Persistent: workgroup b takes tiles b, b + gridDim.x, ... (the grid is a multiple of the
    // XCD count, so each tile stays on the XCD the block order assigns it to); tiles without
    // rows (m0 >= M, converged tokens) are skipped.
    auto next_tile = [&](int t) {
        for (; t < total; t += gridDim.x) {
            int s2, mt2, nt2;
            map_block(t, total, nM, nN, s2, mt2, nt2);
            if (mt2 * BMt < M) return t;
        }
        return total;
    };
    int t = next_tile(blockIdx.x);
    if (t >= total) return;

    // Per-lane source pointers of this wave's DMA blocks for the current tile.  Rows past M or N
    // read row 0 of the operand (their products land in outputs that the epilogue does not
    // store).  B is in the blocked layout (one contiguous 1 KB block per 32 rows x 16 K, see
    // k_split): each DMA block is one such block, lane L taking the chunk its LDS position
    // holds; row groups past N read group 0.
    int s = 0, m0 = 0, n0 = 0;
    static_assert(!PRE || (std::is_same<T, _Float16>::value && TERMS == 3), "pre-split A: fp16 halves");
    // A pre-split by its producer (PRE): fp16 halves hi = f16(x), lo = f16(x - hi) of x = A * asc,
    // asc being the scale derived below, 4 bytes per value as in fp32, each 8 consecutive K values
    // as their 8 hi halves followed by their 8 lo halves (one 16-byte chunk each).  A slice's 64
    // bytes then hold the hi and lo chunks of its K values [0, 8) where the fp32 path has its
    // chunks 0 and 1 and those of [8, 16) at 2 and 3: the loads and fragment reads are the fp32
    // path's, and the fragments are the halves as loaded, with no split work in the k loop.
    const float *Abase = PRE ? p.a_pre : p.A;
    const float *asrc[A_PW];
    const T *bsrc[B_PW][PARTS];
    auto set_tile = [&](int tt) {
        int mt, nt;
        map_block(tt, total, nM, nN, s, mt, nt);
        m0 = mt * BMt;
        n0 = nt * BNt;
#pragma unroll
        for (int j = 0; j < A_PW; ++j) {
            const int row = (wave + NW * j) * 16 + (lane >> 2);
            const int c = (lane & 3) ^ swz_a(row);
            const int m = m0 + row;
            long ar = 0;
            if (m < M) {
                ar = p.a_idx ? (long)p.a_idx[m] : (long)m;
                if (p.a_idx && (ar < 0 || ar >= p.a_idx_max)) {
                    if (p.err) atomicOr(p.err, ADN_DEVERR_TOKEN);
                    ar = 0;
                }
            }
            asrc[j] = Abase + ar * p.a_sm + (long)s * p.a_ss + c * 4;
        }
#pragma unroll
        for (int j = 0; j < B_PW; ++j) {
            const int row = (wave + NW * j) * 32 + (lane >> 1);
            const int c = (lane & 1) ^ swz_b(row);
            const long grp = (n0 >> 5) + wave + NW * j;
            const long off = (long)s * split_slot_stride(p) + (grp * 32 < p.N ? grp : 0) * (p.K / BK) * 512 +
                             (lane >> 1) * 16 + c * 8;
            bsrc[j][0] = reinterpret_cast<const T *>(p.Bhi) + off;
            if constexpr (TERMS == 3) bsrc[j][1] = reinterpret_cast<const T *>(p.Blo) + off;
        }
    };
    auto issue = [&](int kt, int st) {
#pragma unroll
        for (int j = 0; j < A_PW; ++j)
            __builtin_amdgcn_global_load_lds((const void *)(asrc[j] + kt * BK),
                                             (lds_void *)&As[st][(wave + NW * j) * 16][0], 16, 0, 0);
#pragma unroll
        for (int j = 0; j < B_PW; ++j)
#pragma unroll
            for (int q = 0; q < PARTS; ++q)
                __builtin_amdgcn_global_load_lds((const void *)(bsrc[j][q] + kt * 512),
                                                 (lds_void *)&Bs[st][q][(wave + NW * j) * 32][0], 16, 0, 0);
    };

    const int wm = wave / WGN, wn = wave % WGN;
    const int r = lane & 31, hh = lane >> 5;
    const int pb = (hh ^ swz_b(r)) * 8;
    float asc = p.a_scale, osc = p.out_scale;
    if (p.a_absmax) {  // data-dependent A scale (power of two, never above the static one)
        const float mx = __uint_as_float(*p.a_absmax);
        if (mx > 0.0f) {
            const float dyn = exp2f(floorf(log2f(p.a_headroom / mx)));
            if (dyn < asc) {
                osc *= asc / dyn;
                asc = dyn;
            }
        }
    }
    // fragment chunk positions: rows r + 32t share swz(r) (the swizzles read row bits 1..3); a
    // lane's 8 K values are chunks 2 hh and 2 hh + 1 (fp32 values, or their hi and lo halves)
    const int pa0 = ((2 * hh) ^ swz_a(r)) * 4, pa1 = ((2 * hh + 1) ^ swz_a(r)) * 4;
    floatx16 acc[WTM][WTN];

    // Fragments in registers.  B is streamed one 32-column tile at a time through two buffers,
    // tile j + 1 (or the next slice's tile 0) being read while tile j's MFMAs run.  A of the next
    // slice is read raw (fp32) at the top of a slice and split into its halves in pieces placed
    // between the current slice's MFMAs, so that the split's VALU work issues while the matrix
    // core is busy; the split halves are double-buffered (ah/al[P] in use, [P ^ 1] being
    // filled) and the k loop is unrolled by two so that the buffers swap without moves.
    floatx4 anx[WTM][2];
    V8 ah[2][WTM], al[2][WTM];
    V8 bq[2][PARTS];
    auto read_a = [&](int st) {
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
            const int row = (wm * WTM + i) * 32 + r;
            anx[i][0] = *reinterpret_cast<const floatx4 *>(&As[st][row][pa0]);
            anx[i][1] = *reinterpret_cast<const floatx4 *>(&As[st][row][pa1]);
        }
    };
    // The empty asm pins the halves where they are formed: without it the compiler sinks a
    // piece into the next slice's block, after its barrier, out of reach of the MFMAs it is
    // meant to overlap.
    auto split_i = [&](int i, V8 &h, V8 &l) {
        if constexpr (PRE) {
            h = __builtin_bit_cast(V8, anx[i][0]);
            l = __builtin_bit_cast(V8, anx[i][1]);
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float x = anx[i][q >> 2][q & 3] * asc;
                const T hv = (T)x;
                h[q] = hv;
                if constexpr (TERMS == 3) l[q] = (T)(x - (float)hv);
            }
        }
        if constexpr (TERMS == 3)
            asm volatile("" : "+v"(h), "+v"(l));
        else
            asm volatile("" : "+v"(h));
    };
    auto read_b = [&](int st, int j, V8 (&bb)[PARTS]) {
        const int row = (wn * WTN + j) * 32 + r;
#pragma unroll
        for (int q = 0; q < PARTS; ++q) bb[q] = *reinterpret_cast<const V8 *>(&Bs[st][q][row][pb]);
    };
    auto mfma_tile = [&](int j, const V8 (&bb)[PARTS], const V8 (&h)[WTM], const V8 (&l)[WTM]) {
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
            if constexpr (TERMS == 3) {
                acc[i][j] = mfma16(l[i], bb[0], acc[i][j]);
                acc[i][j] = mfma16(h[i], bb[1], acc[i][j]);
            }
            acc[i][j] = mfma16(h[i], bb[0], acc[i][j]);
        }
    };

    const int nk = p.K / BK;
    auto prologue = [&]() {
#pragma unroll
        for (int st = 0; st < STAGES - 1; ++st)
            if (st < nk) issue(st, st);
    };
    // One 16-K slice: P selects the split A buffer in use.
    auto step = [&](int kt, auto par) {
        constexpr int P = decltype(par)::value;
        const int cs = kt % STAGES, ns = (kt + 1) % STAGES;
        if (kt + 1 < nk) {
            // slice kt+1 visible: this wave's loads of it are done once at most STAGES-3 later
            // slices are in flight; the barrier covers the other waves' loads and their reads of
            // the slot about to be refilled (slice kt-1's, last read in the previous step)
            if (kt + STAGES - 2 < nk)
                wait_vmcnt<(STAGES - 3) * LOADS>();
            else
                wait_vmcnt<0>();
            lds_barrier();
            if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        }
        // The reads below are unconditional so that the wait counts stay exact: after the last
        // slice they read a slot no load writes any more, and the values are not used.
        // sched_barrier keeps each tile's reads ahead of the previous tile's MFMAs; within a
        // tile the split pieces are interleaved with the MFMAs.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            if (j == 0) read_a(ns);
            read_b(j + 1 < WTN ? cs : ns, (j + 1) % WTN, bq[(j + 1) & 1]);
            mfma_tile(j, bq[j & 1], ah[P], al[P]);
            if constexpr (WTM == 1 && WTN >= 8 && !PRE) {
                // a single A tile: its split in pieces of one value per tile j = 2..7 (two at
                // j = 1), so that each tile's MFMAs have a few split instructions beside them
                if (j >= 1 && j <= 7) {
#pragma unroll
                    for (int q = (j == 1 ? 0 : j); q <= j; ++q) {
                        const float x = anx[0][q >> 2][q & 3] * asc;
                        const T hv = (T)x;
                        ah[P ^ 1][0][q] = hv;
                        if constexpr (TERMS == 3) al[P ^ 1][0][q] = (T)(x - (float)hv);
                    }
                    if constexpr (TERMS == 3)
                        asm volatile("" : "+v"(ah[P ^ 1][0]), "+v"(al[P ^ 1][0]));
                    else
                        asm volatile("" : "+v"(ah[P ^ 1][0]));
                }
            } else {
                if (j >= 1 && j - 1 < WTM) split_i(j - 1, ah[P ^ 1][j - 1], al[P ^ 1][j - 1]);
            }
            // Order within the tile: its first MFMA (whose operands were read a tile earlier:
            // the wait before it then covers only those), the reads for the next tile, then the
            // remaining MFMAs each followed by up to 6 split instructions.
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, PARTS + 2 * WTM, 0);
#pragma unroll
            for (int u = 1; u < WTM * (TERMS == 3 ? 3 : 1); ++u) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (WTN & 1) {  // the next slice's tile 0 went to buffer 1
#pragma unroll
            for (int q = 0; q < PARTS; ++q) bq[0][q] = bq[1][q];
        }
#pragma unroll
        for (int i = WTN - 1; i < WTM; ++i)
            if (i >= 0) split_i(i, ah[P ^ 1][i], al[P ^ 1][i]);
    };
    set_tile(t);
    prologue();
    bool first = true;
    while (true) {
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    // this wave's loads of the tile's first slice are complete: in a workgroup's first tile at
    // most STAGES-2 later slices are in flight; after an epilogue, whose stores the
    // vector-memory counter also counts, everything is waited for
    if (first && STAGES - 2 < nk)
        wait_vmcnt<(STAGES - 2) * LOADS>();
    else
        wait_vmcnt<0>();
    first = false;
    lds_barrier();
    read_a(0);
    read_b(0, 0, bq[0]);
#pragma unroll
    for (int i = 0; i < WTM; ++i) split_i(i, ah[0][i], al[0][i]);
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        step(kt, std::integral_constant<int, 0>());
        step(kt + 1, std::integral_constant<int, 1>());
    }
    if (kt < nk) step(kt, std::integral_constant<int, 0>());
    lds_barrier();  // every wave is done with the ring
    // The next tile's first slices are loaded into ring slots 0..STAGES-2 while this tile's
    // results are stored; the epilogue's LDS scratch (arg-max partials) is slot STAGES-1.
    const int es = s, em0 = m0, en0 = n0;
    const int tn = next_tile(t + gridDim.x);
    if (tn < total) {
        set_tile(tn);
        prologue();
    }
    epilogue_t<ROLE, WTM, WTN, WGM, WGN>(p, acc, M, es, em0, en0, osc, &As[STAGES - 1][0][0],
                                         reinterpret_cast<int *>(&Bs[STAGES - 1][0][0][0]));
    if (tn >= total) break;
    t = tn;
    }
}

// Skinny GEMM (at most 32 rows: one position of every sequence, a decode step).  There the
// ring kernel's serial k loop (one barrier per 16-K slice) is the whole cost, so here a
// workgroup of KW waves owns a 32 x (32 WTN) output block and wave w multiplies its own K range
// [w K/KW, (w+1) K/KW) straight from global memory into registers, 64 K values per step:
// lane (q = lane & 31, g = lane >> 5) loads the 32 consecutive K values [64i + 32g, +32) of A
// row q and of B row q (of each of the WTN column tiles), and MFMA step j (0..3) takes values
// [8j, 8j + 8) of that run.  A and B use the same K order, so each MFMA still contracts
// matching K indices.  The KW partial blocks are summed in LDS in wave order (deterministic)
// and wave 0 runs the role's epilogue.
//
// ATTN (W_o at a few rows, GemmParams::attn_qkv): A, the attention mix of slot s, is formed here
// from the compact Q|K|V rows (fixed_point_memory_reasoning.rs:1397-1421: scores q_s.k_c / sqrt(d),
// optionally clamped to [-4, 4], softmax with max and sum in key order, mix = sum over c in order
// of w_c v_c), so that the attention needs no kernel of its own; its work is repeated by the
// slot's column blocks, which at a few rows costs less than a launch.  The block forms each row's
// mix in LDS: every thread loads its elements of every key slot at once (clamped addresses, so the
// loads do not wait behind per-slot branches), the score shares are summed over the waves in order,
// and the K loop then reads A from LDS.
//
// UPD (Q|K|V at a few rows, GemmParams::upd_o): A is h after the previous iteration's damped
// update, formed here (fixed_point_memory_reasoning.rs:1386-1393, with k_update_tok's arithmetic
// and summation order: one wave per row, a lane's elements lane + 64e summed in e order, then the
// wave sum) into LDS, so that the update needs no kernel of its own; the slot's first column
// block also stores the row.  Used only where no token can exit before the last iteration, so
// that the update's residual and exit test are not needed.
template <int ROLE, typename T, int TERMS, int KW, int WTN, bool ATTN = false, bool UPD = false>
__global__ __launch_bounds__(64 * KW) void k_gemm_skinny(GemmParams p) {
    typedef typename Vec8<T>::type V8;
    __shared__ float red[KW > 1 ? KW - 1 : 1][WTN * 16][64];  // [wave-1][element][lane]
    // LM head: the 32 rows' (max, arg-max) partials of the block's 128 columns
    __shared__ float am_v[ROLE == ROLE_LMHEAD ? 32 : 1];
    __shared__ int am_i[ROLE == ROLE_LMHEAD ? 32 : 1];
    constexpr int HM = 16;         // slots at most
    constexpr int DM = 2048;       // row width at most
    constexpr int NT = 64 * KW;
    __shared__ float sc_w[ATTN ? ATTN_FUSE_ROWS : 1][ATTN ? KW : 1][HM];  // per row and wave: score shares
    constexpr bool LA = ATTN || UPD;  // A rows formed in LDS
    __shared__ __attribute__((aligned(16))) float mix_l[LA ? ATTN_FUSE_ROWS : 1][LA ? DM : 1];
    __shared__ float hold_l[UPD ? ATTN_FUSE_ROWS : 1][UPD ? DM : 1];
    constexpr int BNt = 32 * WTN;
    const int nN = (p.N + BNt - 1) / BNt;
    int s, mt, nt;
    map_block(blockIdx.x, nN * p.S, 1, nN, s, mt, nt);
    if constexpr (ATTN) {
        if (blockIdx.x == 0 && threadIdx.x == 0) {  // the attention kernel's bookkeeping
            const int n = *p.m_count;
            *p.attn_cnt_next = 0;  // the update of this iteration appends survivors there
            *p.attn_cnt_hist += n;
        }
    }
    const int M = p.m_count ? min(*p.m_count, p.M) : p.M;
    if (M <= 0) return;
    const int n0 = nt * BNt;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int q = lane & 31, g = lane >> 5;
    const int kw = p.K / KW;  // a multiple of 64 (checked by the launcher)
    if constexpr (ATTN) {
        // Wave w takes the elements of its own K range [w kw, (w+1) kw) (lane l: kb + l + 64j), so
        // that the mix it forms there is the A its k loop reads: only the score shares cross the
        // waves (one barrier per row; each row has its own sc_w slice, so none is reused).  Every
        // wave then forms the softmax itself, lane c holding slot c, with the sequential form's
        // order (scores summed over the waves in order, max and sum over the slots in key order).
        const int H = p.S, dd = p.K;
        const long rs3 = 3L * dd;
        const float scale = 1.0f / sqrtf((float)dd);
        const int kb = wave * kw;
        const bool one = kw <= 128;  // the V elements loaded with Q and K, one round trip for the three
        for (int r = 0; r < M; ++r) {  // M <= ATTN_FUSE_ROWS
            const float *row = p.attn_qkv + (long)r * H * rs3;
            float part[HM];
#pragma unroll
            for (int c = 0; c < HM; ++c) part[c] = 0.0f;
            float vpre[HM][2];
            for (int e0 = 0; e0 < kw; e0 += 128) {
                float qv[2], kv[HM][2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int el = e0 + lane + 64 * j;
                    const int e = kb + min(el, kw - 1);
                    qv[j] = el < kw ? row[(long)s * rs3 + e] : 0.0f;
#pragma unroll
                    for (int c = 0; c < HM; ++c) kv[c][j] = row[(long)(c < H ? c : 0) * rs3 + dd + e];
                    if (one) {
#pragma unroll
                        for (int c = 0; c < HM; ++c) vpre[c][j] = row[(long)(c < H ? c : 0) * rs3 + 2 * dd + e];
                    }
                }
#pragma unroll
                for (int c = 0; c < HM; ++c)
#pragma unroll
                    for (int j = 0; j < 2; ++j) part[c] += qv[j] * kv[c][j];
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {  // wave sums, the rounds issued for every slot at once
                float o[HM];
#pragma unroll
                for (int c = 0; c < HM; ++c) o[c] = __shfl_xor(part[c], off, 64);
#pragma unroll
                for (int c = 0; c < HM; ++c) part[c] += o[c];
            }
            if (lane == 0) {
#pragma unroll
                for (int c = 0; c < HM; ++c) sc_w[r][wave][c] = part[c];
            }
            __syncthreads();
            float sc = -INFINITY;
            if (lane < H) {
                float t = 0.0f;
                for (int w = 0; w < KW; ++w) t += sc_w[r][w][lane];
                sc = t * scale;
                if (p.attn_clamp) sc = fminf(fmaxf(sc, -4.0f), 4.0f);
            }
            float mx = -INFINITY;
            for (int c = 0; c < H; ++c) mx = fmaxf(mx, __shfl(sc, c, 64));
            const float ex = lane < H ? expf(sc - mx) : 0.0f;
            float sum = 0.0f;
            for (int c = 0; c < H; ++c) sum += __shfl(ex, c, 64);
            const float wl = ex / sum;
            float wv[HM];
#pragma unroll
            for (int c = 0; c < HM; ++c) wv[c] = c < H ? __shfl(wl, c, 64) : 0.0f;
            for (int e0 = 0; e0 < kw; e0 += 128) {
                float vv[HM][2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int e = kb + min(e0 + lane + 64 * j, kw - 1);
#pragma unroll
                    for (int c = 0; c < HM; ++c)
                        vv[c][j] = one ? vpre[c][j] : row[(long)(c < H ? c : 0) * rs3 + 2 * dd + e];
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    float acc = 0.0f;
#pragma unroll
                    for (int c = 0; c < HM; ++c)
                        if (c < H) acc = acc + vv[c][j] * wv[c];
                    if (e0 + lane + 64 * j < kw) mix_l[r][kb + e0 + lane + 64 * j] = acc;
                }
            }
        }
        // mix_l: each wave reads back only its own K range (a wave's LDS operations complete in order)
    }
    if constexpr (UPD) {
#pragma clang fp contract(off)  // as in k_update_tok
        const int dd = p.K, E = dd / 64;
        const long hd = (long)p.S * dd;
        const float beta = p.upd_beta, omb = 1.0f - beta;
        for (int r = wave; r < M; r += KW) {  // M <= ATTN_FUSE_ROWS
            long t = p.a_idx ? (long)p.a_idx[r] : (long)r;
            if (p.a_idx && (t < 0 || t >= p.a_idx_max)) t = 0;  // flagged below
            const float *o = p.upd_o + ((long)r * p.S + s) * dd;
            const float *sg = p.upd_sig + t * hd + (long)s * dd;
            const float *an = p.upd_anchor + (long)s * dd;
            const float *hp = p.A + t * hd + (long)s * dd;
            float ss = 0.0f;
            for (int e0 = 0; e0 < E; e0 += 8) {  // 8 elements' loads in flight per lane
                float ov[8], sv[8], av[8], hv[8], gv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int idx = lane + 64 * min(e0 + u, E - 1);
                    ov[u] = o[idx];
                    sv[u] = sg[idx];
                    av[u] = an[idx];
                    hv[u] = hp[idx];
                    gv[u] = p.upd_norm[idx];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (e0 + u < E) {
                        const int idx = lane + 64 * (e0 + u);
                        const float as_ = (ov[u] + sv[u]) + 0.0f;  // k_update_tok adds a zero history term
                        const float c = as_ + av[u];
                        ss += p.upd_excl ? as_ * as_ : c * c;
                        mix_l[r][idx] = gv[u] * c;
                        hold_l[r][idx] = hv[u];
                    }
            }
            ss = wave_sum(ss);
            const float rms = sqrtf(ss / (float)dd + 1e-6f);
            float *hw = p.upd_hout + t * hd + (long)s * dd;
            for (int e = 0; e < E; ++e) {  // each lane reads back only what it wrote
                const int idx = lane + 64 * e;
                const float f = mix_l[r][idx] / rms;
                const float hn = f * beta + hold_l[r][idx] * omb;
                mix_l[r][idx] = hn;
                if (nt == 0) hw[idx] = hn;
            }
        }
        __syncthreads();
    }

    // rows past M read row 0, columns past N row 0 of B (their outputs are not stored)
    long ar = 0;
    if (q < M) {
        ar = p.a_idx ? (long)p.a_idx[q] : (long)q;
        if (p.a_idx && (ar < 0 || ar >= p.a_idx_max)) {
            if (p.err) atomicOr(p.err, ADN_DEVERR_TOKEN);
            ar = 0;
        }
    }
    const float *ap = p.A + ar * p.a_sm + (long)s * p.a_ss;
    // B row n in the blocked layout: K values [16b, 16b + 16) at block b of its 32-row group
    const T *bhp[WTN], *blp[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
        const int n = n0 + 32 * j + q;
        const long nn = n < p.N ? n : 0;
        const long boff = (long)s * split_slot_stride(p) + (nn >> 5) * (p.K / 16) * 512 + (nn & 31) * 16;
        bhp[j] = reinterpret_cast<const T *>(p.Bhi) + boff;
        blp[j] = reinterpret_cast<const T *>(TERMS == 3 ? p.Blo : p.Bhi) + boff;
    }

    float asc = p.a_scale, osc = p.out_scale;
    if (p.a_absmax) {  // data-dependent A scale (power of two, never above the static one)
        const float mx = __uint_as_float(*p.a_absmax);
        if (mx > 0.0f) {
            const float dyn = exp2f(floorf(log2f(p.a_headroom / mx)));
            if (dyn < asc) {
                osc *= asc / dyn;
                asc = dyn;
            }
        }
    }
    floatx16 acc[1][WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[0][j][e] = 0.0f;

    for (int k = wave * kw; k < (wave + 1) * kw; k += 64) {
        const int ko = k + 32 * g;
        floatx4 a[8];
        V8 bh[WTN][4], bl[WTN][4];
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const long e = (long)((ko >> 4) + (st >> 1)) * 512 + (st & 1) * 8;
                bh[j][st] = *reinterpret_cast<const V8 *>(bhp[j] + e);
                if constexpr (TERMS == 3) bl[j][st] = *reinterpret_cast<const V8 *>(blp[j] + e);
            }
        if constexpr (LA) {  // the rows formed above (rows past M read row 0)
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const floatx4 *>(&mix_l[q < M ? q : 0][ko + 4 * i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const floatx4 *>(ap + ko + 4 * i);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            V8 ah, al;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = a[2 * st + (e >> 2)][e & 3] * asc;
                const T hv = (T)x;
                ah[e] = hv;
                if constexpr (TERMS == 3) al[e] = (T)(x - (float)hv);
            }
#pragma unroll
            for (int j = 0; j < WTN; ++j) {
                if constexpr (TERMS == 3) {
                    acc[0][j] = mfma16(al, bh[j][st], acc[0][j]);
                    acc[0][j] = mfma16(ah, bl[j][st], acc[0][j]);
                }
                acc[0][j] = mfma16(ah, bh[j][st], acc[0][j]);
            }
        }
    }
    if constexpr (KW > 1) {
        if (wave > 0)
#pragma unroll
            for (int j = 0; j < WTN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) red[wave - 1][j * 16 + e][lane] = acc[0][j][e];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
            for (int j = 0; j < WTN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[0][j][e] += red[w][j * 16 + e][lane];
    }
    epilogue_t<ROLE, 1, WTN, 1, 1>(p, acc, M, s, 0, n0, osc, am_v, am_i);
}

// Weight split at upload: hi = T(w * scale), lo = T(w * scale - hi), from [S][N][K] fp32 into
// the blocked layout: per slot, rows in groups of 32 (N padded to a multiple of 32 with zeros),
// each group's K in blocks of 16, a block (32 rows x 16 halves, 1 KB) contiguous and row-major:
//   (s, n, k) -> s * split_slot_stride + ((n / 32) * (K / 16) + k / 16) * 512 + (n % 32) * 16 + k % 16
// so that a GEMM's 32-row x 16-K load is one contiguous kilobyte.  eye: split w + I instead (square
// matrices), so that a product with a residual, y + W y, runs as the plain product (I + W) y.
template <typename T>
__global__ void k_split(const float *w, int S, int N, int K, float scale, T *hi, T *lo, bool eye) {
    const long np = ((long)N + 31) / 32 * 32, total = (long)S * np * K, kb = K / 16;
    for (long o = (long)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (long)gridDim.x * blockDim.x) {
        const long sl = o / (np * K), ro = o - sl * np * K;
        const long blk = ro >> 9, in = ro & 511;
        const long n = (blk / kb) * 32 + (in >> 4), k = (blk % kb) * 16 + (in & 15);
        const float x = n < N ? (w[(sl * N + n) * K + k] + (eye && n == k ? 1.0f : 0.0f)) * scale : 0.0f;
        const T h = (T)x;
        hi[o] = h;
        if (lo) lo[o] = (T)(x - (float)h);
    }
}

// Grid of the persistent ring kernel: at most `per_cu` resident workgroups on every CU, a
// multiple of the XCD count (block i runs on XCD i % 8), never more than the tiles.
int ring_grid(int total, int per_cu) {
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
        return total;
    long g = (long)ncu * per_cu;
    g -= g % NXCD;
    if (g < NXCD) g = NXCD;
    return (int)std::min<long>(total, g);
}

template <int ROLE, typename T, int TERMS, int WTN, bool ATTN = false, bool UPD = false>
void launch_skinny(const GemmParams &p, int kw, hipStream_t st) {
    const int total = ((p.N + 32 * WTN - 1) / (32 * WTN)) * p.S;
    if (total <= 0) return;
    switch (kw) {  // kw divides K / 64
        case 8: hipLaunchKernelGGL((k_gemm_skinny<ROLE, T, TERMS, 8, WTN, ATTN, UPD>), dim3(total), dim3(512), 0, st, p); break;
        case 4: hipLaunchKernelGGL((k_gemm_skinny<ROLE, T, TERMS, 4, WTN, ATTN, UPD>), dim3(total), dim3(256), 0, st, p); break;
        case 2: hipLaunchKernelGGL((k_gemm_skinny<ROLE, T, TERMS, 2, WTN, ATTN, UPD>), dim3(total), dim3(128), 0, st, p); break;
        default: hipLaunchKernelGGL((k_gemm_skinny<ROLE, T, TERMS, 1, WTN, ATTN, UPD>), dim3(total), dim3(64), 0, st, p); break;
    }
}

// Tile configurations (WTM, WTN, WGM, WGN, STAGES): GEMMs with M >= 1024 and N >= 512 use
// 256x256 blocks of 8 waves (one workgroup per CU, 128 KB of LDS ring); the rest 128x128 blocks
// of 4 waves (two workgroups per CU) so that their grids still cover the chip.  The 256x256
// configuration runs persistent (one resident workgroup per CU walking its share of tiles, the
// next tile's first slices loaded during the epilogue); the smaller ones launch a workgroup per
// tile, whose short k loops would otherwise wait on the previous tile's stores.
template <int ROLE, typename T, int TERMS>
void launch_cfg(const GemmParams &p, hipStream_t st) {
    if constexpr (ROLE == ROLE_LMHEAD) {
        if (p.M <= 32 && p.K % 64 == 0) {
            // skinny LM head (a decode step): 128-column blocks, the arg-max partials' width; at
            // a few rows 64-column blocks with partials per 64 columns (twice the workgroups on
            // the weight stream, as for the other products); K split as below
            const int steps = p.K / 64;
            int kw = steps >= 16 ? 8 : steps >= 8 ? 4 : steps >= 4 ? 2 : 1;
            while (steps % kw) kw >>= 1;
            if (gemm_lm_partial_cols(p.prec, p.M, p.K) == 64)
                launch_skinny<ROLE, T, TERMS, 2>(p, kw, st);
            else
                launch_skinny<ROLE, T, TERMS, 4>(p, kw, st);
            return;
        }
    } else {
        if (p.M <= 32 && p.K % 64 == 0) {
            // skinny: K split over the waves of a workgroup, about two 64-K steps per wave;
            // wide outputs take two column tiles per wave (each A fragment feeds both) except at
            // a few rows, where twice the workgroups stream the weights sooner (decode Q|K|V at
            // one row: 248 -> 238 us per token; at 32 rows the two-tile waves are 7% faster)
            const int steps = p.K / 64;
            int kw = steps >= 16 ? 8 : steps >= 8 ? 4 : steps >= 4 ? 2 : 1;
            while (steps % kw) kw >>= 1;  // each wave's K range is whole 64-K steps
            if constexpr (ROLE == ROLE_WO) {
                if (p.attn_qkv) {  // the attention formed in the kernel (a few rows)
                    launch_skinny<ROLE, T, TERMS, 1, true>(p, kw, st);
                    return;
                }
            }
            if constexpr (ROLE == ROLE_QKV) {
                if (p.upd_o) {  // the previous iteration's update formed in the kernel (a few rows)
                    launch_skinny<ROLE, T, TERMS, 1, false, true>(p, kw, st);
                    return;
                }
            }
            if (p.N >= 1024 && p.M > ATTN_FUSE_ROWS)
                launch_skinny<ROLE, T, TERMS, 2>(p, kw, st);
            else
                launch_skinny<ROLE, T, TERMS, 1>(p, kw, st);
            return;
        }
        if (p.M <= 32) {
            // skinny (at most 32 rows, e.g. one position of every sequence): 32x32 blocks of one
            // wave, an 8-deep ring, so that the weight stream is spread over as many CUs as
            // possible (an LM head with K not a multiple of 64 keeps the 128x128 tiles below: its
            // arg-max partials are per 128 columns)
            const int total = ((p.N + 31) / 32) * p.S;
            if (total > 0)
                hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 1, 1, 1, 1, 8>), dim3(total), dim3(64), 0, st, p);
            return;
        }
    }
    const bool big = p.N >= 512 && p.M >= 1024;  // the configuration gemm_presplit_ok names
    const int bm = big ? 256 : 128, bn = big ? 256 : 128;
    const int total = ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn) * p.S;
    if (total <= 0) return;
    if (big) {
        // the roles whose A a producer writes pre-split (the slot mix, the LM head's normalised row)
        if constexpr (std::is_same<T, _Float16>::value && TERMS == 3 && (ROLE == ROLE_WO || ROLE == ROLE_LMHEAD)) {
            if (p.a_pre) {
                hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 2, 4, 4, 2, 4, true>), dim3(ring_grid(total, 1)),
                                   dim3(512), 0, st, p);
                return;
            }
        }
        if constexpr (ROLE == ROLE_QKV) {
            // waves of 32 x 256 (8 down the block): each A row block is split by one wave only
            hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 1, 8, 8, 1, 4>), dim3(ring_grid(total, 1)), dim3(512), 0, st,
                               p);
            return;
        }
        hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 2, 4, 4, 2, 4>), dim3(ring_grid(total, 1)), dim3(512), 0, st,
                           p);
    }
    else if (p.N <= 64 && p.M >= 1024) {
        // narrow outputs (the carrier's projections, r + 2N = 64 columns): 128 x 64 blocks of two
        // 64 x 64 waves, no zero-padded half tile
        const int t64 = ((p.M + 127) / 128) * ((p.N + 63) / 64) * p.S;
        hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 2, 2, 2, 1, 4>), dim3(t64), dim3(128), 0, st, p);
    } else
        hipLaunchKernelGGL((k_gemm_split<ROLE, T, TERMS, 2, 2, 2, 2, 4>), dim3(total), dim3(256), 0, st, p);
}

template <typename T, int TERMS>
void launch_role(const GemmParams &p, hipStream_t st) {
    switch (p.role) {
        case ROLE_QKV: launch_cfg<ROLE_QKV, T, TERMS>(p, st); break;
        case ROLE_WO: launch_cfg<ROLE_WO, T, TERMS>(p, st); break;
        case ROLE_LMHEAD: launch_cfg<ROLE_LMHEAD, T, TERMS>(p, st); break;
        case ROLE_READOUT: launch_cfg<ROLE_READOUT, T, TERMS>(p, st); break;
        case ROLE_SCAN_PROJ: launch_cfg<ROLE_SCAN_PROJ, T, TERMS>(p, st); break;
        default: launch_cfg<ROLE_SIGNAL, T, TERMS>(p, st); break;
    }
}

}  // namespace

void launch_gemm_split(const GemmParams &p, hipStream_t st) {
    switch (p.prec) {
        case PREC_BF16X3: launch_role<__bf16, 3>(p, st); break;
        case PREC_BF16X1: launch_role<__bf16, 1>(p, st); break;
        default: launch_role<_Float16, 3>(p, st); break;
    }
}

bool gemm_presplit_ok(int prec, int M, int N) { return prec == PREC_F16X3 && M >= 1024 && N >= 512; }

int gemm_lm_partial_cols(int prec, int M, int K) {
    return (prec != PREC_FP32 && M <= ATTN_FUSE_ROWS && K % 64 == 0) ? 64 : GEMM_BN;
}

bool gemm_attn_fusable(int prec, int M, int K, int S) {
    return prec != PREC_FP32 && M <= ATTN_FUSE_ROWS && K % 64 == 0 && K <= 2048 && S <= 16;
}

long split_weight_elems(int S, int N, int K) { return (long)S * ((N + 31) / 32 * 32) * K; }

void launch_split_weights(const float *w, int S, int N, int K, float scale, int prec, void *hi, void *lo,
                          hipStream_t st, bool eye) {
    const long n = split_weight_elems(S, N, K);
    const long blocks = std::min<long>((n + 255) / 256, 8192);
    if (prec == PREC_F16X3)
        hipLaunchKernelGGL(k_split<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st, w, S, N, K, scale,
                           (_Float16 *)hi, (_Float16 *)lo, eye);
    else
        hipLaunchKernelGGL(k_split<__bf16>, dim3((unsigned)blocks), dim3(256), 0, st, w, S, N, K, scale,
                           (__bf16 *)hi, (__bf16 *)lo, eye);
}

}  // namespace adn

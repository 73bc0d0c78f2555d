// Picard-loop kernels of the DEQ solve (everything between the projection GEMMs).
//
// Reference semantics: FixedPointMemoryReasoning::{init, step_with_fixed_hist_ctx,
// cross_slot_attn} (fixed_point_memory_reasoning.rs:1372-1448), rms_norm (:1300-1303),
// damped_update (spectral_norm.rs:93-95), exit on the residual between consecutive iterates
// (aideen-node/src/inference.rs:196-228, ARCHITECTURE.md:178-185) with converged tokens frozen.
//
// All of these kernels are HBM-bound: they touch each state row a small constant number of
// times.  The loop is device-resident: every kernel reads the active-token count from device
// memory and blocks beyond it exit at once, so the host enqueues max_iters iterations without
// reading anything back.
#include "kernels.h"

namespace adn {

namespace {

constexpr int WAVES_PER_BLOCK = 4;

// ---------------------------------------------------------------------------------------
// init: h0 = x + anchor (FPMR:1432-1448) or signal/rms(signal) (UWGSL:900-943); first active
// list = all tokens in order; iteration counts cleared.
// ---------------------------------------------------------------------------------------
__global__ void k_init(Dims D, SolveBuffers b, const float *x_src, const int32_t *tokens, int ntok,
                       const float *anchor) {
    const int wave = blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int row = wave;  // (t, s)
    if (row >= ntok * D.H) return;
    const int t = row / D.H, s = row - t * D.H;
    const int d = D.d;
    float *h = b.h + (long)row * d;
    float mx = 0.0f;  // largest finite |h0| of this lane
    auto put = [&](int i, float v) {
        h[i] = v;
        mx = fmaxf(mx, fabsf(v) < INFINITY ? fabsf(v) : 0.0f);
    };
    if (D.flags & ADN_F_INIT_SIGNAL_RMS) {
        const float *sg = b.signal + (long)row * d;
        float ss = 0.0f;
        for (int i = lane; i < d; i += 64) ss += sg[i] * sg[i];
        ss = wave_sum(ss);
        const float rms = sqrtf(ss / (float)d + 1e-6f);
        for (int i = lane; i < d; i += 64) put(i, sg[i] / rms);
    } else {
        long xr = t;
        if (tokens) {
            xr = tokens[t];
            if (xr < 0 || xr >= D.V) {
                if (lane == 0) atomicOr(b.err, ADN_DEVERR_TOKEN);
                xr = 0;
            }
        }
        const float *x = x_src + xr * d;
        const float *an = anchor + (long)s * d;
        for (int i = lane; i < d; i += 64) put(i, x[i] + an[i]);
    }
    if (b.amax_h) track_absmax(b.amax_h, mx);  // the bound on |h| the split GEMMs scale their A by
    if (s == 0 && lane == 0) {
        b.act[0][t] = t;
        b.iters[t] = 0;
        if (b.rprev) b.rprev[t] = 1.0f;
    }
    if (row == 0 && lane == 0) {
        b.cnt[0] = ntok;
        b.cnt[1] = 0;
    }
    if (row == 0)
        for (int q = lane; q < ADN_PROFILE_MAX_ITERS; q += 64) b.cnt_hist[q] = 0;
}

// ---------------------------------------------------------------------------------------
// Slot attention for one active token (FPMR:1397-1421): scores q_a.k_c/sqrt(d) (optionally
// clamped to [-4,4], PPT:216), max-subtracted softmax over key slots, mix_a = sum_c attn v_c
// folded in slot order.  One wave per (token, group of QA query slots); P = QA*H <= 64 partial
// dot products per lane, all-reduced across the wave so every lane holds every score.
// ---------------------------------------------------------------------------------------
// *p, loaded non-temporally if NT
template <bool NT>
__device__ __forceinline__ float qkv_load(const float *p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

// W_o's A operand written pre-split (b.mix_pre): the scale the split GEMM derives for it (its
// a_scale 1, lowered to 2^floor(log2(headroom / bound)) when the h bound calls for it), and VEC
// consecutive elements of a row from e0 (VEC divides 8) as fp16 halves of x = v * asc,
// hi = f16(x) and lo = f16(x - hi), in the GEMM's pre-split layout: each 8 consecutive
// elements as their 8 hi halves followed by their 8 lo halves (4 bytes per element, as in fp32).
__device__ __forceinline__ float presplit_scale(const SolveBuffers &b) {
    float asc = 1.0f;
    if (b.mix_bound) {
        const float mx = __uint_as_float(*b.mix_bound);
        if (mx > 0.0f) {
            const float dyn = exp2f(floorf(log2f(b.mix_headroom / mx)));
            if (dyn < asc) asc = dyn;
        }
    }
    return asc;
}

template <int VEC>
__device__ __forceinline__ void store_presplit(float *row, int e0, const float (&v)[VEC], float asc) {
    static_assert(8 % VEC == 0, "a run stays inside one group of 8");
    _Float16 hi[VEC], lo[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
        const float x = v[q] * asc;
        hi[q] = (_Float16)x;
        lo[q] = (_Float16)(x - (float)hi[q]);
    }
    _Float16 *hp = reinterpret_cast<_Float16 *>(row) + (e0 >> 3) * 16 + (e0 & 7);
    if constexpr (VEC == 4) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<h4 *>(hp) = h4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<h4 *>(hp + 8) = h4{lo[0], lo[1], lo[2], lo[3]};
    } else if constexpr (VEC == 2) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<h2 *>(hp) = h2{hi[0], hi[1]};
        *reinterpret_cast<h2 *>(hp + 8) = h2{lo[0], lo[1]};
    } else {
        hp[0] = hi[0];
        hp[8] = lo[0];
    }
}

// store_presplit for VEC = 4 when the lanes of a pair (2k, 2k + 1) hold the two halves of one
// group of 8 (elements e0 = 8m and 8m + 4): the pair swaps halves so that the even lane stores the
// group's 16 hi bytes and the odd lane its 16 lo bytes, one 16-byte store per lane
__device__ __forceinline__ void store_presplit_pair(float *row, int e0, const float (&v)[4], float asc, int lane) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 hi, lo;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float x = v[q] * asc;
        hi[q] = (_Float16)x;
        lo[q] = (_Float16)(x - (float)hi[q]);
    }
    const bool odd = (lane & 1) != 0;
    const uint2 mine = __builtin_bit_cast(uint2, odd ? hi : lo);
    const uint2 got = make_uint2((unsigned)__shfl_xor((int)mine.x, 1, 64), (unsigned)__shfl_xor((int)mine.y, 1, 64));
    const uint2 keep = __builtin_bit_cast(uint2, odd ? lo : hi);
    const uint4 out = odd ? make_uint4(got.x, got.y, keep.x, keep.y) : make_uint4(keep.x, keep.y, got.x, got.y);
    *reinterpret_cast<uint4 *>(reinterpret_cast<_Float16 *>(row) + (e0 >> 3) * 16 + (odd ? 8 : 0)) = out;
}

template <int H, int QA, int VEC>
__global__ __launch_bounds__(256) void k_attn(Dims D, SolveBuffers b, int cur, int k) {
    static_assert(QA * H <= 64, "the score butterfly leaves one score per lane: at most 64 per wave");
    constexpr int NG = H / QA;
    const int gw = blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = b.cnt[cur];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        // the update kernel of this iteration appends survivors to the other list
        b.cnt[cur ^ 1] = 0;
        b.cnt_hist[k] += n;  // summed over the positions of a memory-coupled forward
    }
    const int i = gw / NG, g = gw - (gw / NG) * NG;
    if (i >= n) return;
    const int d = D.d;
    const long rowstride = 3L * d;
    // With one wave per token (QA == H) the Q|K|V rows are read once: non-temporal loads keep
    // them from displacing cached data.  With several, the waves of a token share K and V.
    constexpr bool NT = QA == H;
    const float *base = b.qkv + (long)i * H * rowstride;

    float part[QA][H];
#pragma unroll
    for (int a = 0; a < QA; ++a)
#pragma unroll
        for (int c = 0; c < H; ++c) part[a][c] = 0.0f;

    for (int off = lane * VEC; off < d; off += 64 * VEC) {
        float q[QA][VEC];
#pragma unroll
        for (int a = 0; a < QA; ++a)
#pragma unroll
            for (int v = 0; v < VEC; ++v) q[a][v] = qkv_load<NT>(base + (long)(g * QA + a) * rowstride + off + v);
#pragma unroll
        for (int c = 0; c < H; ++c) {
            float kk[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) kk[v] = qkv_load<NT>(base + (long)c * rowstride + d + off + v);
#pragma unroll
            for (int a = 0; a < QA; ++a)
#pragma unroll
                for (int v = 0; v < VEC; ++v) part[a][c] += q[a][v] * kk[v];
        }
    }
    const float scale = 1.0f / sqrtf((float)d);
    constexpr int P = QA * H;
    float w[P];  // the attention weights, index a * H + c, the same in every lane
    if constexpr (P >= 16) {
        // Wave totals of the P = QA*H partial dot products with wave_sum's offsets (32, 16, ..., 1),
        // so that every total is bit-identical to wave_sum's.  Offsets >= P add all P values; below
        // P the lanes also split the indices still held (a transposing butterfly): at offset `off`
        // the lanes with that bit set keep the upper half of the range, the others the lower half,
        // and each adds its partner's partial for the indices it keeps.  Lane L ends with the total
        // of index L % P = a * H + c: 2P - 1 shuffles instead of 6P.
        float t[P];
#pragma unroll
        for (int a = 0; a < QA; ++a)
#pragma unroll
            for (int c = 0; c < H; ++c) t[a * H + c] = part[a][c];
#pragma unroll
        for (int off = 32; off >= P; off >>= 1)
#pragma unroll
            for (int j = 0; j < P; ++j) t[j] += __shfl_xor(t[j], off, 64);
#pragma unroll
        for (int off = (P < 64 ? P : 64) / 2; off > 0; off >>= 1) {
            const bool up = (lane & off) != 0;
#pragma unroll
            for (int j = 0; j < off; ++j) {
                const float send = up ? t[j] : t[j + off];
                const float keep = up ? t[j + off] : t[j];
                t[j] = keep + __shfl_xor(send, off, 64);
            }
        }
        float sc = t[0] * scale;
        if (D.flags & ADN_F_SCORE_CLAMP4) sc = fminf(fmaxf(sc, -4.0f), 4.0f);
        // softmax over the key slots of this lane's query (lanes gb .. gb + H - 1), max and sum
        // taken in key order as in the sequential form
        const int gb = lane & ~(H - 1);
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < H; ++c) mx = fmaxf(mx, __shfl(sc, gb + c, 64));
        const float ex = expf(sc - mx);
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < H; ++c) sum += __shfl(ex, gb + c, 64);
        const float w_own = ex / sum;
        // every weight to every lane as a wave-uniform value (lane i holds index i)
#pragma unroll
        for (int q = 0; q < P; ++q) w[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_own), q));
    } else {
        // few scores: one wave_sum each and the softmax in every lane (the same totals)
#pragma unroll
        for (int a = 0; a < QA; ++a) {
            float mx = -INFINITY;
            float e[H];
#pragma unroll
            for (int c = 0; c < H; ++c) {
                float sc = wave_sum(part[a][c]) * scale;
                if (D.flags & ADN_F_SCORE_CLAMP4) sc = fminf(fmaxf(sc, -4.0f), 4.0f);
                e[c] = sc;
                mx = fmaxf(mx, sc);
            }
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < H; ++c) {
                e[c] = expf(e[c] - mx);
                sum += e[c];
            }
#pragma unroll
            for (int c = 0; c < H; ++c) w[a * H + c] = e[c] / sum;
        }
    }

    float *mixbase = b.mix + (long)i * H * d;
    const float asc = b.mix_pre ? presplit_scale(b) : 1.0f;
    for (int off = lane * VEC; off < d; off += 64 * VEC) {
        float acc[QA][VEC];
#pragma unroll
        for (int a = 0; a < QA; ++a)
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[a][v] = 0.0f;
#pragma unroll
        for (int c = 0; c < H; ++c) {
            float vv[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) vv[v] = qkv_load<NT>(base + (long)c * rowstride + 2 * d + off + v);
#pragma unroll
            for (int a = 0; a < QA; ++a)
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[a][v] = acc[a][v] + vv[v] * w[a * H + c];
        }
        if (b.mix_pre) {
#pragma unroll
            for (int a = 0; a < QA; ++a) {
                if constexpr (VEC == 4)  // lane pairs hold whole groups of 8 (off = 4 lane + 256 j)
                    store_presplit_pair(mixbase + (long)(g * QA + a) * d, off, acc[a], asc, lane);
                else
                    store_presplit<VEC>(mixbase + (long)(g * QA + a) * d, off, acc[a], asc);
            }
        } else {
#pragma unroll
            for (int a = 0; a < QA; ++a)
#pragma unroll
                for (int v = 0; v < VEC; ++v) mixbase[(long)(g * QA + a) * d + off + v] = acc[a][v];
        }
    }
}

// The same attention for any slot count H <= 16 (read at run time): one wave per (token, query
// slot), the scores summed and the softmax formed as in k_attn's few-score path (the same
// per-lane partial sums, one wave_sum per score, max and sum in key order).
template <int VEC>
__global__ __launch_bounds__(256) void k_attn_rt(Dims D, SolveBuffers b, int cur, int k) {
    constexpr int HM = 16;
    const int H = D.H;
    const int gw = blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = b.cnt[cur];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        b.cnt[cur ^ 1] = 0;
        b.cnt_hist[k] += n;
    }
    const int i = gw / H, a = gw - (gw / H) * H;
    if (i >= n) return;
    const int d = D.d;
    const long rowstride = 3L * d;
    const float *base = b.qkv + (long)i * H * rowstride;
    float part[HM];
#pragma unroll
    for (int c = 0; c < HM; ++c) part[c] = 0.0f;
    for (int off = lane * VEC; off < d; off += 64 * VEC) {
        float q[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) q[v] = base[(long)a * rowstride + off + v];
#pragma unroll
        for (int c = 0; c < HM; ++c) {
            if (c < H) {
#pragma unroll
                for (int v = 0; v < VEC; ++v) part[c] += q[v] * base[(long)c * rowstride + d + off + v];
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)d);
    float e[HM];
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < HM; ++c) {
        if (c < H) {
            float sc = wave_sum(part[c]) * scale;
            if (D.flags & ADN_F_SCORE_CLAMP4) sc = fminf(fmaxf(sc, -4.0f), 4.0f);
            e[c] = sc;
            mx = fmaxf(mx, sc);
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < HM; ++c) {
        if (c < H) {
            e[c] = expf(e[c] - mx);
            sum += e[c];
        }
    }
#pragma unroll
    for (int c = 0; c < HM; ++c)
        if (c < H) e[c] = e[c] / sum;
    float *mixrow = b.mix + ((long)i * H + a) * d;
    const float asc = b.mix_pre ? presplit_scale(b) : 1.0f;
    for (int off = lane * VEC; off < d; off += 64 * VEC) {
        float acc[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
#pragma unroll
        for (int c = 0; c < HM; ++c) {
            if (c < H) {
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[v] = acc[v] + base[(long)c * rowstride + 2 * d + off + v] * e[c];
            }
        }
        if (b.mix_pre) {
            store_presplit<VEC>(mixrow, off, acc, asc);
        } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) mixrow[off + v] = acc[v];
        }
    }
}

// Token residual modes: max-abs over [H][d] (default), L2 over [H][d] (ADN_F_RESID_L2), or the
// largest per-slot relative RMS change (ADN_F_RESID_RELRMS).  Per slot, `acc` is the max |dh|
// (mode 0) or the sum of dh^2 (modes 1, 2) after the wave reduction; `rms` the slot's RMSNorm
// denominator.
// A non-finite difference (a state that turned NaN or inf) counts as an infinite residual, so
// such a token never passes the exit test and runs to the iteration cap unconverged (the
// reference guards its state the same way, finite_or in deq_slot_attn_unified_clean.wgsl:99-108;
// fmaxf alone would drop a NaN and report the token converged).
__device__ __forceinline__ float nan_to_inf(float v) { return v == v ? v : INFINITY; }
__device__ __forceinline__ float slot_resid(int mode, float acc, float rms, int d) {
    return nan_to_inf(mode == 2 ? sqrtf(acc / (float)d + 1e-12f) / fmaxf(rms, 1e-6f) : acc);
}
__device__ __forceinline__ float combine_resid(int mode, float tok, float slot) {
    return mode == 1 ? tok + slot : fmaxf(tok, slot);
}
// Exit test after update k (0-based) of a token with residual r: converged when below eps or
// (with rprev) on the homeostatic plateau of deq_slot_attn_unified_clean.wgsl:1786-1793
// (k+1 >= 4, r <= max(eps, 0.15 * 0.2), |r - r_prev| <= 0.10 max(r_prev, eps)); r_prev is the
// previous update's residual (1 before the first), replaced by r here (`store`: this lane
// writes).  Returns 1 (converged), 2 (unconverged at the iteration cap) or 0 (continue).
__device__ __forceinline__ int token_exit(float r, float eps, int k, int max_iters, float *rprev, bool store) {
    bool conv = r < eps;
    if (rprev) {
        const float rp = *rprev;
        if (k + 1 >= 4 && r <= fmaxf(eps, 0.15f * 0.2f) && fabsf(r - rp) / fmaxf(rp, eps) <= 0.10f) conv = true;
        if (store) *rprev = r;
    }
    return conv ? 1 : (k + 1 >= max_iters ? 2 : 0);
}

// ---------------------------------------------------------------------------------------
// Damped update and exit test of one active token (one wave; FPMR:1386-1393): per slot
// c = o + signal + anchor, f = g*c/sqrt(mean(c^2)+1e-6), h' = f*beta + h*(1-beta); the token's
// residual (max-abs, or L2 over [H*d]) decides the exit: a done token records k+1 applied
// updates, a continuing one is appended to the next active list (one atomic per workgroup).
// The list order is not deterministic, which is harmless: every token's arithmetic is
// independent of its position.
// ---------------------------------------------------------------------------------------
// With the slot count HT known at compile time (and d <= 1024) the slots are walked with the
// next slot's rows loaded into a second register set before this slot's h is stored: a load
// issued after stores is waited for behind them (the vector-memory counter retires in issue
// order), and a fully unrolled walk lets the compiler count the loads exactly.  HT = 0: the
// slot count is read at run time (one slot at a time).  HIST: the memory-coupled history term.
template <int E, int HT, bool HIST, bool PART>
__global__ __launch_bounds__(256) void k_update(Dims D, SolveBuffers b, int cur, int k, int max_iters,
                                                float eps, const float *anchor, const float *norm_scale,
                                                float beta) {
    // no contracted multiply-adds: every kernel that forms the update (this one, k_update_tok and
    // the Q|K|V product that applies it at a few rows) rounds each operation alike
#pragma clang fp contract(off)
    __shared__ int keep_s[WAVES_PER_BLOCK];
    __shared__ int tok_s[WAVES_PER_BLOCK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = b.cnt[cur];
    if (blockIdx.x * WAVES_PER_BLOCK >= n) return;
    const int i = blockIdx.x * WAVES_PER_BLOCK + wave;
    const int H = HT > 0 ? HT : D.H;
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const bool excl = (D.flags & ADN_F_RMS_EXCL_ANCHOR) != 0;
    const int rmode = (D.flags & ADN_F_RESID_L2) ? 1 : (D.flags & ADN_F_RESID_RELRMS) ? 2 : 0;
    bool keep = false;
    int t = -1;
    if (i < n) {
        t = b.act[cur][i];
        float g[E];
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = (!PART || e < er) ? norm_scale[lane + 64 * e] : 0.0f;
        const float omb = 1.0f - beta;
        float rtok = 0.0f;
        const float *hc_tok = HIST ? b.mem_hist + (long)(t / b.mem_T) * H * d : nullptr;
        struct SlotIn {
            float o[E], sg[E], an[E], h[E], hc[HIST ? E : 1];
        };
        // combined = attn + input signal + history, then + slot anchor (FPMR:1386-1389); o and
        // the signal are loaded non-temporally (o is read once; an iteration's working set is
        // larger than the caches, so keeping the signal cached only displaces h, which the next
        // Q|K|V product reads)
        auto load = [&](int s, SlotIn &q) {
            const float *o = b.o + ((long)i * H + s) * d;
            const float *sg = b.signal + ((long)t * H + s) * d;
            const float *an = anchor + (long)s * d;
            const float *h = b.h + ((long)t * H + s) * d;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int idx = lane + 64 * e;
                const bool on = !PART || e < er;  // zeros outside the row add nothing below
                q.o[e] = on ? __builtin_nontemporal_load(o + idx) : 0.0f;
                q.sg[e] = on ? __builtin_nontemporal_load(sg + idx) : 0.0f;
                q.an[e] = on ? an[idx] : 0.0f;
                q.h[e] = on ? h[idx] : 0.0f;
                if constexpr (HIST) q.hc[e] = on ? hc_tok[(long)s * d + idx] : 0.0f;
            }
        };
        auto step = [&](int s, const SlotIn &q) {
            float *h = (b.h_out ? b.h_out : b.h) + ((long)t * H + s) * d;
            float *h2 = b.h_both ? b.h + ((long)t * H + s) * d : nullptr;
            float cval[E];
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float as_ = (q.o[e] + q.sg[e]) + (HIST ? q.hc[e] : 0.0f);
                const float c = as_ + q.an[e];
                cval[e] = c;
                ss += excl ? as_ * as_ : c * c;
            }
            ss = wave_sum(ss);
            const float rms = sqrtf(ss / (float)d + 1e-6f);
            float r = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float f = g[e] * cval[e] / rms;
                const float hn = f * beta + q.h[e] * omb;
                if (!PART || e < er) {
                    h[lane + 64 * e] = hn;
                    if (h2) h2[lane + 64 * e] = hn;
                }
                const float df = hn - q.h[e];
                r = rmode ? r + df * df : fmaxf(r, nan_to_inf(fabsf(df)));
            }
            r = rmode ? wave_sum(r) : wave_max(r);
            rtok = combine_resid(rmode, rtok, slot_resid(rmode, r, rms, d));
        };
        if constexpr (HT > 0) {
            static_assert(E <= 16, "two register sets of slot rows");
            SlotIn q[2];
            load(0, q[0]);
#pragma unroll
            for (int s = 0; s < HT; ++s) {
                if (s + 1 < HT) load(s + 1, q[(s + 1) & 1]);
                step(s, q[s & 1]);
            }
        } else {
            for (int s = 0; s < H; ++s) {
                SlotIn q;
                load(s, q);
                step(s, q);
            }
        }
        if (rmode == 1) rtok = nan_to_inf(sqrtf(rtok));
        const int ex = token_exit(rtok, eps, k, max_iters, b.rprev ? b.rprev + t : nullptr, lane == 0);
        if (ex && lane == 0) {
            b.iters[t] = k + 1;
            if (b.conv) b.conv[t] = ex == 1;
        }
        keep = !ex || (ex == 2 && b.cap_mix);
    }
    if (lane == 0) {
        keep_s[wave] = keep;
        tok_s[wave] = t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int nk = 0;
        for (int w = 0; w < WAVES_PER_BLOCK; ++w) nk += keep_s[w];
        if (nk) {
            int pos = atomicAdd(&b.cnt[cur ^ 1], nk);
            for (int w = 0; w < WAVES_PER_BLOCK; ++w)
                if (keep_s[w]) b.act[cur ^ 1][pos++] = tok_s[w];
        }
    }
}

// ---------------------------------------------------------------------------------------
// Anderson mixing for the tokens still active after iteration k (forward use of the
// reference's scheme, staged_adjoint_picard_clean.wgsl:1012-1134 with the store-then-mix
// order of gpu_deq.rs:4278-4293): ring slot k % m <- un-mixed iterate g; for k >= 2 and
// n_res = min(k, m-1) >= 2 solve (G + reg I) beta = 1 over the pseudo-residuals
// X_{k-i} - X_{k-i-1}, clamp, normalise and set h = sum_i beta_i X_{k-i}.
// ---------------------------------------------------------------------------------------
__device__ void anderson_coeffs(int n, const float *g, float *beta) {
    if (n == 2) {
        const float reg = fmaxf(1e-8f, 1e-4f * (fabsf(g[0]) + fabsf(g[3])));
        const float g00 = g[0] + reg, g01 = g[1], g10 = g[2], g11 = g[3] + reg;
        const float det = g00 * g11 - g01 * g10;
        const float sdet = det < 0.0f ? fminf(det, -1e-10f) : fmaxf(det, 1e-10f);
        beta[0] = (g11 - g01) / sdet;
        beta[1] = (g00 - g10) / sdet;
    } else if (n == 3) {
        const float reg = fmaxf(1e-8f, 1e-4f * (fabsf(g[0]) + fabsf(g[4]) + fabsf(g[8])));
        const float g00 = g[0] + reg, g01 = g[1], g02 = g[2];
        const float g10 = g[3], g11 = g[4] + reg, g12 = g[5];
        const float g20 = g[6], g21 = g[7], g22 = g[8] + reg;
        const float det = g00 * (g11 * g22 - g12 * g21) - g01 * (g10 * g22 - g12 * g20) +
                          g02 * (g10 * g21 - g11 * g20);
        const float sdet = det < 0.0f ? fminf(det, -1e-8f) : fmaxf(det, 1e-8f);
        beta[0] = (1.0f * (g11 * g22 - g12 * g21) - g01 * (g22 - g12) + g02 * (g21 - g11)) / sdet;
        beta[1] = (g00 * (g22 - g12) - 1.0f * (g10 * g22 - g12 * g20) + g02 * (g10 - g20)) / sdet;
        beta[2] = (g00 * (g11 - g21) - g01 * (g10 - g20) + 1.0f * (g10 * g21 - g11 * g20)) / sdet;
    } else {
        float a[16];
        float tr = 0.0f;
        for (int q = 0; q < 4; ++q) tr += fabsf(g[q * 4 + q]);
        const float reg = fmaxf(1e-8f, 1e-4f * tr);
        for (int q = 0; q < 16; ++q) a[q] = g[q];
        for (int q = 0; q < 4; ++q) a[q * 4 + q] += reg;
        auto m3 = [](const float *m, int r0, int r1, int r2, int c0, int c1, int c2) {
            return m[r0 * 4 + c0] * (m[r1 * 4 + c1] * m[r2 * 4 + c2] - m[r1 * 4 + c2] * m[r2 * 4 + c1]) -
                   m[r0 * 4 + c1] * (m[r1 * 4 + c0] * m[r2 * 4 + c2] - m[r1 * 4 + c2] * m[r2 * 4 + c0]) +
                   m[r0 * 4 + c2] * (m[r1 * 4 + c0] * m[r2 * 4 + c1] - m[r1 * 4 + c1] * m[r2 * 4 + c0]);
        };
        auto det4 = [&](const float *m) {
            return m[0] * m3(m, 1, 2, 3, 1, 2, 3) - m[1] * m3(m, 1, 2, 3, 0, 2, 3) +
                   m[2] * m3(m, 1, 2, 3, 0, 1, 3) - m[3] * m3(m, 1, 2, 3, 0, 1, 2);
        };
        const float det = det4(a);
        const float sdet = det < 0.0f ? fminf(det, -1e-8f) : fmaxf(det, 1e-8f);
        for (int col = 0; col < 4; ++col) {
            float bm[16];
            for (int q = 0; q < 16; ++q) bm[q] = a[q];
            for (int rr = 0; rr < 4; ++rr) bm[rr * 4 + col] = 1.0f;
            beta[col] = det4(bm) / sdet;
        }
    }
    float s = 0.0f;
    for (int q = 0; q < n; ++q) {
        beta[q] = fminf(fmaxf(beta[q], -2.0f), 3.0f);
        s += beta[q];
    }
    if (fabsf(s) < 1e-6f) {
        for (int q = 0; q < n; ++q) beta[q] = 0.0f;
        beta[0] = 1.0f;
    } else {
        for (int q = 0; q < n; ++q) beta[q] = beta[q] / s;
    }
}

// Update for few tokens (one position of every sequence, a decode step): one block per token
// and one wave per slot, so that the slots' row updates run side by side instead of one after
// another in a single wave.  Same arithmetic as k_update (the token residual is combined over
// the slots in slot order).
template <int E, bool PART>
__global__ __launch_bounds__(1024) void k_update_tok(Dims D, SolveBuffers b, int cur, int k, int max_iters,
                                                     float eps, const float *anchor, const float *norm_scale,
                                                     float beta) {
#pragma clang fp contract(off)  // as in k_update
    __shared__ float rs[16];
    extern __shared__ float hl[];  // [H][d] the new rows, with b.pool
    const int i = blockIdx.x;
    if (i >= b.cnt[cur]) return;
    const int s = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = D.H;
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const bool excl = (D.flags & ADN_F_RMS_EXCL_ANCHOR) != 0;
    const int rmode = (D.flags & ADN_F_RESID_L2) ? 1 : (D.flags & ADN_F_RESID_RELRMS) ? 2 : 0;
    const int t = b.act[cur][i];
    const float *o = b.o + ((long)i * H + s) * d;
    const float *sg = b.signal + ((long)t * H + s) * d;
    const float *an = anchor + (long)s * d;
    const float *hc = b.mem_hist ? b.mem_hist + ((long)(t / b.mem_T) * H + s) * d : nullptr;
    float *h = b.h + ((long)t * H + s) * d;
    float *hw = (b.h_out ? b.h_out : b.h) + ((long)t * H + s) * d;
    // every load (the norm scale too) before the first store of h: a load issued after stores
    // is waited for behind them (the vector-memory counter retires in issue order)
    float cval[E], hold[E], gs[E];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        const float as_ = on ? (o[idx] + sg[idx]) + (hc ? hc[idx] : 0.0f) : 0.0f;
        const float c = as_ + (on ? an[idx] : 0.0f);
        cval[e] = c;
        hold[e] = on ? h[idx] : 0.0f;
        gs[e] = on ? norm_scale[idx] : 0.0f;
        ss += excl ? as_ * as_ : c * c;
    }
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-6f);
    const float omb = 1.0f - beta;
    float r = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float f = gs[e] * cval[e] / rms;
        const float hn = f * beta + hold[e] * omb;
        if (!PART || e < er) {
            hw[lane + 64 * e] = hn;
            if (b.h_both) h[lane + 64 * e] = hn;
            if (b.pool) hl[s * d + lane + 64 * e] = hn;
        }
        const float df = hn - hold[e];
        r = rmode ? r + df * df : fmaxf(r, nan_to_inf(fabsf(df)));
    }
    r = rmode ? wave_sum(r) : wave_max(r);
    if (lane == 0) rs[s] = slot_resid(rmode, r, rms, d);
    __syncthreads();
    if (threadIdx.x == 0) {
        float rtok = 0.0f;
        for (int q = 0; q < H; ++q) rtok = combine_resid(rmode, rtok, rs[q]);
        if (rmode == 1) rtok = nan_to_inf(sqrtf(rtok));
        const int ex = token_exit(rtok, eps, k, max_iters, b.rprev ? b.rprev + t : nullptr, true);
        if (ex) {
            b.iters[t] = k + 1;
            if (b.conv) b.conv[t] = ex == 1;
        }
        if (!ex || (ex == 2 && b.cap_mix)) {
            const int pos = atomicAdd(&b.cnt[cur ^ 1], 1);
            b.act[cur ^ 1][pos] = t;
        }
    }
    if (b.pool && threadIdx.x < 64) {  // the token's LM-head prologue, the slots summed in order as k_pool_norm does
        float pv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) pv[e] = 0.0f;
        for (int q = 0; q < H; ++q)
#pragma unroll
            for (int e = 0; e < E; ++e) pv[e] = pv[e] + ((!PART || e < er) ? hl[q * d + lane + 64 * e] : 0.0f);
        pool_finish<E>(pv, H, d, er, lane, t, b.pool_g, b.pool_out, b.pool_norm, 0.0f);
    }
}

constexpr int AND_NT = 256;
// at most this many tokens in flight: the few-token kernel shapes (more waves per token)
constexpr int SMALL_ROWS = 512;

// The Anderson mix as one multiply-add chain per element, acc = fma(c_n-1, x_n-1, ... fma(c_0, x_0, 0)):
// the fused update recomputes the previous iteration's mix with it, so both must round alike.
// Terms x[OFF + ri][e], ri < n <= NX - OFF.
template <int OFF, int NX, int E>
__device__ __forceinline__ float mix_chain(int n, const float *c, const float (&x)[NX][E], int e) {
    float acc = 0.0f;
#pragma unroll
    for (int ri = 0; ri + OFF < NX; ++ri)
        if (ri < n) acc = fmaf(c[ri], x[OFF + ri][e], acc);
    return acc;
}

// Thread 0 of a fused update-and-mix block: the token residual from the slot residuals rs (combined
// in slot order), the exit test, and for a token that is mixed (continuing, or stopped at the cap
// unconverged) the Gram matrix from the waves' partials red (summed in wave order), the
// coefficients into cf and mix_coef, and the token's place in the next list.  Returns whether the
// token is mixed.
template <int NRES>
__device__ bool update_mix_decide(const SolveBuffers &b, int cur, int k, int max_iters, float eps, int t, int H,
                                  int rmode, const float *rs, const float (*red)[NRES * (NRES + 1) / 2], float *cf) {
    float rtok = 0.0f;
    for (int q = 0; q < H; ++q) rtok = combine_resid(rmode, rtok, rs[q]);
    if (rmode == 1) rtok = nan_to_inf(sqrtf(rtok));
    const int ex = token_exit(rtok, eps, k, max_iters, b.rprev ? b.rprev + t : nullptr, true);
    if (ex) {
        b.iters[t] = k + 1;
        if (b.conv) b.conv[t] = ex == 1;
    }
    const bool mixit = !ex || (ex == 2 && b.cap_mix);
    if (mixit) {
        float g[16];
        int q = 0;
        for (int ri = 0; ri < NRES; ++ri)
            for (int rj = ri; rj < NRES; ++rj) {
                float v = 0.0f;
                for (int w = 0; w < H; ++w) v += red[w][q];
                g[ri * NRES + rj] = v;
                g[rj * NRES + ri] = v;
                ++q;
            }
        float bt[4];
        anderson_coeffs(NRES, g, bt);
        for (int q2 = 0; q2 < NRES; ++q2) {
            cf[q2] = bt[q2];
            b.mix_coef[(long)t * 4 + q2] = bt[q2];
        }
        const int pos = atomicAdd(&b.cnt[cur ^ 1], 1);
        b.act[cur ^ 1][pos] = t;
    }
    return mixit;
}

// Damped update and Anderson mix in one pass, one block per active token and one wave per slot
// (the update of FPMR:1386-1393, then the mixing of staged_adjoint_picard_clean.wgsl:1012-1134 in
// the store-then-mix order of gpu_deq.rs:4278-4293), at iterations k >= 2 with NRES = min(k, m-1)
// >= 2 residuals.  The iterate is formed as k_update_tok forms it (the same elements per lane,
// wave sums and slot order) from the previous iterate, which is not read from h: a token active
// at iteration k continued at k - 1, so its h is the mix formed then from ring slots X(k-1) ..
// X(k-pn) that this kernel loads anyway (pn = the previous mix's term count, its coefficients
// kept per token in mix_coef; pn = 0: no mix at k - 1, h = X(k-1)), and mix_chain recomputes it
// bit for bit.  The iterate goes to ring slot k % m; h gets the mix, or the iterate for a token
// that converged at this step (a token stopped at the cap unconverged is mixed).  The Gram sums:
// per lane over its elements, the wave sums, then the waves in slot order.  Per token 2 + NRES
// state vectors are read and 2 written, where the update and a mixing pass read 4 + NRES and
// write 2.
template <int E, bool PART, int NRES, bool HIST>
__global__ __launch_bounds__(1024) void k_update_mix(Dims D, SolveBuffers b, int cur, int k, int m, int ntok, int pn,
                                                     int max_iters, float eps, const float *anchor,
                                                     const float *norm_scale, float beta) {
#pragma clang fp contract(off)  // the update as in k_update; the mix by explicit multiply-adds
    constexpr int NPK = NRES * (NRES + 1) / 2;
    __shared__ float rs[16];
    __shared__ float red[16][NPK];
    __shared__ float cf_s[4];
    __shared__ int mix_s;
    const int i = blockIdx.x;
    if (i >= b.cnt[cur]) return;
    const int s = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = D.H;
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const bool excl = (D.flags & ADN_F_RMS_EXCL_ANCHOR) != 0;
    const int rmode = (D.flags & ADN_F_RESID_L2) ? 1 : (D.flags & ADN_F_RESID_RELRMS) ? 2 : 0;
    const int t = b.act[cur][i];
    const long hd = (long)H * d, row = (long)s * d;
    auto X = [&](int j) { return b.hist + ((long)(j % m) * ntok + t) * hd + row; };
    const float *o = b.o + ((long)i * H + s) * d;
    const float *sg = b.signal + (long)t * hd + row;
    const float *an = anchor + row;
    const float *hc = HIST ? b.mem_hist + ((long)(t / b.mem_T) * H + s) * d : nullptr;
    // x[0]: this iteration's iterate, x[ri]: X(k - ri); every load before the first store
    float x[NRES + 1][E], cval[E], gs[E];
    float ss = 0.0f;
#pragma unroll
    for (int ri = 1; ri <= NRES; ++ri) {
        const float *src = X(k + m - ri);
#pragma unroll
        for (int e = 0; e < E; ++e) x[ri][e] = (!PART || e < er) ? src[lane + 64 * e] : 0.0f;
    }
    float cp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) cp[q] = q < pn ? b.mix_coef[(long)t * 4 + q] : 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = lane + 64 * e;
        const bool on = !PART || e < er;  // zeros outside the row add nothing below
        const float as_ =
            on ? (__builtin_nontemporal_load(o + idx) + __builtin_nontemporal_load(sg + idx)) + (HIST ? hc[idx] : 0.0f)
               : 0.0f;
        const float c = as_ + (on ? an[idx] : 0.0f);
        cval[e] = c;
        gs[e] = on ? norm_scale[idx] : 0.0f;
        ss += excl ? as_ * as_ : c * c;
    }
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-6f);
    const float omb = 1.0f - beta;
    float r = 0.0f;
    float *slot = X(k);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        // the previous iterate: X(k-1), or the mix of X(k-1) .. X(k-pn) (x[1 ..] here, x[0 ..] then)
        const float hold = pn ? mix_chain<1>(pn, cp, x, e) : x[1][e];
        const float f = gs[e] * cval[e] / rms;
        const float hn = f * beta + hold * omb;
        x[0][e] = hn;
        if (!PART || e < er) slot[lane + 64 * e] = hn;
        const float df = hn - hold;
        r = rmode ? r + df * df : fmaxf(r, nan_to_inf(fabsf(df)));
    }
    r = rmode ? wave_sum(r) : wave_max(r);
    // the Gram partials of the pseudo-residuals X(k-ri) - X(k-ri-1), the NPK wave sums interleaved
    float gp[NPK];
#pragma unroll
    for (int q = 0; q < NPK; ++q) gp[q] = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        float dl[NRES];
#pragma unroll
        for (int ri = 0; ri < NRES; ++ri) dl[ri] = x[ri][e] - x[ri + 1][e];
        int p = 0;
#pragma unroll
        for (int ri = 0; ri < NRES; ++ri)
#pragma unroll
            for (int rj = ri; rj < NRES; ++rj) gp[p++] += dl[ri] * dl[rj];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float ov[NPK];
#pragma unroll
        for (int q = 0; q < NPK; ++q) ov[q] = __shfl_xor(gp[q], off, 64);
#pragma unroll
        for (int q = 0; q < NPK; ++q) gp[q] += ov[q];
    }
    if (lane == 0) {
        rs[s] = slot_resid(rmode, r, rms, d);
#pragma unroll
        for (int q = 0; q < NPK; ++q) red[s][q] = gp[q];
    }
    __syncthreads();
    if (threadIdx.x == 0) mix_s = update_mix_decide<NRES>(b, cur, k, max_iters, eps, t, H, rmode, rs, red, cf_s);
    __syncthreads();
    float *h = b.h + (long)t * hd + row;
    if (mix_s) {
        float bl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) bl[q] = q < NRES ? cf_s[q] : 0.0f;
        float hmax = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float v = mix_chain<0>(NRES, bl, x, e);
            if (!PART || e < er) {
                h[lane + 64 * e] = v;
                hmax = fmaxf(hmax, fabsf(v) < INFINITY ? fabsf(v) : 0.0f);
            }
        }
        if (b.amax_h) track_absmax(b.amax_h, hmax);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (!PART || e < er) h[lane + 64 * e] = x[0][e];
    }
}

// k_update_mix for rows of 1024 or 2048 floats (E = 16, 32), whose ring values do not fit in
// registers: a lane walks its elements in groups of SUB, two groups per pass of a loop that is not
// unrolled (unrolled, the per-element addresses alone overflow the registers), each group's ring
// values and norm scale loaded into a register set before the previous group's iterate is stored;
// the row's c values and then its iterate are kept in LDS (H * d floats, dynamic).  After the
// coefficient solve the mix reads X(k-1) .. X(k-NRES+1) again (mostly from the caches: the block
// read them a moment before).  Same arithmetic per element as k_update_mix (a lane's Gram partials
// in element order).  Per token 2 + NRES vectors read and 2 written, plus the NRES - 1 re-read;
// the update and the two-pass mixing read 4 + 2 NRES + 1 and write 3.
template <int E, bool PART, int NRES, bool HIST>
__global__ __launch_bounds__(1024) void k_update_mix_wide(Dims D, SolveBuffers b, int cur, int k, int m, int ntok,
                                                          int pn, int max_iters, float eps, const float *anchor,
                                                          const float *norm_scale, float beta) {
#pragma clang fp contract(off)  // as in k_update_mix
    constexpr int SUB = 4, NG = E / SUB;
    static_assert(NG % 2 == 0, "pairs of element groups");
    constexpr int NPK = NRES * (NRES + 1) / 2;
    __shared__ float rs[16];
    __shared__ float red[16][NPK];
    __shared__ float cf_s[4];
    __shared__ int mix_s;
    extern __shared__ float cl[];  // [H][E][64]: a lane's c values, then its iterate
    const int i = blockIdx.x;
    if (i >= b.cnt[cur]) return;
    const int s = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = D.H;
    const int d = PART ? D.d : 64 * E, er = PART ? D.d / 64 : E;  // chunks e >= er are outside the row
    const bool excl = (D.flags & ADN_F_RMS_EXCL_ANCHOR) != 0;
    const int rmode = (D.flags & ADN_F_RESID_L2) ? 1 : (D.flags & ADN_F_RESID_RELRMS) ? 2 : 0;
    const int t = b.act[cur][i];
    const long hd = (long)H * d, row = (long)s * d;
    auto X = [&](int j) { return b.hist + ((long)(j % m) * ntok + t) * hd + row; };
    const float *o = b.o + ((long)i * H + s) * d;
    const float *sg = b.signal + (long)t * hd + row;
    const float *an = anchor + row;
    const float *hc = HIST ? b.mem_hist + ((long)(t / b.mem_T) * H + s) * d : nullptr;
    const float *xr[NRES + 1];  // xr[ri] = X(k - ri), ri >= 1
#pragma unroll
    for (int ri = 1; ri <= NRES; ++ri) xr[ri] = X(k + m - ri);
    float *slot = X(k);
    float *h = b.h + (long)t * hd + row;
    float cp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) cp[q] = q < pn ? b.mix_coef[(long)t * 4 + q] : 0.0f;
    float *cv = cl + (long)s * E * 64 + lane;  // element e of this lane at cv[64 e]
    // element ee of a lane is lane + 64 ee; groups past the row (PART) load zeros and store nothing
    auto on = [&](int ee) { return !PART || ee < er; };

    // c = o + signal (+ history) + anchor into LDS, and the sum of squares
    float ss = 0.0f;
    struct In {
        float o[SUB], sg[SUB], an[SUB], hc[HIST ? SUB : 1];
    };
    auto load_in = [&](int j, In &q) {
#pragma unroll
        for (int e = 0; e < SUB; ++e) {
            const int ee = j * SUB + e, idx = lane + 64 * ee;
            q.o[e] = on(ee) ? __builtin_nontemporal_load(o + idx) : 0.0f;
            q.sg[e] = on(ee) ? __builtin_nontemporal_load(sg + idx) : 0.0f;
            q.an[e] = on(ee) ? an[idx] : 0.0f;
            if constexpr (HIST) q.hc[e] = on(ee) ? hc[idx] : 0.0f;
        }
    };
    auto sum_in = [&](int j, const In &q) {
#pragma unroll
        for (int e = 0; e < SUB; ++e) {
            const float as_ = (q.o[e] + q.sg[e]) + (HIST ? q.hc[e] : 0.0f);
            const float c = as_ + q.an[e];
            cv[64 * (j * SUB + e)] = c;
            ss += excl ? as_ * as_ : c * c;
        }
    };
    {
        In in0, in1;
        load_in(0, in0);
#pragma unroll 1
        for (int j = 0; j < NG; j += 2) {
            load_in(j + 1, in1);
            sum_in(j, in0);
            load_in(j + 2 < NG ? j + 2 : NG - 1, in0);  // clamped: the last pass loads a group again
            sum_in(j + 1, in1);
        }
    }
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)d + 1e-6f);
    const float omb = 1.0f - beta;

    // the iterate into the ring slot and LDS, the residual and the Gram partials
    struct Grp {
        float x[NRES + 1][SUB];  // x[ri]: X(k - ri) for ri >= 1 (x[0] unused)
        float g[SUB];
    };
    auto load_grp = [&](int j, Grp &q) {
#pragma unroll
        for (int ri = 1; ri <= NRES; ++ri)
#pragma unroll
            for (int e = 0; e < SUB; ++e) {
                const int ee = j * SUB + e;
                q.x[ri][e] = on(ee) ? xr[ri][lane + 64 * ee] : 0.0f;
            }
#pragma unroll
        for (int e = 0; e < SUB; ++e) {
            const int ee = j * SUB + e;
            q.g[e] = on(ee) ? norm_scale[lane + 64 * ee] : 0.0f;
        }
    };
    float r = 0.0f;
    float gp[NPK];
#pragma unroll
    for (int q = 0; q < NPK; ++q) gp[q] = 0.0f;
    auto upd = [&](int j, const Grp &q) {
#pragma unroll
        for (int e = 0; e < SUB; ++e) {
            const int ee = j * SUB + e;
            const float hold = pn ? mix_chain<1>(pn, cp, q.x, e) : q.x[1][e];
            const float f = q.g[e] * cv[64 * ee] / rms;
            const float hn = f * beta + hold * omb;
            cv[64 * ee] = hn;
            if (on(ee)) slot[lane + 64 * ee] = hn;
            const float df = hn - hold;
            r = rmode ? r + df * df : fmaxf(r, nan_to_inf(fabsf(df)));
            float dl[NRES];
            dl[0] = hn - q.x[1][e];
#pragma unroll
            for (int ri = 1; ri < NRES; ++ri) dl[ri] = q.x[ri][e] - q.x[ri + 1][e];
            int p = 0;
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri)
#pragma unroll
                for (int rj = ri; rj < NRES; ++rj) gp[p++] += dl[ri] * dl[rj];
        }
    };
    {
        Grp g0, g1;
        load_grp(0, g0);
#pragma unroll 1
        for (int j = 0; j < NG; j += 2) {
            load_grp(j + 1, g1);
            upd(j, g0);
            load_grp(j + 2 < NG ? j + 2 : NG - 1, g0);
            upd(j + 1, g1);
        }
    }
    r = rmode ? wave_sum(r) : wave_max(r);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float ov[NPK];
#pragma unroll
        for (int q = 0; q < NPK; ++q) ov[q] = __shfl_xor(gp[q], off, 64);
#pragma unroll
        for (int q = 0; q < NPK; ++q) gp[q] += ov[q];
    }
    if (lane == 0) {
        rs[s] = slot_resid(rmode, r, rms, d);
#pragma unroll
        for (int q = 0; q < NPK; ++q) red[s][q] = gp[q];
    }
    __syncthreads();
    if (threadIdx.x == 0) mix_s = update_mix_decide<NRES>(b, cur, k, max_iters, eps, t, H, rmode, rs, red, cf_s);
    __syncthreads();
    if (mix_s) {
        float bl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) bl[q] = q < NRES ? cf_s[q] : 0.0f;
        float hmax = 0.0f;
        // the mix's terms: the iterate from LDS and X(k-1) .. X(k-NRES+1) read again
        auto load_mix = [&](int j, float (&xq)[NRES][SUB]) {
#pragma unroll
            for (int ri = 1; ri < NRES; ++ri)
#pragma unroll
                for (int e = 0; e < SUB; ++e) {
                    const int ee = j * SUB + e;
                    xq[ri][e] = on(ee) ? xr[ri][lane + 64 * ee] : 0.0f;
                }
        };
        auto mix = [&](int j, float (&xq)[NRES][SUB]) {
#pragma unroll
            for (int e = 0; e < SUB; ++e) xq[0][e] = cv[64 * (j * SUB + e)];
#pragma unroll
            for (int e = 0; e < SUB; ++e) {
                const int ee = j * SUB + e;
                const float v = mix_chain<0>(NRES, bl, xq, e);
                if (on(ee)) {
                    h[lane + 64 * ee] = v;
                    hmax = fmaxf(hmax, fabsf(v) < INFINITY ? fabsf(v) : 0.0f);
                }
            }
        };
        float x0[NRES][SUB], x1[NRES][SUB];
        load_mix(0, x0);
#pragma unroll 1
        for (int j = 0; j < NG; j += 2) {
            load_mix(j + 1, x1);
            mix(j, x0);
            load_mix(j + 2 < NG ? j + 2 : NG - 1, x0);
            mix(j + 1, x1);
        }
        if (b.amax_h) track_absmax(b.amax_h, hmax);
    } else {
#pragma unroll 1
        for (int e = 0; e < E; ++e)
            if (on(e)) h[lane + 64 * e] = cv[64 * e];
    }
}

// NRES = 0: store only; NRES in 2..4: store, Gram, solve, mix.
template <int NRES>
__global__ __launch_bounds__(AND_NT) void k_anderson(Dims D, SolveBuffers b, int nxt, int ntok, int k,
                                                     int m) {
    __shared__ float red[AND_NT / 64][10];
    __shared__ float beta_s[4];
    const int i = blockIdx.x;
    if (i >= b.cnt[nxt]) return;
    const int t = b.act[nxt][i];
    const long hd = (long)D.H * D.d;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *h = b.h + (long)t * hd;
    auto X = [&](int j) { return b.hist + ((long)(j % m) * ntok + t) * hd; };
    float *slot = X(k);
    // Copies and the final mix go AB elements per thread at a time, loads before stores: a load
    // issued after stores is waited for behind them (the vector-memory counter retires in issue
    // order).
    constexpr int AB = 8;
    for (long e0 = tid; e0 < hd; e0 += AB * AND_NT) {
        float v[AB];
#pragma unroll
        for (int q = 0; q < AB; ++q) {
            const long e = e0 + (long)q * AND_NT;
            v[q] = e < hd ? h[e] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < AB; ++q) {
            const long e = e0 + (long)q * AND_NT;
            if (e < hd) slot[e] = v[q];
        }
    }
    if constexpr (NRES >= 2) {
        constexpr int NPK = NRES * (NRES + 1) / 2;
        float gp[NPK];
#pragma unroll
        for (int q = 0; q < NPK; ++q) gp[q] = 0.0f;
        for (long e = tid; e < hd; e += AND_NT) {
            float dl[NRES];
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri) dl[ri] = X(k + m - ri)[e] - X(k + m - ri - 1)[e];
            int q = 0;
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri)
#pragma unroll
                for (int rj = ri; rj < NRES; ++rj) gp[q++] += dl[ri] * dl[rj];
        }
#pragma unroll
        for (int q = 0; q < NPK; ++q) {
            const float v = wave_sum(gp[q]);
            if (lane == 0) red[wave][q] = v;
        }
        __syncthreads();
        if (tid == 0) {
            float g[16];
            int q = 0;
            for (int ri = 0; ri < NRES; ++ri)
                for (int rj = ri; rj < NRES; ++rj) {
                    float v = 0.0f;
                    for (int w = 0; w < AND_NT / 64; ++w) v += red[w][q];
                    g[ri * NRES + rj] = v;
                    g[rj * NRES + ri] = v;
                    ++q;
                }
            float bt[4];
            anderson_coeffs(NRES, g, bt);
            for (int q2 = 0; q2 < NRES; ++q2) beta_s[q2] = bt[q2];
        }
        __syncthreads();
        float hmax = 0.0f;
        for (long e0 = tid; e0 < hd; e0 += AB * AND_NT) {
            float acc[AB];
#pragma unroll
            for (int q = 0; q < AB; ++q) {
                const long e = e0 + (long)q * AND_NT;
                acc[q] = 0.0f;
                if (e < hd) {
#pragma unroll
                    for (int ri = 0; ri < NRES; ++ri) acc[q] += beta_s[ri] * X(k + m - ri)[e];
                }
            }
#pragma unroll
            for (int q = 0; q < AB; ++q) {
                const long e = e0 + (long)q * AND_NT;
                if (e < hd) {
                    h[e] = acc[q];
                    hmax = fmaxf(hmax, fabsf(acc[q]) < INFINITY ? fabsf(acc[q]) : 0.0f);
                }
            }
        }
        // a mixed iterate can leave the update's bound (the coefficients are normalised by their
        // sum), so the mix raises the bound on |h| itself
        if (b.amax_h) track_absmax(b.amax_h, hmax);
    }
}

// One-pass form of k_anderson (NRES in 2..4) for token states of at most AND_NT * EPT floats: each
// thread holds its elements of the current iterate and of the NRES previous ones in registers, so
// the ring is read once per iteration (NRES + 1 vectors read, the ring slot and h written) instead
// of twice (2 NRES + 2 read); after an update that wrote the slot itself (SLOT), NRES + 1 read and
// h alone written.  Element e = tid + q AND_NT of thread tid, q ascending: the same assignment and
// summation order as k_anderson's Gram and mix, so the results are bit-identical.
// (EXACT: the state is exactly AND_NT * EPT floats, so no element needs a bounds test.)
// SLOT: the update wrote its iterate into ring slot k % m (SolveBuffers::h_out) and list `lst` is
// the update's own list: a token that exited at iteration k (iters = k + 1) or any token while
// NRES = 0 gets h = its iterate; a continuing one the mix, without writing the slot again.
// Otherwise list `lst` holds the continuing tokens, whose iterate is in h.
template <int NRES, int EPT, bool EXACT, bool SLOT>
__global__ __launch_bounds__(AND_NT) void k_anderson_reg(Dims D, SolveBuffers b, int lst, int ntok, int k,
                                                         int m) {
    __shared__ float red[AND_NT / 64][10];
    __shared__ float beta_s[4];
    const int i = blockIdx.x;
    if (i >= b.cnt[lst]) return;
    const int t = b.act[lst][i];
    const int hd = D.H * D.d;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *h = b.h + (long)t * hd;
    auto X = [&](int j) { return b.hist + ((long)(j % m) * ntok + t) * hd; };
    float *slot = X(k);
    if constexpr (SLOT) {
        // h = the update's iterate: a token that exited at this iteration (unless it stopped at the
        // cap unconverged, which is mixed), or any token while there is nothing to mix
        if (NRES == 0 || (b.iters[t] == k + 1 && !(b.cap_mix && !b.conv[t]))) {
            float v[EPT];
#pragma unroll
            for (int q = 0; q < EPT; ++q) {
                const int e = tid + q * AND_NT;
                v[q] = (EXACT || e < hd) ? slot[e] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < EPT; ++q) {
                const int e = tid + q * AND_NT;
                if (EXACT || e < hd) h[e] = v[q];
            }
            return;
        }
    }
    if constexpr (NRES >= 2) {
        // every load before the first store (the vector-memory counter retires in issue order)
        float x[NRES + 1][EPT];  // x[0] = X(k) (in h, or in the slot), x[ri] = X(k - ri)
#pragma unroll
        for (int ri = 0; ri <= NRES; ++ri) {
            const float *src = ri == 0 ? (SLOT ? slot : h) : X(k + m - ri);
#pragma unroll
            for (int q = 0; q < EPT; ++q) {
                const int e = tid + q * AND_NT;
                x[ri][q] = (EXACT || e < hd) ? src[e] : 0.0f;
            }
        }
        if constexpr (!SLOT) {
#pragma unroll
            for (int q = 0; q < EPT; ++q) {
                const int e = tid + q * AND_NT;
                if (EXACT || e < hd) slot[e] = x[0][q];
            }
        }
        constexpr int NPK = NRES * (NRES + 1) / 2;
        float gp[NPK];
#pragma unroll
        for (int q = 0; q < NPK; ++q) gp[q] = 0.0f;
#pragma unroll
        for (int q = 0; q < EPT; ++q) {
            float dl[NRES];
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri) dl[ri] = x[ri][q] - x[ri + 1][q];
            int p = 0;
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri)
#pragma unroll
                for (int rj = ri; rj < NRES; ++rj) gp[p++] += dl[ri] * dl[rj];
        }
        // the NPK wave sums interleaved (wave_sum's pairings, each round issued for all of them at once)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            float o[NPK];
#pragma unroll
            for (int q = 0; q < NPK; ++q) o[q] = __shfl_xor(gp[q], off, 64);
#pragma unroll
            for (int q = 0; q < NPK; ++q) gp[q] += o[q];
        }
        if (lane == 0) {
#pragma unroll
            for (int q = 0; q < NPK; ++q) red[wave][q] = gp[q];
        }
        __syncthreads();
        if (tid == 0) {
            float g[16];
            int q = 0;
            for (int ri = 0; ri < NRES; ++ri)
                for (int rj = ri; rj < NRES; ++rj) {
                    float v = 0.0f;
                    for (int w = 0; w < AND_NT / 64; ++w) v += red[w][q];
                    g[ri * NRES + rj] = v;
                    g[rj * NRES + ri] = v;
                    ++q;
                }
            float bt[4];
            anderson_coeffs(NRES, g, bt);
            for (int q2 = 0; q2 < NRES; ++q2) beta_s[q2] = bt[q2];
        }
        __syncthreads();
        float bl[NRES];
#pragma unroll
        for (int ri = 0; ri < NRES; ++ri) bl[ri] = beta_s[ri];
        float hmax = 0.0f;
#pragma unroll
        for (int q = 0; q < EPT; ++q) {
            const int e = tid + q * AND_NT;
            float acc = 0.0f;
#pragma unroll
            for (int ri = 0; ri < NRES; ++ri) acc += bl[ri] * x[ri][q];
            if (EXACT || e < hd) {
                h[e] = acc;
                hmax = fmaxf(hmax, fabsf(acc) < INFINITY ? fabsf(acc) : 0.0f);
            }
        }
        if (b.amax_h) track_absmax(b.amax_h, hmax);
    }
}

template <int H, int QA>
void attn_dispatch_vec(const Dims &D, const SolveBuffers &b, int cur, int k, int ntok, hipStream_t st) {
    constexpr int NG = H / QA;
    const long waves = (long)ntok * NG;
    const dim3 grid((unsigned)((waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK));
    if (D.d % 256 == 0)
        hipLaunchKernelGGL((k_attn<H, QA, 4>), grid, dim3(256), 0, st, D, b, cur, k);
    else if (D.d % 128 == 0)
        hipLaunchKernelGGL((k_attn<H, QA, 2>), grid, dim3(256), 0, st, D, b, cur, k);
    else
        hipLaunchKernelGGL((k_attn<H, QA, 1>), grid, dim3(256), 0, st, D, b, cur, k);
}

}  // namespace

void launch_init(const Dims &D, const SolveBuffers &b, const float *x_src, const int32_t *tokens,
                 int ntok, const float *anchor, hipStream_t st) {
    const long waves = (long)ntok * D.H;
    hipLaunchKernelGGL(k_init, dim3((unsigned)((waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK)),
                       dim3(64 * WAVES_PER_BLOCK), 0, st, D, b, x_src, tokens, ntok, anchor);
}

void launch_attn(const Dims &D, const SolveBuffers &b, int cur, int k, int ntok, hipStream_t st) {
    if (D.H & (D.H - 1)) {  // slot counts other than powers of two
        const dim3 grid((unsigned)(((long)ntok * D.H + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK));
        if (D.d % 256 == 0)
            hipLaunchKernelGGL(k_attn_rt<4>, grid, dim3(256), 0, st, D, b, cur, k);
        else if (D.d % 128 == 0)
            hipLaunchKernelGGL(k_attn_rt<2>, grid, dim3(256), 0, st, D, b, cur, k);
        else
            hipLaunchKernelGGL(k_attn_rt<1>, grid, dim3(256), 0, st, D, b, cur, k);
        return;
    }
    if (ntok <= SMALL_ROWS) {  // one wave per (token, query slot): the same scores, more waves
        switch (D.H) {
            case 1: attn_dispatch_vec<1, 1>(D, b, cur, k, ntok, st); break;
            case 2: attn_dispatch_vec<2, 1>(D, b, cur, k, ntok, st); break;
            case 4: attn_dispatch_vec<4, 1>(D, b, cur, k, ntok, st); break;
            case 8: attn_dispatch_vec<8, 1>(D, b, cur, k, ntok, st); break;
            case 16: attn_dispatch_vec<16, 1>(D, b, cur, k, ntok, st); break;
            default: break;
        }
        return;
    }
    switch (D.H) {
        case 1: attn_dispatch_vec<1, 1>(D, b, cur, k, ntok, st); break;
        case 2: attn_dispatch_vec<2, 2>(D, b, cur, k, ntok, st); break;
        case 4: attn_dispatch_vec<4, 4>(D, b, cur, k, ntok, st); break;
        case 8: attn_dispatch_vec<8, 8>(D, b, cur, k, ntok, st); break;
        case 16: attn_dispatch_vec<16, 4>(D, b, cur, k, ntok, st); break;
        default: break;  // other slot counts take k_attn_rt
    }
}

// k_update for d = 64 E: the slot count as a template argument (1, 2, 4, 8, 16) up to d = 1024
// for power-of-two rows without the history term, read at run time otherwise.
template <int E, bool PART>
void launch_update_e(const Dims &D, const SolveBuffers &b, int cur, int k, int max_iters, float eps,
                     const float *anchor, const float *norm_scale, float beta, dim3 grid, dim3 blk,
                     hipStream_t st) {
#define ADN_UPD_ARGS D, b, cur, k, max_iters, eps, anchor, norm_scale, beta
    if (b.mem_hist) {
        hipLaunchKernelGGL((k_update<E, 0, true, PART>), grid, blk, 0, st, ADN_UPD_ARGS);
        return;
    }
    if constexpr (E <= 16 && !PART) {
        switch (D.H) {
            case 1: hipLaunchKernelGGL((k_update<E, 1, false, false>), grid, blk, 0, st, ADN_UPD_ARGS); return;
            case 2: hipLaunchKernelGGL((k_update<E, 2, false, false>), grid, blk, 0, st, ADN_UPD_ARGS); return;
            case 4: hipLaunchKernelGGL((k_update<E, 4, false, false>), grid, blk, 0, st, ADN_UPD_ARGS); return;
            case 8: hipLaunchKernelGGL((k_update<E, 8, false, false>), grid, blk, 0, st, ADN_UPD_ARGS); return;
            case 16: hipLaunchKernelGGL((k_update<E, 16, false, false>), grid, blk, 0, st, ADN_UPD_ARGS); return;
            default: break;
        }
    }
    hipLaunchKernelGGL((k_update<E, 0, false, PART>), grid, blk, 0, st, ADN_UPD_ARGS);
#undef ADN_UPD_ARGS
}

void launch_update(const Dims &D, const SolveBuffers &b, int cur, int k, int max_iters, float eps, int ntok,
                   const float *anchor, const float *norm_scale, float beta, hipStream_t st) {
    if (ntok <= SMALL_ROWS) {
        const dim3 tgrid((unsigned)ntok), tblk(64 * D.H);
        const size_t lds = b.pool ? (size_t)D.H * D.d * sizeof(float) : 0;
        dispatch_width(D.d, [&](auto Ec, auto Pc) {
            hipLaunchKernelGGL((k_update_tok<decltype(Ec)::value, decltype(Pc)::value>), tgrid, tblk, lds, st, D, b,
                               cur, k, max_iters, eps, anchor, norm_scale, beta);
        });
        return;
    }
    const dim3 grid((unsigned)((ntok + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK)), blk(64 * WAVES_PER_BLOCK);
    dispatch_width(D.d, [&](auto Ec, auto Pc) {
        launch_update_e<decltype(Ec)::value, decltype(Pc)::value>(D, b, cur, k, max_iters, eps, anchor, norm_scale,
                                                                  beta, grid, blk, st);
    });
}

void launch_anderson(const Dims &D, const SolveBuffers &b, int nxt, int ntok, int rows, int k, int m,
                     hipStream_t st) {
    const int n_res = k < m - 1 ? k : m - 1;
    const int nres = (k >= 2 && n_res >= 2) ? n_res : 0;
    const dim3 grid((unsigned)rows), blk(AND_NT);
    const long hd = (long)D.H * D.d;
    // the one-pass form where a thread's elements fit in registers (16 per vector: at most 157 VGPRs,
    // 3 waves per SIMD; 32 would take 256, one wave per SIMD)
    if (nres >= 2 && hd <= 16L * AND_NT) {
        auto go = [&](auto ept) {
            constexpr int EPT = decltype(ept)::value;
            auto go2 = [&](auto exact) {
                constexpr bool EX = decltype(exact)::value;
                switch (nres) {
                    case 2: hipLaunchKernelGGL((k_anderson_reg<2, EPT, EX, false>), grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
                    case 3: hipLaunchKernelGGL((k_anderson_reg<3, EPT, EX, false>), grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
                    default: hipLaunchKernelGGL((k_anderson_reg<4, EPT, EX, false>), grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
                }
            };
            if (hd == (long)EPT * AND_NT)
                go2(std::true_type{});
            else
                go2(std::false_type{});
        };
        if (hd <= 4L * AND_NT)
            go(std::integral_constant<int, 4>{});
        else if (hd <= 8L * AND_NT)
            go(std::integral_constant<int, 8>{});
        else
            go(std::integral_constant<int, 16>{});
        return;
    }
    switch (nres) {
        case 0: hipLaunchKernelGGL(k_anderson<0>, grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
        case 2: hipLaunchKernelGGL(k_anderson<2>, grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
        case 3: hipLaunchKernelGGL(k_anderson<3>, grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
        default: hipLaunchKernelGGL(k_anderson<4>, grid, blk, 0, st, D, b, nxt, ntok, k, m); break;
    }
}

bool anderson_from_slot_ok(const Dims &D) { return (long)D.H * D.d <= 16L * AND_NT; }

void launch_anderson_from_slot(const Dims &D, const SolveBuffers &b, int cur, int ntok, int rows, int k, int m,
                               hipStream_t st) {
    const int n_res = k < m - 1 ? k : m - 1;
    const int nres = (k >= 2 && n_res >= 2) ? n_res : 0;
    const dim3 grid((unsigned)rows), blk(AND_NT);
    const long hd = (long)D.H * D.d;
    auto go = [&](auto ept) {
        constexpr int EPT = decltype(ept)::value;
        auto go2 = [&](auto exact) {
            constexpr bool EX = decltype(exact)::value;
            switch (nres) {
                case 0: hipLaunchKernelGGL((k_anderson_reg<0, EPT, EX, true>), grid, blk, 0, st, D, b, cur, ntok, k, m); break;
                case 2: hipLaunchKernelGGL((k_anderson_reg<2, EPT, EX, true>), grid, blk, 0, st, D, b, cur, ntok, k, m); break;
                case 3: hipLaunchKernelGGL((k_anderson_reg<3, EPT, EX, true>), grid, blk, 0, st, D, b, cur, ntok, k, m); break;
                default: hipLaunchKernelGGL((k_anderson_reg<4, EPT, EX, true>), grid, blk, 0, st, D, b, cur, ntok, k, m); break;
            }
        };
        if (hd == (long)EPT * AND_NT)
            go2(std::true_type{});
        else
            go2(std::false_type{});
    };
    if (hd <= 4L * AND_NT)
        go(std::integral_constant<int, 4>{});
    else if (hd <= 8L * AND_NT)
        go(std::integral_constant<int, 8>{});
    else
        go(std::integral_constant<int, 16>{});
}

bool update_mix_ok(const Dims &D) {
    if (D.H < 1 || D.H > 16 || D.d > 2048) return false;
    if (D.d <= 512) return true;
    // rows above 512 floats keep a token's rows in LDS (a padded 64 * E floats per row)
    int dev = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return false;
    const long e = D.d <= 1024 ? 16 : 32;
    return (long)D.H * e * 64 * (long)sizeof(float) + 1024 <= max_lds;
}

void launch_update_mix(const Dims &D, const SolveBuffers &b, int cur, int k, int m, int ntok, int rows,
                       int max_iters, float eps, const float *anchor, const float *norm_scale, float beta,
                       hipStream_t st) {
    const int nres = k < m - 1 ? k : m - 1;                  // >= 2 (k >= 2, m >= 3)
    const int pn = k - 1 >= 2 ? (k - 1 < m - 1 ? k - 1 : m - 1) : 0;  // terms of the mix at k - 1
    const dim3 grid((unsigned)rows), blk(64 * D.H);
    dispatch_width(D.d, [&](auto Ec, auto Pc) {
        constexpr int E = decltype(Ec)::value;
        constexpr bool P = decltype(Pc)::value;
        if constexpr (E <= 32) {
            auto go = [&](auto hist) {
                constexpr bool HS = decltype(hist)::value;
#define ADN_UM_ARGS D, b, cur, k, m, ntok, pn, max_iters, eps, anchor, norm_scale, beta
                if constexpr (E <= 8) {
                    switch (nres) {
                        case 2: hipLaunchKernelGGL((k_update_mix<E, P, 2, HS>), grid, blk, 0, st, ADN_UM_ARGS); break;
                        case 3: hipLaunchKernelGGL((k_update_mix<E, P, 3, HS>), grid, blk, 0, st, ADN_UM_ARGS); break;
                        default: hipLaunchKernelGGL((k_update_mix<E, P, 4, HS>), grid, blk, 0, st, ADN_UM_ARGS); break;
                    }
                } else {
                    const size_t lds = (size_t)D.H * E * 64 * sizeof(float);
                    switch (nres) {
                        case 2: hipLaunchKernelGGL((k_update_mix_wide<E, P, 2, HS>), grid, blk, lds, st, ADN_UM_ARGS); break;
                        case 3: hipLaunchKernelGGL((k_update_mix_wide<E, P, 3, HS>), grid, blk, lds, st, ADN_UM_ARGS); break;
                        default: hipLaunchKernelGGL((k_update_mix_wide<E, P, 4, HS>), grid, blk, lds, st, ADN_UM_ARGS); break;
                    }
                }
#undef ADN_UM_ARGS
            };
            if (b.mem_hist)
                go(std::true_type{});
            else
                go(std::false_type{});
        }
    });
}

}  // namespace adn

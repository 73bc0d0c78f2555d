// Weight preparation and the two small trait surfaces of the boundary.
//
//  * spectral norm by power iteration (spectral_norm.rs:25-80, spectral_renorm.wgsl:83-196)
//  * BlockBackend::fpm_batch_step ZOH step (gpu_backend.rs:18-56)
//  * ComputeBackend::ffn_forward column-major GEMV (aideen-engine ffn_forward.wgsl:22-37)
//  * layout helpers (tiled transpose, fill)
#include <cstring>

#include "kernels.h"

namespace adn {

namespace {

constexpr int SN_NT = 1024;

__device__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
    return t;
}

// One workgroup per matrix.  u0 = 1/sqrt(rows); per iteration v = W^T u / ||.||,
// u = W v / ||.||, sigma = (u^T W) v.  W^T u of the next iteration is the u^T W of the sigma
// step, so each iteration streams W twice.  work: [rows + 2*cols] floats.
__global__ __launch_bounds__(SN_NT) void k_spectral_norm(const float *w, int rows, int cols, int n_iter,
                                                         float *sigma_out, float *work) {
    __shared__ float red[SN_NT / 64];
    float *u = work;             // [rows]
    float *v = work + rows;      // [cols]
    float *z = v + cols;         // [cols] = W^T u
    const float inv = 1.0f / sqrtf((float)rows);
    for (int i = threadIdx.x; i < rows; i += SN_NT) u[i] = inv;
    __syncthreads();
    // z = W^T u (each output accumulates over rows in order)
    for (int j = threadIdx.x; j < cols; j += SN_NT) {
        float acc = 0.0f;
        for (int i = 0; i < rows; ++i) acc += w[(long)i * cols + j] * u[i];
        z[j] = acc;
    }
    __syncthreads();
    float sigma = 1.0f;
    bool zero = false;
    for (int it = 0; it < n_iter; ++it) {
        float p = 0.0f;
        for (int j = threadIdx.x; j < cols; j += SN_NT) p += z[j] * z[j];
        const float nv = sqrtf(block_sum(p, red));
        if (nv < 1e-12f) {
            zero = true;
            break;
        }
        for (int j = threadIdx.x; j < cols; j += SN_NT) v[j] = z[j] / nv;
        __syncthreads();
        // u = W v (wave per row)
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int i = wave; i < rows; i += SN_NT / 64) {
            float acc = 0.0f;
            for (int j = lane; j < cols; j += 64) acc += w[(long)i * cols + j] * v[j];
            acc = wave_sum(acc);
            if (lane == 0) u[i] = acc;
        }
        __syncthreads();
        p = 0.0f;
        for (int i = threadIdx.x; i < rows; i += SN_NT) p += u[i] * u[i];
        const float nu = sqrtf(block_sum(p, red));
        if (nu < 1e-12f) {
            zero = true;
            break;
        }
        for (int i = threadIdx.x; i < rows; i += SN_NT) u[i] = u[i] / nu;
        __syncthreads();
        for (int j = threadIdx.x; j < cols; j += SN_NT) {
            float acc = 0.0f;
            for (int i = 0; i < rows; ++i) acc += w[(long)i * cols + j] * u[i];
            z[j] = acc;
        }
        __syncthreads();
        p = 0.0f;
        for (int j = threadIdx.x; j < cols; j += SN_NT) p += z[j] * v[j];
        sigma = block_sum(p, red);
    }
    if (threadIdx.x == 0) {
        const float a = fabsf(sigma);
        *sigma_out = zero ? 0.0f : (a > 1e-12f ? a : 1e-12f);
    }
}

__global__ void k_scale_if(float *w, long n, const float *sigma, float threshold) {
    const float sg = *sigma;
    if (!(sg > threshold)) return;
    const float sc = threshold / sg;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        w[i] *= sc;
}

__global__ void k_zoh(int d, const float *x, const float *dt, const float *a, const float *b,
                      const float *c, float *y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d) return;
    const float abar = expf(dt[i] * a[i]);
    const float bbar = fabsf(a[i]) > 1e-8f ? (abar - 1.0f) / a[i] * b[i] : dt[i] * b[i];
    const float hn = bbar * x[i];
    y[i] = c[i] * hn;
}

__global__ void k_gemv_colmajor(const float *w, const float *x, int in_dim, int out_dim, float *y) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= out_dim) return;
    float acc = 0.0f;
    for (int i = 0; i < in_dim; ++i) acc = acc + x[i] * w[(long)i * out_dim + row];
    y[row] = acc;
}

// dst[b][c][r] = src[b][r][c]
__global__ void k_transpose(const float *src, int rows, int cols, float *dst) {
    __shared__ float tile[32][33];
    const long b = blockIdx.z;
    const float *s = src + b * (long)rows * cols;
    float *o = dst + b * (long)rows * cols;
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int k = threadIdx.y; k < 32; k += blockDim.y) {
        const int r = r0 + k, c = c0 + threadIdx.x;
        if (r < rows && c < cols) tile[k][threadIdx.x] = s[(long)r * cols + c];
    }
    __syncthreads();
    for (int k = threadIdx.y; k < 32; k += blockDim.y) {
        const int c = c0 + k, r = r0 + threadIdx.x;
        if (r < rows && c < cols) o[(long)c * rows + r] = tile[threadIdx.x][k];
    }
}

__global__ void k_fill_i32(int32_t *p, int32_t v, long n) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        p[i] = v;
}

// The operand bounds of one forward: words[0] = w0 (float bits), the other ADN_BOUNDS - 1 zero;
// also *zero = 0 when given (the signal GEMM's A-magnitude word).
__global__ void k_reset_bounds(unsigned *words, unsigned w0, unsigned *zero) {
    const int i = threadIdx.x;
    if (i < ADN_BOUNDS) words[i] = i == 0 ? w0 : 0u;
    if (i == ADN_BOUNDS && zero) *zero = 0u;
}

// The GPU spectral renormalisation (spectral_renorm.wgsl:83-196): one workgroup of 256 per matrix.
// The shader indexes its buffer as wg[i*d + j]; with the matrix M as stored here (row-major
// [d][d]) that buffer is M^T (RENORM_T, the per-slot Q/K/V/O and W_out, whose reference buffers
// are [in][out]), M itself (RENORM_N: W_in, uploaded row-major) or a diagonal (RENORM_DIAG: W_x,
// of which the carrier keeps the diagonal).  u = 1/sqrt(d); per iteration v = wg^T u / sqrt(|.|^2 +
// 1e-12), u = wg v, sigma = sqrt(|u|^2 + 1e-12), u /= sigma; then, when sigma exceeds the
// matrix's threshold, M *= threshold / sigma.  Thread t owns rows t, t + 256, ...: every dot
// product is summed over j in order and every squared norm by the shader's tree, without
// contracted multiply-adds, as the oracle restates it.
constexpr int RN_NT = 256;
constexpr int RN_MAXD = 2048;

__device__ float rn_tree(float v, float *part) {
    __syncthreads();
    part[threadIdx.x] = v;
    __syncthreads();
    for (int stride = RN_NT / 2; stride > 0; stride >>= 1) {
        if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
        __syncthreads();
    }
    return part[0];
}

__global__ __launch_bounds__(RN_NT) void k_spectral_renorm(const RenormJob *jobs, int d, int n_iters,
                                                           float *sigmas) {
#pragma clang fp contract(off)
    __shared__ float u[RN_MAXD], v[RN_MAXD], part[RN_NT];
    const RenormJob J = jobs[blockIdx.x];
    const float *M = J.m;
    const int tid = threadIdx.x;
    // wg[a][b] of the shader's buffer
    auto wg = [&](int a, int b) {
        return J.kind == RENORM_T ? M[(long)b * d + a] : J.kind == RENORM_N ? M[(long)a * d + b] : (a == b ? M[a] : 0.0f);
    };
    for (int i = tid; i < d; i += RN_NT) u[i] = 1.0f / sqrtf((float)d);
    __syncthreads();
    float sigma = 1.0f;
    for (int it = 0; it < n_iters; ++it) {
        float acc = 0.0f;
        for (int row = tid; row < d; row += RN_NT) {
            float vt = 0.0f;
            if (J.kind == RENORM_DIAG) {
                vt = M[row] * u[row];  // the other terms of the shader's sum are zero
            } else {
                for (int j = 0; j < d; ++j) vt += wg(j, row) * u[j];
            }
            v[row] = vt;
            acc += vt * vt;
        }
        const float vn = sqrtf(rn_tree(acc, part) + 1e-12f);
        for (int row = tid; row < d; row += RN_NT) v[row] = v[row] / vn;
        __syncthreads();
        acc = 0.0f;
        for (int row = tid; row < d; row += RN_NT) {
            float ut = 0.0f;
            if (J.kind == RENORM_DIAG) {
                ut = M[row] * v[row];
            } else {
                for (int j = 0; j < d; ++j) ut += wg(row, j) * v[j];
            }
            u[row] = ut;
            acc += ut * ut;
        }
        sigma = sqrtf(rn_tree(acc, part) + 1e-12f);
        for (int row = tid; row < d; row += RN_NT) u[row] = u[row] / sigma;
        __syncthreads();
    }
    if (tid == 0) sigmas[J.out] = sigma;
    if (sigma > J.threshold) {
        const float scale = J.threshold / sigma;
        const long n = J.kind == RENORM_DIAG ? d : (long)d * d;
        for (long e = tid; e < n; e += RN_NT) J.m[e] = M[e] * scale;
    }
}

}  // namespace

void launch_reset_bounds(unsigned *words, float h_bound, unsigned *zero, hipStream_t st) {
    unsigned bits;
    memcpy(&bits, &h_bound, sizeof bits);
    hipLaunchKernelGGL(k_reset_bounds, dim3(1), dim3(64), 0, st, words, bits, zero);
}

void launch_spectral_norm(const float *w, int rows, int cols, int n_iter, float *sigma, float *work,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_spectral_norm, dim3(1), dim3(SN_NT), 0, st, w, rows, cols, n_iter, sigma, work);
}

void launch_scale_if(float *w, long n, const float *sigma, float threshold, hipStream_t st) {
    const long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_scale_if, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st, w, n,
                       sigma, threshold);
}

void launch_zoh(int d, const float *x, const float *dt, const float *a, const float *b,
                const float *c, float *y, hipStream_t st) {
    hipLaunchKernelGGL(k_zoh, dim3((unsigned)((d + 255) / 256)), dim3(256), 0, st, d, x, dt, a, b, c, y);
}

void launch_gemv_colmajor(const float *w, const float *x, int in_dim, int out_dim, float *y,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_gemv_colmajor, dim3((unsigned)((out_dim + 63) / 64)), dim3(64), 0, st, w, x, in_dim,
                       out_dim, y);
}

void launch_transpose(const float *src, int rows, int cols, long batch, float *dst, hipStream_t st) {
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32), (unsigned)batch);
    hipLaunchKernelGGL(k_transpose, grid, dim3(32, 8), 0, st, src, rows, cols, dst);
}

// max |x| over the finite elements, as the bit pattern of a non-negative float (which orders
// like the float), one atomic per wave.  NaN and inf elements are skipped: they stay non-finite
// in their own output rows, and must not turn the scale of every other row into 0 or NaN.
__global__ void k_absmax(const float *x, long n, unsigned *out) {
    unsigned m = 0;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
        const float a = fabsf(x[i]);
        if (a < INFINITY) m = max(m, __float_as_uint(a));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, off, 64));
    if ((threadIdx.x & 63) == 0 && m) atomicMax(out, m);
}

void launch_absmax(const float *x, long n, unsigned *out, hipStream_t st) {
    const long blocks = std::min<long>((n + 255) / 256, 2048);
    hipLaunchKernelGGL(k_absmax, dim3((unsigned)(blocks > 0 ? blocks : 1)), dim3(256), 0, st, x, n, out);
}

void launch_fill_i32(int32_t *p, int32_t v, long n, hipStream_t st) {
    const long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096)),
                       dim3(256), 0, st, p, v, n);
}

void launch_spectral_renorm(const RenormJob *jobs, int njobs, int d, int n_iters, float *sigmas, hipStream_t st) {
    if (njobs > 0)
        hipLaunchKernelGGL(k_spectral_renorm, dim3((unsigned)njobs), dim3(RN_NT), 0, st, jobs, d, n_iters, sigmas);
}

}  // namespace adn

// k_backend.hip -- kernels behind the reference's Backend function table
// (sys/src/lib.rs:29-38: dot256, axpy256, add256, max256, sum256, scale_mul)
// and the jit_* helpers of ops/src/kernels.rs:1035-1113 that have no
// counterpart elsewhere in this library (layernorm, bias, outer).
//
// Elementwise results are bitwise the reference's: the FMA-or-not choice of
// each element follows the reference's 8-lane blocks and scalar tail.
// dot / sum are deterministic two-level tree sums (not the reference's
// serial 8-lane chains, which cannot run in parallel bit for bit); max is
// bitwise, including the MAXPS treatment of NaN and signed zeros.
#include "internal.hpp"

namespace vmlm {

// ---------------------------------------------------------------- dot / sum
// Block b sums the contiguous chunk [b * chunk, min(n, (b + 1) * chunk)):
// thread t takes elements t, t + 256, ... (FMA chain for dot, adds for sum),
// then the 4 waves' sums are added in wave order. The final kernel adds the
// block partials the same way. The order depends on n only.
template <int DOT>
__global__ __launch_bounds__(256) void bk_reduce_kernel(const float *__restrict__ a,
                                                        const float *__restrict__ b, size_t n,
                                                        size_t chunk, float *__restrict__ part) {
    __shared__ float sh[4];
    const size_t lo = (size_t)blockIdx.x * chunk;
    const size_t hi = lo + chunk < n ? lo + chunk : n;
    float acc = 0.0f;
    for (size_t i = lo + threadIdx.x; i < hi; i += 256)
        acc = DOT ? __builtin_fmaf(a[i], b[i], acc) : acc + a[i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

__global__ __launch_bounds__(256) void bk_reduce_final_kernel(const float *__restrict__ part,
                                                              int nb, float *__restrict__ out) {
    __shared__ float sh[4];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < nb; i += 256) acc = acc + part[i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

constexpr int BK_MAX_BLOCKS = 256;

int bk_reduce_work_floats() { return BK_MAX_BLOCKS; }

int launch_bk_reduce(const float *a, const float *b, size_t n, bool dot, float *part, float *out,
                     hipStream_t st) {
    size_t nb = cdiv(n, (size_t)8192);
    nb = nb < 1 ? 1 : nb > BK_MAX_BLOCKS ? BK_MAX_BLOCKS : nb;
    const size_t chunk = n == 0 ? 0 : (n + nb - 1) / nb;
    if (dot)
        bk_reduce_kernel<1><<<(unsigned)nb, 256, 0, st>>>(a, b, n, chunk, part);
    else
        bk_reduce_kernel<0><<<(unsigned)nb, 256, 0, st>>>(a, b, n, chunk, part);
    VMLM_HIP_CHECK(hipGetLastError());
    bk_reduce_final_kernel<<<1, 256, 0, st>>>(part, (int)nb, out);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- max
// max256_f32 scans each of the 8 lanes l (elements 8j + l of the 8-blocks)
// with m = m > x ? m : x from -inf (MAXPS keeps the second operand on NaN or
// equality), folds the lanes and finishes the tail with a strict `>`.
//
// A lane's scan is split over threads and blocks as an ordered monoid: a
// segment is summarised by what it does to the incoming value m:
//   EMPTY          m
//   NONAN(v)       m > v ? m : v      (no NaN in the segment; v its scan)
//   RESET(v)       v                  (after its last NaN the scan restarts:
//                                      v is NaN if the NaN ends the segment)
// Composition of an earlier segment A with a later B: B if B is RESET or A
// is EMPTY; A if B is EMPTY; else A's kind with A.v > B.v ? A.v : B.v.
struct MaxSeg {
    int kind;  // 0 EMPTY, 1 NONAN, 2 RESET
    float v;
};
__device__ __forceinline__ MaxSeg max_combine(MaxSeg A, MaxSeg B) {
    if (B.kind == 2 || A.kind == 0) return B;
    if (B.kind == 0) return A;
    return MaxSeg{A.kind, A.v > B.v ? A.v : B.v};
}
__device__ __forceinline__ MaxSeg max_push(MaxSeg S, float x) {
    if (!(x == x)) return MaxSeg{2, x};
    if (S.kind == 0) return MaxSeg{1, x};
    return MaxSeg{S.kind, S.v > x ? S.v : x};
}

// Block b covers 8-blocks [b * per, min(n8, (b + 1) * per)); thread t a
// contiguous run of them; runs are combined in thread order.
__global__ __launch_bounds__(256) void bk_max_partial_kernel(const float *__restrict__ x,
                                                             size_t n8, size_t per,
                                                             MaxSeg *__restrict__ part) {
    __shared__ MaxSeg sh[256][8];
    const size_t ob = (size_t)blockIdx.x * per;
    const size_t oe = ob + per < n8 ? ob + per : n8;
    const size_t q = (per + 255) / 256;
    const size_t t0 = ob + threadIdx.x * q;
    const size_t t1 = t0 + q < oe ? t0 + q : oe;
    MaxSeg s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s[l] = MaxSeg{0, 0.0f};
    for (size_t o = t0; o < t1; ++o) {
#pragma unroll
        for (int l = 0; l < 8; ++l) s[l] = max_push(s[l], x[8 * o + l]);
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) sh[threadIdx.x][l] = s[l];
    __syncthreads();
    for (int w = 1; w < 256; w <<= 1) {
        if ((threadIdx.x & (2 * w - 1)) == 0)
#pragma unroll
            for (int l = 0; l < 8; ++l)
                sh[threadIdx.x][l] = max_combine(sh[threadIdx.x][l], sh[threadIdx.x + w][l]);
        __syncthreads();
    }
    if (threadIdx.x < 8) part[(size_t)blockIdx.x * 8 + threadIdx.x] = sh[0][threadIdx.x];
}

// One thread: the blocks' segments in order, each lane applied to -inf, the
// lane fold of max256_f32 (max(lo, hi), max with movehl, max with lane 1)
// and the scalar tail.
__global__ void bk_max_final_kernel(const MaxSeg *__restrict__ part, int nb,
                                    const float *__restrict__ x, size_t n8, size_t n,
                                    float *__restrict__ out) {
    if (threadIdx.x != 0) return;
    float m[8];
    for (int l = 0; l < 8; ++l) {
        MaxSeg s{0, 0.0f};
        for (int b = 0; b < nb; ++b) s = max_combine(s, part[(size_t)b * 8 + l]);
        const float ninf = -__builtin_inff();
        m[l] = s.kind == 0 ? ninf : s.kind == 1 ? (ninf > s.v ? ninf : s.v) : s.v;
    }
    float s4[4];
    for (int l = 0; l < 4; ++l) s4[l] = m[l] > m[l + 4] ? m[l] : m[l + 4];
    const float t0 = s4[0] > s4[2] ? s4[0] : s4[2];
    const float t1 = s4[1] > s4[3] ? s4[1] : s4[3];
    float r = t0 > t1 ? t0 : t1;
    for (size_t i = 8 * n8; i < n; ++i)
        if (x[i] > r) r = x[i];
    out[0] = r;
}

size_t bk_max_work_bytes() { return (size_t)BK_MAX_BLOCKS * 8 * sizeof(MaxSeg); }

int launch_bk_max(const float *x, size_t n, void *work, float *out, hipStream_t st) {
    const size_t n8 = n / 8;
    size_t nb = cdiv(n8, (size_t)1024);
    nb = nb < 1 ? 1 : nb > BK_MAX_BLOCKS ? BK_MAX_BLOCKS : nb;
    const size_t per = n8 == 0 ? 0 : (n8 + nb - 1) / nb;
    MaxSeg *part = (MaxSeg *)work;
    bk_max_partial_kernel<<<(unsigned)nb, 256, 0, st>>>(x, n8, per, part);
    VMLM_HIP_CHECK(hipGetLastError());
    bk_max_final_kernel<<<1, 64, 0, st>>>(part, (int)nb, x, n8, n, out);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- elementwise
// axpy256_f32 (sys/src/x86_avx2/simd.rs:70-95): fused on the 8-blocks, a * x
// then + on the tail. add256_f32: y + x. scale_mul_avx2: a * src.
__global__ __launch_bounds__(256) void bk_axpy_kernel(float *__restrict__ y,
                                                      const float *__restrict__ x, float a,
                                                      size_t n, size_t n8) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        y[i] = i < n8 ? __builtin_fmaf(a, x[i], y[i]) : y[i] + a * x[i];
}
__global__ __launch_bounds__(256) void bk_add_kernel(float *__restrict__ y,
                                                     const float *__restrict__ x, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = y[i] + x[i];
}
__global__ __launch_bounds__(256) void bk_scale_mul_kernel(float *__restrict__ d,
                                                           const float *__restrict__ s, float a,
                                                           size_t n) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) d[i] = a * s[i];
}

static unsigned ew_blocks(size_t n) {
    size_t b = cdiv(n, (size_t)256);
    return (unsigned)(b < 1 ? 1 : b > 8192 ? 8192 : b);
}

int launch_bk_axpy(float *y, const float *x, float a, size_t n, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    bk_axpy_kernel<<<ew_blocks(n), 256, 0, st>>>(y, x, a, n, n / 8 * 8);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}
int launch_bk_add(float *y, const float *x, size_t n, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    bk_add_kernel<<<ew_blocks(n), 256, 0, st>>>(y, x, n);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}
int launch_bk_scale_mul(float *d, const float *s, float a, size_t n, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    bk_scale_mul_kernel<<<ew_blocks(n), 256, 0, st>>>(d, s, a, n);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- jit helpers
// ops/src/kernels.rs:1308-1333 layernorm, in place, one workgroup per row:
// mean and variance as fixed-order tree sums, inv = 1/sqrt(var + eps)
// (IEEE sqrt, as sqrt_f), then y = (x - mean) * inv * g + b per element.
__global__ __launch_bounds__(256) void layernorm_kernel(float *__restrict__ x,
                                                        const float *__restrict__ g,
                                                        const float *__restrict__ b, int cols,
                                                        float eps) {
    __shared__ float sh[4];
    float *p = x + (size_t)blockIdx.x * cols;
    float s = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) s = s + p[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    const float mean = ((sh[0] + sh[1]) + (sh[2] + sh[3])) / (float)cols;
    __syncthreads();
    float v = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) {
        const float d = p[i] - mean;
        v = v + d * d;
    }
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float var = ((sh[0] + sh[1]) + (sh[2] + sh[3])) / (float)cols;
    const float inv = 1.0f / __builtin_sqrtf(var + eps);
    for (int i = threadIdx.x; i < cols; i += 256) p[i] = (p[i] - mean) * inv * g[i] + b[i];
}

int launch_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                     float eps, hipStream_t st) {
    if (rows == 0 || cols == 0) return VMLM_OK;
    VMLM_GUARD(rows <= 0x7fffffffu && cols <= 0x7fffffffu, "layernorm: shape too large");
    layernorm_kernel<<<(unsigned)rows, 256, 0, st>>>(x, g, b, (int)cols, eps);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ops/src/kernels.rs:1058-1065 jit_bias: d[i, j] += b[j].
__global__ __launch_bounds__(256) void bias_kernel(float *__restrict__ d,
                                                   const float *__restrict__ b, size_t rows,
                                                   size_t cols) {
    const size_t n = rows * cols, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride)
        d[e] = d[e] + b[e % cols];
}

int launch_bias(float *d, const float *b, size_t rows, size_t cols, hipStream_t st) {
    if (rows == 0 || cols == 0) return VMLM_OK;
    bias_kernel<<<ew_blocks(rows * cols), 256, 0, st>>>(d, b, rows, cols);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ops/src/kernels.rs:1416-1448 outer (outer_avx2): vi = v[i] * sc; fused
// vi * k[j] + s on the 8-blocks of j, s + v[i] * sc * k[j] on the tail.
__global__ __launch_bounds__(256) void outer_kernel(float *__restrict__ s,
                                                    const float *__restrict__ v,
                                                    const float *__restrict__ k, size_t m,
                                                    size_t n, float sc) {
    const size_t total = m * n, n8 = n / 8 * 8, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += stride) {
        const size_t i = e / n, j = e % n;
        const float vi = v[i] * sc;
        s[e] = j < n8 ? __builtin_fmaf(vi, k[j], s[e]) : s[e] + vi * k[j];
    }
}

int launch_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc,
                 hipStream_t st) {
    if (m == 0 || n == 0) return VMLM_OK;
    outer_kernel<<<ew_blocks(m * n), 256, 0, st>>>(s, v, k, m, n, sc);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

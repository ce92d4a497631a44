// k_b1.hip -- B1 sparse-connection forward (ops/src/b1_pure.rs, ops/src/kernels.rs).
//
// Activations are kept source-major, xt[d][t8] (transpose_t8_avx2's layout,
// ops/src/kernels.rs:1881): a wavefront's 64 lanes are 64 consecutive tokens
// of one neuron, so for a connection (i, j) every lane reads the same source
// row src[i][j] at consecutive addresses -- the gather becomes one coalesced
// 256-byte read, and w[i][j] / src[i][j] are wave-uniform scalar loads.
//
// Two accumulation contracts, both reproduced bit for bit:
//  * T8: ops/src/kernels.rs:2163-2188 -- j ascending, first term assigned,
//    multiply then add (the contract of b1_forward_t8).
//  * FOLD: ops/src/kernels.rs:1773-1804 -- 8 partial sums (lane l takes
//    j = l mod 8 over the full 8-blocks, each starting at +0.0), the fixed
//    fold ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)), then the ascending tail; the
//    small-k0 packed groupings of b1_forward_packed_avx2 (:2720-2800) for
//    k0 in {1, 4, 8} (the contract of b1_forward).
// An optional activation (VMLM_ACT_*) is applied to each output (tanh_f for
// the layer stack), bitwise like act_scalar.
#include "internal.hpp"

namespace vmlm {

enum { B1_T8 = 0, B1_FOLD = 1 };

__device__ __forceinline__ float b1_fold(const float *__restrict__ w,
                                         const uint32_t *__restrict__ src,
                                         const float *__restrict__ xt, size_t t8, int t,
                                         int k0) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    int j = 0;
    for (; j + 8 <= k0; j += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + w[j + l] * xt[(size_t)src[j + l] * t8 + t];
    }
    float s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
    for (; j < k0; ++j) s += w[j] * xt[(size_t)src[j] * t8 + t];
    return s;
}

__device__ __forceinline__ float hsum4(float v0, float v1, float v2, float v3) {
    return (v0 + v2) + (v1 + v3);
}

// grid: (ceil(n_tokens/64), n); block 64 (one neuron, 64 tokens)
__global__ __launch_bounds__(64) void b1_forward_kernel(const float *__restrict__ w,
                                                        const uint32_t *__restrict__ src,
                                                        int n, int k0,
                                                        const float *__restrict__ xt,
                                                        size_t t8, int n_tokens,
                                                        float *__restrict__ yt, int mode,
                                                        int act) {
    const int i = blockIdx.y;
    const int t = blockIdx.x * 64 + threadIdx.x;
    if (t >= n_tokens) return;
    const float *wi = w + (size_t)i * k0;
    const uint32_t *si = src + (size_t)i * k0;
    float y;
    if (k0 == 0) {
        y = 0.0f;
    } else if (mode == B1_T8) {
        float acc = wi[0] * xt[(size_t)si[0] * t8 + t];
        for (int j = 1; j < k0; ++j) acc = acc + wi[j] * xt[(size_t)si[j] * t8 + t];
        y = acc;
    } else {
        // b1_forward: packed rows for k0 in {1,4,8} (k0 == 2 computes the row
        // sum; see the header note on the reference's k0 == 2 branch)
        if (k0 == 1 && i < (n / 8) * 8) {
            y = wi[0] * xt[(size_t)si[0] * t8 + t];
        } else if (k0 == 4 && i < (n / 2) * 2) {
            float p[4];
#pragma unroll
            for (int l = 0; l < 4; ++l) p[l] = wi[l] * xt[(size_t)si[l] * t8 + t];
            y = hsum4(p[0], p[1], p[2], p[3]);
        } else if (k0 == 8) {
            float p[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) p[l] = wi[l] * xt[(size_t)si[l] * t8 + t];
            y = hsum4(p[0] + p[4], p[1] + p[5], p[2] + p[6], p[3] + p[7]);
        } else {
            y = b1_fold(wi, si, xt, t8, t, k0);
        }
    }
    if (act >= 0) y = act_scalar(y, act);
    yt[(size_t)i * t8 + t] = y;
}

int launch_b1_forward(const float *w, const uint32_t *src, int n, int k0, const float *xt,
                      size_t t8, int n_tokens, float *yt, int mode, int act, hipStream_t st) {
    if (n == 0 || n_tokens == 0) return VMLM_OK;
    dim3 grid(cdiv(n_tokens, 64), n);
    b1_forward_kernel<<<grid, 64, 0, st>>>(w, src, n, k0, xt, t8, n_tokens, yt, mode, act);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// T8 layer with the sources staged in LDS: a workgroup owns 16 tokens and a
// group of neurons. The 16-token slice of every source row (d rows, 64 bytes
// each) is copied into LDS once, so a source row is fetched once per 16 tokens
// and workgroup rather than once per connection; then thread (slot, token)
// computes neurons slot, slot + 64, ... of the group with the T8 contract
// (j ascending, first product assigned, multiply then add). Indices are
// clamped to the staged rows.
constexpr int B1S_TB = 16;
constexpr int B1S_PIECES = 9;  // 16-byte staging pieces per thread: d <= 2304
__global__ __launch_bounds__(1024) void b1_t8_staged_kernel(const float *__restrict__ w,
                                                            const uint32_t *__restrict__ src,
                                                            int n, int k0, int d,
                                                            const float *__restrict__ xt,
                                                            size_t t8, int n_tokens,
                                                            float *__restrict__ yt, int act,
                                                            int group) {
    extern __shared__ float4 xs4[];  // [d][4] float4 = [d][16] floats
    const float *xs = (const float *)xs4;
    const int t0 = blockIdx.x * B1S_TB;
    {
        // every staging load of the thread goes out before any is stored;
        // pieces past d * 4 re-read the last one and store it again (same
        // value, same place), so neither the loads nor the stores branch
        float4 stg[B1S_PIECES];
        int pcs[B1S_PIECES];
#pragma unroll
        for (int k = 0; k < B1S_PIECES; ++k) {
            const int pc = threadIdx.x + k * 1024;
            pcs[k] = pc < d * 4 ? pc : d * 4 - 1;
            stg[k] = *(const float4 *)(xt + (size_t)(pcs[k] >> 2) * t8 + t0 + (pcs[k] & 3) * 4);
        }
#pragma unroll
        for (int k = 0; k < B1S_PIECES; ++k) xs4[pcs[k]] = stg[k];
    }
    __syncthreads();
    const int tok = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const int t = t0 + tok;
    const int i_end = (int)blockIdx.y * group + group < n ? (int)blockIdx.y * group + group : n;
    for (int i = (int)blockIdx.y * group + slot; i < i_end; i += 64) {
        const float *wi = w + (size_t)i * k0;
        const uint32_t *si = src + (size_t)i * k0;
        float acc = 0.0f;
        // batches of 32 connections: indices and weights loaded together
        // (clamped past k0), then the in-order sum; a full batch has no branch
        for (int j0 = 0; j0 < k0; j0 += 32) {
            uint32_t sv[32];
            float wv[32];
#pragma unroll
            for (int jj = 0; jj < 32; ++jj) {
                const int j = j0 + jj < k0 ? j0 + jj : k0 - 1;
                sv[jj] = si[j];
                wv[jj] = wi[j];
            }
            if (j0 + 32 <= k0) {
#pragma unroll
                for (int jj = 0; jj < 32; ++jj) {
                    const uint32_t srow = sv[jj] < (uint32_t)d ? sv[jj] : (uint32_t)(d - 1);
                    const float p = wv[jj] * xs[srow * B1S_TB + tok];
                    acc = j0 + jj == 0 ? p : acc + p;
                }
            } else {
                for (int jj = 0; j0 + jj < k0; ++jj) {
                    const uint32_t srow = sv[jj] < (uint32_t)d ? sv[jj] : (uint32_t)(d - 1);
                    const float p = wv[jj] * xs[srow * B1S_TB + tok];
                    acc = j0 + jj == 0 ? p : acc + p;
                }
            }
        }
        if (act >= 0) acc = act_scalar(acc, act);
        if (t < n_tokens) yt[(size_t)i * t8 + t] = acc;
    }
}

int launch_b1_t8_layer(const float *w, const uint32_t *src, int n, int k0, int d,
                       const float *xt, size_t t8, int n_tokens, float *yt, int act,
                       hipStream_t st) {
    const size_t lds = (size_t)d * B1S_TB * sizeof(float);
    if (n == 0 || n_tokens == 0) return VMLM_OK;
    if (k0 == 0 || d == 0 || d * 4 > B1S_PIECES * 1024 || t8 % B1S_TB)
        return launch_b1_forward(w, src, n, k0, xt, t8, n_tokens, yt, B1_T8, act, st);
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    // about one workgroup per CU: token blocks x neuron groups
    const int ntb = (int)((size_t)(n_tokens + B1S_TB - 1) / B1S_TB);
    int groups = cus / ntb;
    groups = groups < 1 ? 1 : groups > (n + 63) / 64 ? (n + 63) / 64 : groups;
    const int group = (n + groups - 1) / groups;
    b1_t8_staged_kernel<<<dim3(ntb, (n + group - 1) / group), 1024, lds, st>>>(
        w, src, n, k0, d, xt, t8, n_tokens, yt, act, group);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// xt[s*t8 + t] = x[t*d + s] for t < T, 0 for T <= t < t8 (32x32 LDS tiles).
__global__ __launch_bounds__(256) void transpose_t8_kernel(const float *__restrict__ x, int T,
                                                           int d, float *__restrict__ xt,
                                                           size_t t8) {
    __shared__ float tile[32][33];
    const int t0 = blockIdx.x * 32, s0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        int t = t0 + r, s = s0 + tx;
        tile[r][tx] = (t < T && s < d) ? x[(size_t)t * d + s] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int s = s0 + r, t = t0 + tx;
        if (s < d && (size_t)t < t8) xt[(size_t)s * t8 + t] = tile[tx][r];
    }
}

int launch_transpose_t8(const float *x, size_t T, size_t d, float *xt, size_t t8,
                        hipStream_t st) {
    if (d == 0 || t8 == 0) return VMLM_OK;
    dim3 grid(cdiv(t8, 32), cdiv(d, 32));
    transpose_t8_kernel<<<grid, 256, 0, st>>>(x, (int)T, (int)d, xt, t8);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// out[i*os + s] = a[s*in_stride + i], s < rows, i < cols (ops/src/kernels.rs:3307).
__global__ __launch_bounds__(256) void transpose_back_kernel(const float *__restrict__ a,
                                                             int rows, int cols,
                                                             float *__restrict__ out,
                                                             size_t os, size_t in_stride) {
    __shared__ float tile[32][33];
    const int i0 = blockIdx.x * 32, s0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        int s = s0 + r, i = i0 + tx;
        tile[r][tx] = (s < rows && i < cols) ? a[(size_t)s * in_stride + i] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int i = i0 + r, s = s0 + tx;
        if (i < cols && s < rows) out[(size_t)i * os + s] = tile[tx][r];
    }
}

int launch_transpose_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                          size_t in_stride, hipStream_t st) {
    if (rows == 0 || cols == 0) return VMLM_OK;
    dim3 grid(cdiv(cols, 32), cdiv(rows, 32));
    transpose_back_kernel<<<grid, 256, 0, st>>>(a, (int)rows, (int)cols, out, os, in_stride);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

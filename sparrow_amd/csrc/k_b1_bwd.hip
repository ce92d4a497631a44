// k_b1_bwd.hip -- B1 sparse-connection backward (ops/src/b1_pure.rs:410-490,
// 642-656; ops/src/kernels.rs:2401-2478, 3229-3275), bitwise.
//
// dw is elementwise: each connection (i, j) gets one update from its own
// neuron's dy and source activation. dx is a scatter: source s sums
// dy[i] * w[i][j] over every connection that reads it, in (i, j) ascending
// order (the reference's loop order; its fused AVX2 kernel keeps that order
// by scattering one lane at a time). The GPU keeps the order without
// atomics through a reverse index: the connections sorted by source with a
// stable radix sort (connection numbers e = i * k0 + j ascending inside each
// source), so one thread per source (or per (source, token)) replays its
// connections in the reference's order.
#include <hipcub/hipcub.hpp>

#include "internal.hpp"

namespace vmlm {

// Rust's `f as usize` for the f32 ids of SparseConnW.src
__device__ __forceinline__ size_t b1_usize(float f) {
    return f > 0.0f ? (f >= 1.8446744e19f ? ~(size_t)0 : (size_t)f) : 0;
}

__global__ __launch_bounds__(256) void b1_iota_kernel(uint32_t *v, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) v[e] = (uint32_t)e;
}

// off[s] = first position of source s in the sorted ids (binary search),
// s = 0 .. d; ids >= d sort after off[d] and are never replayed.
__global__ __launch_bounds__(256) void b1_rev_offsets_kernel(const uint32_t *keys, size_t E,
                                                             size_t d, uint32_t *off) {
    const size_t s = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (s > d) return;
    size_t lo = 0, hi = E;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (keys[mid] < s) lo = mid + 1;
        else hi = mid;
    }
    off[s] = (uint32_t)lo;
}

// dw[e] += dy[e / k0] * x[src[e]] (f32 ids when srcf, else u32); an id past
// the source dimension sets the guard and skips the connection.
__global__ __launch_bounds__(256) void b1_bwd_dw_kernel(const float *dy, const float *x,
                                                        const float *srcf, const uint32_t *src,
                                                        size_t E, size_t k0, size_t d, float *dw,
                                                        int *guard) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < E; e += stride) {
        const size_t s = srcf ? b1_usize(srcf[e]) : src[e];
        if (s >= d) {
            atomicOr(guard, 1);
            continue;
        }
        dw[e] = dw[e] + dy[e / k0] * x[s];
    }
}

// dx[s] += dy[i] * w[e] over source s's connections in ascending e.
__global__ __launch_bounds__(256) void b1_bwd_dx_kernel(const uint32_t *perm, const uint32_t *off,
                                                        const float *w, const float *dy,
                                                        size_t k0, size_t d, float *dx) {
    const size_t s = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (s >= d) return;
    float acc = dx[s];
    for (uint32_t t = off[s]; t < off[s + 1]; ++t) {
        const uint32_t e = perm[t];
        acc = acc + dy[e / k0] * w[e];
    }
    dx[s] = acc;
}

// t8 dw: eight lanes per connection, lane l the FMA chain over tokens
// p = l, l + 8, ... (ops/src/kernels.rs:3245-3262), then the chains folded in
// hsum256's order ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) and added to dw.
__global__ __launch_bounds__(256) void b1_bwd_t8_dw_kernel(const uint32_t *src, const float *xt,
                                                           const float *dyt, size_t t8, size_t E,
                                                           size_t k0, size_t d, float *dw,
                                                           int *guard) {
    const size_t g = ((size_t)blockIdx.x * 256 + threadIdx.x) / 8;  // connection
    const int l = threadIdx.x & 7;
    const bool live = g < E;
    const size_t e = live ? g : 0;
    const size_t s = src[e];
    const bool ok = live && s < d;
    if (live && !ok && l == 0) atomicOr(guard, 1);
    float acc = 0.0f;
    if (ok) {
        const float *dr = dyt + (e / k0) * t8, *xr = xt + s * t8;
        for (size_t p = l; p < t8; p += 8) acc = __builtin_fmaf(dr[p], xr[p], acc);
    }
    const int base = (threadIdx.x & 63) & ~7;
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = __shfl(acc, base + q, 64);
    if (ok && l == 0) {
        const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
        dw[e] = dw[e] + ((s0 + s1) + (s2 + s3));
    }
}

// t8 dx: one thread per (source, token): dxt[s][p] = fma(dyt[i][p], w[e],
// dxt[s][p]) over the source's connections in ascending e.
__global__ __launch_bounds__(256) void b1_bwd_t8_dx_kernel(const uint32_t *perm,
                                                           const uint32_t *off, const float *w,
                                                           const float *dyt, size_t t8, size_t k0,
                                                           size_t d, float *dxt) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= d * t8) return;
    const size_t s = idx / t8, p = idx % t8;
    float acc = dxt[idx];
    for (uint32_t t = off[s]; t < off[s + 1]; ++t) {
        const uint32_t e = perm[t];
        acc = __builtin_fmaf(dyt[(e / k0) * t8 + p], w[e], acc);
    }
    dxt[idx] = acc;
}

static unsigned bwd_blocks(size_t n) {
    size_t b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : b);
}

// Workspace of the reverse index: sorted ids, two permutation buffers, the
// offsets and the radix sort's temporary storage (16-byte aligned pieces).
static size_t sort_temp_bytes(size_t E) {
    size_t bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const uint32_t *)nullptr,
                                             (uint32_t *)nullptr, (const uint32_t *)nullptr,
                                             (uint32_t *)nullptr, (int)E, 0, 32, (hipStream_t)0);
    return bytes;
}
static size_t a16(size_t x) { return (x + 15) / 16 * 16; }

size_t b1_rev_work_bytes(size_t E, size_t d) {
    return 3 * a16(E * 4 + 4) + a16((d + 1) * 4) + a16(sort_temp_bytes(E) + 16);
}

struct RevIndex {
    uint32_t *perm, *off;
};

static int build_rev(const uint32_t *src, size_t E, size_t d, void *work, RevIndex &r,
                     hipStream_t st) {
    VMLM_GUARD(E <= 0x7fffffffu && d < 0xffffffffu, "B1 backward: %zu connections", E);
    char *p = (char *)work;
    uint32_t *keys = (uint32_t *)p;
    p += a16(E * 4 + 4);
    uint32_t *iota = (uint32_t *)p;
    p += a16(E * 4 + 4);
    r.perm = (uint32_t *)p;
    p += a16(E * 4 + 4);
    r.off = (uint32_t *)p;
    p += a16((d + 1) * 4);
    size_t tb = sort_temp_bytes(E);
    if (E) {
        b1_iota_kernel<<<bwd_blocks(E), 256, 0, st>>>(iota, E);
        VMLM_HIP_CHECK(hipGetLastError());
        VMLM_HIP_CHECK(hipcub::DeviceRadixSort::SortPairs(p, tb, src, keys, iota, r.perm, (int)E, 0,
                                                          32, st));
    }
    b1_rev_offsets_kernel<<<bwd_blocks(d + 1), 256, 0, st>>>(keys, E, d, r.off);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_b1_backward(const float *w, const float *srcf, const uint32_t *src, size_t n,
                       size_t k0, const float *dy, const float *x, float *dw, float *dx,
                       void *work, hipStream_t st) {
    const size_t E = n * k0, d = n;
    if (E == 0) return VMLM_OK;
    int rc;
    if (dw) {
        b1_bwd_dw_kernel<<<bwd_blocks(E), 256, 0, st>>>(dy, x, srcf, src, E, k0, d, dw,
                                                        guard_flag_ptr());
        VMLM_HIP_CHECK(hipGetLastError());
    }
    if (dx) {
        RevIndex r;
        if ((rc = build_rev(src, E, d, work, r, st))) return rc;
        b1_bwd_dx_kernel<<<bwd_blocks(d), 256, 0, st>>>(r.perm, r.off, w, dy, k0, d, dx);
        VMLM_HIP_CHECK(hipGetLastError());
    }
    return VMLM_OK;
}

int launch_b1_backward_t8(const float *w, const uint32_t *src, const float *xt, const float *dyt,
                          size_t t8, size_t n, size_t k0, float *dxt, float *dw, void *work,
                          hipStream_t st) {
    VMLM_GUARD(t8 % 8 == 0, "B1_T8 backward: t8 = %zu is not a multiple of 8", t8);
    const size_t E = n * k0, d = n;
    if (E == 0 || t8 == 0) return VMLM_OK;
    RevIndex r;
    int rc = build_rev(src, E, d, work, r, st);
    if (rc) return rc;
    b1_bwd_t8_dw_kernel<<<bwd_blocks(E * 8), 256, 0, st>>>(src, xt, dyt, t8, E, k0, d, dw,
                                                           guard_flag_ptr());
    VMLM_HIP_CHECK(hipGetLastError());
    b1_bwd_t8_dx_kernel<<<bwd_blocks(d * t8), 256, 0, st>>>(r.perm, r.off, w, dyt, t8, k0, d, dxt);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

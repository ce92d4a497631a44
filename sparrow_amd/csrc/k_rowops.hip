// k_rowops.hip -- row and elementwise kernels of the VM opcode set.
//
// Elementwise kernels (act, ew_op, scale, RoPE, EMB) perform the same
// operations in the same order as the reference and are bitwise equal to
// it. Row reductions (RMSNORM sum of squares, SOFTMAX sum) are tree sums
// across a workgroup instead of the reference's left-to-right loop; the max
// and every per-element operation remain exact.
#include "internal.hpp"

namespace vmlm {

// Block-wide sum for 256 threads (4 wavefronts).
__device__ __forceinline__ float block_sum256(float v, float *sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_max256(float v, float *sh) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

// ops/src/kernels.rs:1346-1368 -- y = (x * inv) * g, inv = 1/sqrt(mean(x^2)+eps).
// Optionally also writes the T bf16 terms of y (GEMV activation operand).
__global__ __launch_bounds__(256) void rmsnorm_kernel(float *__restrict__ dst,
                                                      const float *__restrict__ src,
                                                      const float *__restrict__ g, int cols,
                                                      float eps, uint16_t *__restrict__ terms,
                                                      int T, int ld_terms, int rows) {
    __shared__ float sh[4];
    const int row = blockIdx.x;
    const float *p = src + (size_t)row * cols;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) ss += p[i] * p[i];
    ss = block_sum256(ss, sh);
    ss = ss / (float)cols;
    const float inv = 1.0f / sqrtf(ss + eps);
    float *q = dst ? dst + (size_t)row * cols : nullptr;
    for (int i = threadIdx.x; i < cols; i += 256) {
        float y = p[i] * inv * g[i];
        if (q) q[i] = y;
        if (terms) {
            for (int t = 0; t < T; ++t) {
                uint32_t h = bf16_rne_bits(y);
                y = term_rem(y, h);
                terms[((size_t)t * rows + row) * ld_terms + i] = (uint16_t)h;
            }
        }
    }
    if (terms) {  // zero the K padding of the terms
        for (int i = cols + threadIdx.x; i < ld_terms; i += 256)
            for (int t = 0; t < T; ++t) terms[((size_t)t * rows + row) * ld_terms + i] = 0;
    }
}

// Same operations for cols % 4 == 0, cols <= 4096: the row is read once into
// registers (float4 per thread, all loads issued together), so the kernel
// costs one memory round trip; terms are stored 4 bf16 (8 bytes) at a time.
template <int U>
__global__ __launch_bounds__(256) void rmsnorm_v4_kernel(float *__restrict__ dst,
                                                         const float *__restrict__ src,
                                                         const float *__restrict__ g, int cols,
                                                         float eps, uint16_t *__restrict__ terms,
                                                         int T, int ld_terms, int rows) {
    __shared__ float sh[4];
    const int row = blockIdx.x, n4 = cols >> 2;
    const float4 *p = (const float4 *)(src + (size_t)row * cols);
    const float4 *g4 = (const float4 *)g;
    float4 x[U], gg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = threadIdx.x + u * 256;
        x[u] = c < n4 ? p[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        gg[u] = c < n4 ? g4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        ss += x[u].x * x[u].x;
        ss += x[u].y * x[u].y;
        ss += x[u].z * x[u].z;
        ss += x[u].w * x[u].w;
    }
    ss = block_sum256(ss, sh);
    ss = ss / (float)cols;
    const float inv = 1.0f / sqrtf(ss + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = threadIdx.x + u * 256;
        if (c >= n4) continue;
        float y[4] = {x[u].x * inv * gg[u].x, x[u].y * inv * gg[u].y, x[u].z * inv * gg[u].z,
                      x[u].w * inv * gg[u].w};
        if (dst) ((float4 *)(dst + (size_t)row * cols))[c] = make_float4(y[0], y[1], y[2], y[3]);
        if (terms) {
            for (int t = 0; t < T; ++t) {
                uint32_t h[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    h[q] = bf16_rne_bits(y[q]);
                    y[q] = term_rem(y[q], h[q]);
                }
                uint2 pk = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                *(uint2 *)(terms + ((size_t)t * rows + row) * ld_terms + 4 * c) = pk;
            }
        }
    }
    if (terms) {
        for (int i = cols + threadIdx.x; i < ld_terms; i += 256)
            for (int t = 0; t < T; ++t) terms[((size_t)t * rows + row) * ld_terms + i] = 0;
    }
}

int launch_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                   float eps, uint16_t *terms, int T, int ld_terms, hipStream_t st) {
    if (rows == 0) return VMLM_OK;
    const bool aligned = cols % 4 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)g & 15) == 0 &&
                         (!dst || ((uintptr_t)dst & 15) == 0) &&
                         (!terms || (((uintptr_t)terms & 7) == 0 && ld_terms % 4 == 0));
    const size_t u = (cols / 4 + 255) / 256;
    if (aligned && u >= 1 && u <= 4) {
        switch (u) {
#define RMS_CASE(U)                                                                            \
    case U:                                                                                    \
        rmsnorm_v4_kernel<U><<<(unsigned)rows, 256, 0, st>>>(dst, src, g, (int)cols, eps,     \
                                                              terms, T, ld_terms, (int)rows); \
        break;
            RMS_CASE(1)
            RMS_CASE(2)
            RMS_CASE(3)
            RMS_CASE(4)
#undef RMS_CASE
        }
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    rmsnorm_kernel<<<(unsigned)rows, 256, 0, st>>>(dst, src, g, (int)cols, eps, terms, T,
                                                   ld_terms, (int)rows);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Residual add of a k-split projection fused with the RMSNorm that follows
// it (OP_GEMM + OP_EWADD + OP_RMSNORM of the decoder program): per row,
//   x = base + (sum_ks part[ks]) * scale      (slices summed in order)
//   resid = x;  y = x * (1 / sqrt(mean(x^2) + eps)) * g  -> T bf16 terms.
// One thread per 4 columns (cols <= 4096); every slice of a column is loaded
// up front (index clamped, KS_MAX slots) so the reads take one round trip.
constexpr int KS_MAX = 16;

__global__ __launch_bounds__(1024) void rmsnorm_resid_kernel(
    const float *__restrict__ base, const float *__restrict__ part, int ks, int ldp,
    const float *__restrict__ scale, float *__restrict__ resid, const float *__restrict__ g,
    int cols, float eps, uint16_t *__restrict__ terms, int T, int ld_terms, int rows) {
    __shared__ float sh[16];
    const int row = blockIdx.x, n4 = cols >> 2;
    const int c = threadIdx.x < n4 ? threadIdx.x : n4 - 1;
    float4 pv[KS_MAX];
#pragma unroll
    for (int k = 0; k < KS_MAX; ++k) {
        const int kk = k < ks ? k : ks - 1;
        pv[k] = ((const float4 *)(part + ((size_t)kk * rows + row) * ldp))[c];
    }
    const float4 sc = ((const float4 *)scale)[c];
    const float4 bb = ((const float4 *)(base + (size_t)row * cols))[c];
    const float4 gg = ((const float4 *)g)[c];
    float4 acc = pv[0];
#pragma unroll
    for (int k = 1; k < KS_MAX; ++k) {
        if (k < ks) {
            acc.x += pv[k].x;
            acc.y += pv[k].y;
            acc.z += pv[k].z;
            acc.w += pv[k].w;
        }
    }
    const float4 x = make_float4(bb.x + acc.x * sc.x, bb.y + acc.y * sc.y, bb.z + acc.z * sc.z,
                                 bb.w + acc.w * sc.w);
    const bool live = threadIdx.x < n4;
    float ss = live ? x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w : 0.0f;
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) ss += sh[w];
    ss = ss / (float)cols;
    const float inv = 1.0f / sqrtf(ss + eps);
    if (!live) return;
    ((float4 *)(resid + (size_t)row * cols))[c] = x;
    float y[4] = {x.x * inv * gg.x, x.y * inv * gg.y, x.z * inv * gg.z, x.w * inv * gg.w};
    for (int t = 0; t < T; ++t) {
        uint32_t h[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h[q] = bf16_rne_bits(y[q]);
            y[q] = term_rem(y[q], h[q]);
        }
        *(uint2 *)(terms + ((size_t)t * rows + row) * ld_terms + 4 * c) =
            make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
}

int launch_rmsnorm_resid(const float *base, const float *part, int ks, int ldp,
                         const float *scale, float *resid, size_t rows, size_t cols,
                         const float *g, float eps, uint16_t *terms, int T, int ld_terms,
                         hipStream_t st) {
    if (rows == 0) return VMLM_OK;
    VMLM_GUARD(cols % 4 == 0 && cols <= 4096 && ldp % 4 == 0 && ks >= 1 && ks <= KS_MAX &&
                   (int)cols == ld_terms,
               "rmsnorm_resid: cols %% 4 (<= 4096), ldp %% 4, 1 <= ks <= %d, ld_terms == cols",
               KS_MAX);
    const unsigned threads = (unsigned)((cols / 4 + 63) / 64 * 64);
    rmsnorm_resid_kernel<<<(unsigned)rows, threads, 0, st>>>(base, part, ks, ldp, scale, resid,
                                                             g, (int)cols, eps, terms, T,
                                                             ld_terms, (int)rows);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// One wave per (segment, row): the residual add of a k-split projection and
// the int8 input of the next k-slice GEMVs (see launch_resid_q8). One wave
// per workgroup: grouping 4, 8 or 16 rows of a segment in one workgroup
// (whole 128-byte lines of the blocked output from one CU) measured 0.5 to
// 7 % slower over the batch-16 decode step; the latency of the partial
// reads, not the write-back, sets this kernel's time. Lane l
// holds columns 4c..4c+3 of the segment, c = l + 64i (i < SI); all slices of
// a column are loaded up front so the reads take one round trip. The segment's power-of-two factor comes from its own max |x * g|.
template <int SI, int KSN, bool BLK>
__global__ __launch_bounds__(64) void resid_q8_kernel(
    const float *__restrict__ base, const float *__restrict__ part, int ks, int ldp,
    const float *__restrict__ scale, float *__restrict__ resid, const float *__restrict__ g,
    int cols, int rows, int seg, int8_t *__restrict__ q8, float *__restrict__ q8s,
    float *__restrict__ ssp) {
    const int sgi = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
    const int n4 = seg >> 2;
    float4 xg[SI], xb[SI];  // x * g, and x (the residual sum, stored last)
    float ss = 0.0f, mg = 0.0f;
#pragma unroll
    for (int i = 0; i < SI; ++i) {
        const int c = lane + 64 * i;
        const bool live = c < n4;
        const int col = sgi * seg + 4 * (live ? c : n4 - 1);
        float4 bb = *(const float4 *)(base + (size_t)row * cols + col);
        const float4 gg = *(const float4 *)(g + col);
        if (ks > 0) {
            float4 pv[KSN];
#pragma unroll
            for (int k = 0; k < KSN; ++k) {  // the slices there are (a uniform branch)
                pv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k < ks) pv[k] = *(const float4 *)(part + ((size_t)k * rows + row) * ldp + col);
            }
            const float4 sc = *(const float4 *)(scale + col);
            float4 acc = pv[0];
#pragma unroll
            for (int k = 1; k < KSN; ++k) {
                if (k < ks) {
                    acc.x += pv[k].x;
                    acc.y += pv[k].y;
                    acc.z += pv[k].z;
                    acc.w += pv[k].w;
                }
            }
            bb = make_float4(bb.x + acc.x * sc.x, bb.y + acc.y * sc.y, bb.z + acc.z * sc.z,
                             bb.w + acc.w * sc.w);
        }
        xb[i] = bb;
        xg[i] = make_float4(bb.x * gg.x, bb.y * gg.y, bb.z * gg.z, bb.w * gg.w);
        if (live) {
            ss += bb.x * bb.x + bb.y * bb.y + bb.z * bb.z + bb.w * bb.w;
            mg = fmaxf(mg, fmaxf(fmaxf(q8_mag(xg[i].x), q8_mag(xg[i].y)),
                                 fmaxf(q8_mag(xg[i].z), q8_mag(xg[i].w))));
        }
    }
    ss = wave_sum_dpp(ss);
    mg = wave_max_nonneg(mg);
    const int k = q8_row_k(mg);
    if (lane == 0) {
        q8s[(size_t)sgi * rows + row] = q8_factor(k);
        ssp[(size_t)sgi * rows + row] = ss;
    }
#pragma unroll
    for (int i = 0; i < SI; ++i) {
        const int c = lane + 64 * i;
        if (c >= n4) continue;
        const int col = sgi * seg + 4 * c;
        int a[4][Q8_T];
        q8_split(xg[i].x, k, a[0]);
        q8_split(xg[i].y, k, a[1]);
        q8_split(xg[i].z, k, a[2]);
        q8_split(xg[i].w, k, a[3]);
        // blocked: column col of k-block col / 64 sits in lane (g, row), g =
        // (col % 32) / 8, at byte 8 * (col % 64 >= 32) + col % 8
        const int o = col & 63;
        const size_t boff = ((size_t)(col >> 6) * 1024) + 16 * (16 * ((o & 31) >> 3) + row) +
                            8 * (o >> 5) + (o & 7);
#pragma unroll
        for (int t = 0; t < Q8_T; ++t) {
            const uint32_t v = pack_i8x4(a[0][t], a[1][t], a[2][t], a[3][t]);
            if constexpr (BLK)
                *(uint32_t *)(q8 + (size_t)t * (cols >> 6) * 1024 + boff) = v;
            else
                *(uint32_t *)(q8 + ((size_t)t * rows + row) * cols + col) = v;
        }
    }
    // The residual sum is stored after everything else: vmcnt counts stores
    // too, and with the store issued before the reductions the wait for the
    // gains there also waited for the store (batch-16 decode 8,338 -> 8,397
    // tokens/s, the same tokens).
    if (ks > 0) {
#pragma unroll
        for (int i = 0; i < SI; ++i) {
            const int c = lane + 64 * i;
            if (c < n4) *(float4 *)(resid + (size_t)row * cols + sgi * seg + 4 * c) = xb[i];
        }
    }
}

int launch_resid_q8(const float *base, const float *part, int ks, int ldp, const float *scale,
                    float *resid, const float *g, size_t rows, size_t cols, int seg, int8_t *q8,
                    float *q8s, float *ssp, hipStream_t st, bool blocked) {
    if (rows == 0) return VMLM_OK;
    VMLM_GUARD(!blocked || (rows <= 16 && cols % 64 == 0 && ((uintptr_t)q8 & 15) == 0),
               "resid_q8: blocked rows need at most 16 rows, 64-column blocks, 16-byte alignment");
    VMLM_GUARD(seg >= 64 && seg <= 512 && seg % 64 == 0 && cols % seg == 0 && cols / seg <= 65535,
               "resid_q8: segments of 64..512 columns (multiple of 64) tiling the row");
    VMLM_GUARD(ks >= 0 && ks <= KS_MAX && (ks == 0 || (part && scale && resid && ldp % 4 == 0)),
               "resid_q8: 0 <= ks <= %d; a k-split needs partials, scales and a residual", KS_MAX);
    VMLM_GUARD(((uintptr_t)base & 15) == 0 && ((uintptr_t)g & 15) == 0 && ((uintptr_t)q8 & 3) == 0 &&
                   q8s && ssp && rows <= 65535,
               "resid_q8: aligned rows and outputs");
    const dim3 grid((unsigned)(cols / seg), (unsigned)rows);
    // slice loads sized to the slice count of the decoder's projections (9
    // for K = 2304, 15 for K = 5760), else 4 or 16 (loads past ks skipped)
#define RQ_LAUNCH(SI, KSN)                                                                      \
    do {                                                                                        \
        if (blocked)                                                                            \
            resid_q8_kernel<SI, KSN, true><<<grid, 64, 0, st>>>(base, part, ks, ldp, scale,    \
                                                                resid, g, (int)cols, (int)rows, \
                                                                seg, q8, q8s, ssp);             \
        else                                                                                    \
            resid_q8_kernel<SI, KSN, false><<<grid, 64, 0, st>>>(base, part, ks, ldp, scale,   \
                                                                 resid, g, (int)cols,           \
                                                                 (int)rows, seg, q8, q8s, ssp); \
    } while (0)
#define RQ_KS(SI)                                                                               \
    if (ks == 9) RQ_LAUNCH(SI, 9);                                                              \
    else if (ks == 15) RQ_LAUNCH(SI, 15);                                                       \
    else if (ks <= 4) RQ_LAUNCH(SI, 4);                                                         \
    else RQ_LAUNCH(SI, 16);
    if (seg <= 256) {
        RQ_KS(1)
    } else {
        RQ_KS(2)
    }
#undef RQ_KS
#undef RQ_LAUNCH
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// SiLU(gate) * up as the int8 input of the down projection's k-slice GEMV.
// The gate/up projection interleaves its rows in blocks of 16 (rows
// 32t..32t+15 gate, 32t+16..32t+31 up, for outputs 16t..16t+15); its k-slice
// partials are summed in slice order and scaled, then
// y = (gate / (1 + exp_f(-gate))) * up, the element operations of ACT silu
// then EWMUL. One workgroup per (segment of `seg` columns, row), one thread
// per 4 columns; the segment's power-of-two factor from its own max |y|.
template <int KSN>
__global__ __launch_bounds__(128) void silu_q8_kernel(const float *__restrict__ part, int ks,
                                                      int ldp, const float *__restrict__ sgu,
                                                      int rows, int I, int seg,
                                                      int8_t *__restrict__ q8,
                                                      float *__restrict__ q8s) {
    __shared__ float sh[2];
    const int sgi = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int n4 = seg >> 2;
    const bool live = tid < n4;
    const int jo = sgi * seg + 4 * (live ? tid : n4 - 1);
    const int jg = (jo >> 4) * 32 + (jo & 15), ju = jg + 16;  // gate/up tiles interleave by 16
    float4 gv[KSN], uv[KSN];
#pragma unroll
    for (int k = 0; k < KSN; ++k) {  // the slices there are (a uniform branch)
        gv[k] = uv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < ks) {
            const float *pr = part + ((size_t)k * rows + row) * ldp;
            gv[k] = *(const float4 *)(pr + jg);
            uv[k] = *(const float4 *)(pr + ju);
        }
    }
    const float4 sg = *(const float4 *)(sgu + jg), su = *(const float4 *)(sgu + ju);
    float4 ga = gv[0], ua = uv[0];
#pragma unroll
    for (int k = 1; k < KSN; ++k) {
        if (k < ks) {
            ga.x += gv[k].x, ga.y += gv[k].y, ga.z += gv[k].z, ga.w += gv[k].w;
            ua.x += uv[k].x, ua.y += uv[k].y, ua.z += uv[k].z, ua.w += uv[k].w;
        }
    }
    float y[4];
    const float gs[4] = {ga.x * sg.x, ga.y * sg.y, ga.z * sg.z, ga.w * sg.w};
    const float us[4] = {ua.x * su.x, ua.y * su.y, ua.z * su.z, ua.w * su.w};
    float mx = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        y[q] = (gs[q] / (1.0f + exp_f(-gs[q]))) * us[q];
        mx = fmaxf(mx, q8_mag(y[q]));
    }
    mx = wave_max(live ? mx : 0.0f);
    if ((tid & 63) == 0) sh[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(sh[0], blockDim.x > 64 ? sh[1] : 0.0f);
    const int k = q8_row_k(mx);
    if (tid == 0) q8s[(size_t)sgi * rows + row] = q8_factor(k);
    if (!live) return;
    int a[4][Q8_T];
#pragma unroll
    for (int q = 0; q < 4; ++q) q8_split(y[q], k, a[q]);
#pragma unroll
    for (int t = 0; t < Q8_T; ++t)
        *(uint32_t *)(q8 + ((size_t)t * rows + row) * I + jo) =
            pack_i8x4(a[0][t], a[1][t], a[2][t], a[3][t]);
}

int launch_silu_q8(const float *part, int ks, int ldp, const float *sgu, int rows, int I, int seg,
                   int8_t *q8, float *q8s, hipStream_t st) {
    VMLM_GUARD(I % 16 == 0 && ks >= 1 && ks <= KS_MAX && rows >= 1 && rows <= 65535 &&
                   seg >= 64 && seg <= 512 && seg % 64 == 0 && I % seg == 0 && ldp % 4 == 0 &&
                   ((uintptr_t)part & 15) == 0 && ((uintptr_t)sgu & 15) == 0 &&
                   ((uintptr_t)q8 & 3) == 0 && q8s,
               "silu_q8: I %% seg, segments of 64..512 columns, 1 <= ks <= %d, aligned", KS_MAX);
    const unsigned threads = (unsigned)((seg / 4 + 63) / 64 * 64);
    const dim3 grid((unsigned)(I / seg), (unsigned)rows);
#define SQ_LAUNCH(KSN) \
    silu_q8_kernel<KSN><<<grid, threads, 0, st>>>(part, ks, ldp, sgu, rows, I, seg, q8, q8s)
    if (ks == 9) SQ_LAUNCH(9);
    else if (ks <= 4) SQ_LAUNCH(4);
    else SQ_LAUNCH(16);
#undef SQ_LAUNCH
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Rows as the int8 input of the int8-row GEMM: y = x, or with g the RMSNorm
// y = (x * inv) * g, inv = 1 / sqrt(mean(x^2) + eps) (ops/src/kernels.rs:
// 1346-1368); then Q8_T int8 terms of y with the row's power-of-two factor
// (q8_split), q8s[row] = 2^-k. The terms are written in 1 KiB blocks of 16
// rows x 64 k in MFMA operand order (the layout of launch_rows_q8), so that
// the GEMM copies each block into LDS with one contiguous 16-byte-per-lane
// load. Lane piece p of a row: k-block p / 4, lane group g = p % 4, values
// k = 64 (p / 4) + 8 g + 0..7 and 64 (p / 4) + 32 + 8 g + 0..7; rows past
// the last (to the tile count) hold zero terms.
// At least 2048 rows: rows_q8_wave_kernel (below), one launch. Between 256
// and 2048 rows: two launches. rows_q8_stats_kernel (one workgroup per row) finds
// inv and the factor, rows_q8_terms_kernel (one workgroup per 16 rows x 32
// lane pieces) forms y again with the same operations and writes the terms,
// the 16 threads of a piece index writing 256 contiguous bytes of a block.
// Few rows (RQ_ONE_MAX or fewer): rows_q8_stats_kernel<true> alone, one
// workgroup per row that also writes its row's terms (4 bytes of a lane
// piece per store), which saves the second launch where the grid is small.
// These two give the same bits: the same sums in the same order. The wave
// kernel sums x^2 in another order (a lane's pieces, then across the wave),
// so with a norm its rows can differ from theirs in the last bit of inv;
// without one (the maximum alone) all three give the same bits.
// With ra / rb the rows are first formed as x = ra + rb (a residual add, the
// f32 add of EWADD) and written to x; the terms kernel then reads them there.
// rb may instead be k-slices (rbs.part, row stride cols): each element of rb
// is then the slices summed in order times the column scale, as the slice
// reduction would have written it.
constexpr int RQ_U = 8;  // 4-column groups per thread in the stats kernel (cols <= 8192)
constexpr size_t RQ_ONE_MAX = 256;
template <bool TERMS>
__global__ __launch_bounds__(256) void rows_q8_stats_kernel(
    float *x, int ldx, const float *__restrict__ ra, const float *__restrict__ rb, Slices rbs,
    const float *__restrict__ g, float eps, int cols, int rows, int row_tiles,
    float *__restrict__ inv_out, float *__restrict__ q8s, int8_t *__restrict__ q8) {
    __shared__ float sh[4];
    const int row = blockIdx.x, n4 = cols >> 2;
    // byte offset in a term plane of the terms of columns 4c..4c+3
    auto term_off = [&](int c) {
        const int kk = 4 * c, w = kk & 63;
        return ((size_t)(row >> 4) * (cols >> 6) + (kk >> 6)) * 1024 +
               (size_t)((((w & 31) >> 3) * 16 + (row & 15)) * 16 + (w >> 5) * 8 + (w & 4));
    };
    const size_t plane = (size_t)row_tiles * cols * 16;
    if (TERMS && row >= rows) {  // a row past the last: zero terms
#pragma unroll
        for (int u = 0; u < RQ_U; ++u) {
            const int c = threadIdx.x + u * 256;
            if (c >= n4) continue;
#pragma unroll
            for (int tt = 0; tt < Q8_T; ++tt) *(uint32_t *)(q8 + tt * plane + term_off(c)) = 0u;
        }
        return;
    }
    float4 *xr = (float4 *)(x + (size_t)row * ldx);
    float4 v[RQ_U];
    float ss = 0.0f;
    if (ra) {
        const float4 *ar = (const float4 *)(ra + (size_t)row * ldx);
        const float4 *br = (const float4 *)(rbs.part ? rbs.part + (size_t)row * cols
                                                     : rb + (size_t)row * ldx);
#pragma unroll
        for (int u = 0; u < RQ_U; ++u) {
            const int c = threadIdx.x + u * 256;
            if (c < n4) {
                const float4 a = ar[c];
                float4 b = br[c];
                if (rbs.part) {  // slices in order, then the column scale
                    for (int s = 1; s < rbs.ks; ++s) {
                        const float4 t = br[(size_t)s * (rbs.pst / 4) + c];
                        b = make_float4(b.x + t.x, b.y + t.y, b.z + t.z, b.w + t.w);
                    }
                    const float4 sc = ((const float4 *)rbs.scale)[c];
                    b = make_float4(b.x * sc.x, b.y * sc.y, b.z * sc.z, b.w * sc.w);
                }
                v[u] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                xr[c] = v[u];
            } else {
                v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < RQ_U; ++u) {
            const int c = threadIdx.x + u * 256;
            v[u] = c < n4 ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int u = 0; u < RQ_U; ++u)
        ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
    float inv = 1.0f;
    if (g) {
        ss = block_sum256(ss, sh);
        inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
        for (int u = 0; u < RQ_U; ++u) {
            const int c = threadIdx.x + u * 256;
            if (c >= n4) continue;
            const float4 gg = ((const float4 *)g)[c];
            v[u] = make_float4(v[u].x * inv * gg.x, v[u].y * inv * gg.y, v[u].z * inv * gg.z,
                               v[u].w * inv * gg.w);
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < RQ_U; ++u)
        mx = fmaxf(mx, fmaxf(fmaxf(q8_mag(v[u].x), q8_mag(v[u].y)), fmaxf(q8_mag(v[u].z), q8_mag(v[u].w))));
    mx = block_max256(mx, sh);
    const int k = q8_row_k(mx);
    if (threadIdx.x == 0) {
        q8s[row] = q8_factor(k);
        if (!TERMS) inv_out[row] = inv;
    }
    if constexpr (TERMS) {
#pragma unroll
        for (int u = 0; u < RQ_U; ++u) {
            const int c = threadIdx.x + u * 256;
            if (c >= n4) continue;
            int a[4][Q8_T];
            q8_split(v[u].x, k, a[0]);
            q8_split(v[u].y, k, a[1]);
            q8_split(v[u].z, k, a[2]);
            q8_split(v[u].w, k, a[3]);
            const size_t off = term_off(c);
#pragma unroll
            for (int tt = 0; tt < Q8_T; ++tt)
                *(uint32_t *)(q8 + tt * plane + off) = pack_i8x4(a[0][tt], a[1][tt], a[2][tt], a[3][tt]);
        }
    }
}

constexpr int RQ_J = 32;  // lane pieces per terms workgroup (16 rows each)
__global__ __launch_bounds__(16 * RQ_J) void rows_q8_terms_kernel(
    const float *__restrict__ x, int ldx, const float *__restrict__ g, int cols, int rows,
    int row_tiles, const float *__restrict__ inv_in, const float *__restrict__ q8s,
    int8_t *__restrict__ q8) {
    const int t = threadIdx.x, r = t & 15;
    const int row = (int)blockIdx.x * 16 + r, pc = (int)blockIdx.y * RQ_J + (t >> 4);
    const int npc = cols >> 4, nkb = cols >> 6;
    if (pc >= npc) return;
    const bool live = row < rows;
    const int rowc = live ? row : rows - 1;
    const float *xr = x + (size_t)rowc * ldx;
    const int k0 = (pc >> 2) * 64 + 8 * (pc & 3);
    float v[16];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float4 a = *(const float4 *)(xr + k0 + 32 * h);
        const float4 b = *(const float4 *)(xr + k0 + 32 * h + 4);
        v[8 * h + 0] = a.x, v[8 * h + 1] = a.y, v[8 * h + 2] = a.z, v[8 * h + 3] = a.w;
        v[8 * h + 4] = b.x, v[8 * h + 5] = b.y, v[8 * h + 6] = b.z, v[8 * h + 7] = b.w;
    }
    if (g) {  // the stats kernel's operations: (x * inv) * g
        const float inv = inv_in[rowc];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 ga = *(const float4 *)(g + k0 + 32 * h);
            const float4 gb = *(const float4 *)(g + k0 + 32 * h + 4);
            const float e[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[8 * h + i] = v[8 * h + i] * inv * e[i];
        }
    }
    // the row's k from its factor 2^-k (NaN: a non-finite row)
    const float f = q8s[rowc];
    const int k = f == f ? -ilogbf(f) : Q8_NONFINITE;
    uint32_t w[Q8_T][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int a[4][Q8_T];
#pragma unroll
        for (int e = 0; e < 4; ++e) q8_split(live ? v[4 * q + e] : 0.0f, k, a[e]);
#pragma unroll
        for (int tt = 0; tt < Q8_T; ++tt) w[tt][q] = pack_i8x4(a[0][tt], a[1][tt], a[2][tt], a[3][tt]);
    }
    const size_t plane = (size_t)row_tiles * cols * 16;
    const size_t off = ((size_t)blockIdx.x * nkb + (pc >> 2)) * 1024 + (size_t)((pc & 3) * 16 + r) * 16;
#pragma unroll
    for (int tt = 0; tt < Q8_T; ++tt)
        *(u32x4 *)(q8 + tt * plane + off) = u32x4{w[tt][0], w[tt][1], w[tt][2], w[tt][3]};
}

// One launch for any row count: one wave per row, RW_ROWS rows per
// workgroup. Lane l takes lane pieces l, l + 64, ... of its row (16 values
// each: k-block p / 4, values 64 (p / 4) + 8 (p % 4) + 0..7 and + 32 ..), so
// four adjacent lanes read one 64-column block with 16-byte loads, the row's
// sum of squares and maximum reduce across the wave with DPP (no barrier),
// and each term store is a whole 16-byte piece. The eight rows' pieces of a
// 128-byte line of a block come from one workgroup, so the line is whole in
// one L2 before it is written back (pieces of one line from different
// workgroups, possibly on different XCDs, measured 5 % slower over the
// batch-16 prefill than a second launch that re-reads the rows).
constexpr int RW_ROWS = 8;
template <int P>  // lane pieces per lane: cols <= 1024 * P
__global__ __launch_bounds__(64 * RW_ROWS) void rows_q8_wave_kernel(
    float *x, int ldx, const float *__restrict__ ra, const float *__restrict__ rb, Slices rbs,
    const float *__restrict__ g, float eps, int cols, int rows, int row_tiles,
    float *__restrict__ q8s, int8_t *__restrict__ q8) {
    const int lane = threadIdx.x & 63;
    const int row = (int)blockIdx.x * RW_ROWS + (int)(threadIdx.x >> 6);
    const int npc = cols >> 4, nkb = cols >> 6;
    const size_t plane = (size_t)row_tiles * cols * 16;
    auto piece_off = [&](int pc) {
        return ((size_t)(row >> 4) * nkb + (pc >> 2)) * 1024 +
               (size_t)((pc & 3) * 16 + (row & 15)) * 16;
    };
    if (row >= rows) {  // a row past the last (to the tile count): zero terms
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int pc = lane + 64 * i;
            if (pc >= npc) continue;
#pragma unroll
            for (int tt = 0; tt < Q8_T; ++tt) *(u32x4 *)(q8 + tt * plane + piece_off(pc)) = u32x4{0, 0, 0, 0};
        }
        return;
    }
    float *xr = x + (size_t)row * ldx;
    const float *ar = ra ? ra + (size_t)row * ldx : nullptr;
    const float *br = rbs.part ? rbs.part + (size_t)row * cols : rb ? rb + (size_t)row * ldx : nullptr;
    // piece i: values k0 .. k0 + 7 in v[i][0..1], k0 + 32 .. in v[i][2..3]
    auto kof = [&](int pc, int j) { return (pc >> 2) * 64 + 8 * (pc & 3) + 32 * (j >> 1) + 4 * (j & 1); };
    float4 v[P][4];
    constexpr bool RA = P <= 6;  // registers for both rows
    if (RA && ar && !rbs.part) {
        // the residual add: every load of the row first, then the sums and
        // their stores (a store to x between the loads would make each wait
        // for it: one piece in flight per wave)
        float4 bv[RA ? P : 1][4];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int pc = lane + 64 * i;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                bv[RA ? i : 0][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (pc >= npc) continue;
                const int kk = kof(pc, j);
                v[i][j] = *(const float4 *)(ar + kk);
                bv[RA ? i : 0][j] = *(const float4 *)(br + kk);
            }
        }
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int pc = lane + 64 * i;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (pc >= npc) continue;
                const float4 a = v[i][j], b = bv[RA ? i : 0][j];
                v[i][j] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                *(float4 *)(xr + kof(pc, j)) = v[i][j];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int pc = lane + 64 * i;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (pc >= npc) continue;
                const int kk = kof(pc, j);
                if (ar) {
                    const float4 a = *(const float4 *)(ar + kk);
                    float4 b = *(const float4 *)(br + kk);
                    // slices in order, then the column scale
                    for (int sl = 1; sl < rbs.ks; ++sl) {
                        const float4 t = *(const float4 *)(br + (size_t)sl * rbs.pst + kk);
                        b = make_float4(b.x + t.x, b.y + t.y, b.z + t.z, b.w + t.w);
                    }
                    const float4 sc = *(const float4 *)(rbs.scale + kk);
                    b = make_float4(b.x * sc.x, b.y * sc.y, b.z * sc.z, b.w * sc.w);
                    v[i][j] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                    *(float4 *)(xr + kk) = v[i][j];
                } else {
                    v[i][j] = *(const float4 *)(xr + kk);
                }
            }
        }
    }
    if (g) {
        // the gains issued before the sum is reduced (up to 4 pieces per
        // lane: registers), so they are in by the time they are needed
        constexpr bool HG = P <= 4;
        float4 gv[HG ? P : 1][4];
        if constexpr (HG) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int pc = lane + 64 * i;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    gv[i][j] = pc < npc ? *(const float4 *)(g + kof(pc, j)) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ss += v[i][j].x * v[i][j].x + v[i][j].y * v[i][j].y + v[i][j].z * v[i][j].z +
                      v[i][j].w * v[i][j].w;
        ss = wave_sum_dpp(ss);
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int pc = lane + 64 * i;
            if (pc >= npc) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float4 gg;
                if constexpr (HG) gg = gv[i][j];
                else gg = *(const float4 *)(g + kof(pc, j));
                v[i][j] = make_float4(v[i][j].x * inv * gg.x, v[i][j].y * inv * gg.y,
                                      v[i][j].z * inv * gg.z, v[i][j].w * inv * gg.w);
            }
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            mx = fmaxf(mx, fmaxf(fmaxf(q8_mag(v[i][j].x), q8_mag(v[i][j].y)),
                                 fmaxf(q8_mag(v[i][j].z), q8_mag(v[i][j].w))));
    const int k = q8_row_k(wave_max_nonneg(mx));
    if (lane == 0) q8s[row] = q8_factor(k);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int pc = lane + 64 * i;
        if (pc >= npc) continue;
        uint32_t w[Q8_T][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int a[4][Q8_T];
            q8_split(v[i][j].x, k, a[0]);
            q8_split(v[i][j].y, k, a[1]);
            q8_split(v[i][j].z, k, a[2]);
            q8_split(v[i][j].w, k, a[3]);
#pragma unroll
            for (int tt = 0; tt < Q8_T; ++tt) w[tt][j] = pack_i8x4(a[0][tt], a[1][tt], a[2][tt], a[3][tt]);
        }
        const size_t off = piece_off(pc);
#pragma unroll
        for (int tt = 0; tt < Q8_T; ++tt)
            *(u32x4 *)(q8 + tt * plane + off) = u32x4{w[tt][0], w[tt][1], w[tt][2], w[tt][3]};
    }
}

size_t q8_rows_tiles(size_t rows) { return (rows + 63) / 64 * 4; }
// the term planes, then one float per row (inv of the RMSNorm, kept between
// the two launches)
size_t q8_rows_bytes(size_t rows, size_t cols) {
    return (size_t)Q8_T * q8_rows_tiles(rows) * 16 * cols + q8_rows_tiles(rows) * 16 * sizeof(float);
}

int launch_rows_q8(const float *x, size_t ldx, const float *g, float eps, size_t rows, size_t cols,
                   int8_t *q8, float *q8s, hipStream_t st, const float *ra, const float *rb,
                   const Slices &rbs) {
    if (rows == 0) return VMLM_OK;
    const float *rbx = rbs.part ? rbs.part : rb;
    VMLM_GUARD(!ra == !rbx && (!ra || (((uintptr_t)ra & 15) == 0 && ((uintptr_t)rbx & 15) == 0)),
               "rows_q8: a residual add needs both 16-byte aligned operands");
    VMLM_GUARD(!rbs.part || (ra && rbs.ks >= 1 && rbs.pst % 4 == 0 && rbs.pst >= rows * cols &&
                             rbs.scale && ((uintptr_t)rbs.scale & 15) == 0),
               "rows_q8: k-slices of the added rows need ks >= 1, a slice stride of at least "
               "rows x cols floats (a multiple of 4) and 16-byte aligned column scales");
    VMLM_GUARD(cols % 64 == 0 && cols >= 64 && cols <= 4 * 256 * RQ_U && ldx % 4 == 0 &&
                   ldx >= cols && ((uintptr_t)x & 15) == 0 && (!g || ((uintptr_t)g & 15) == 0) &&
                   ((uintptr_t)q8 & 15) == 0 && q8s && rows <= 0x7fffffff,
               "rows_q8: cols %% 64 == 0, 64 <= cols <= %d, 16-byte aligned rows", 4 * 256 * RQ_U);
    const size_t tiles = q8_rows_tiles(rows);
    // a grid of at least 256 workgroups of eight rows (M >= 2048: the batch-16
    // prefill, 19.73 -> 19.35 ms); with fewer rows a wave per row leaves
    // the CUs idle (the batch-1 prefill, 128 rows: 4.62 -> 5.87 ms)
    if (rows >= (size_t)256 * RW_ROWS) {
        const unsigned grid = (unsigned)(tiles * 16 / RW_ROWS);
#define RW_LAUNCH(PV)                                                                            \
    rows_q8_wave_kernel<PV><<<grid, 64 * RW_ROWS, 0, st>>>((float *)x, (int)ldx, ra, rb, rbs, g,  \
                                                         eps, (int)cols, (int)rows, (int)tiles, \
                                                         q8s, q8)
        if (cols <= 1024 * 3) RW_LAUNCH(3);
        else if (cols <= 1024 * 6) RW_LAUNCH(6);
        else RW_LAUNCH(8);
#undef RW_LAUNCH
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    if (rows <= RQ_ONE_MAX) {
        rows_q8_stats_kernel<true><<<(unsigned)(tiles * 16), 256, 0, st>>>(
            (float *)x, (int)ldx, ra, rb, rbs, g, eps, (int)cols, (int)rows, (int)tiles, nullptr,
            q8s, q8);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    float *inv = (float *)(q8 + (size_t)Q8_T * tiles * 16 * cols);
    rows_q8_stats_kernel<false><<<(unsigned)rows, 256, 0, st>>>(
        (float *)x, (int)ldx, ra, rb, rbs, g, eps, (int)cols, (int)rows, (int)tiles, inv, q8s, q8);
    VMLM_HIP_CHECK(hipGetLastError());
    const dim3 grid((unsigned)((rows + 15) / 16), (unsigned)((cols / 16 + RQ_J - 1) / RQ_J));
    rows_q8_terms_kernel<<<grid, 16 * RQ_J, 0, st>>>(x, (int)ldx, g, (int)cols, (int)rows,
                                                     (int)tiles, inv, q8s, q8);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ops/src/kernels.rs:1388-1414 -- max, exp_f(x-max), sum, * (1/sum), causal tail 0.
__global__ __launch_bounds__(256) void softmax_kernel(float *__restrict__ p, int cols,
                                                      int causal) {
    __shared__ float sh[4];
    const int r = blockIdx.x;
    float *row = p + (size_t)r * cols;
    int lim = causal ? (r + 1 < cols ? r + 1 : cols) : cols;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < lim; i += 256) mx = fmaxf(mx, row[i]);
    mx = block_max256(mx, sh);
    float s = 0.0f;
    for (int i = threadIdx.x; i < lim; i += 256) {
        float e = exp_f(row[i] - mx);
        row[i] = e;
        s += e;
    }
    s = block_sum256(s, sh);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < lim; i += 256) row[i] *= inv;
    for (int i = lim + threadIdx.x; i < cols; i += 256) row[i] = 0.0f;
}

// Rows of at most 64 * SM_R values: one wavefront per row (four rows per
// workgroup), the row read once into registers (lane l holds l, l + 64, ...),
// max and sum reduced across the wave without barriers, written once.
constexpr int SM_R = 16;
__global__ __launch_bounds__(256) void softmax_wave_kernel(float *__restrict__ p, int rows,
                                                           int cols, int causal) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    float *row = p + (size_t)r * cols;
    const int lim = causal ? (r + 1 < cols ? r + 1 : cols) : cols;
    float x[SM_R];
#pragma unroll
    for (int k = 0; k < SM_R; ++k) {
        const int i = lane + 64 * k;
        x[k] = row[i < cols ? i : cols - 1];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SM_R; ++k)
        if (lane + 64 * k < lim) mx = fmaxf(mx, x[k]);
    mx = wave_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < SM_R; ++k) {
        if (lane + 64 * k < lim) {
            x[k] = exp_f(x[k] - mx);
            s += x[k];
        }
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int k = 0; k < SM_R; ++k) {
        const int i = lane + 64 * k;
        if (i < lim) row[i] = x[k] * inv;
        else if (i < cols) row[i] = 0.0f;
    }
}

int launch_softmax(float *p, size_t rows, size_t cols, bool causal, hipStream_t st) {
    if (rows == 0 || cols == 0) return VMLM_OK;
    if (cols <= 64 * SM_R)
        softmax_wave_kernel<<<(unsigned)cdiv(rows, (size_t)4), 256, 0, st>>>(
            p, (int)rows, (int)cols, causal ? 1 : 0);
    else
        softmax_kernel<<<(unsigned)rows, 256, 0, st>>>(p, (int)cols, causal ? 1 : 0);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Element kernels: four elements per thread through float4 loads and stores
// when every pointer is 16-byte aligned (the scalar form otherwise); the tail
// past the last full quad is done element by element. Each element gets the
// reference's operation, so vector and scalar forms agree bit for bit.
static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ops/src/kernels.rs:1144-1167 -- RELU: maxps(v,0) on the 8-wide body
// (returns 0 unless v > 0), `if x < 0 {0}` on the tail; others act_scalar.
__device__ __forceinline__ float act_elem(float x, size_t i, size_t n8, int kind) {
    if (kind == VMLM_ACT_RELU) return i < n8 ? (x > 0.0f ? x : 0.0f) : (x < 0.0f ? 0.0f : x);
    return act_scalar(x, kind);
}
template <bool V4>
__global__ __launch_bounds__(256) void act_kernel(float *__restrict__ d, size_t n, int kind) {
    const size_t n8 = n / 8 * 8;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (V4) {
        const size_t i = 4 * t;
        if (i + 4 <= n) {
            float4 v = *(const float4 *)(d + i);
            v.x = act_elem(v.x, i, n8, kind);
            v.y = act_elem(v.y, i + 1, n8, kind);
            v.z = act_elem(v.z, i + 2, n8, kind);
            v.w = act_elem(v.w, i + 3, n8, kind);
            *(float4 *)(d + i) = v;
        } else {
            for (size_t k = i; k < n; ++k) d[k] = act_elem(d[k], k, n8, kind);
        }
    } else if (t < n) {
        d[t] = act_elem(d[t], t, n8, kind);
    }
}

int launch_act(float *dst, size_t n, int kind, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    if (aligned16(dst))
        act_kernel<true><<<cdiv(cdiv(n, 4), 256), 256, 0, st>>>(dst, n, kind);
    else
        act_kernel<false><<<cdiv(n, 256), 256, 0, st>>>(dst, n, kind);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ops/src/kernels.rs:1115-1142
__device__ __forceinline__ float ew_elem(float a, float b, int op) {
    switch (op) {
    case VMLM_OP_EWADD: return a + b;
    case VMLM_OP_EWMUL: return a * b;
    case VMLM_OP_EWSUB: return a - b;
    default: return a / b;
    }
}
template <bool V4>
__global__ __launch_bounds__(256) void ew_kernel(float *__restrict__ d, const float *__restrict__ x,
                                                 const float *__restrict__ y, size_t n, int op) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (V4) {
        const size_t i = 4 * t;
        if (i + 4 <= n) {
            const float4 a = *(const float4 *)(x + i), b = *(const float4 *)(y + i);
            *(float4 *)(d + i) = make_float4(ew_elem(a.x, b.x, op), ew_elem(a.y, b.y, op),
                                             ew_elem(a.z, b.z, op), ew_elem(a.w, b.w, op));
        } else {
            for (size_t k = i; k < n; ++k) d[k] = ew_elem(x[k], y[k], op);
        }
    } else if (t < n) {
        d[t] = ew_elem(x[t], y[t], op);
    }
}

int launch_ew(float *dst, const float *x, const float *y, size_t n, int op, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    if (aligned16(dst) && aligned16(x) && aligned16(y))
        ew_kernel<true><<<cdiv(cdiv(n, 4), 256), 256, 0, st>>>(dst, x, y, n, op);
    else
        ew_kernel<false><<<cdiv(n, 256), 256, 0, st>>>(dst, x, y, n, op);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// core/src/interp.rs:1225-1235
template <bool V4>
__global__ __launch_bounds__(256) void scale_kernel(float *__restrict__ d,
                                                    const float *__restrict__ s, size_t n,
                                                    float a) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (V4) {
        const size_t i = 4 * t;
        if (i + 4 <= n) {
            const float4 v = *(const float4 *)(s + i);
            *(float4 *)(d + i) = make_float4(v.x * a, v.y * a, v.z * a, v.w * a);
        } else {
            for (size_t k = i; k < n; ++k) d[k] = s[k] * a;
        }
    } else if (t < n) {
        d[t] = s[t] * a;
    }
}

int launch_scale(float *dst, const float *src, size_t n, float s, hipStream_t st) {
    if (n == 0) return VMLM_OK;
    if (aligned16(dst) && aligned16(src))
        scale_kernel<true><<<cdiv(cdiv(n, 4), 256), 256, 0, st>>>(dst, src, n, s);
    else
        scale_kernel<false><<<cdiv(n, 256), 256, 0, st>>>(dst, src, n, s);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Zero fill as a kernel, so that a caller's stream capture records only
// kernel nodes. `head` bytes up to the first 16-byte boundary, `n16` 16-byte
// stores, then `tail` bytes.
__global__ __launch_bounds__(256) void fill_zero_kernel(uint8_t *__restrict__ p, size_t head,
                                                        size_t n16, size_t tail) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 256;
    if (tid < head) p[tid] = 0;
    uint4 *q = (uint4 *)(p + head);
    for (size_t i = tid; i < n16; i += stride) q[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < tail) p[head + 16 * n16 + tid] = 0;
}

int launch_fill_zero(void *ptr, size_t bytes, hipStream_t st) {
    if (bytes == 0) return VMLM_OK;
    uint8_t *p = (uint8_t *)ptr;
    size_t head = (16 - ((uintptr_t)p & 15)) & 15;
    if (head > bytes) head = bytes;
    const size_t n16 = (bytes - head) / 16, tail = bytes - head - 16 * n16;
    size_t blocks = cdiv(n16 > 0 ? n16 : 1, (size_t)256);
    if (blocks > 4096) blocks = 4096;
    fill_zero_kernel<<<(unsigned)blocks, 256, 0, st>>>(p, head, n16, tail);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// core/src/interp.rs:1159-1223 -- one thread per (row, pair).
__global__ void rope_kernel(float *__restrict__ dst, const float *__restrict__ src, int rows,
                            int hd, size_t ld, float step, float pos0, int heads) {
    const int half = hd / 2;
    // rows * heads * half < 2^32 (checked by the launcher): 32-bit index math
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint32_t)rows * (uint32_t)heads * (uint32_t)half) return;
    const uint32_t rh = idx / (uint32_t)half;
    const int i = (int)(idx - rh * (uint32_t)half);
    const int row = (int)(rh / (uint32_t)heads);
    const int h = (int)(rh - (uint32_t)row * (uint32_t)heads);
    const float pos = pos0 + (float)row;
    const float *sr = src + (size_t)row * ld + (size_t)h * hd;
    float *dr = dst + (size_t)row * ld + (size_t)h * hd;
    float y1, y2;
    rope_pair(sr[i], sr[i + half], pos, i, step, &y1, &y2);
    dr[i] = y1;
    dr[i + half] = y2;
}

int launch_rope(float *dst, const float *src, size_t rows, size_t hd, size_t ld, float theta,
                float pos0, int heads, hipStream_t st) {
    VMLM_GUARD(hd >= 2 && (hd & 1) == 0, "ROPE: hd must be even >= 2 (hd=%zu)", hd);
    VMLM_GUARD(theta > 0.0f, "ROPE: theta must be > 0");
    if (rows == 0) return VMLM_OK;
    // step = -2/hd * ln_f(theta), evaluated on the host with the same operations
    float step = -2.0f / (float)hd * host_ln_f(theta);
    size_t n = rows * heads * (hd / 2);
    VMLM_GUARD(n <= 0xFFFFFF00u, "ROPE: rows * heads * hd / 2 = %zu exceeds 2^32 - 256", n);
    rope_kernel<<<cdiv(n, 256), 256, 0, st>>>(dst, src, (int)rows, (int)hd, ld, step, pos0,
                                              heads);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// core/src/interp.rs:1351-1436 -- validate the f32 row index, then widen.
// `rowf` (f32 indices) or `rowi` (int32 ids) per output row.
__global__ void emb_bf16_kernel(float *__restrict__ dst, size_t ldd,
                                const uint16_t *__restrict__ table, size_t rows, int cols,
                                const float *__restrict__ rowf,
                                const int32_t *__restrict__ rowi, int *guard) {
    const int r = blockIdx.x;
    float f = rowf ? rowf[r] : (float)rowi[r];
    bool bad = !(f >= 0.0f) || f >= (float)rows;
    size_t row = 0;
    if (!bad) {
        row = (size_t)f;
        bad = (float)row != f;
    }
    if (bad) {
        if (threadIdx.x == 0) atomicOr(guard, 1);
        return;
    }
    const uint16_t *s = table + row * cols;
    float *d = dst + (size_t)r * ldd;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) d[i] = bf16_bits_to_f32(s[i]);
}

int launch_emb_bf16(float *dst, size_t ldd, const uint16_t *table, size_t rows, size_t cols,
                    const float *rowf, const int32_t *rowi, int n, hipStream_t st, int *guard) {
    if (n == 0) return VMLM_OK;
    emb_bf16_kernel<<<n, 256, 0, st>>>(dst, ldd, table, rows, (int)cols, rowf, rowi,
                                       guard ? guard : guard_flag_ptr());
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// core/src/interp.rs:1649-1681 -- argmax with the scan's semantics: a larger
// value wins, equal values keep the lower index, NaN never wins except that
// a NaN at index 0 blocks every candidate (nothing compares > NaN).
__device__ __forceinline__ void am_merge(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Two launches. The row is split over at most ARGMAX_KEYS / 4 workgroups:
// each thread scans AM_E values per sweep (loads issued together, index
// clamped), the wave reduces (value, index) pairs with the strict-`>` /
// lowest-index rule and writes its order-preserving 64-bit key (0: no
// candidate) to keys[wave]. One workgroup then takes the largest key (a max,
// so the order of the waves does not matter) and turns it into the index.
constexpr int AM_E = 8;

__global__ __launch_bounds__(256) void argmax_keys_kernel(const float *__restrict__ src, int cols,
                                                          unsigned long long *__restrict__ keys) {
    const int stride = gridDim.x * 256;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i0 = blockIdx.x * 256 + threadIdx.x; i0 < cols; i0 += AM_E * stride) {
        float v[AM_E];
#pragma unroll
        for (int e = 0; e < AM_E; ++e) {
            const int i = i0 + e * stride;
            v[e] = src[i < cols ? i : cols - 1];
        }
#pragma unroll
        for (int e = 0; e < AM_E; ++e) {
            const int i = i0 + e * stride;
            if (i < cols && v[e] == v[e]) am_merge(bv, bi, v[e], i);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        am_merge(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0)
        keys[blockIdx.x * 4 + (threadIdx.x >> 6)] =
            bi != 0x7fffffff ? argmax_key(bv, (uint32_t)bi) : 0ull;
}

__global__ __launch_bounds__(256) void argmax_final_kernel(
    const float *__restrict__ src, const unsigned long long *__restrict__ keys, int nkeys,
    float *dst_f, int32_t *dst_i) {
    __shared__ unsigned long long sk[4];
    unsigned long long k = 0ull;
    for (int i = threadIdx.x; i < nkeys; i += 256) k = keys[i] > k ? keys[i] : k;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long ok = __shfl_xor(k, o, 64);
        k = ok > k ? ok : k;
    }
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < 4; ++w) k = sk[w] > k ? sk[w] : k;
    const float x0 = src[0];
    const int bi = (x0 != x0 || k == 0ull) ? 0 : argmax_key_index(k);  // NaN at 0, or all NaN
    if (dst_f) dst_f[0] = (float)bi;
    if (dst_i) dst_i[0] = bi;
}

int launch_argmax(const float *src, size_t cols, float *dst_f, int32_t *dst_i,
                  unsigned long long *keys, hipStream_t st) {
    VMLM_GUARD(cols >= 1 && cols <= 0x7f000000u, "TOPK_IDX: %zu values", cols);
    const size_t want = (size_t)cdiv(cols, (size_t)256 * AM_E);
    const unsigned nwg = (unsigned)(want < ARGMAX_KEYS / 4 ? want : ARGMAX_KEYS / 4);
    argmax_keys_kernel<<<nwg, 256, 0, st>>>(src, (int)cols, keys);
    argmax_final_kernel<<<1, 256, 0, st>>>(src, keys, (int)nwg * 4, dst_f, dst_i);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

// k_gemv.hip -- weight-streaming GEMV for decode (M <= 16 rows of activations).
//
// Replaces gemm_nt_int8 (ops/src/kernels.rs:1256-1287) and gemm_nt_bf16
// (:1199-1227) on the decode path, where every weight byte is read once per
// step and the kernel is bound by HBM bandwidth.
//
// Design (gfx950):
//  * One workgroup = 8 wavefronts on one 16-row output tile (or a pair of
//    tiles); the waves split K and meet in LDS, so every weight row is one
//    contiguous stream of 16-byte loads per lane (a wave reads 16 rows x
//    64 B per load instruction).
//  * The dot products run on v_mfma_f32_16x16x32_bf16. int8 weights convert
//    to bf16 exactly (|q| <= 127 needs 8 significant bits); the f32
//    activations arrive pre-split into T bf16 terms (hi+mid+lo), each an
//    exact product with the weight, accumulated in f32 by the MFMA. Batch
//    rows are the MFMA's A rows, so M = 1..16 costs the same weight traffic.
//  * Epilogues fuse the scale multiply and the adjacent elementwise ops of
//    the VM program (EWADD residual; ACT silu + EWMUL with the up
//    projection) with the same per-element operation order as the
//    reference's separate kernels.
#include "internal.hpp"

namespace vmlm {

struct GemvParams {
    const uint8_t *W;
    const float *scale;
    const uint16_t *A;
    float *Y;
    const float *Rr;
    uint16_t *Aout;
    size_t tstride;
    int lda, M, N, K, ldy, ldr, ldaout, Tout, epi;
};

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 ldg16(const void *p) {
    return __builtin_nontemporal_load((const u32x4 *)p);
}
__device__ __forceinline__ u32x4 ldg16_cached(const void *p) { return *(const u32x4 *)p; }

constexpr int GEMV_NW = 8;  // wavefronts per workgroup (split of K)
constexpr int GEMV_U = 4;   // 64-wide K steps in flight per wave

template <bool WI8, int T, int R>
__global__ __launch_bounds__(GEMV_NW * 64) void gemv_kernel(GemvParams p) {
    __shared__ f32x4 red[GEMV_NW][R][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, rr = lane & 15;
    const int S = p.K >> 6;
    const int s0 = (S * wave) / GEMV_NW, s1 = (S * (wave + 1)) / GEMV_NW;
    constexpr int WB = WI8 ? 64 : 128;  // weight bytes per 64-wide K step and row
    constexpr int WL = WI8 ? 1 : 2;     // 16-byte loads per lane per step

    const uint8_t *wrow[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
        int j = (blockIdx.x * R + t) * 16 + rr;
        j = j < p.N ? j : p.N - 1;
        wrow[t] = p.W + (size_t)j * p.K * (WI8 ? 1 : 2) + g * (WB / 4);
    }
    const bool arow = rr < p.M;
    const uint16_t *abase = p.A + (size_t)(arow ? rr : 0) * p.lda + g * 16;
    const size_t tstride = p.tstride;

    f32x4 acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto step = [&](const u32x4 (&wv)[R][WL], const u32x4 (&av)[T][2]) {
#pragma unroll
        for (int t = 0; t < R; ++t) {
            u32x4 b0, b1;
            if constexpr (WI8) {
                i8x16_to_bf16(wv[t][0], b0, b1);
            } else {
                b0 = wv[t][0];
                b1 = wv[t][1];
            }
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                acc[t] = mfma_bf16(av[tt][0], b0, acc[t]);
                acc[t] = mfma_bf16(av[tt][1], b1, acc[t]);
            }
        }
    };

    int s = s0;
    for (; s + GEMV_U <= s1; s += GEMV_U) {
        u32x4 wv[GEMV_U][R][WL];
        u32x4 av[GEMV_U][T][2];
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u)
#pragma unroll
            for (int t = 0; t < R; ++t)
#pragma unroll
                for (int l = 0; l < WL; ++l)
                    wv[u][t][l] = ldg16(wrow[t] + (size_t)(s + u) * WB + l * 16);
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u)
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                if (arow) {
                    const uint16_t *ap = abase + tt * tstride + (size_t)(s + u) * 64;
                    av[u][tt][0] = ldg16_cached(ap);
                    av[u][tt][1] = ldg16_cached(ap + 8);
                } else {
                    av[u][tt][0] = u32x4{0u, 0u, 0u, 0u};
                    av[u][tt][1] = u32x4{0u, 0u, 0u, 0u};
                }
            }
#pragma unroll
        for (int u = 0; u < GEMV_U; ++u) step(wv[u], av[u]);
    }
    for (; s < s1; ++s) {
        u32x4 wv[R][WL];
        u32x4 av[T][2];
#pragma unroll
        for (int t = 0; t < R; ++t)
#pragma unroll
            for (int l = 0; l < WL; ++l) wv[t][l] = ldg16(wrow[t] + (size_t)s * WB + l * 16);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            if (arow) {
                const uint16_t *ap = abase + tt * tstride + (size_t)s * 64;
                av[tt][0] = ldg16_cached(ap);
                av[tt][1] = ldg16_cached(ap + 8);
            } else {
                av[tt][0] = u32x4{0u, 0u, 0u, 0u};
                av[tt][1] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        step(wv, av);
    }

#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave != 0) return;
    f32x4 v[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
        v[t] = red[0][t][lane];
        for (int w = 1; w < GEMV_NW; ++w) v[t] += red[w][t][lane];
    }

    if (p.epi == EPI_SILU_MUL) {
        // tile 0 = gate rows, tile 1 = up rows of the same 16 output columns
        const int jg = blockIdx.x * 32 + rr, ju = jg + 16;
        const int jo = blockIdx.x * 16 + rr;
        const float sg = p.scale[jg], su = p.scale[ju];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = g * 4 + i;
            if (b >= p.M) break;
            float gate = v[0][i] * sg;
            float up = v[R - 1][i] * su;
            float a = (gate / (1.0f + exp_f(-gate))) * up;
            p.Y[(size_t)b * p.ldy + jo] = a;
            float r = a;
            for (int tt = 0; tt < p.Tout; ++tt) {
                uint32_t h = bf16_rne_bits(r);
                r = r - bf16_bits_to_f32(h);
                p.Aout[((size_t)tt * p.M + b) * p.ldaout + jo] = (uint16_t)h;
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int j = (blockIdx.x * R + t) * 16 + rr;
        if (j >= p.N) continue;
        const float sc = p.scale ? p.scale[j] : 1.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = g * 4 + i;
            if (b >= p.M) break;
            float y = p.scale ? v[t][i] * sc : v[t][i];
            if (p.epi == EPI_RESIDUAL) y = p.Rr[(size_t)b * p.ldr + j] + y;
            p.Y[(size_t)b * p.ldy + j] = y;
        }
    }
}

__global__ void split_terms_kernel(const float *__restrict__ x, size_t ldx, int rows, int K,
                                   int ldo, int T, uint16_t *__restrict__ out) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)rows * ldo;
    if (idx >= total) return;
    int r = (int)(idx / ldo), k = (int)(idx % ldo);
    float v = k < K ? x[(size_t)r * ldx + k] : 0.0f;
    for (int t = 0; t < T; ++t) {
        uint32_t h = bf16_rne_bits(v);
        v = v - bf16_bits_to_f32(h);
        out[((size_t)t * rows + r) * ldo + k] = (uint16_t)h;
    }
}

int launch_split_terms(const float *x, size_t ldx, int rows, int K, int T, uint16_t *out,
                       int ld_out, hipStream_t st) {
    if (rows <= 0) return VMLM_OK;
    size_t total = (size_t)rows * ld_out;
    split_terms_kernel<<<cdiv(total, 256), 256, 0, st>>>(x, ldx, rows, K, ld_out, T, out);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

template <bool WI8, int T, int R>
static int launch_t(const GemvParams &p, hipStream_t st) {
    int tiles = (p.N + 16 * R - 1) / (16 * R);
    if (p.epi == EPI_SILU_MUL) tiles = p.N / 32;
    gemv_kernel<WI8, T, R><<<tiles, GEMV_NW * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

template <bool WI8, int R>
static int launch_r(const GemvParams &p, int T, hipStream_t st) {
    switch (T) {
    case 1: return launch_t<WI8, 1, R>(p, st);
    case 2: return launch_t<WI8, 2, R>(p, st);
    case 3: return launch_t<WI8, 3, R>(p, st);
    default: return fail(VMLM_ERR_UNIMPL, "gemv: %d activation terms unsupported", T);
    }
}

int launch_gemv(const GemvArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.M <= 16, "gemv: M=%d outside 1..16", a.M);
    VMLM_GUARD(a.K > 0 && a.K % 64 == 0, "gemv: K=%d not a positive multiple of 64", a.K);
    VMLM_GUARD(a.N > 0, "gemv: N=%d", a.N);
    VMLM_GUARD(((uintptr_t)a.W & 15) == 0 && ((uintptr_t)a.A & 15) == 0 && a.lda % 64 == 0,
               "gemv: operands must be 16-byte aligned with lda %% 64 == 0");
    GemvParams p;
    p.W = (const uint8_t *)a.W;
    p.scale = a.scale;
    p.A = a.A;
    p.Y = a.Y;
    p.Rr = a.R;
    p.Aout = a.Aout;
    p.lda = a.lda;
    p.tstride = a.a_tstride ? a.a_tstride : (size_t)a.M * a.lda;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    p.ldy = a.ldy;
    p.ldr = a.ldr;
    p.ldaout = a.ldaout;
    p.Tout = a.Tout;
    p.epi = a.epi;
    if (a.epi == EPI_SILU_MUL) {
        VMLM_GUARD(a.N % 32 == 0 && a.scale && a.Aout, "gemv silu: N %% 32, scale, Aout");
        return a.w_int8 ? launch_r<true, 2>(p, a.T, st) : launch_r<false, 2>(p, a.T, st);
    }
    return a.w_int8 ? launch_r<true, 1>(p, a.T, st) : launch_r<false, 1>(p, a.T, st);
}

}  // namespace vmlm

// k_gemv.hip -- weight-streaming GEMV for decode (M <= 16 rows of activations).
//
// Replaces gemm_nt_int8 (ops/src/kernels.rs:1256-1287) and gemm_nt_bf16
// (:1199-1227) on the decode path, where every weight byte is read once per
// step and the kernel is bound by HBM bandwidth.
//
// Design (gfx950):
//  * One workgroup = 8 wavefronts on one 16-row output tile (or a gate/up
//    pair of tiles). The waves split K; each wave issues ALL of its weight
//    loads (16 bytes per lane per 64-wide K step, a wave reading 16 rows x
//    64 B per instruction) before it consumes any, so a launch costs one HBM
//    round trip plus streaming time; the waves meet in LDS.
//  * The dot products run on v_mfma_f32_16x16x32_bf16. int8 weights convert
//    to bf16 exactly (|q| <= 127 needs 8 significant bits); the f32
//    activations arrive pre-split into T bf16 terms (hi+mid+lo, split_bf16),
//    each an exact product with the weight, accumulated in f32 by the MFMA.
//    With T*M <= 16 the (term, batch) pairs are the MFMA's A rows (one A
//    fragment per step, the terms summed in the epilogue); otherwise the
//    batch rows are the A rows and each term is a separate MFMA.
//  * Epilogues fuse the scale multiply and the adjacent elementwise ops of
//    the VM program (EWADD residual; ACT silu + EWMUL with the up
//    projection; TOPK_IDX argmax after the LM head) with the reference's
//    per-element operation order.
#include "internal.hpp"

namespace vmlm {

struct GemvParams {
    const uint8_t *W;
    const float *scale;
    const uint16_t *A;
    float *Y;
    const float *Rr;
    uint16_t *Aout;
    unsigned long long *keys;
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

constexpr int GEMV_NW = 8;     // wavefronts per workgroup (split of K)
constexpr int GEMV_MAXS = 12;  // 64-wide K steps per wave per pass (all loads in flight)

template <bool WI8, int T, int R, bool BT>
__global__ __launch_bounds__(GEMV_NW * 64) void gemv_kernel(GemvParams p) {
    constexpr int TA = BT ? 1 : T;  // A fragment sets per 32-wide half step
    constexpr int WB = WI8 ? 64 : 128;  // weight bytes per 64-wide K step and row
    constexpr int WL = WI8 ? 1 : 2;     // 16-byte loads per lane per step
    __shared__ f32x4 red[GEMV_NW][R][64];
    __shared__ float ys[R][16][17];
    __shared__ float ssc[R][16];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, rr = lane & 15;
    const int S = p.K >> 6;
    const int arows = BT ? T * p.M : p.M;
    const bool arow = rr < arows;
    const uint16_t *abase = p.A + (size_t)(arow ? rr : 0) * p.lda + g * 16;

    const uint8_t *wrow[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
        int j = (blockIdx.x * R + t) * 16 + rr;
        j = j < p.N ? j : p.N - 1;
        wrow[t] = p.W + (size_t)j * p.K * (WI8 ? 1 : 2) + g * (WB / 4);
    }
    if (tid < R * 16) {  // scales for the epilogue, fetched while the weights stream
        const int t = tid >> 4, c = tid & 15;
        int j = (blockIdx.x * R + t) * 16 + c;
        j = j < p.N ? j : p.N - 1;
        ssc[t][c] = p.scale ? p.scale[j] : 1.0f;
    }

    f32x4 acc[R];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int base = 0; base < S; base += GEMV_NW * GEMV_MAXS) {
        const int Sp = (S - base) < GEMV_NW * GEMV_MAXS ? (S - base) : GEMV_NW * GEMV_MAXS;
        const int s0 = base + (Sp * wave) / GEMV_NW;
        const int n = base + (Sp * (wave + 1)) / GEMV_NW - s0;
        u32x4 wv[GEMV_MAXS][R][WL];
#pragma unroll
        for (int i = 0; i < GEMV_MAXS; ++i)
            if (i < n) {
#pragma unroll
                for (int t = 0; t < R; ++t)
#pragma unroll
                    for (int l = 0; l < WL; ++l)
                        wv[i][t][l] = ldg16(wrow[t] + (size_t)(s0 + i) * WB + l * 16);
            }
        u32x4 av[3][TA][2];
        auto load_a = [&](int i, u32x4 (&dst)[TA][2]) {
#pragma unroll
            for (int tt = 0; tt < TA; ++tt) {
                if (arow) {
                    const uint16_t *ap = abase + (BT ? 0 : tt * p.tstride) + (size_t)(s0 + i) * 64;
                    dst[tt][0] = ldg16_cached(ap);
                    dst[tt][1] = ldg16_cached(ap + 8);
                } else {
                    dst[tt][0] = u32x4{0u, 0u, 0u, 0u};
                    dst[tt][1] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        };
        if (n > 0) load_a(0, av[0]);
        if (n > 1) load_a(1, av[1]);
#pragma unroll
        for (int i = 0; i < GEMV_MAXS; ++i) {
            if (i < n) {
                if (i + 2 < n) load_a(i + 2, av[(i + 2) % 3]);
#pragma unroll
                for (int t = 0; t < R; ++t) {
                    u32x4 b0, b1;
                    if constexpr (WI8) {
                        i8x16_to_bf16(wv[i][t][0], b0, b1);
                    } else {
                        b0 = wv[i][t][0];
                        b1 = wv[i][t][1];
                    }
#pragma unroll
                    for (int tt = 0; tt < TA; ++tt) {
                        acc[t] = mfma_bf16(av[i % 3][tt][0], b0, acc[t]);
                        acc[t] = mfma_bf16(av[i % 3][tt][1], b1, acc[t]);
                    }
                }
            }
        }
    }

    // ---- cross-wave reduction: D[row = 4g+i][col = rr] of each tile
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    for (int e = tid; e < R * 256; e += GEMV_NW * 64) {
        const int t = e >> 8, row = (e >> 4) & 15, col = e & 15;
        const int ln = (row >> 2) * 16 + col, i = row & 3;
        float v = red[0][t][ln][i];
        for (int w = 1; w < GEMV_NW; ++w) v += red[w][t][ln][i];
        ys[t][row][col] = v;
    }
    __syncthreads();

    // ---- epilogue over (tile, batch row, column)
    auto rowval = [&](int t, int b, int col) {
        if constexpr (BT) {
            float v = ys[t][b][col];
#pragma unroll
            for (int tt = 1; tt < T; ++tt) v += ys[t][tt * p.M + b][col];
            return v;
        } else {
            return ys[t][b][col];
        }
    };
    if (p.epi == EPI_SILU_MUL) {  // tile 0 = gate rows, tile 1 = up rows
        for (int e = tid; e < p.M * 16; e += GEMV_NW * 64) {
            const int b = e >> 4, col = e & 15;
            const int jo = blockIdx.x * 16 + col;
            const float gate = rowval(0, b, col) * ssc[0][col];
            const float up = rowval(R - 1, b, col) * ssc[R - 1][col];
            float a = (gate / (1.0f + exp_f(-gate))) * up;
            p.Y[(size_t)b * p.ldy + jo] = a;
            for (int tt = 0; tt < p.Tout; ++tt) {
                const uint32_t h = bf16_rne_bits(a);
                a = a - bf16_bits_to_f32(h);
                p.Aout[((size_t)tt * p.M + b) * p.ldaout + jo] = (uint16_t)h;
            }
        }
        return;
    }
    for (int e = tid; e < R * p.M * 16; e += GEMV_NW * 64) {
        const int t = e / (p.M * 16), b = (e >> 4) % p.M, col = e & 15;
        const int j = (blockIdx.x * R + t) * 16 + col;
        float y = 0.0f;
        const bool in = j < p.N;
        if (in) {
            y = p.scale ? rowval(t, b, col) * ssc[t][col] : rowval(t, b, col);
            if (p.epi == EPI_RESIDUAL) y = p.Rr[(size_t)b * p.ldr + j] + y;
            p.Y[(size_t)b * p.ldy + j] = y;
        }
        if (p.epi == EPI_ARGMAX) {
            // 16 consecutive threads hold the 16 columns of row b: reduce keys
            unsigned long long k = 0;
            if (in && y == y) k = argmax_key(y, (uint32_t)j);
            if (in && j == 0 && y != y) k = ARGMAX_NAN0_KEY;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                unsigned long long ok = __shfl_xor(k, o, 64);
                k = ok > k ? ok : k;
            }
            if (col == 0 && k) atomicMax(p.keys + (size_t)b * KEY_SLOTS + (blockIdx.x & (KEY_SLOTS - 1)), k);
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

template <bool WI8, int T, int R, bool BT>
static int launch_t(const GemvParams &p, hipStream_t st) {
    int tiles = (p.N + 16 * R - 1) / (16 * R);
    if (p.epi == EPI_SILU_MUL) tiles = p.N / 32;
    gemv_kernel<WI8, T, R, BT><<<tiles, GEMV_NW * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

template <bool WI8, int R>
static int launch_r(const GemvParams &p, int T, bool bt, hipStream_t st) {
    switch (T) {
    case 1: return launch_t<WI8, 1, R, false>(p, st);
    case 2: return bt ? launch_t<WI8, 2, R, true>(p, st) : launch_t<WI8, 2, R, false>(p, st);
    case 3: return bt ? launch_t<WI8, 3, R, true>(p, st) : launch_t<WI8, 3, R, false>(p, st);
    default: return fail(VMLM_ERR_UNIMPL, "gemv: %d activation terms unsupported", T);
    }
}

int launch_gemv(const GemvArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.M <= 16, "gemv: M=%d outside 1..16", a.M);
    VMLM_GUARD(a.K > 0 && a.K % 64 == 0, "gemv: K=%d not a positive multiple of 64", a.K);
    VMLM_GUARD(a.N > 0, "gemv: N=%d", a.N);
    VMLM_GUARD(((uintptr_t)a.W & 15) == 0 && ((uintptr_t)a.A & 15) == 0 && a.lda % 64 == 0,
               "gemv: operands must be 16-byte aligned with lda %% 64 == 0");
    VMLM_GUARD(a.epi != EPI_ARGMAX || a.keys, "gemv argmax: keys buffer required");
    GemvParams p;
    p.W = (const uint8_t *)a.W;
    p.scale = a.scale;
    p.A = a.A;
    p.Y = a.Y;
    p.Rr = a.R;
    p.Aout = a.Aout;
    p.keys = a.keys;
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
    // (term, batch) rows need the planes contiguous: row r = buffer row r
    const bool bt = a.T > 1 && a.T * a.M <= 16 && p.tstride == (size_t)a.M * a.lda;
    if (a.epi == EPI_SILU_MUL) {
        VMLM_GUARD(a.N % 32 == 0 && a.scale && a.Aout && a.w_int8,
                   "gemv silu: int8 weights, N %% 32, scale, Aout");
        return launch_r<true, 2>(p, a.T, bt, st);
    }
    return a.w_int8 ? launch_r<true, 1>(p, a.T, bt, st) : launch_r<false, 1>(p, a.T, bt, st);
}

}  // namespace vmlm

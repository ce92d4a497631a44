// k_gemm.hip -- LDS-tiled MFMA GEMM for M > 16 (prefill, dense bf16 shape).
//
// C[M,N] = A[M,K] . W[N,K]^T (* scale[n]) with W int8 (converted exactly to
// bf16 when staged into LDS) or bf16, and A given as T bf16 term planes
// (T = 1 for bf16 activations, 3 for f32 activations; see split_bf16).
// Replaces gemm_nt_int8 / gemm_nt_bf16 (ops/src/kernels.rs:1199-1287) for
// multi-row activations; f32 accumulation in the MFMA, order differs from the
// reference's 8-lane FMA chains (E contract).
//
// Tile BM x BN x 64 per workgroup of 4 wavefronts (2 x 2), each wavefront
// (BM/2) x (BN/2) as 16x16 v_mfma_f32_16x16x32_bf16 sub-tiles. The next K
// tile is prefetched into registers while the current one is consumed.
#include "internal.hpp"

namespace vmlm {

struct GemmParams {
    const uint8_t *W;
    const float *scale;
    const uint16_t *A;
    float *C;
    size_t tstride;
    int lda, M, N, K, ldc;
};

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

constexpr int G_BK = 64;
constexpr int G_LDK = G_BK + 8;  // padded LDS row (bf16 elements)

template <bool WI8, int T, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;     // per-wave tile
    constexpr int TM = WM / 16, TN = WN / 16;   // MFMA sub-tiles per wave
    __shared__ uint16_t As[T][BM][G_LDK];
    __shared__ uint16_t Bs[BN][G_LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r = lane & 15;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // global -> register staging: A: T*BM rows x 64 bf16 (8 chunks of 16 B per row)
    constexpr int A_CHUNKS = T * BM * 8;
    constexpr int A_PER = (A_CHUNKS + 255) / 256;
    constexpr int B_CHUNKS = WI8 ? BN * 4 : BN * 8;  // 16-byte chunks per K tile
    constexpr int B_PER = (B_CHUNKS + 255) / 256;
    u32x4 ra[A_PER], rb[B_PER];

    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            int c = tid + i * 256;
            if (c < A_CHUNKS) {
                int t = c / (BM * 8), rem = c % (BM * 8);
                int row = rem / 8, ch = rem % 8;
                int gm = m0 + row;
                gm = gm < p.M ? gm : p.M - 1;
                ra[i] = *(const u32x4 *)(p.A + t * p.tstride + (size_t)gm * p.lda + k0 + ch * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            int c = tid + i * 256;
            if (c < B_CHUNKS) {
                constexpr int CPR = WI8 ? 4 : 8;  // chunks per row
                int row = c / CPR, ch = c % CPR;
                int gn = n0 + row;
                gn = gn < p.N ? gn : p.N - 1;
                const uint8_t *src = p.W + ((size_t)gn * p.K + k0) * (WI8 ? 1 : 2) + ch * 16;
                rb[i] = __builtin_nontemporal_load((const u32x4 *)src);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            int c = tid + i * 256;
            if (c < A_CHUNKS) {
                int t = c / (BM * 8), rem = c % (BM * 8);
                int row = rem / 8, ch = rem % 8;
                *(u32x4 *)&As[t][row][ch * 8] = ra[i];
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            int c = tid + i * 256;
            if (c < B_CHUNKS) {
                if constexpr (WI8) {
                    int row = c / 4, ch = c % 4;
                    u32x4 lo, hi;
                    i8x16_to_bf16(rb[i], lo, hi);
                    *(u32x4 *)&Bs[row][ch * 16] = lo;
                    *(u32x4 *)&Bs[row][ch * 16 + 8] = hi;
                } else {
                    int row = c / 8, ch = c % 8;
                    *(u32x4 *)&Bs[row][ch * 8] = rb[i];
                }
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = p.K / G_BK;
    load_tile(0);
    for (int kt = 0; kt < nk; ++kt) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (kt + 1 < nk) load_tile((kt + 1) * G_BK);
#pragma unroll
        for (int ks = 0; ks < G_BK / 32; ++ks) {
            u32x4 bf[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *(const u32x4 *)&Bs[wn * WN + j * 16 + r][ks * 32 + g * 8];
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    u32x4 af = *(const u32x4 *)&As[t][wm * WM + i * 16 + r][ks * 32 + g * 8];
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af, bf[j], acc[i][j]);
                }
            }
        }
    }

    // D layout: lane (g, r) holds rows 4g..4g+3 of the A sub-tile, column r
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 16 + r;
            if (col >= p.N) continue;
            const float sc = p.scale ? p.scale[col] : 1.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = m0 + wm * WM + i * 16 + g * 4 + q;
                if (row < p.M) {
                    float v = acc[i][j][q];
                    p.C[(size_t)row * p.ldc + col] = p.scale ? v * sc : v;
                }
            }
        }
}

template <bool WI8, int T>
static int launch_g(const GemmParams &p, hipStream_t st) {
    constexpr int BM = 64, BN = 64;
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
    gemm_kernel<WI8, T, BM, BN><<<grid, 256, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_gemm(const GemmArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.N >= 1, "gemm: empty shape");
    VMLM_GUARD(a.K > 0 && a.K % 64 == 0, "gemm: K=%d not a positive multiple of 64", a.K);
    VMLM_GUARD(((uintptr_t)a.W & 15) == 0 && ((uintptr_t)a.A & 15) == 0 && a.lda % 8 == 0,
               "gemm: operands must be 16-byte aligned");
    GemmParams p;
    p.W = (const uint8_t *)a.W;
    p.scale = a.scale;
    p.A = a.A;
    p.C = a.C;
    p.tstride = (size_t)a.M * a.lda;
    p.lda = a.lda;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    p.ldc = a.ldc;
    if (a.w_int8) {
        switch (a.T) {
        case 1: return launch_g<true, 1>(p, st);
        case 2: return launch_g<true, 2>(p, st);
        case 3: return launch_g<true, 3>(p, st);
        }
    } else {
        switch (a.T) {
        case 1: return launch_g<false, 1>(p, st);
        case 2: return launch_g<false, 2>(p, st);
        case 3: return launch_g<false, 3>(p, st);
        }
    }
    return fail(VMLM_ERR_UNIMPL, "gemm: %d activation terms unsupported", a.T);
}

}  // namespace vmlm

// k_gemm.hip -- LDS-tiled MFMA GEMM for M > 16 (prefill, dense bf16 shape).
//
// C[M,N] = A[M,K] . W[N,K]^T (* scale[n]) with W int8 (converted exactly to
// bf16 when staged into LDS) or bf16, and A given as T bf16 term planes
// (T = 1 for bf16 activations, 3 for f32 activations; see split_bf16).
// Replaces gemm_nt_int8 / gemm_nt_bf16 (ops/src/kernels.rs:1199-1287) for
// multi-row activations; f32 accumulation in the MFMA, order differs from the
// reference's 8-lane FMA chains (E contract).
//
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

// Workgroup tile BM x BN (A rows x W rows) x 64 k, 4 wavefronts as 2 x 2,
// each (BM/2) x (BN/2) of 16x16 MFMA blocks. Per k-step every thread loads
// its share of the next tile into registers (unconditionally: rows clamped,
// the last step reloads itself) while the current tile is consumed from LDS.
template <bool WI8, int T, int BM, int BN>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;    // per-wave tile
    constexpr int TM = WM / 16, TN = WN / 16;  // MFMA blocks per wave
    __shared__ __attribute__((aligned(16))) uint16_t As[T][BM][G_LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN][G_LDK];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r = lane & 15;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // 16-byte pieces per k-step: A: T*BM rows x 8; W: BN rows x 4 (int8) or 8
    constexpr int A_CHUNKS = T * BM * 8;
    static_assert(A_CHUNKS % 256 == 0, "A tile pieces per thread");
    constexpr int A_PER = A_CHUNKS / 256;
    constexpr int CPR = WI8 ? 4 : 8;
    constexpr int B_CHUNKS = BN * CPR;
    static_assert(B_CHUNKS % 256 == 0, "W tile pieces per thread");
    constexpr int B_PER = B_CHUNKS / 256;
    const uint16_t *asrc[A_PER];
    const uint8_t *bsrc[B_PER];
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
        const int c = tid + i * 256, t = c / (BM * 8), rem = c % (BM * 8);
        int gm = m0 + rem / 8;
        gm = gm < p.M ? gm : p.M - 1;
        asrc[i] = p.A + t * p.tstride + (size_t)gm * p.lda + (rem % 8) * 8;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
        const int c = tid + i * 256;
        int gn = n0 + c / CPR;
        gn = gn < p.N ? gn : p.N - 1;
        bsrc[i] = p.W + (size_t)gn * p.K * (WI8 ? 1 : 2) + (c % CPR) * 16;
    }
    u32x4 ra[A_PER], rb[B_PER];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) ra[i] = *(const u32x4 *)(asrc[i] + k0);
#pragma unroll
        for (int i = 0; i < B_PER; ++i)
            rb[i] = __builtin_nontemporal_load((const u32x4 *)(bsrc[i] + (size_t)k0 * (WI8 ? 1 : 2)));
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * 256, t = c / (BM * 8), rem = c % (BM * 8);
            *(u32x4 *)&As[t][rem / 8][(rem % 8) * 8] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * 256;
            if constexpr (WI8) {
                u32x4 lo, hi;
                i8x16_to_bf16(rb[i], lo, hi);
                *(u32x4 *)&Bs[c / 4][(c % 4) * 16] = lo;
                *(u32x4 *)&Bs[c / 4][(c % 4) * 16 + 8] = hi;
            } else {
                *(u32x4 *)&Bs[c / 8][(c % 8) * 8] = rb[i];
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
        load_tile((kt + 1 < nk ? kt + 1 : kt) * G_BK);
        __builtin_amdgcn_sched_barrier(0);  // the next tile's loads go out before the MFMAs
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
                    const u32x4 af = *(const u32x4 *)&As[t][wm * WM + i * 16 + r][ks * 32 + g * 8];
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af, bf[j], acc[i][j]);
                }
            }
        }
    }

    // D layout: lane (g, r) holds rows 4g..4g+3 of the A block, column r
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 16 + r;
        if (col >= p.N) continue;
        const float sc = p.scale ? p.scale[col] : 1.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = m0 + wm * WM + i * 16 + g * 4 + q;
                if (row < p.M) {
                    const float v = acc[i][j][q];
                    p.C[(size_t)row * p.ldc + col] = p.scale ? v * sc : v;
                }
            }
    }
}

template <bool WI8, int T>
static int launch_g(const GemmParams &p, hipStream_t st) {
    // 128 x 128 tiles, or 64 x 128 when that leaves fewer workgroups than CUs
    const int n_blocks = (p.N + 127) / 128;
    if (((p.M + 127) / 128) * n_blocks >= 256) {
        const dim3 grid(n_blocks, (p.M + 127) / 128);
        gemm_kernel<WI8, T, 128, 128><<<grid, 256, 0, st>>>(p);
    } else {
        const dim3 grid(n_blocks, (p.M + 63) / 64);
        gemm_kernel<WI8, T, 64, 128><<<grid, 256, 0, st>>>(p);
    }
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

// k_fullk.hip -- full-K int8 GEMV for decode batches of up to 16 rows, with
// the projection's row operations in its epilogue.
//
// Each projection of the decoder layer is the q8 kernel gemm_nt_int8
// (ops/src/kernels.rs:1256-1287: C = (sum_k A[i,k] * (f32)Q[j,k]) * scale[j])
// at M = 16 decode rows. The k-slice form (ks_gemv_i8_kernel) leaves raw
// slice sums in HBM for a second kernel; here one workgroup covers its rows
// over the whole K and reduces on chip, so the projection is one launch and
// writes only its result:
//   FQ_STORE  Y[m][j] = acc[m][j] * scale[j] * inv[m]   (the q/k/v rows)
//   FQ_SILU   over a gate/up tile pair: act[m][16p + r] =
//             silu(gate * sg) * (up * su), gate = acc * inv on row 32p + r,
//             up on row 32p + 16 + r (ACT silu then EWMUL,
//             tools/p12_build_minicpm.py:975-978)
// inv[m] = 1 / sqrt(sum of the segment sums of squares / K + eps) is the
// RMSNorm of the input row (ops/src/kernels.rs:1346-1368), whose gain the
// producer already applied: the rows arrive as int8 terms of x * g.
//
// Design (gfx950):
//  * Input: Q8_T int8 term planes of the M <= 16 rows in 1 KiB blocks in MFMA
//    operand order, [Q8_T][K/64][1 KiB]: lane l = (g = l / 16, n = l % 16) of
//    block (t, kb) holds row n, k = 64 kb + 8g .. +7 and 64 kb + 32 + 8g .. +7
//    (rows past M are zero). Each B fragment is one contiguous 1 KiB load, an
//    L2 hit after its first use on the XCD. Each (row, segment of the
//    producer's window) has a power-of-two factor a8s[seg][m].
//  * Weights: the session's swizzled copy (the A fragments, 1 KiB per 16-row
//    tile and 64-wide k-block).
//  * A workgroup of NW waves owns TW 16-row tiles; wave w takes k-blocks
//    w*KB .. w*KB + KB - 1 and issues all of its loads (weights, B fragments,
//    factors) before it waits on any. Per block and tile, Q8_T
//    v_mfma_i32_16x16x64_i8 straight on the int8 weights give exact int32 sums
//    of each term; they combine as (s0 + s1 / 2^7) + s2 / 2^14 times the
//    block's segment factor, accumulated in f32 per block in k order.
//  * The waves' tiles meet in LDS and are summed in wave order: the result
//    does not depend on scheduling, and is the same for every batch size.
#include "internal.hpp"

namespace vmlm {

namespace {

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

struct FqParams {
    const uint8_t *W;    // swizzled [N/16][K/64][64][16]
    const float *scale;  // [N]
    const int8_t *A8;    // blocked terms [Q8_T][K/64][1 KiB]
    const float *a8s;    // [K/seg][M] segment factors
    const float *ssp;    // [K/seg][M] segment sums of squares (RMSNorm), or null
    float eps;
    int seg_kb;          // 64-wide blocks per segment
    float *Y;
    int ldy;
    int M, N, K;
};

template <int KB, int NW, int TW, int EPI, int WPE>
__global__ __launch_bounds__(NW * 64, WPE) void fq_gemv_kernel(FqParams p) {
    static_assert(EPI != FQ_SILU || TW % 2 == 0, "SiLU pairs a gate tile and an up tile");
    constexpr int SMAX = 16;  // segments whose sums of squares are read
    __shared__ float red[TW][NW][16][17];
    __shared__ float ssp_s[SMAX][16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int nkb = p.K >> 6;
    const int kb0 = wave * KB;
    const int tile0 = blockIdx.x * TW;
    const int nr = n < p.M ? n : 0;

    // 1. every global read up front: B fragments, weights, segment factors,
    // and (threads 0..15) the row's segment sums of squares. The fragments
    // go first: loads return in order, so block i's products wait only for
    // the weights up to block i, not for the whole run
    i32x4 b[KB][Q8_T];
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
        for (int q = 0; q < Q8_T; ++q)
            b[i][q] = *(const i32x4 *)(p.A8 + ((size_t)q * nkb + kb0 + i) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wr[TW][KB];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const uint8_t *wt = p.W + ((size_t)(tile0 + t) * nkb + kb0) * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < KB; ++i)
            wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + (size_t)i * 1024));
    }
    // the wave's run is one segment (KB == seg_kb, checked at launch)
    const float segf = p.a8s[wave * p.M + nr];
    const int nseg = nkb / KB;
    // thread e < 16 * nseg: segment e / 16's sum of squares of row e % 16
    const int er = tid & 15;
    const float sspv = p.ssp && tid < 16 * nseg ? p.ssp[(tid >> 4) * p.M + (er < p.M ? er : 0)]
                                                : 0.0f;
    // the scales of the thread's first epilogue output (e = tid; one output
    // per thread at the launch shapes), loaded with everything else
    constexpr int NOUT = EPI == FQ_STORE ? TW * 256 : TW * 128;
    const int e0 = tid < NOUT ? tid : 0;
    const int row0 = EPI == FQ_STORE ? (tile0 + (e0 >> 8)) * 16 + (e0 & 15)
                                     : (tile0 + 2 * (e0 >> 8)) * 16 + (e0 & 15);
    const float sc0 = p.scale[row0];
    const float sc1 = EPI == FQ_STORE ? 0.0f : p.scale[row0 + 16];
    __builtin_amdgcn_sched_barrier(0);

    // 2. per tile: Q8_T MFMAs per block, exact int32 sums of each term over
    // the run (|sum| < 127 * 127 * 256 < 2^22), combined once. The term
    // weights and the factor are powers of two, so each fmaf rounds once, as
    // the separate multiply and add would.
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        i32x4 s[Q8_T];
#pragma unroll
        for (int q = 0; q < Q8_T; ++q) s[q] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            const i32x4 a = __builtin_bit_cast(i32x4, wr[t][i]);
#pragma unroll
            for (int q = 0; q < Q8_T; ++q)
                s[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[i][q], s[q], 0, 0, 0);
        }
        // D[row 4g + j][token n]
        const int g = lane >> 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float f = (float)s[0][j];
#pragma unroll
            for (int u = 1; u < Q8_T; ++u) f = __builtin_fmaf((float)s[u][j], q8_term_weight(u), f);
            red[t][wave][4 * g + j][n] = f * segf;
        }
    }
    if (tid < 16 * nseg) ssp_s[tid >> 4][er] = sspv;
    __syncthreads();
    // the RMSNorm of row m: 1 / sqrt(sum of its segments' squares in order / K + eps)
    auto inv_of = [&](int m) {
        if (!p.ssp) return 1.0f;
        float ss = ssp_s[0][m];
        for (int sg = 1; sg < nseg; ++sg) ss += ssp_s[sg][m];
        ss = ss / (float)p.K;
        return 1.0f / sqrtf(ss + p.eps);
    };

    // 3. the waves' partial tiles summed in wave order, then the epilogue:
    // consecutive threads take consecutive rows of one token (contiguous
    // stores)
    if constexpr (EPI == FQ_STORE) {
        for (int e = tid; e < TW * 256; e += NW * 64) {
            const int t = e >> 8, m = (e >> 4) & 15, r = e & 15;
            float s = red[t][0][r][m];
#pragma unroll
            for (int w = 1; w < NW; ++w) s += red[t][w][r][m];
            const int row = (tile0 + t) * 16 + r;
            if (m < p.M) p.Y[(size_t)m * p.ldy + row] = (s * (e == tid ? sc0 : p.scale[row])) * inv_of(m);
        }
    } else {
        // pair pp: gate tile 2pp, up tile 2pp + 1, outputs 16 (pair index) + r
        for (int e = tid; e < 128 * TW; e += NW * 64) {
            const int pp = e >> 8, m = (e >> 4) & 15, r = e & 15;
            float sg = red[2 * pp][0][r][m], su = red[2 * pp + 1][0][r][m];
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                sg += red[2 * pp][w][r][m];
                su += red[2 * pp + 1][w][r][m];
            }
            const float inv = inv_of(m);
            const int row = (tile0 + 2 * pp) * 16 + r;
            const float gs = (sg * (e == tid ? sc0 : p.scale[row])) * inv;
            const float us = (su * (e == tid ? sc1 : p.scale[row + 16])) * inv;
            if (m < p.M)
                p.Y[(size_t)m * p.ldy + (tile0 / 2 + pp) * 16 + r] = (gs / (1.0f + exp_f(-gs))) * us;
        }
    }
}

// WPE: waves per SIMD the registers must allow (two workgroups per CU)
template <int KB, int NW, int TW, int EPI, int WPE>
int launch_fq_t(const FqParams &p, hipStream_t st) {
    const unsigned grid = (unsigned)(p.N / 16 / TW);
    fq_gemv_kernel<KB, NW, TW, EPI, WPE><<<grid, NW * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace

// K as waves of one segment of 4 64-wide blocks each (the producer's window:
// 256 columns): 3, 6 or 9 waves (K = 768, 1536, 2304)
static int fq_waves(int K) {
    const int nw = K % 256 == 0 ? K / 256 : 0;
    return nw == 3 || nw == 6 || nw == 9 ? nw : 0;
}

bool fq_gemv_ok(int M, int N, int K, int epi, int tw) {
    const bool tw_ok = epi == FQ_SILU ? tw == 2 || tw == 4 : tw == 1 || tw == 2 || tw == 4;
    return M >= 1 && M <= 16 && fq_waves(K) && tw_ok && N % (16 * tw) == 0;
}

int launch_fq_gemv(const FqArgs &a, hipStream_t st) {
    const int tw = a.tw;
    VMLM_GUARD(a.M <= 16, "full-K int8 GEMV: at most 16 rows");
    VMLM_GUARD(fq_gemv_ok(a.M, a.N, a.K, a.epi, tw),
               "full-K int8 GEMV: shape M=%d N=%d K=%d (K = 768, 1536 or 2304) unsupported", a.M,
               a.N, a.K);
    VMLM_GUARD(a.W && a.scale && a.A8 && a.a8s && a.Y && ((uintptr_t)a.A8 & 15) == 0 &&
                   a.seg_kb == 4 && a.K / 256 <= 16,
               "full-K int8 GEMV: operands, 16-byte aligned blocked rows, 256-column segments");
    FqParams p;
    p.W = (const uint8_t *)a.W;
    p.scale = a.scale;
    p.A8 = a.A8;
    p.a8s = a.a8s;
    p.ssp = a.ssp;
    p.eps = a.eps;
    p.seg_kb = a.seg_kb;
    p.Y = a.Y;
    p.ldy = a.ldy;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    // one wave per 256-column segment (K = 2304: 9 waves of 4 blocks), two
    // workgroups per CU
#define FQ_NW(NWV)                                                                   \
    if (fq_waves(a.K) == NWV) {                                                      \
        if (a.epi == FQ_SILU)                                                        \
            return tw == 4 ? launch_fq_t<4, NWV, 4, FQ_SILU, 4>(p, st)               \
                           : launch_fq_t<4, NWV, 2, FQ_SILU, 5>(p, st);              \
        if (tw == 4) return launch_fq_t<4, NWV, 4, FQ_STORE, 4>(p, st);              \
        if (tw == 2) return launch_fq_t<4, NWV, 2, FQ_STORE, 5>(p, st);              \
        return launch_fq_t<4, NWV, 1, FQ_STORE, 5>(p, st);                           \
    }
    FQ_NW(3)
    FQ_NW(6)
    FQ_NW(9)
#undef FQ_NW
    return fail(VMLM_ERR_GUARD, "full-K int8 GEMV: K=%d", a.K);
}

}  // namespace vmlm

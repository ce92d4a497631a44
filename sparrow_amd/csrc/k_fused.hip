// k_fused.hip -- full-K decode GEMV for small batches (M <= 5), with the
// neighbouring row operations of the VM's decoder program fused in.
//
// The decoder layer of tools/p12_build_minicpm.py:941-981 runs, per token,
//   RMSNORM -> GEMM(q,k,v) -> attention -> GEMM(o) -> EWADD -> RMSNORM ->
//   GEMM(gate), GEMM(up) -> ACT silu -> EWMUL -> GEMM(down) -> EWADD
// with every GEMM the q8 kernel gemm_nt_int8 (ops/src/kernels.rs:1256-1287,
// C = (sum_k A[i,k] * (f32)Q[j,k]) * scale[j]). At a decode batch of a few
// tokens each projection is a weight stream, and each launch boundary costs
// more than the arithmetic of the ops around it. Here one launch covers
//   prologue  RMSNorm of the input rows (ops/src/kernels.rs:1346-1368:
//             ss = sum x^2, ss /= cols, inv = 1/sqrt(ss + eps), y = (x*inv)*g)
//   body      the projection over the full K (no k-slice partials)
//   epilogue  * scale[j], then EWADD with the residual row, or ACT silu of
//             the gate row times the up row (x / (1 + exp_f(-x)), then *)
// so a layer is five launches: qkv(+norm), attention, o(+residual),
// gate/up(+norm, silu*up), down(+residual).
//
// The RMSNorm is split between the producer and the consumer of the
// residual row: the residual epilogue writes the row x, the bf16 terms of
// x * g (the next norm's gain) and a sum of x^2 per 16 columns; the consumer
// sums the partials to ss and multiplies its dot products by
// inv = 1 / sqrt(ss / K + eps). That is y . w = inv * ((x * g) . w): the same
// value as the reference's ((x * inv) * g) . w up to f32 rounding order.
//
// Design (gfx950):
//  * Weights are read from a copy swizzled at load time into MFMA operand
//    order: block (16-row tile t, 64-wide k-block kb) is 1 KiB, lane l =
//    (g = l / 16, r = l % 16) holds row 16t + r, bytes kb*64 + 8g .. +7 and
//    kb*64 + 32 + 8g .. +7 (the A fragments of two v_mfma_f32_16x16x32_bf16).
//    One 16-byte load per lane reads a whole 1 KiB block: every load
//    instruction is contiguous, and no LDS transpose is needed.
//  * A workgroup owns one 16-row tile (two for the gate/up pair) over the full
//    K; its waves split K into runs of KB blocks. Each wave issues all of its
//    loads (inputs, weights, epilogue operands) before it waits on any, so a
//    launch costs one memory round trip.
//  * Inputs arrive as three bf16 term planes (hi + mid + lo = the f32 value,
//    written by the producer); each MFMA column is one (term, token) pair and
//    a lane loads its B fragments straight from the planes. Every
//    term x int8-weight product is exact in f32; the MFMA accumulates in f32.
//    Columns past 3*M are zero.
//  * The waves' partial tiles meet in LDS and are summed in wave order, so
//    the result does not depend on scheduling.
#include "internal.hpp"

namespace vmlm {

namespace {

constexpr int FK_T = 3;        // bf16 terms per f32 input value
constexpr int FK_MAXW = 16;    // wavefronts per workgroup
constexpr int FK_SSPF = 768;   // most sum-of-squares partial floats (partials x rows)

struct FkParams {
    const uint8_t *W;   // swizzled weights [N/16][K/64][64][16]
    const float *scale; // [N]
    const uint16_t *A;  // bf16 term planes [3][M][lda] of the input rows
    int lda;
    const float *ssp;   // RMSNorm of the input: partial sums of squares [nssp][M]
    int nssp;
    float eps;
    float *Y;
    int ldy;
    const float *R;     // residual rows [M][ldr] (FK_RESID)
    int ldr;
    uint16_t *Aout;     // term planes [3][M][ldy] of Y (FK_SILU) or of Y * gout (FK_RESID)
    const float *gout;  // FK_RESID: the next RMSNorm's gain [N]
    float *ssp_out;     // FK_RESID: partial sums of squares of Y, [N / 16][M]
    int M, N, K;
    int epi;
    const float *apart; // AP: the attention's position-range partials [K/64][FK_APART][68]
};

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Writes the three bf16 terms of v to planes [3][rows][ld] at offset o.
__device__ __forceinline__ void store_terms(uint16_t *dst, size_t plane, size_t o, float v) {
#pragma unroll
    for (int q = 0; q < FK_T; ++q) {
        const uint32_t hb = bf16_rne_bits(v);
        v = term_rem(v, hb);
        dst[q * plane + o] = (uint16_t)hb;
    }
}

// Sum over the 16 lanes of a DPP row (fixed butterfly order), in every lane.
__device__ __forceinline__ float row16_sum(float v) {
    v = v + __shfl_xor(v, 8, 64);
    v = v + __shfl_xor(v, 4, 64);
    v = v + __shfl_xor(v, 2, 64);
    v = v + __shfl_xor(v, 1, 64);
    return v;
}

// KB: k-blocks per wave; WPT: waves (the k-runs of the full K); TPW: 16-row
// tiles per workgroup (2: the gate/up pair of FK_SILU). Every wave covers all
// TPW tiles over its k-run, so its input fragments serve each tile.
// BL (one input row): the wave reads its k-run of the three term planes with
// one or two coalesced 16-byte loads per lane into a wave-private LDS slot
// and takes its B fragments from there, instead of 2 KB fragment loads on
// the live lanes (measured 0.3 - 0.9 us per launch faster at the MiniCPM-2B
// shapes).
// AP (one input row, the o projection): the run's KB heads arrive as the
// attention's FK_APART position-range partials (max m, sum l, O[64]) each;
// every wave merges its heads in range order -- M = max m, f = exp_f(m - M),
// L = sum l f, O = sum O f (FMAs in range order), y = O / L -- and writes the
// three bf16 terms of y into its LDS slot, which the attention would
// otherwise have written to the term planes.
template <int KB, int WPT, int TPW, bool BL, bool AP = false>
__global__ __launch_bounds__(WPT * 64) void fk_gemv_kernel(FkParams p) {
    static_assert(!AP || (BL && KB * FK_APART <= 64), "one lane per (head, range) weight");
    constexpr int NTH = WPT * 64;
    constexpr int RUN = KB * 64;              // bf16 of one term plane in a k-run
    constexpr int PCS = FK_T * RUN / 8;        // its 16-byte pieces over the planes
    constexpr int PQ = (PCS + 63) / 64;        // pieces per lane
    __shared__ float dw[TPW][WPT][16][17];
    __shared__ float inv_s[8];
    __shared__ __attribute__((aligned(16))) uint16_t bs[BL ? WPT : 1][BL ? FK_T * RUN : 8];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nkb = p.K >> 6;
    const int M = p.M;
    const int g = lane >> 4, n = lane & 15;
    const bool live = n < FK_T * M;  // column n = (term n / M, token n % M)
    const int tt = live ? n / M : 0, b = live ? n - tt * M : 0;
    const int kb0 = wave * KB;

    // 1. every global read up front: the lane's B fragments from the term
    // planes (row (tt, b), k = kb*64 + 8g .. +7 and kb*64 + 32 + 8g .. +7),
    // the weight blocks of its k-run for each tile, the norm partials, the
    // epilogue's scales and residual
    // Only the live lanes load (address work scales with the active lanes);
    // the other columns of the MFMA hold whatever the registers held and are
    // never read: each output column depends on its own B column only.
    u32x4 av[KB][2];
    u32x4 bq[BL && !AP ? PQ : 1];
    float ap_o[AP ? KB : 1][FK_APART];
    float2 ap_ml[AP ? KB : 1][FK_APART];
    if constexpr (AP) {  // head j of the run: range z's O[lane], (m, l)
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const int hd = kb0 + j < nkb ? kb0 + j : nkb - 1;
#pragma unroll
            for (int z = 0; z < FK_APART; ++z) {
                const float *pz = p.apart + ((size_t)hd * FK_APART + z) * ATTN_PART;
                ap_o[j][z] = pz[4 + lane];
                ap_ml[j][z] = *(const float2 *)pz;
            }
        }
    } else if constexpr (BL) {  // piece e: plane e / (RUN / 8), bf16 8 (e % (RUN / 8)) of the run
#pragma unroll
        for (int q = 0; q < PQ; ++q) {
            int e = lane + 64 * q;
            e = e < PCS ? e : PCS - 1;
            int k = kb0 * 64 + (e % (RUN / 8)) * 8;
            k = k < p.K ? k : p.K - 8;  // the last wave's run may pass K (its blocks are skipped)
            bq[q] = *(const u32x4 *)(p.A + (size_t)(e / (RUN / 8)) * p.lda + k);
        }
    } else if (live) {
        const uint16_t *ar = p.A + ((size_t)tt * M + b) * p.lda + 8 * g;
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            const int kb = kb0 + i < nkb ? kb0 + i : nkb - 1;
            av[i][0] = *(const u32x4 *)(ar + kb * 64);
            av[i][1] = *(const u32x4 *)(ar + kb * 64 + 32);
        }
    }
    // norm partials [nssp][M] (nssp * M <= FK_SSPF floats): wave 0, lane l
    // holds floats 4l .. 4l + 3, 256 + 4l .., 512 + 4l .. (zero past the end)
    float4 sp[3];
    const bool norm = p.ssp != nullptr;
    const int nsf = p.nssp * M;
    if (norm && wave == 0) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int f = 4 * lane + 256 * i;
            sp[i] = f < nsf ? *(const float4 *)(p.ssp + f) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // block-major, the order the k-run below consumes them in (loads return
    // in order: block i's products then wait only for blocks 0 .. i)
    u32x4 wr[TPW][KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const int kb = kb0 + i < nkb ? kb0 + i : nkb - 1;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const uint8_t *wt = p.W + ((size_t)(blockIdx.x * TPW + t) * nkb) * 1024 + lane * 16;
            wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + (size_t)kb * 1024));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // epilogue operands of thread tid's first output (row r, token bb):
    // unconditional loads (SILU: gate and up scales; else scale, residual)
    const int nout = 16 * M;
    const int e0 = tid < nout ? tid : 0;
    const int r0 = e0 & 15, bb0 = e0 >> 4;
    const bool silu = p.epi == FK_SILU;
    const int js0 = silu ? blockIdx.x * 32 + r0 : blockIdx.x * 16 + r0;
    const float sc0 = p.scale[js0];
    const float sc1 = p.scale[silu ? js0 + 16 : js0];
    const float res0 = *(p.R ? p.R + (size_t)bb0 * p.ldr + blockIdx.x * 16 + r0 : p.scale);
    const float go0 = *(p.gout ? p.gout + blockIdx.x * 16 + r0 : p.scale);

    // 2. RMSNorm of the input rows: inv = 1 / sqrt(ss / K + eps), ss summed
    // from the partials in a fixed order (identical in every workgroup)
    if (norm && wave == 0) {
        float ss[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const float v[4] = {sp[i].x, sp[i].y, sp[i].z, sp[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int row = (4 * lane + 256 * i + c) % M;
#pragma unroll
                for (int q = 0; q < 5; ++q)
                    if (q == row) ss[q] = ss[q] + v[c];
            }
        }
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            if (q < M) {  // uniform
                const float t = wave_sum(ss[q]);
                if (lane == 0) inv_s[q] = 1.0f / sqrtf(t / (float)p.K + p.eps);
            }
        }
    }

    if constexpr (BL) {  // the run into the wave's LDS slot, then the live lanes' fragments
        if constexpr (AP) {
            // the KB x FK_APART weights e^{m - M} in one exp_f: lane
            // j * FK_APART + z takes (j, z), then each weight is read back
            // as a wave-uniform value
            float xm = 0.0f;
#pragma unroll
            for (int j = 0; j < KB; ++j) {
                float M = ap_ml[j][0].x;
#pragma unroll
                for (int z = 1; z < FK_APART; ++z) M = fmaxf(M, ap_ml[j][z].x);
#pragma unroll
                for (int z = 0; z < FK_APART; ++z)
                    if (lane == j * FK_APART + z) xm = ap_ml[j][z].x - M;
            }
            const float ex = exp_f(xm);
#pragma unroll
            for (int j = 0; j < KB; ++j) {
                float L = 0.0f, O = 0.0f;
#pragma unroll
                for (int z = 0; z < FK_APART; ++z) {
                    const float f = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), j * FK_APART + z));
                    L = __builtin_fmaf(ap_ml[j][z].y, f, L);
                    O = __builtin_fmaf(ap_o[j][z], f, O);
                }
                float y = O / L;
#pragma unroll
                for (int t = 0; t < FK_T; ++t) {
                    const uint32_t hb = bf16_rne_bits(y);
                    y = term_rem(y, hb);
                    bs[wave][t * RUN + j * 64 + lane] = (uint16_t)hb;
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < PQ; ++q) {
                const int e = lane + 64 * q;
                if (e < PCS) *(u32x4 *)&bs[wave][e * 8] = bq[q];
            }
        }
        if (live) {
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                av[i][0] = *(const u32x4 *)&bs[wave][tt * RUN + i * 64 + 8 * g];
                av[i][1] = *(const u32x4 *)&bs[wave][tt * RUN + i * 64 + 32 + 8 * g];
            }
        }
    }

    // 3. the k-run: two MFMAs per 64-wide block and tile
    f32x4 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        if (kb0 + i < nkb) {
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                u32x4 a0, a1;
                i8x16_to_bf16(wr[t][i], a0, a1);
                acc[t] = mfma16(a0, av[i][0], acc[t]);
                acc[t] = mfma16(a1, av[i][1], acc[t]);
            }
        }
    }
    // D[row 4g + i][column n]
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[t][wave][4 * g + i][n] = acc[t][i];
    __syncthreads();

    // 4. epilogue: (row, token) pairs; wave partials summed in wave order
    auto tile_sum = [&](int t, int r, int bt) {
        float v = 0.0f;
        for (int w = 0; w < WPT; ++w) {
            float s = dw[t][w][r][bt];
#pragma unroll
            for (int q = 1; q < FK_T; ++q) s = s + dw[t][w][r][q * M + bt];
            v = v + s;
        }
        if (norm) v = v * inv_s[bt];
        return v;
    };
    const size_t plane = (size_t)M * p.ldy;
    for (int e = tid; e < nout; e += NTH) {
        const int r = e & 15, bt = e >> 4;
        const bool first = e == tid;
        if (silu) {  // tile 0: gate rows, tile 1: up rows
            const int jg = blockIdx.x * 32 + r;
            const float gate = tile_sum(0, r, bt) * (first ? sc0 : p.scale[jg]);
            const float up = tile_sum(1, r, bt) * (first ? sc1 : p.scale[jg + 16]);
            const float a = (gate / (1.0f + exp_f(-gate))) * up;
            const size_t o = (size_t)bt * p.ldy + blockIdx.x * 16 + r;
            if (p.Y) p.Y[o] = a;
            if (p.Aout) store_terms(p.Aout, plane, o, a);
        } else {
            const int j = blockIdx.x * 16 + r;
            float y = tile_sum(0, r, bt) * (first ? sc0 : p.scale[j]);
            if (p.epi == FK_RESID) y = (first ? res0 : p.R[(size_t)bt * p.ldr + j]) + y;
            const size_t o = (size_t)bt * p.ldy + j;
            p.Y[o] = y;
            if (p.ssp_out) {  // the next RMSNorm's input: terms of y * g, and sum y^2
                store_terms(p.Aout, plane, o, y * (first ? go0 : p.gout[j]));
                const float s2 = row16_sum(y * y);  // the 16 rows of token bt (16 lanes)
                if (r == 0) p.ssp_out[(size_t)blockIdx.x * M + bt] = s2;
            }
        }
    }
}

// k-slice GEMV for decode batches of 6..16 rows, over the swizzled weights.
// Workgroup (row group, k-slice): NWV waves each own TW 16-row tiles over the
// slice's KB 64-wide blocks. The slice of the three term planes
// ([3][16 tokens][KB*64] bf16, rows past M repeat row 0) is staged once in
// LDS; each wave reads a B fragment once per block and term and uses it for
// all TW tiles. Output: raw slice sums Y[ks][M][ldy] (no scale), reduced in
// slice order by the consumer (attention, residual RMSNorm, SiLU).
struct KsParams {
    const uint8_t *W;   // swizzled [N/16][K/64][64][16]
    const uint16_t *A;  // [3][M][lda] bf16 term planes, or
    const int8_t *A8;   // [Q8_T][M][lda] int8 rows, slice factors a8s[ks][M], or
    const float *X;     // f32 rows [M][lda], split into int8 terms while staged
    const float *a8s;
    const float *ssp;   // [ks][M] segment sums of squares (RMSNorm), or null
    float eps;
    int lda;
    float *Y;
    int ldy;
    int M, N, K;
};

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
constexpr int KS_SSP_MAX = 16;  // k-slices whose segment sums are read up front

// The int8 form: the slice of the Q8_T int8 term planes is staged in LDS; per
// block and term one v_mfma_i32_16x16x64_i8 per tile straight on the int8
// weights (no conversion), accumulated exactly in int32 (|sum| < 2^24 over
// a slice of at most 6 blocks). The epilogue forms
// (s0 + s1 / 2^7) + s2 / 2^14 in f32 (q8_term_weight), times the row factor:
// the slice's segment factor a8s[slice][row], and with ssp the RMSNorm's
// 1 / sqrt(sum ssp[.][row] / K + eps) (the int8 terms are of x * g).
// The swizzled weight bytes of lane (g, r) are k = 8g .. +7 and 32 + 8g .. +7
// of the block; the B fragment of lane (g, n) takes the same k of token n,
// so each product pairs matching k whatever order the MFMA sums them in.
template <int KB, int TW, int NWV, bool XF>
__global__ __launch_bounds__(NWV * 64) void ks_gemv_i8_kernel(KsParams p) {
    constexpr int NTH = NWV * 64;
    constexpr int KW = KB * 64;
    constexpr int ALD = KW + 16;     // padded LDS row (bytes)
    static_assert(!XF || NTH == 256, "f32 staging: 16 threads per row");
    __shared__ __attribute__((aligned(16))) int8_t as8[Q8_T][16][ALD];
    __shared__ float ssp_s[KS_SSP_MAX][16];
    __shared__ float xf_s[XF ? 16 : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int nkb = p.K >> 6;
    const int kb0 = blockIdx.y * KB;
    const int tile0 = (blockIdx.x * NWV + wave) * TW;

    constexpr int PIECES = Q8_T * 16 * (KW / 16);
    constexpr int PER = XF ? 1 : (PIECES + NTH - 1) / NTH;
    constexpr int XPER = KW / 64;  // XF: float4 pieces per thread (16 threads per row)
    u32x4 ap[PER];
    float4 xv[XF ? XPER : 1];
    const int xr = tid >> 4, xc = tid & 15;  // XF: row, and the thread's pieces xc + 16 i
    if constexpr (XF) {
        const float *xrow = p.X + (size_t)(xr < p.M ? xr : 0) * p.lda + (size_t)kb0 * 64;
#pragma unroll
        for (int i = 0; i < XPER; ++i) xv[i] = *(const float4 *)(xrow + 4 * (xc + 16 * i));
    } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int e = tid + i * NTH;
            e = e < PIECES ? e : PIECES - 1;
            const int t = e / (16 * (KW / 16)), r = (e / (KW / 16)) % 16, c16 = e % (KW / 16);
            const int rs = r < p.M ? r : 0;
            ap[i] = *(const u32x4 *)(p.A8 + ((size_t)t * p.M + rs) * p.lda + (size_t)kb0 * 64 + c16 * 16);
        }
    }
    // the row factor: this slice's segment factor, times the RMSNorm's
    // 1 / sqrt(mean(x^2) + eps) from the segment sums (one load per thread
    // into LDS; summed per row in segment order after the barrier)
    const int nr = n < p.M ? n : 0;
    const float segf = XF ? 0.0f : p.a8s[blockIdx.y * p.M + nr];
    const int nsl = (int)gridDim.y;
    constexpr int SPER = (KS_SSP_MAX * 16 + NTH - 1) / NTH;
    float sspv[SPER];
#pragma unroll
    for (int i = 0; i < SPER; ++i) {
        int e = tid + i * NTH;
        e = e < nsl * 16 ? e : 0;
        const int r = e & 15;
        sspv[i] = p.ssp ? p.ssp[(e >> 4) * p.M + (r < p.M ? r : 0)] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wr[TW][KB];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int tl = tile0 + t < (p.N >> 4) ? tile0 + t : (p.N >> 4) - 1;
        const uint8_t *wt = p.W + ((size_t)tl * nkb + kb0) * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < KB; ++i)
            wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + (size_t)i * 1024));
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XF) {
        // the slice of row xr as int8 terms with the power-of-two factor of
        // its own maximum (q8_row_k over the 16 threads of the row)
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < XPER; ++i)
            mx = fmaxf(mx, fmaxf(fmaxf(q8_mag(xv[i].x), q8_mag(xv[i].y)),
                                 fmaxf(q8_mag(xv[i].z), q8_mag(xv[i].w))));
        mx = row16_max_nonneg(mx);
        const int k = q8_row_k(mx);
        if (xc == 0) xf_s[xr] = q8_factor(k);
#pragma unroll
        for (int i = 0; i < XPER; ++i) {
            int a[4][Q8_T];
            q8_split(xv[i].x, k, a[0]);
            q8_split(xv[i].y, k, a[1]);
            q8_split(xv[i].z, k, a[2]);
            q8_split(xv[i].w, k, a[3]);
#pragma unroll
            for (int t = 0; t < Q8_T; ++t)
                *(uint32_t *)&as8[t][xr][4 * (xc + 16 * i)] =
                    pack_i8x4(a[0][t], a[1][t], a[2][t], a[3][t]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = tid + i * NTH;
            if (e < PIECES) {
                const int t = e / (16 * (KW / 16)), r = (e / (KW / 16)) % 16, c16 = e % (KW / 16);
                *(u32x4 *)&as8[t][r][c16 * 16] = ap[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < SPER; ++i) {
        const int e = tid + i * NTH;
        if (e < nsl * 16) ssp_s[e >> 4][e & 15] = sspv[i];
    }
    __syncthreads();
    float rowf = XF ? xf_s[n] : segf;
    if (p.ssp) {
        float ss = ssp_s[0][n];
        for (int s = 1; s < nsl; ++s) ss += ssp_s[s][n];
        ss = ss / (float)p.K;
        rowf = rowf * (1.0f / sqrtf(ss + p.eps));
    }

    // the B fragments of every block and term, then the tiles one at a time
    // in load order: a tile's partial row is stored as soon as its weights
    // have arrived and been multiplied, so the stores overlap the later
    // tiles' loads instead of following the whole load stream
    i32x4 b[KB][Q8_T];
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
        for (int q = 0; q < Q8_T; ++q) {
            const uint2 lo = *(const uint2 *)&as8[q][n][i * 64 + 8 * g];
            const uint2 hi = *(const uint2 *)&as8[q][n][i * 64 + 32 + 8 * g];
            b[i][q] = i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
        }
    float *yr = p.Y + ((size_t)blockIdx.y * p.M + n) * p.ldy;
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        i32x4 acc[Q8_T];
#pragma unroll
        for (int q = 0; q < Q8_T; ++q) acc[q] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            const i32x4 a = __builtin_bit_cast(i32x4, wr[t][i]);
#pragma unroll
            for (int q = 0; q < Q8_T; ++q)
                acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[i][q], acc[q], 0, 0, 0);
        }
        const int tl = tile0 + t;
        if (n < p.M && tl < (p.N >> 4)) {
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float f = (float)acc[0][j];
#pragma unroll
                for (int u = 1; u < Q8_T; ++u) f = f + (float)acc[u][j] * q8_term_weight(u);
                v[j] = f * rowf;
            }
            *(f32x4 *)(yr + tl * 16 + 4 * g) = v;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int KB, int TW, int NWV>
__global__ __launch_bounds__(NWV * 64) void ks_gemv_kernel(KsParams p) {
    constexpr int NTH = NWV * 64;
    constexpr int KW = KB * 64;      // k of the slice
    constexpr int ALD = KW + 8;      // padded LDS row (16 B): rows start on different banks
    __shared__ __attribute__((aligned(16))) uint16_t as[FK_T][16][ALD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int nkb = p.K >> 6;
    const int kb0 = blockIdx.y * KB;
    const int tile0 = (blockIdx.x * NWV + wave) * TW;

    // 1. the activation slice (16-byte pieces, all issued before anything waits)
    constexpr int PIECES = FK_T * 16 * (KW / 8);
    constexpr int PER = (PIECES + NTH - 1) / NTH;
    u32x4 ap[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        int e = tid + i * NTH;
        e = e < PIECES ? e : PIECES - 1;
        const int t = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
        const int rs = r < p.M ? r : 0;
        ap[i] = *(const u32x4 *)(p.A + ((size_t)t * p.M + rs) * p.lda + (size_t)kb0 * 64 + c8 * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. this wave's weight blocks
    u32x4 wr[TW][KB];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int tl = tile0 + t < (p.N >> 4) ? tile0 + t : (p.N >> 4) - 1;
        const uint8_t *wt = p.W + ((size_t)tl * nkb + kb0) * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < KB; ++i)
            wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + (size_t)i * 1024));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = tid + i * NTH;
        if (e < PIECES) {
            const int t = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
            *(u32x4 *)&as[t][r][c8 * 8] = ap[i];
        }
    }
    __syncthreads();

    // 3. per block: the B fragments of the three terms (lane (g, n): token n,
    // k = 8g .. +7 and 32 + 8g .. +7), then 2 x 3 MFMAs per tile
    f32x4 acc[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        u32x4 b[FK_T][2];
#pragma unroll
        for (int q = 0; q < FK_T; ++q) {
            b[q][0] = *(const u32x4 *)&as[q][n][i * 64 + 8 * g];
            b[q][1] = *(const u32x4 *)&as[q][n][i * 64 + 32 + 8 * g];
        }
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            u32x4 a0, a1;
            i8x16_to_bf16(wr[t][i], a0, a1);
#pragma unroll
            for (int q = 0; q < FK_T; ++q) {
                acc[t] = mfma16(a0, b[q][0], acc[t]);
                acc[t] = mfma16(a1, b[q][1], acc[t]);
            }
        }
    }
    // 4. D[row 4g + i][token n]: rows 4g .. 4g + 3 of the tile are 16 contiguous
    // bytes of the token's partial row
    if (n < p.M) {
        float *yr = p.Y + ((size_t)blockIdx.y * p.M + n) * p.ldy;
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            const int tl = tile0 + t;
            if (tl < (p.N >> 4))
                *(f32x4 *)(yr + tl * 16 + 4 * g) = acc[t];
        }
    }
}

template <int KB, int TW, int NWV>
int launch_ks_t(const KsParams &p, int ks, hipStream_t st) {
    const int rows = 16 * TW * NWV;
    const dim3 grid((unsigned)((p.N + rows - 1) / rows), (unsigned)ks);
    if (p.X) {
        if constexpr (NWV == 4)
            ks_gemv_i8_kernel<KB, TW, NWV, true><<<grid, NWV * 64, 0, st>>>(p);
        else
            return fail(VMLM_ERR_UNIMPL, "k-slice GEMV: f32 rows need 4 waves per workgroup");
    } else if (p.A8)
        ks_gemv_i8_kernel<KB, TW, NWV, false><<<grid, NWV * 64, 0, st>>>(p);
    else
        ks_gemv_kernel<KB, TW, NWV><<<grid, NWV * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// (N, K) int8 row-major -> swizzled blocks (see the header comment). One
// thread per 16-byte lane of a block.
__global__ void swizzle_w_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                 int N, int K) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nkb = K >> 6;
    const size_t total = (size_t)(N >> 4) * nkb * 64;
    if (idx >= total) return;
    const int l = (int)(idx & 63);
    const size_t blk = idx >> 6;
    const int kb = (int)(blk % nkb);
    const size_t t = blk / nkb;
    const int r = l & 15, g = l >> 4;
    const uint8_t *row = src + (t * 16 + r) * (size_t)K + (size_t)kb * 64 + 8 * g;
    const uint2 lo = *(const uint2 *)row;
    const uint2 hi = *(const uint2 *)(row + 32);
    *(u32x4 *)(dst + idx * 16) = u32x4{lo.x, lo.y, hi.x, hi.y};
}

template <int KB, int WPT, int TPW>
int launch_fk_t(const FkParams &p, hipStream_t st) {
    const unsigned grid = (unsigned)(p.N / 16 / TPW);
    if (p.apart) {
        if constexpr ((KB == 2 || KB == 3) && TPW == 1)  // fk_apart_ok: the o projection
            fk_gemv_kernel<KB, WPT, TPW, true, true><<<grid, WPT * 64, 0, st>>>(p);
        else
            return fail(VMLM_ERR_UNIMPL, "fused GEMV: attention partials need runs of 2 or 3 "
                                         "blocks and one tile");
    } else if (p.M == 1)
        fk_gemv_kernel<KB, WPT, TPW, true><<<grid, WPT * 64, 0, st>>>(p);
    else
        fk_gemv_kernel<KB, WPT, TPW, false><<<grid, WPT * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace

// k-run per wave: the smallest of 2, 3, 4, 6, 8 blocks that keeps the
// workgroup within 16 waves (the most waves, hence loads in flight, per
// workgroup; measured best for the MiniCPM shapes: 12 waves at K = 2304,
// 15 at K = 5760).
static int fk_kb(int nkb) {
    for (int kb : {2, 3, 4, 6, 8})
        if (nkb <= kb * FK_MAXW) return kb;
    return 0;
}

bool fk_apart_ok(int K) {
    const int kb = K % 64 ? 0 : fk_kb(K / 64);
    return kb == 2 || kb == 3;
}

bool fk_gemv_ok(int M, int N, int K, int epi) {
    const int tpw = epi == FK_SILU ? 2 : 1;
    return M >= 1 && M <= 5 && K >= 64 && K % 64 == 0 && N % (16 * tpw) == 0 &&
           fk_kb(K / 64) > 0;
}

int launch_fk_gemv(const FkArgs &a, hipStream_t st) {
    VMLM_GUARD(fk_gemv_ok(a.M, a.N, a.K, a.epi), "fused GEMV: shape M=%d N=%d K=%d unsupported",
               a.M, a.N, a.K);
    VMLM_GUARD(a.A && a.lda % 8 == 0 && ((uintptr_t)a.A & 15) == 0,
               "fused GEMV: term planes must be 16-byte aligned");
    VMLM_GUARD(!a.ssp || (a.nssp >= 1 && a.nssp * a.M <= FK_SSPF && ((uintptr_t)a.ssp & 15) == 0),
               "fused GEMV: %d norm partials x %d rows", a.nssp, a.M);
    VMLM_GUARD(a.epi == FK_SILU ? a.Y || a.Aout : !!a.Y, "fused GEMV: no output");
    VMLM_GUARD(!a.apart || (a.M == 1 && a.epi != FK_SILU && !a.ssp && ((uintptr_t)a.apart & 7) == 0),
               "fused GEMV: attention partials go with one row, no input norm, no SiLU pair");
    VMLM_GUARD(!a.ssp_out || (a.epi == FK_RESID && a.Aout && a.gout),
               "fused GEMV: the norm partials out need FK_RESID, terms and the gain");
    FkParams p;
    p.W = (const uint8_t *)a.W;
    p.scale = a.scale;
    p.A = a.A;
    p.lda = a.lda;
    p.ssp = a.ssp;
    p.nssp = a.nssp;
    p.eps = a.eps;
    p.Y = a.Y;
    p.ldy = a.ldy;
    p.R = a.R;
    p.ldr = a.ldr;
    p.Aout = a.Aout;
    p.gout = a.gout;
    p.ssp_out = a.ssp_out;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    p.epi = a.epi;
    p.apart = a.apart;
    const bool pair = a.epi == FK_SILU;
    const int nkb = a.K / 64;
    const int kb = a.kb ? a.kb : fk_kb(nkb), w = (nkb + kb - 1) / kb;
    VMLM_GUARD((kb == 2 || kb == 3 || kb == 4 || kb == 6 || kb == 8) && w <= FK_MAXW,
               "fused GEMV: k-run of %d blocks over %d", kb, nkb);
#define FK_W(KBV, TPWV)                                                 \
    switch (w) {                                                        \
    case 1: return launch_fk_t<KBV, 1, TPWV>(p, st);                \
    case 2: return launch_fk_t<KBV, 2, TPWV>(p, st);                \
    case 3: return launch_fk_t<KBV, 3, TPWV>(p, st);                \
    case 4: return launch_fk_t<KBV, 4, TPWV>(p, st);                \
    case 5: return launch_fk_t<KBV, 5, TPWV>(p, st);                \
    case 6: return launch_fk_t<KBV, 6, TPWV>(p, st);                \
    case 7: return launch_fk_t<KBV, 7, TPWV>(p, st);                \
    case 8: return launch_fk_t<KBV, 8, TPWV>(p, st);                \
    case 9: return launch_fk_t<KBV, 9, TPWV>(p, st);                \
    case 10: return launch_fk_t<KBV, 10, TPWV>(p, st);              \
    case 11: return launch_fk_t<KBV, 11, TPWV>(p, st);              \
    case 12: return launch_fk_t<KBV, 12, TPWV>(p, st);              \
    case 13: return launch_fk_t<KBV, 13, TPWV>(p, st);              \
    case 14: return launch_fk_t<KBV, 14, TPWV>(p, st);              \
    case 15: return launch_fk_t<KBV, 15, TPWV>(p, st);              \
    default: return launch_fk_t<KBV, 16, TPWV>(p, st);              \
    }
    switch (kb * 2 + (pair ? 1 : 0)) {
    case 4: FK_W(2, 1)
    case 5: FK_W(2, 2)
    case 6: FK_W(3, 1)
    case 7: FK_W(3, 2)
    case 8: FK_W(4, 1)
    case 9: FK_W(4, 2)
    case 12: FK_W(6, 1)
    case 13: FK_W(6, 2)
    case 16: FK_W(8, 1)
    default: FK_W(8, 2)
    }
#undef FK_W
}

// Terms of h * g and the partial sums of squares of h (16 columns per
// partial, as the FK_RESID epilogue writes them) for rows that enter the
// fused path without a producer GEMV (the embedding rows).
__global__ void fk_norm_prep_kernel(const float *__restrict__ h, int ldh, const float *__restrict__ g,
                                    int M, int N, uint16_t *__restrict__ terms, int ldt,
                                    float *__restrict__ ssp) {
    const int lane = threadIdx.x, r = lane & 15, q = lane >> 4;
    const int j = blockIdx.x * 16 + r;
    for (int bt = q; bt < ((M + 3) & ~3); bt += 4) {  // uniform trip count for the shuffles
        const bool ok = bt < M;
        const float y = ok ? h[(size_t)bt * ldh + j] : 0.0f;
        if (ok) store_terms(terms, (size_t)M * ldt, (size_t)bt * ldt + j, y * g[j]);
        const float s2 = row16_sum(y * y);
        if (ok && r == 0) ssp[(size_t)blockIdx.x * M + bt] = s2;
    }
}

int launch_fk_norm_prep(const float *h, int ldh, const float *g, int M, int N, uint16_t *terms,
                        int ldt, float *ssp, hipStream_t st) {
    VMLM_GUARD(N % 16 == 0 && M >= 1, "norm prep: N %% 16 must be 0");
    fk_norm_prep_kernel<<<(unsigned)(N / 16), 64, 0, st>>>(h, ldh, g, M, N, terms, ldt, ssp);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int ks_gemv_slices(int K) {
    const int nkb = K / 64;
    return nkb % 4 == 0 ? nkb / 4 : nkb % 6 == 0 ? nkb / 6 : nkb % 2 == 0 ? nkb / 2 : nkb;
}

int launch_ks_gemv(const KsArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.M <= 16 && a.K % 64 == 0 && a.K >= 64 && a.N % 16 == 0 && a.N >= 16,
               "k-slice GEMV: shape M=%d N=%d K=%d unsupported", a.M, a.N, a.K);
    VMLM_GUARD((a.A != nullptr) + (a.A8 != nullptr) + (a.X != nullptr) == 1 && (!a.A8 || a.a8s),
               "k-slice GEMV: bf16 term planes, int8 rows with their factors, or f32 rows");
    VMLM_GUARD(!a.ssp || ((a.A8 || a.X) && ks_gemv_slices(a.K) <= KS_SSP_MAX),
               "k-slice GEMV: segment sums go with int8 or f32 rows of at most %d slices",
               KS_SSP_MAX);
    VMLM_GUARD(!a.X || (a.K / ks_gemv_slices(a.K)) % 64 == 0,
               "k-slice GEMV: f32 rows need slices of whole 64-column blocks");
    const void *ain = a.A ? (const void *)a.A : a.A8 ? (const void *)a.A8 : (const void *)a.X;
    VMLM_GUARD(a.lda % 16 == 0 && ((uintptr_t)ain & 15) == 0 &&
                   a.Y && a.ldy % 4 == 0 && ((uintptr_t)a.Y & 15) == 0,
               "k-slice GEMV: input rows and partial rows must be 16-byte aligned");
    KsParams p;
    p.W = (const uint8_t *)a.W;
    p.A = a.A;
    p.A8 = a.A8;
    p.X = a.X;
    p.a8s = a.a8s;
    p.ssp = a.ssp;
    p.eps = a.eps;
    p.lda = a.lda;
    p.Y = a.Y;
    p.ldy = a.ldy;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    const int nkb = a.K / 64, ks = ks_gemv_slices(a.K), kb = nkb / ks;
    const int tw = a.tw ? a.tw : 2, nwv = a.nwv ? a.nwv : 4;
#define KS_CASE(KBV)                                                                  \
    if (kb == KBV) {                                                                  \
        if (tw == 1 && nwv == 8) return launch_ks_t<KBV, 1, 8>(p, ks, st);            \
        if (tw == 2 && nwv == 8) return launch_ks_t<KBV, 2, 8>(p, ks, st);            \
        if (tw == 3 && nwv == 4) return launch_ks_t<KBV, 3, 4>(p, ks, st);            \
        if (tw == 4 && nwv == 2) return launch_ks_t<KBV, 4, 2>(p, ks, st);            \
        if (tw == 4 && nwv == 4) return launch_ks_t<KBV, 4, 4>(p, ks, st);            \
        return launch_ks_t<KBV, 2, 4>(p, ks, st);                                     \
    }
    KS_CASE(1)
    KS_CASE(2)
    KS_CASE(4)
    KS_CASE(6)
#undef KS_CASE
    return fail(VMLM_ERR_GUARD, "k-slice GEMV: K=%d", a.K);
}

int launch_swizzle_w(const int8_t *src, int8_t *dst, int N, int K, hipStream_t st) {
    VMLM_GUARD(N % 16 == 0 && K % 64 == 0, "swizzle: N %% 16 and K %% 64 must be 0");
    const size_t total = (size_t)(N / 16) * (K / 64) * 64;
    if (!total) return VMLM_OK;
    swizzle_w_kernel<<<cdiv(total, 256), 256, 0, st>>>((const uint8_t *)src, (uint8_t *)dst, N, K);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

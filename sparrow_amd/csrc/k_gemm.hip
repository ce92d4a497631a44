// k_gemm.hip -- LDS-tiled MFMA GEMM for M > 16 (prefill, dense bf16 shape).
//
// C[M,N] = A[M,K] . W[N,K]^T (* scale[n]) with W int8 (kept int8 in LDS and
// converted exactly to bf16 per MFMA fragment) or bf16, and A given as T bf16
// term planes
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
    const int8_t *A8;   // int8 rows: Q8_T blocked term planes (launch_rows_q8), tstride
    const float *a8s;   // bytes apart, and row factors [M] (gemm_dma_i8_kernel)
    float *part;        // k-slices > 1: raw sums times the row factor [ks][M][N]
    int group;          // tile order: 0 as dispatched, g > 0 XCD-grouped (gemm_tile)
    int silu;           // int8 rows: C = SiLU(gate) * up of interleaved pairs (GemmArgs)
};

// The (N-block, M-block) tile of this workgroup. Workgroups are dispatched
// round-robin over the 8 XCDs (workgroup i on XCD i % 8), each with its own
// L2. With `group` > 0 (and the tile count a multiple of 8), XCD x takes the
// x-th eighth of the tiles in a grouped order -- `group` M-blocks at a time,
// N-blocks walked inside the group -- so the workgroups resident on one XCD
// at once share A rows and W rows through its L2. A bijection on the tiles.
__device__ __forceinline__ void gemm_tile(int group, int &bx, int &by) {
    const int nbx = (int)gridDim.x, nby = (int)gridDim.y, n = nbx * nby;
    int id = (int)blockIdx.y * nbx + (int)blockIdx.x;
    if (group <= 0) {
        bx = (int)blockIdx.x;
        by = (int)blockIdx.y;
        return;
    }
    if (n % 8 == 0) id = (id % 8) * (n / 8) + id / 8;
    const int per = group * nbx;
    const int m0 = id / per * group, r = id % per;
    const int gm = nby - m0 < group ? nby - m0 : group;
    by = m0 + r % gm;
    bx = r / gm;
}

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int gi32x4;

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) that waits for the vector-memory
// counter to drop to n and leaves the other counters unconstrained.
constexpr int waitcnt_vm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// One 16-byte-per-lane copy from global memory into LDS: lane i's 16 bytes
// at gptr land at LDS byte address lds_base + 16 * i (lds_base wave-uniform).
// Issued as inline assembly so that the compiler does not order every later
// LDS read behind it; the callers wait for the copies with explicit vmcnt
// waits and publish them with barriers. m0 is not used by anything else in
// these kernels.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; nothing else here uses it
__device__ __forceinline__ void dma16(const void *gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gptr), "s"(lds_base)
                 : "memory", "m0");
}

// The same copy with a wave-uniform base held in SGPRs (sbase) and a 32-bit
// per-lane byte offset: one VGPR per distinct offset instead of a 64-bit
// address per copy.
__device__ __forceinline__ void dma16s(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t *)p;
}

// 8 int8 weights -> 8 bf16 (exact).
__device__ __forceinline__ u32x4 i8x8_to_bf16(uint32_t w0, uint32_t w1) {
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t x = q ? w1 : w0;
        d[2 * q] = pack_hi16((float)(int)(int8_t)(x & 0xffu), (float)(int)(int8_t)((x >> 8) & 0xffu));
        d[2 * q + 1] = pack_hi16((float)(int)(int8_t)((x >> 16) & 0xffu), (float)(int)(int8_t)(x >> 24));
    }
    return u32x4{d[0], d[1], d[2], d[3]};
}

// GEMM with the tiles copied straight from global memory into LDS
// (global_load_lds_dwordx4: no register staging) through an NS-stage ring:
// the copy of k-step kt + NS - 1 is issued while step kt is consumed, and one
// barrier per step both publishes step kt and retires the reads of step
// kt - 1, whose stage the new copy overwrites. Copies past the last step
// re-read it into a stage that is never consumed again, so every step waits
// for the same number of outstanding copies.
//
// LDS rows hold 64 k: A (bf16 terms) and bf16 W 128 bytes, int8 W 64 bytes.
// The 16-byte pieces of a row are XOR-swizzled (piece c of row R sits in
// slot c ^ (R & 7); int8: c ^ ((R >> 1) & 3)) so that the 16 rows of an MFMA
// fragment read spread over the banks. Each copy instruction fills 1 KB of
// consecutive LDS (8 rows of 128 B or 16 of 64 B); the swizzle is applied by
// choosing which global piece each lane fetches.
//
// The epilogue stages each wave's 16-row slabs through LDS so that rows go
// out as 16-byte stores.
template <bool WI8, int T, int BM, int BN, int NS>
__global__ __launch_bounds__(256, 1) void gemm_dma_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int A_ROW = 128, B_ROW = WI8 ? 64 : 128;
    constexpr int A_BYTES = T * BM * A_ROW, B_BYTES = BN * B_ROW;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int C_LD = WN + 4;
    constexpr int C_BYTES = 4 * 16 * C_LD * 4;
    constexpr int SMEM = NS * STAGE > C_BYTES ? NS * STAGE : C_BYTES;
    constexpr int A_INS = A_BYTES / 1024 / 4, B_INS = B_BYTES / 1024 / 4;  // per wave per step
    static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "copy instructions per wave");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r = lane & 15;
    int tbx, tby;
    gemm_tile(p.group, tbx, tby);
    const int m0 = tby * BM, n0 = tbx * BN;
    const int nk = p.K / 64;

    // copy plan: global source of this lane (k-step 0) per instruction
    const uint8_t *a_src[A_INS];
    const uint8_t *b_src[B_INS];
#pragma unroll
    for (int q = 0; q < A_INS; ++q) {
        const int rowg = (q * 4 + wave) * 8 + (lane >> 3);  // over the T*BM rows
        const int t = rowg / BM, R = rowg % BM;
        const int c = (lane & 7) ^ (R & 7);
        int gm = m0 + R;
        gm = gm < p.M ? gm : p.M - 1;
        a_src[q] = (const uint8_t *)(p.A + t * p.tstride + (size_t)gm * p.lda) + c * 16;
    }
#pragma unroll
    for (int q = 0; q < B_INS; ++q) {
        int R, c;
        if constexpr (WI8) {
            R = (q * 4 + wave) * 16 + (lane >> 2);
            c = (lane & 3) ^ ((R >> 1) & 3);
        } else {
            R = (q * 4 + wave) * 8 + (lane >> 3);
            c = (lane & 7) ^ (R & 7);
        }
        int gn = n0 + R;
        gn = gn < p.N ? gn : p.N - 1;
        b_src[q] = p.W + (size_t)gn * p.K * (WI8 ? 1 : 2) + c * 16;
    }
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
    auto issue = [&](int kt) {
        const int kc = kt < nk ? kt : nk - 1;
        const uint32_t sb = lds0 + (uint32_t)((kt % NS) * STAGE);
#pragma unroll
        for (int q = 0; q < A_INS; ++q)
            dma16(a_src[q] + (size_t)kc * A_ROW, sb + (q * 4 + wave) * 1024);
#pragma unroll
        for (int q = 0; q < B_INS; ++q)
            dma16(b_src[q] + (size_t)kc * B_ROW, sb + A_BYTES + (q * 4 + wave) * 1024);
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const uint8_t *sA) {
        const uint8_t *sB = sA + A_BYTES;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            u32x4 bf[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int R = wn * WN + j * 16 + r;
                if constexpr (WI8) {
                    const int c = ks * 2 + (g >> 1);
                    const uint2 v = *(const uint2 *)(sB + R * 64 + ((c ^ ((R >> 1) & 3)) * 16) +
                                                     (g & 1) * 8);
                    bf[j] = i8x8_to_bf16(v.x, v.y);
                } else {
                    const int c = ks * 4 + g;
                    bf[j] = *(const u32x4 *)(sB + R * 128 + ((c ^ (R & 7)) * 16));
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int R = wm * WM + i * 16 + r;
                    const int c = ks * 4 + g;
                    const u32x4 af =
                        *(const u32x4 *)(sA + (t * BM + R) * 128 + ((c ^ (R & 7)) * 16));
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af, bf[j], acc[i][j]);
                }
        }
    };

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s);
    for (int kt = 0; kt < nk; ++kt) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * (A_INS + B_INS)));
        __syncthreads();
        issue(kt + NS - 1);
        compute(smem + (kt % NS) * STAGE);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // copies past the end land before reuse
    __syncthreads();

    // epilogue: 16-row slabs of this wave's tile through LDS, 16-byte stores
    float *cs = (float *)smem + wave * 16 * C_LD;
    const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)p.C & 15) == 0;
    constexpr int LPR = WN / 4, RPP = 64 / LPR;  // lanes per row, rows per pass
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) cs[(g * 4 + q) * C_LD + j * 16 + r] = acc[i][j][q];
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's slab is in LDS
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int pass = 0; pass < 16 / RPP; ++pass) {
            const int rr_ = pass * RPP + lane / LPR, c4 = (lane % LPR) * 4;
            float4 v = *(const float4 *)&cs[rr_ * C_LD + c4];
            const int row = m0 + wm * WM + i * 16 + rr_, col = n0 + wn * WN + c4;
            if (row >= p.M || col >= p.N) continue;
            float y[4] = {v.x, v.y, v.z, v.w};
            if (p.scale) {
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = y[e] * p.scale[col + e < p.N ? col + e : col];
            }
            float *dst = p.C + (size_t)row * p.ldc + col;
            if (vec && col + 3 < p.N) {
                *(float4 *)dst = make_float4(y[0], y[1], y[2], y[3]);
            } else {
                for (int e = 0; e < 4 && col + e < p.N; ++e) dst[e] = y[e];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

// The same pipeline for int8 weights and int8 rows (Q8_T term planes of
// each row with a power-of-two row factor, from launch_rows_q8): both tiles
// stay int8 in LDS, and each 64-wide k-step runs one v_mfma_i32_16x16x64_i8
// per term and 16 x 16 tile, exact int32 sums per term. The rows arrive in
// 1 KiB blocks of 16 rows x 64 k in MFMA lane order (lane (g, r): row r, k
// 8g .. 8g + 7 and 32 + 8g .. +7), so each copy instruction moves one
// contiguous block and each fragment read is one conflict-free 16-byte LDS
// read per lane. The weights are either the same blocks (WB: the swizzled
// copy of launch_swizzle_w) or row-major [N][K] (64-byte LDS rows, the int8
// XOR swizzle; lane (g, r) reads the two 8-byte halves of row r at k 8g and
// 32 + 8g); both pair the same k as the rows' fragments. Rows of 64 bytes fill half a cache line
// per copy lane; whole blocks fill full lines, which measured 25-30 % faster
// at the prefill shapes. The epilogue forms (s0 + s1/2^7) + s2/2^14 in f32
// (q8_term_weight), times the row factor and the column scale. No int8 ->
// bf16 conversion, and Q8_T MFMAs of 8 passes per k-step against six for
// three bf16 terms.
template <int BM, int BN, int NS, bool WB, int OCC = 2, int WMW = 2, int WNW = 2>
__global__ __launch_bounds__(64 * WMW * WNW) __attribute__((amdgpu_waves_per_eu(OCC))) void gemm_dma_i8_kernel(GemmParams p) {
    // WMW x WNW waves, each owning a WM x WN sub-tile
    constexpr int NW = WMW * WNW;
    constexpr int WM = BM / WMW, WN = BN / WNW;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int ROW = 64;  // bytes of a row-major W row in LDS (64 k of int8)
    constexpr int ABLK = Q8_T * BM / 16;  // 1 KiB blocks of A per k-step
    constexpr int BBLK = BN / 16;         // 1 KiB copies of W per k-step
    constexpr int A_BYTES = ABLK * 1024, B_BYTES = BN * ROW;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int C_LD = WN + 4;
    constexpr int C_BYTES = NW * 16 * C_LD * 4;
    constexpr int SMEM = NS * STAGE > C_BYTES ? NS * STAGE : C_BYTES;
    // copy instructions per wave and step: the step's ABLK + BBLK blocks
    // (A first, then W; block b at stage byte 1024 b) dealt round-robin to
    // the waves, block q * NW + wave to this wave. An uneven deal (64 x 96:
    // 5, 5, 4, 4) needs the two-stage wait (wait for all).
    constexpr int NBLK = ABLK + BBLK, INS = (NBLK + NW - 1) / NW;
    static_assert(WM % 16 == 0 && WN % 16 == 0 && BN % 16 == 0, "16 x 16 MFMA tiles");
    static_assert(NBLK % NW == 0 || NS == 2, "uneven copies need the two-stage wait");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int g = lane >> 4, r = lane & 15;
    int tbx, tby;
    gemm_tile(p.group, tbx, tby);
    const int m0 = tby * BM, n0 = tbx * BN;
    // this workgroup's k-steps [kb0, kb0 + nk): all, or k-slice blockIdx.z
    const int nkt = p.K / 64, ksl = (int)gridDim.z;
    const int kb0 = (int)blockIdx.z * nkt / ksl;
    const int nk = ((int)blockIdx.z + 1) * nkt / ksl - kb0;

    // copy plan: A block blk = term blk / (BM / 16), row tile blk % (BM / 16)
    // of this tile (the planes are p.tstride bytes apart, row tiles nkt KiB);
    // W blocks of the swizzled copy, or 16 rows x 64 B of row-major W per
    // instruction with lane i bringing piece (i & 3) ^ ((R >> 1) & 3) of row
    // R = 16 * instr + i / 4. Copy q reads base[q] (wave-uniform, advancing
    // kstr[q] bytes per k-step) plus the lane's offset voff[q]: 16 * lane for
    // whole blocks, the row and piece within the tile for row-major W.
    const uint8_t *base[INS];
    uint32_t voff[INS];
    int kstr[INS];
#pragma unroll
    for (int q = 0; q < INS; ++q) {
        const int blk0 = q * NW + wave, blk = blk0 < NBLK ? blk0 : NBLK - 1;
        voff[q] = (uint32_t)lane * 16;
        kstr[q] = 1024;
        if (blk < ABLK) {
            const int t = blk / (BM / 16), i = blk % (BM / 16);
            base[q] = (const uint8_t *)p.A8 + t * p.tstride + ((size_t)(m0 / 16 + i) * nkt) * 1024;
        } else if constexpr (WB) {
            int tn = n0 / 16 + (blk - ABLK);
            tn = tn < p.N / 16 ? tn : p.N / 16 - 1;
            base[q] = p.W + ((size_t)tn * nkt) * 1024;
        } else {
            const int R = (blk - ABLK) * 16 + (lane >> 2);
            const int c = (lane & 3) ^ ((R >> 1) & 3);
            int gn = n0 + R;
            gn = gn < p.N ? gn : p.N - 1;
            base[q] = p.W + (size_t)n0 * p.K;
            voff[q] = (uint32_t)((gn - n0) * p.K + c * 16);  // < BN * K (launch_gemm bounds K)
            kstr[q] = ROW;
        }
    }
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
    auto issue = [&](int kt) {
        const int kc = kb0 + (kt < nk ? kt : nk - 1);
        const uint32_t sb = lds0 + (uint32_t)((kt % NS) * STAGE);
#pragma unroll
        for (int q = 0; q < INS; ++q)
            if (NBLK % NW == 0 || q * NW + wave < NBLK)  // wave-uniform
                dma16s(base[q] + (size_t)kc * kstr[q], voff[q], sb + (q * NW + wave) * 1024);
    };

    gi32x4 acc[Q8_T][TM][TN];
#pragma unroll
    for (int t = 0; t < Q8_T; ++t)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[t][i][j] = gi32x4{0, 0, 0, 0};

    auto compute = [&](const uint8_t *sA) {
        const uint8_t *sB = sA + A_BYTES;
        gi32x4 bf[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if constexpr (WB) {
                bf[j] = *(const gi32x4 *)(sB + (wn * TN + j) * 1024 + lane * 16);
            } else {  // k 8g .. 8g + 7 (in piece g / 2) and 32 + 8g .. (piece 2 + g / 2)
                const int R = wn * WN + j * 16 + r, sw = (R >> 1) & 3;
                const uint2 lo = *(const uint2 *)(sB + R * ROW + (((g >> 1) ^ sw) * 16) + (g & 1) * 8);
                const uint2 hi =
                    *(const uint2 *)(sB + R * ROW + (((2 + (g >> 1)) ^ sw) * 16) + (g & 1) * 8);
                bf[j] = gi32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
        }
#pragma unroll
        for (int t = 0; t < Q8_T; ++t)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const gi32x4 af =
                    *(const gi32x4 *)(sA + (t * (BM / 16) + wm * TM + i) * 1024 + lane * 16);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[t][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[j], acc[t][i][j], 0, 0, 0);
            }
    };

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s);
    for (int kt = 0; kt < nk; ++kt) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * INS));
        __syncthreads();
        issue(kt + NS - 1);
        compute(smem + (kt % NS) * STAGE);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // copies past the end land before reuse
    __syncthreads();

    // epilogue: the terms combined, 16-row slabs through LDS, 16-byte stores
    float *cs = (float *)smem + wave * 16 * C_LD;
    const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)p.C & 15) == 0;
    // lanes per row, rows per pass (the last pass may be partial)
    constexpr int LPR = WN / 4, RPP = 64 / LPR, NPASS = (16 + RPP - 1) / RPP;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float f = (float)acc[0][i][j][q];
#pragma unroll
                for (int t = 1; t < Q8_T; ++t) f = f + (float)acc[t][i][j][q] * q8_term_weight(t);
                cs[(g * 4 + q) * C_LD + j * 16 + r] = f;
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's slab is in LDS
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int pass = 0; pass < NPASS; ++pass) {
            const int rr_ = pass * RPP + lane / LPR, c4 = (lane % LPR) * 4;
            if (lane >= RPP * LPR || rr_ >= 16) continue;
            float4 v = *(const float4 *)&cs[rr_ * C_LD + c4];
            const int row = m0 + wm * WM + i * 16 + rr_, col = n0 + wn * WN + c4;
            if (row >= p.M || col >= p.N) continue;
            const float rf = p.a8s[row];
            if (WN % 32 == 0 && p.silu) {
                // the slab's 64 columns are two (16 gate, 16 up) pairs: a gate
                // lane takes its up values 16 columns on, as silu_mul would
                // read them from C (the same scaled f32 results)
                if (c4 & 16) continue;
                const float4 u = *(const float4 *)&cs[rr_ * C_LD + c4 + 16];
                const float gv[4] = {v.x, v.y, v.z, v.w}, uv[4] = {u.x, u.y, u.z, u.w};
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gate = (gv[e] * rf) * p.scale[col + e];
                    const float up = (uv[e] * rf) * p.scale[col + 16 + e];
                    y[e] = act_scalar(gate, VMLM_ACT_SILU) * up;
                }
                *(float4 *)(p.C + (size_t)row * p.ldc + (col - 16 * (col >> 5))) =
                    make_float4(y[0], y[1], y[2], y[3]);
                continue;
            }
            float y[4] = {v.x * rf, v.y * rf, v.z * rf, v.w * rf};
            if (p.scale && ksl == 1) {
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = y[e] * p.scale[col + e < p.N ? col + e : col];
            }
            float *dst = ksl == 1 ? p.C + (size_t)row * p.ldc + col
                                  : p.part + ((size_t)blockIdx.z * p.M + row) * p.N + col;
            if ((ksl > 1 || vec) && col + 3 < p.N) {
                *(float4 *)dst = make_float4(y[0], y[1], y[2], y[3]);
            } else {
                for (int e = 0; e < 4 && col + e < p.N; ++e) dst[e] = y[e];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

constexpr int DMA_LDS_MAX = 160 * 1024;
constexpr int dma_stage_bytes(bool wi8, int T, int BM, int BN) {
    return T * BM * 128 + BN * (wi8 ? 64 : 128);
}

template <bool WI8, int T, int BM, int BN, int NS>
static int launch_dma_ns(const GemmParams &p, hipStream_t st) {
    if constexpr (NS * dma_stage_bytes(WI8, T, BM, BN) <= DMA_LDS_MAX) {
        const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
        gemm_dma_kernel<WI8, T, BM, BN, NS><<<grid, 256, 0, st>>>(p);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    } else {
        return fail(VMLM_ERR_UNIMPL, "gemm: %d LDS stages exceed the LDS", NS);
    }
}

template <bool WI8, int T, int BM, int BN>
static int launch_dma(const GemmParams &p, int ns, hipStream_t st) {
    switch (ns) {
    case 2: return launch_dma_ns<WI8, T, BM, BN, 2>(p, st);
    case 3: return launch_dma_ns<WI8, T, BM, BN, 3>(p, st);
    case 4: return launch_dma_ns<WI8, T, BM, BN, 4>(p, st);
    default: return fail(VMLM_ERR_UNIMPL, "gemm: %d LDS stages", ns);
    }
}

template <bool WI8, int T>
static int launch_g(const GemmParams &p, int bm, int ns, hipStream_t st) {
    // Tiles: 128 x 128 for single-term (bf16) activations when that still
    // gives two workgroups per CU (512 on this device), else 64 x 128 (and
    // always with three terms, whose 128-row stage would leave one workgroup
    // per CU). Two LDS stages keep two workgroups resident per CU.
    // Single-term grids of at most one 64 x 128 tile per CU (config 1: 1024
    // x 2048 x 512 gives 256, each CU streaming one tile's K and then writing
    // 32 KB of results while nothing else runs): 64 x 64 tiles, two per CU,
    // 6.6 -> 5.75 us; 32 x 64 and 32 x 128 tiles, three or four stages, or
    // the XCD-grouped order were slower.
    if (bm == 0 && T == 1 && (size_t)((p.M + 63) / 64) * ((p.N + 127) / 128) <= 256)
        return launch_dma<WI8, T, 64, 64>(p, ns ? ns : 2, st);
    if (bm == 0) bm = T == 1 && ((p.M + 127) / 128) * ((p.N + 127) / 128) >= 512 ? 128 : 64;
    VMLM_GUARD(bm == 64 || bm == 128, "gemm: tile rows %d (64 or 128)", bm);
    if (ns == 0) ns = 2;
    VMLM_GUARD(ns >= 2 && ns <= 4 && ns * dma_stage_bytes(WI8, T, bm, 128) <= DMA_LDS_MAX,
               "gemm: %d LDS stages of %d bytes", ns, dma_stage_bytes(WI8, T, bm, 128));
    return bm == 128 ? launch_dma<WI8, T, 128, 128>(p, ns, st) : launch_dma<WI8, T, 64, 128>(p, ns, st);
}

template <int BM, int BN, int NS, int WMW = 2, int WNW = 2>
static int launch_i8(const GemmParams &p, bool wb, int ksl, bool keep, hipStream_t st) {
    constexpr int stage = Q8_T * BM * 64 + BN * 64;
    static_assert(NS * stage <= DMA_LDS_MAX, "int8 gemm stages exceed the LDS");
    const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, ksl);
    // two stages over blocked weights: registers for four workgroups per CU
    // (128 VGPRs, the LDS holds four 40 KiB rings); 2 % faster than three at
    // the prefill's q/k/v and gate/up shapes, where 128 x 256 tiles of eight
    // waves (one workgroup per CU, two to four stages) measured 7 to 14 %
    // slower than either, and 128 x 128 or 64 x 256 tiles of eight waves (two
    // workgroups per CU, a quarter to a third fewer copy bytes per MFMA) 6 to
    // 7 % slower over the whole batch-16 prefill; 64 x 64 tiles (five
    // workgroups per CU) 20 to 60 % slower
    if (!wb)
        gemm_dma_i8_kernel<BM, BN, NS, false, 2, WMW, WNW><<<grid, 64 * WMW * WNW, 0, st>>>(p);
    else if constexpr (NS == 2)
        gemm_dma_i8_kernel<BM, BN, NS, true, 4, WMW, WNW><<<grid, 64 * WMW * WNW, 0, st>>>(p);
    else
        gemm_dma_i8_kernel<BM, BN, NS, true, 2, WMW, WNW><<<grid, 64 * WMW * WNW, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    if (ksl == 1 || keep) return VMLM_OK;
    return launch_gemv_reduce(p.part, ksl, p.M, p.N, p.scale, p.C, p.ldc, st);
}

int gemm_i8_kslices(int M, int N, int K) {
    if (N % 4) return 1;  // the partial rows are written as 16-byte stores
    const int wgs = ((N + 127) / 128) * ((M + 63) / 64), nk = K / 64;
    const int ks = wgs < 64 ? 4 : wgs < 160 ? 2 : 1;  // fill the 256 CUs
    return nk >= 8 * ks ? ks : 1;
}

// Rows of an int8-row GEMM whose factor is NaN (a NaN or infinite input,
// q8_row_k) are recomputed here in f32 in the reference's order
// (ops/src/kernels.rs:1256-1287: eight FMA lanes over k, the 8 -> 1 fold,
// the scalar tail, then the scale), so their +-inf / NaN pattern is the
// reference's. One thread per output column; each workgroup scans the row
// factors 256 at a time into an LDS list and skips clean rows, so a GEMM
// without such rows pays one short launch.
__global__ __launch_bounds__(256) void gemm_i8_nonfinite_rows_kernel(
    const float *__restrict__ a, int lda, const int8_t *__restrict__ q, int ldq,
    const float *__restrict__ scale, const float *__restrict__ a8s, float *__restrict__ c,
    int ldc, int M, int N, int K) {
    __shared__ int list[256];
    __shared__ int cnt;
    const int j = blockIdx.x * 256 + threadIdx.x;
    for (int base = 0; base < M; base += 256) {
        if (threadIdx.x == 0) cnt = 0;
        __syncthreads();
        const int r = base + threadIdx.x;
        if (r < M) {
            const float f = a8s[r];
            if (!(f == f)) list[atomicAdd(&cnt, 1)] = r;
        }
        __syncthreads();
        const int n = cnt;
        for (int e = 0; e < n && j < N; ++e) {
            const int i = list[e];
            const float *ar = a + (size_t)i * lda;
            const int8_t *qr = q + (size_t)j * ldq;
            float acc[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
            int kk = 0;
            for (; kk + 8 <= K; kk += 8) {
#pragma unroll
                for (int l = 0; l < 8; ++l)
                    acc[l] = __builtin_fmaf(ar[kk + l], (float)qr[kk + l], acc[l]);
            }
            float s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
            for (; kk < K; ++kk) s += ar[kk] * (float)qr[kk];
            c[(size_t)i * ldc + j] = s * scale[j];
        }
        __syncthreads();
    }
}

int launch_gemm_i8_nonfinite_rows(const float *a, int lda, const int8_t *q, int ldq,
                                  const float *scale, const float *a8s, float *c, int ldc, int M,
                                  int N, int K, hipStream_t st) {
    if (M <= 0 || N <= 0) return VMLM_OK;
    gemm_i8_nonfinite_rows_kernel<<<(N + 255) / 256, 256, 0, st>>>(a, lda, q, ldq, scale, a8s, c,
                                                                   ldc, M, N, K);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_gemm(const GemmArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.N >= 1, "gemm: empty shape");
    if (a.A8) {  // int8 rows x int8 weights
        VMLM_GUARD(a.w_int8 && a.a8s && a.K > 0 && a.K % 64 == 0 && ((uintptr_t)a.W & 15) == 0 &&
                       ((uintptr_t)a.A8 & 15) == 0 && (!a.w_blocked || a.N % 16 == 0),
                   "gemm (int8 rows): int8 weights, row factors, K %% 64 == 0, 16-byte aligned "
                   "operands, whole 16-row weight blocks");
        // row-major weights: a lane's offset within a tile's rows is 32-bit
        VMLM_GUARD(a.w_blocked || a.K <= (1 << 22), "gemm (int8 rows): K=%d above 2^22 needs "
                   "blocked weights", a.K);
        VMLM_GUARD(!a.silu_pairs || (a.N % 32 == 0 && a.scale && a.ldc % 4 == 0 &&
                                     a.ldc >= a.N / 2 && ((uintptr_t)a.C & 15) == 0),
                   "gemm (int8 rows, SiLU pairs): N %% 32 == 0, column scales, 16-byte aligned "
                   "output rows of at least N / 2");
        GemmParams p{};
        p.W = (const uint8_t *)a.W;
        p.scale = a.scale;
        p.C = a.C;
        p.tstride = q8_rows_tiles((size_t)a.M) * 16 * (size_t)a.K;  // bytes per term plane
        p.lda = a.K;
        p.M = a.M;
        p.N = a.N;
        p.K = a.K;
        p.ldc = a.ldc;
        // XCD-grouped tile order, 5 M-blocks per group (the prefill shapes,
        // M = 2048: 7 to 12 % faster than the dispatch order; over the whole
        // batch-16 prefill, groups of 3, 5 or 6 M-blocks measured 3.5 to 4 %
        // faster than groups of 4 or 8, and 2 % faster than groups of 2)
        p.group = a.group >= 0 ? a.group : 5;
        p.A8 = a.A8;
        p.a8s = a.a8s;
        // skinny grids: ordered k-slices through `work`, then the in-order
        // slice reduction applies the column scale
        const int ksl = a.work && !a.silu_pairs ? gemm_i8_kslices(a.M, a.N, a.K) : 1;
        VMLM_GUARD(ksl == 1 || (size_t)ksl * a.M * a.N <= a.work_floats,
                   "gemm (int8 rows): %d k-slices need %zu work floats, %zu given", ksl,
                   (size_t)ksl * a.M * a.N, a.work_floats);
        p.part = a.work;
        p.silu = a.silu_pairs ? 1 : 0;
        const int ns = a.stages ? a.stages : 2;
        // 64 x 128 tiles: 128-row tiles need 256 accumulator registers, run one
        // wave per SIMD and measured 30 % slower at the prefill shapes. Two
        // stages (48 KB, 166 VGPRs) keep three workgroups per CU, three
        // stages (72 KB) two: 4 to 8 % faster at the prefill shapes.
        // 64 x 96 tiles where they load the CUs more evenly: the busiest CU
        // holds ceil(tiles / 256) workgroups, each copying 12 KiB of rows and
        // BN / 16 KiB of weights per k-step (N = 2304: 768 tiles, three on
        // every CU, instead of 576 with three on a quarter of them)
        auto tiles = [&](int bn) {
            return (size_t)((a.N + bn - 1) / bn) * ((a.M + 63) / 64) * ksl;
        };
        auto load = [&](int bn) {
            return (tiles(bn) + 255) / 256 * (size_t)(Q8_T * 4 * 1024 + bn * 64);
        };
        // A grid of at most one workgroup per CU (small M) waits on each
        // copy: four stages (80 KB) keep three steps in flight. Batch-1
        // prefill (M = 128) 5.63 -> 4.60 ms; five and six stages were slower.
        if (!a.stages && tiles(128) <= 256) return launch_i8<64, 128, 4>(p, a.w_blocked, ksl, a.keep_slices, st);
        const bool bn96 = !a.silu_pairs && ns == 2 && a.N % 96 == 0 && load(96) < load(128);
        switch (ns) {
        case 2:
            return bn96 ? launch_i8<64, 96, 2>(p, a.w_blocked, ksl, a.keep_slices, st)
                        : launch_i8<64, 128, 2>(p, a.w_blocked, ksl, a.keep_slices, st);
        case 3: return launch_i8<64, 128, 3>(p, a.w_blocked, ksl, a.keep_slices, st);
        case 4: return launch_i8<64, 128, 4>(p, a.w_blocked, ksl, a.keep_slices, st);
        }
        return fail(VMLM_ERR_UNIMPL, "gemm (int8 rows): %d LDS stages", ns);
    }
    VMLM_GUARD(a.K > 0 && a.K % 64 == 0, "gemm: K=%d not a positive multiple of 64", a.K);
    VMLM_GUARD(((uintptr_t)a.W & 15) == 0 && ((uintptr_t)a.A & 15) == 0 && a.lda % 8 == 0,
               "gemm: operands must be 16-byte aligned");
    GemmParams p{};
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
    p.group = a.group >= 0 ? a.group : 0;
    if (a.w_int8) {
        switch (a.T) {
        case 1: return launch_g<true, 1>(p, a.bm, a.stages, st);
        case 2: return launch_g<true, 2>(p, a.bm, a.stages, st);
        case 3: return launch_g<true, 3>(p, a.bm, a.stages, st);
        }
    } else {
        switch (a.T) {
        case 1: return launch_g<false, 1>(p, a.bm, a.stages, st);
        case 2: return launch_g<false, 2>(p, a.bm, a.stages, st);
        case 3: return launch_g<false, 3>(p, a.bm, a.stages, st);
        }
    }
    return fail(VMLM_ERR_UNIMPL, "gemm: %d activation terms unsupported", a.T);
}

}  // namespace vmlm

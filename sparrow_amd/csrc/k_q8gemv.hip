// k_q8gemv.hip -- the standalone q8 GEMM at a few f32 rows (M <= 4) as one
// launch: C[m][j] = (sum_k X[m][k] * (f32)W[j][k]) * scale[j]
// (gemm_nt_int8, ops/src/kernels.rs:1256-1287) on rows and int8 weights the
// caller owns -- the call of the FFI crate's gemm_nt_int8 and of the device
// VM's OP_GEMM at decode rows.
//
// Design (gfx950):
//  * A workgroup of NW waves owns TW 16-row tiles over the whole K; wave w
//    takes the k-run of 64-wide blocks w*KB .. w*KB + KB - 1 (NW * KB = K/64)
//    and issues all of its loads (the run of each input row, its weight
//    blocks) before it waits on any.
//  * The wave splits its run of each input row itself: every lane takes
//    16-byte pieces of the row, the wave finds the row's maximum over the
//    run and splits each value into Q8_T int8 terms with the power-of-two
//    factor of that maximum (q8_row_k, q8_split) into a wave-private LDS
//    slot; the live lanes read their B fragments from there. A row costs
//    about 20 VALU operations per value and per workgroup, which is why
//    this form stops at 4 rows.
//  * Per block and tile Q8_T v_mfma_i32_16x16x64_i8 straight on the int8
//    weights give exact int32 sums of each term over the run, combined once
//    as (s0 + s1 / 2^7) + s2 / 2^14 times the row's run factor.
//  * Weights row-major as passed (lane (g, r) reads bytes 16g .. 16g + 15 of
//    the block on row r: one 16-byte load), or a swizzled copy (1 KiB MFMA
//    blocks, lane (g, r) holding bytes 8g .. +7 and 32 + 8g .. +7). The B
//    fragment of lane (g, n) takes the same k of row n, so each product
//    pairs matching k.
//  * The waves' partial tiles meet in LDS and are summed in wave order: the
//    result does not depend on scheduling.
//  * Non-finite rows: q8 gives a row holding NaN or +-inf a NaN factor, so
//    its sums are NaN; the epilogue then classifies the row's products
//    x * w in f32 (a NaN product, or both infinities: NaN; else the
//    infinity that occurs), the reference's f32 value whatever its
//    summation order.
#include "internal.hpp"

namespace vmlm {

namespace {

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

// Up to three output segments over one input (the q/k/v projections of a
// decoder layer in one launch). Tiles 0 .. tstart[1] - 1 belong to segment
// 0, and so on; with `pair`, workgroup i instead computes tile i of segment
// 0 (gate) and tile i of segment 1 (up) and also writes act = silu(gate) *
// up (the ACT and EWMUL after the gate/up projections). Every segment's
// outputs are what its own launch would give: a tile's sums do not depend
// on the tiles beside it.
struct FxSeg {
    const int8_t *W;     // row-major [N][ldw], or swizzled [N/16][K/64][1 KiB]
    const float *scale;  // [N]
    float *C;            // [M][ldc]
    int N, ldc;
};
struct FxParams {
    FxSeg seg[3];
    int nseg;
    int tstart[3];       // first tile of each segment
    int pair;            // gate/up pair (TW == 2)
    float *act;          // pair: [M][ldact]
    int ldact;
    const float *radd;   // one segment: also z = radd + C (the EWADD after the
    float *zadd;         // GEMM), both [M][ldc] of segment 0
    const float *norm_g; // NORM: the gain of the RMSNorm of the input rows,
    float *norm_out;     // the normalized rows [M][K] (written by workgroup 0)
    float norm_eps;
    int ldw;
    const float *X;      // [M][ldx]
    int ldx;
    int M, K;
};

// W[j][k] of weights W as f32 (the classification of non-finite rows)
template <bool RM>
__device__ __forceinline__ float fx_w(const int8_t *W, int ldw, int K, int j, int k) {
    if constexpr (RM) return (float)W[(size_t)j * ldw + k];
    const int o = k & 63, g = (o & 31) >> 3;
    const size_t blk = (size_t)(j >> 4) * (K >> 6) + (k >> 6);
    return (float)W[blk * 1024 + (size_t)(16 * g + (j & 15)) * 16 + (o >> 5) * 8 + (o & 7)];
}

// Row m . weight row j when row m holds a NaN or an infinity: NaN if a
// product x * w is NaN or both infinities occur, else the infinity that
// occurs; v (the q8 value) if no product is non-finite. With a gain gn the
// row is the normalized one, (x * inv) * gn.
template <bool RM>
__device__ float fx_nonfinite(const FxParams &p, const int8_t *W, int m, int j, float v,
                              float inv, const float *gn) {
    const float *x = p.X + (size_t)m * p.ldx;
    bool nan = false, pos = false, neg = false;
    for (int k = 0; k < p.K; ++k) {
        const float xk = gn ? x[k] * inv * gn[k] : x[k];
        const float t = xk * fx_w<RM>(W, p.ldw, p.K, j, k);
        nan = nan || t != t;
        pos = pos || t == __builtin_inff();
        neg = neg || t == -__builtin_inff();
    }
    if (nan || (pos && neg)) return __builtin_nanf("");
    return pos ? __builtin_inff() : neg ? -__builtin_inff() : v;
}

// Segment s, where s may differ between lanes: every field is selected from
// the three segments' scalar copies, so the kernel arguments are never read
// with a vector load (whose wait would also wait for every weight load
// issued before it).
// a load and a store through global pointers the compiler can no longer
// prove global (after in_sgpr): global, not flat, instructions, so the
// memory-counter waits before them stay exact
__device__ __forceinline__ float ld_g(const float *q) {
    return *(const __attribute__((address_space(1))) float *)q;
}
__device__ __forceinline__ void st_g(float *q, float v) {
    *(__attribute__((address_space(1))) float *)q = v;
}
template <class T>
__device__ __forceinline__ T in_sgpr(T v) {  // an opaque scalar: selects stay selects of values
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ FxSeg fx_seg(const FxParams &p, int s) {
    FxSeg r;
    r.W = in_sgpr(p.seg[0].W);
    r.scale = in_sgpr(p.seg[0].scale);
    r.C = in_sgpr(p.seg[0].C);
    r.N = in_sgpr(p.seg[0].N);
    r.ldc = in_sgpr(p.seg[0].ldc);
#pragma unroll
    for (int i = 1; i < 3; ++i) {
        const int8_t *w = in_sgpr(p.seg[i].W);
        const float *sc = in_sgpr(p.seg[i].scale);
        float *c = in_sgpr(p.seg[i].C);
        const int n = in_sgpr(p.seg[i].N), ld = in_sgpr(p.seg[i].ldc);
        if (s == i) {
            r.W = w;
            r.scale = sc;
            r.C = c;
            r.N = n;
            r.ldc = ld;
        }
    }
    return r;
}

// The segment and the tile within it of this workgroup's tile t (uniform).
__device__ __forceinline__ void fx_tile(const FxParams &p, int tw, int t, int &s, int &lt) {
    if (p.pair) {
        s = t;
        lt = blockIdx.x;
        return;
    }
    const int gt = blockIdx.x * tw + t;
    s = p.nseg > 2 && gt >= p.tstart[2] ? 2 : p.nseg > 1 && gt >= p.tstart[1] ? 1 : 0;
    const int t0 = in_sgpr(p.tstart[0]), t1 = in_sgpr(p.tstart[1]), t2 = in_sgpr(p.tstart[2]);
    lt = gt - (s == 2 ? t2 : s == 1 ? t1 : t0);  // selects of scalar copies
}

// With NORM the input row (M = 1) is first normalized (the RMSNORM opcode
// before the GEMMs): its sum of squares is formed exactly as
// rmsnorm_v4_kernel's 256 threads form it (thread t: float4 pieces t + 256 u;
// the wave sums of its four waves, then (w0 + w1) + (w2 + w3)), wave w taking
// that kernel's waves w, w + NW, ..., so inv and every y = (x * inv) * g are
// that kernel's bits.
template <int KB, int NW, int TW, bool RM, bool NORM = false>
__global__ __launch_bounds__(NW * 64) void fx_gemv_kernel(FxParams p) {
    constexpr int RUN = KB * 64;        // k of a wave's run
    constexpr int PR = RUN / 4;         // 16-byte f32 pieces of a row's run
    constexpr int XI = (PR + 63) / 64;  // pieces per lane and row
    constexpr int SLD = RUN + 16;       // padded LDS row of the terms (bytes)
    __shared__ __attribute__((aligned(16))) int8_t xs8[NW][Q8_T][FX_ROWS][SLD];
    __shared__ float red[TW][NW][16][17];
    __shared__ float nsh[4];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int nkb = p.K >> 6;
    const int kb0 = wave * KB;
    const int M = p.M;

    // 1. every global read up front: the run of each input row (piece
    // lane + 64 i), then the weight blocks of the run for each tile (rows
    // past N read row N - 1)
    float4 xv[FX_ROWS][XI];
#pragma unroll
    for (int m = 0; m < FX_ROWS; ++m) {
        if (m < M) {  // uniform
            const float *xrow = p.X + (size_t)m * p.ldx + (size_t)kb0 * 64;
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const int e = lane + 64 * i < PR ? lane + 64 * i : PR - 1;
                xv[m][i] = *(const float4 *)(xrow + 4 * e);
            }
        }
    }
    // NORM: the gain at the run's pieces, and the whole row for the sum
    // (four float4 pieces at most per thread of the 256-thread kernel: K <=
    // 4096), for its waves wave + NW v
    constexpr int VW = NORM ? (4 + NW - 1) / NW : 1;
    float4 gv[NORM ? XI : 1];
    float4 xn[VW][4];
    const int n4 = p.K >> 2, nu = (n4 + 255) >> 8;
    if constexpr (NORM) {
        const float *grun = p.norm_g + (size_t)kb0 * 64;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int e = lane + 64 * i < PR ? lane + 64 * i : PR - 1;
            gv[i] = *(const float4 *)(grun + 4 * e);
        }
#pragma unroll
        for (int v = 0; v < VW; ++v)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int vw = wave + NW * v, c = vw * 64 + lane + 256 * u;
                xn[v][u] = vw < 4 && u < nu && c < n4 ? ((const float4 *)p.X)[c]
                                                      : make_float4(0.f, 0.f, 0.f, 0.f);
            }
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wr[TW][KB];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        int sg, lt;
        fx_tile(p, TW, t, sg, lt);
        const FxSeg &S = p.seg[sg];
        const int ntile = (S.N + 15) >> 4;
        const int tl = lt < ntile ? lt : ntile - 1;
        if constexpr (RM) {
            const int row = tl * 16 + n < S.N ? tl * 16 + n : S.N - 1;
            const int8_t *wt = S.W + (size_t)row * p.ldw + (size_t)kb0 * 64 + 16 * g;
#pragma unroll
            for (int i = 0; i < KB; ++i)
                wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + 64 * i));
        } else {
            const int8_t *wt = S.W + ((size_t)tl * nkb + kb0) * 1024 + lane * 16;
#pragma unroll
            for (int i = 0; i < KB; ++i)
                wr[t][i] = __builtin_nontemporal_load((const u32x4 *)(wt + (size_t)i * 1024));
        }
    }
    // the scales of the thread's first epilogue output (row e0 % 16 of tile
    // e0 / (16 M), e0 = tid; with `pair`, of both tiles)
    const int nout = (p.pair ? 16 : TW * 16) * M;
    const int e0 = tid < nout ? tid : 0;
    int sg0, lt0;
    fx_tile(p, TW, e0 / (16 * M), sg0, lt0);
    const int row0 = lt0 * 16 + (e0 & 15);
    const FxSeg S0 = fx_seg(p, sg0);
    const float sc0 = ld_g(S0.scale + (row0 < S0.N ? row0 : S0.N - 1));
    const float sc1 = p.pair ? p.seg[1].scale[row0 < p.seg[1].N ? row0 : p.seg[1].N - 1] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    // NORM: the row's inv, the run normalized in place; workgroup 0 also
    // writes the normalized row
    float ninv = 0.0f;
    if constexpr (NORM) {
#pragma unroll
        for (int v = 0; v < VW; ++v) {
            const int vw = wave + NW * v;
            if (vw >= 4) continue;  // uniform
            float ss = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (u >= nu) continue;
                ss += xn[v][u].x * xn[v][u].x;
                ss += xn[v][u].y * xn[v][u].y;
                ss += xn[v][u].z * xn[v][u].z;
                ss += xn[v][u].w * xn[v][u].w;
            }
            ss = wave_sum(ss);
            if (lane == 0) nsh[vw] = ss;
        }
        __syncthreads();
        const float ss = ((nsh[0] + nsh[1]) + (nsh[2] + nsh[3])) / (float)p.K;
        const float inv = 1.0f / sqrtf(ss + p.norm_eps);
        ninv = inv;
        float *orow = p.norm_out + (size_t)kb0 * 64;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const float4 x = xv[0][i], gg = gv[i];
            xv[0][i] = make_float4(x.x * inv * gg.x, x.y * inv * gg.y, x.z * inv * gg.z,
                                   x.w * inv * gg.w);
            if (blockIdx.x == 0 && lane + 64 * i < PR)
                *(float4 *)(orow + 4 * (lane + 64 * i)) = xv[0][i];
        }
    }

    // 2. each row's run as int8 terms with the factor of its own maximum,
    // into the wave's LDS slot (read back below by this wave only: its LDS
    // operations complete in order)
    float fac[FX_ROWS];
#pragma unroll
    for (int m = 0; m < FX_ROWS; ++m) {
        fac[m] = 0.0f;
        if (m < M) {
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < XI; ++i)
                if (lane + 64 * i < PR)
                    mx = fmaxf(mx, fmaxf(fmaxf(q8_mag(xv[m][i].x), q8_mag(xv[m][i].y)),
                                         fmaxf(q8_mag(xv[m][i].z), q8_mag(xv[m][i].w))));
            const int k = q8_row_k(wave_max_nonneg(mx));
            fac[m] = q8_factor(k);
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const int e = lane + 64 * i;
                if (e < PR) {
                    int a[4][Q8_T];
                    q8_split(xv[m][i].x, k, a[0]);
                    q8_split(xv[m][i].y, k, a[1]);
                    q8_split(xv[m][i].z, k, a[2]);
                    q8_split(xv[m][i].w, k, a[3]);
#pragma unroll
                    for (int q = 0; q < Q8_T; ++q)
                        *(uint32_t *)&xs8[wave][q][m][4 * e] =
                            pack_i8x4(a[0][q], a[1][q], a[2][q], a[3][q]);
                }
            }
        }
    }
    // the lanes of rows past M read row 0 (their columns are never stored)
    const int nr = n < M ? n : 0;
    i32x4 b[KB][Q8_T];
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
        for (int q = 0; q < Q8_T; ++q) {
            if constexpr (RM) {
                b[i][q] = *(const i32x4 *)&xs8[wave][q][nr][i * 64 + 16 * g];
            } else {
                const uint2 lo = *(const uint2 *)&xs8[wave][q][nr][i * 64 + 8 * g];
                const uint2 hi = *(const uint2 *)&xs8[wave][q][nr][i * 64 + 32 + 8 * g];
                b[i][q] = i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            }
        }
    float rowf = fac[0];
#pragma unroll
    for (int m = 1; m < FX_ROWS; ++m)
        if (n == m) rowf = fac[m];

    // 3. per tile: Q8_T MFMAs per block, the run's exact int32 term sums
    // combined once (the term weights and the factor are powers of two)
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
        // D[row 4g + j][column n]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float f = (float)s[0][j];
#pragma unroll
            for (int u = 1; u < Q8_T; ++u) f = __builtin_fmaf((float)s[u][j], q8_term_weight(u), f);
            red[t][wave][4 * g + j][n] = f * rowf;
        }
    }
    __syncthreads();

    // 4. the waves' partial tiles summed in wave order, scaled and stored:
    // consecutive threads take consecutive rows of one input row
    auto tile_out = [&](int t, int m, int r, int row, const FxSeg &S, float scl) {
        float v = red[t][0][r][m];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[t][w][r][m];
        if (v != v) v = fx_nonfinite<RM>(p, S.W, m, row, v, ninv, NORM ? p.norm_g : nullptr);
        v = v * scl;
        st_g(S.C + (size_t)m * S.ldc + row, v);
        return v;
    };
    for (int e = tid; e < nout; e += NW * 64) {
        const int t = e / (16 * M), m = (e >> 4) % M, r = e & 15;
        int sg, lt;
        fx_tile(p, TW, t, sg, lt);
        const FxSeg S = fx_seg(p, sg);
        const int row = lt * 16 + r;
        if (row >= S.N) continue;
        const float v = tile_out(t, m, r, row, S, e == tid ? sc0 : ld_g(S.scale + row));
        if (p.zadd) p.zadd[(size_t)m * S.ldc + row] = p.radd[(size_t)m * S.ldc + row] + v;
        if (p.pair) {  // t == 0: the gate; the up value of the same output
            const float u = tile_out(1, m, r, row, p.seg[1], e == tid ? sc1 : p.seg[1].scale[row]);
            p.act[(size_t)m * p.ldact + row] = act_scalar(v, VMLM_ACT_SILU) * u;
        }
    }
}

template <int KB, int NW, int TW, bool RM, bool NORM = false>
int launch_fx_t(const FxParams &p, unsigned grid, hipStream_t st) {
    fx_gemv_kernel<KB, NW, TW, RM, NORM><<<grid, NW * 64, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace

// (blocks per run, waves) pairs with a kernel: the decoder programs' K
// (hidden 2304 or 768, inter 5760 or 2048) and small shapes
#define FX_SHAPES(X) \
    X(4, 9) X(6, 15) X(4, 3) X(4, 8) X(4, 6) X(4, 4) X(4, 2) X(4, 1) X(4, 16) X(2, 1) X(3, 1) X(6, 1)

// The k-run per wave for K: K / 64 = waves * blocks with a kernel (4 blocks
// preferred); 0 when there is none.
int fx_run_blocks(int K) {
    if (K < 128 || K % 64) return 0;
    const int nkb = K / 64;
    for (int kb : {4, 6, 3, 2}) {
        if (nkb % kb) continue;
        const int nw = nkb / kb;
#define FX_HAS(KBV, NWV) \
    if (kb == KBV && nw == NWV) return kb;
        FX_SHAPES(FX_HAS)
#undef FX_HAS
    }
    return 0;
}

// Checks shared by both entry points: the run split of K, the input rows.
static int fx_check(int M, int K, int kb, int nw, const float *X, int ldx) {
    VMLM_GUARD(M >= 1 && M <= FX_ROWS && kb && K == 64 * kb * nw,
               "q8 GEMV: shape M=%d K=%d (M <= %d, K / 64 = waves x blocks)", M, K, FX_ROWS);
    VMLM_GUARD(X && ((uintptr_t)X & 15) == 0 && ldx % 4 == 0 && ldx >= K,
               "q8 GEMV: 16-byte aligned input rows");
    return VMLM_OK;
}
static int fx_seg_check(const FxSeg &S, bool swizzled, int ldw, int K) {
    VMLM_GUARD(S.W && S.scale && S.C && S.N >= 1 && S.ldc >= S.N && ((uintptr_t)S.W & 15) == 0 &&
                   (swizzled ? S.N % 16 == 0 : ldw % 16 == 0 && ldw >= K),
               "q8 GEMV: weights, scales and outputs (16-byte aligned rows)");
    return VMLM_OK;
}

// (blocks per run, waves) pairs with a normalizing kernel (swizzled weights):
// the decoder programs' hidden sizes 2304 and 768
#define FX_NORM_SHAPES(X) X(4, 9) X(4, 3)

bool fx_norm_ok(int K) {
    const int kb = fx_run_blocks(K), nw = kb ? K / 64 / kb : 0;
#define FX_NHAS(KBV, NWV) \
    if (kb == KBV && nw == NWV) return K % 4 == 0 && K <= 4096;
    FX_NORM_SHAPES(FX_NHAS)
#undef FX_NHAS
    return false;
}

static int fx_dispatch(const FxParams &p, int kb, int nw, int tw, bool swizzled, unsigned grid,
                       hipStream_t st) {
    if (p.norm_g) {
#define FX_NLAUNCH(KBV, NWV)                                                   \
    if (kb == KBV && nw == NWV && swizzled)                                    \
        return tw == 2 ? launch_fx_t<KBV, NWV, 2, false, true>(p, grid, st)    \
                       : launch_fx_t<KBV, NWV, 1, false, true>(p, grid, st);
        FX_NORM_SHAPES(FX_NLAUNCH)
#undef FX_NLAUNCH
        return fail(VMLM_ERR_UNIMPL, "q8 GEMV: no normalizing kernel for K=%d (%d waves of %d "
                                     "blocks, %s weights)", p.K, nw, kb,
                    swizzled ? "swizzled" : "row-major");
    }
#define FX_LAUNCH(KBV, NWV)                                                    \
    if (kb == KBV && nw == NWV) {                                              \
        if (swizzled)                                                          \
            return tw == 2 ? launch_fx_t<KBV, NWV, 2, false>(p, grid, st)      \
                           : launch_fx_t<KBV, NWV, 1, false>(p, grid, st);     \
        return tw == 2 ? launch_fx_t<KBV, NWV, 2, true>(p, grid, st)           \
                       : launch_fx_t<KBV, NWV, 1, true>(p, grid, st);          \
    }
    FX_SHAPES(FX_LAUNCH)
#undef FX_LAUNCH
    return fail(VMLM_ERR_UNIMPL, "q8 GEMV: no kernel for K=%d (%d waves of %d blocks)", p.K, nw,
                kb);
}

int launch_fx_gemv(const FxArgs &a, hipStream_t st) {
    const int kb = a.kb ? a.kb : fx_run_blocks(a.K);
    const int nw = kb ? a.K / 64 / kb : 0;
    // two tiles per workgroup for wide outputs (fewer, longer workgroups),
    // one where the run is long (15 waves of 6 blocks: registers)
    const int tw = a.tw ? a.tw : a.N >= 4096 && kb <= 4 ? 2 : 1;
    int rc = fx_check(a.M, a.K, kb, nw, a.X, a.ldx);
    if (rc) return rc;
    VMLM_GUARD(tw == 1 || tw == 2, "q8 GEMV: %d tiles per workgroup", tw);
    FxParams p{};
    p.seg[0] = FxSeg{(const int8_t *)a.W, a.scale, a.C, a.N, a.ldc};
    if ((rc = fx_seg_check(p.seg[0], a.swizzled, a.ldw, a.K))) return rc;
    p.nseg = 1;
    p.ldw = a.ldw;
    p.X = a.X;
    p.ldx = a.ldx;
    p.M = a.M;
    p.K = a.K;
    return fx_dispatch(p, kb, nw, tw, a.swizzled,
                       (unsigned)((a.N + 16 * tw - 1) / (16 * tw)), st);
}

int launch_fx_multi(const FxMultiArgs &a, hipStream_t st) {
    const int kb = fx_run_blocks(a.K);
    const int nw = kb ? a.K / 64 / kb : 0;
    int rc = fx_check(a.M, a.K, kb, nw, a.X, a.ldx);
    if (rc) return rc;
    const bool pair = a.act != nullptr;
    VMLM_GUARD(a.nseg >= 1 && a.nseg <= 3 && (!pair || (a.nseg == 2 && a.seg[0].N == a.seg[1].N &&
                                                        a.ldact >= a.seg[0].N)),
               "q8 GEMV: 1..3 segments; a gate/up pair has two of one width");
    VMLM_GUARD(!a.zadd || (a.nseg == 1 && !pair && a.radd),
               "q8 GEMV: the residual add takes one segment and its addend");
    VMLM_GUARD(!a.norm_g || (a.norm_out && a.M == 1 && a.K % 4 == 0 && a.K <= 4096 &&
                             ((uintptr_t)a.norm_g & 15) == 0 && ((uintptr_t)a.norm_out & 15) == 0),
               "q8 GEMV: the RMSNorm of the input takes one row of K <= 4096 (K %% 4 == 0), "
               "a 16-byte aligned gain and output");
    FxParams p{};
    int tiles = 0;
    for (int i = 0; i < a.nseg; ++i) {
        p.seg[i] = FxSeg{(const int8_t *)a.seg[i].W, a.seg[i].scale, a.seg[i].C, a.seg[i].N,
                         a.seg[i].ldc};
        if ((rc = fx_seg_check(p.seg[i], a.swizzled, a.ldw, a.K))) return rc;
        p.tstart[i] = tiles;
        tiles += (a.seg[i].N + 15) / 16;
    }
    p.nseg = a.nseg;
    p.pair = pair;
    p.act = a.act;
    p.ldact = a.ldact;
    p.radd = a.radd;
    p.zadd = a.zadd;
    p.norm_g = a.norm_g;
    p.norm_out = a.norm_out;
    p.norm_eps = a.norm_eps;
    p.ldw = a.ldw;
    p.X = a.X;
    p.ldx = a.ldx;
    p.M = a.M;
    p.K = a.K;
    const unsigned grid = (unsigned)(pair ? (a.seg[0].N + 15) / 16 : tiles);
    return fx_dispatch(p, kb, nw, pair ? 2 : 1, a.swizzled, grid, st);
}

}  // namespace vmlm

// k_gemv.hip -- weight-streaming GEMV for decode (M <= 16 rows of activations).
//
// Replaces gemm_nt_int8 (ops/src/kernels.rs:1256-1287) and gemm_nt_bf16
// (:1199-1227) on the decode path, where every weight byte is read once per
// step and the kernel is bound by HBM bandwidth.
//
// Design (gfx950):
//  * One workgroup = 8 wavefronts on one 16-row output tile (or a gate/up
//    pair of tiles); the waves split K into 128-byte chunks and meet in LDS.
//  * Loads are shaped for full cache lines: a chunk (16 rows x 128 B) is two
//    load instructions of 8 rows x 128 B, every lane 16 B. Each wave issues
//    all of its chunk loads before consuming any (one HBM round trip per
//    launch), then passes each chunk through a 2.3 KB per-wave LDS buffer to
//    the MFMA operand layout (lane (g, r) <- row r, bytes 32g..32g+31).
//  * The dot products run on v_mfma_f32_16x16x32_bf16. int8 weights convert
//    to bf16 exactly (|q| <= 127 needs 8 significant bits); the f32
//    activations arrive pre-split into T bf16 terms (hi+mid+lo, split_bf16),
//    each an exact product with the weight, accumulated in f32 by the MFMA.
//    With T*M <= 16 the (term, batch) pairs are the MFMA's A rows (one A
//    fragment per MFMA, the terms summed in the epilogue); otherwise the
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

// Orders one wavefront's LDS writes before its following LDS reads (other
// lanes' data); LDS operations of a wavefront execute in order.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int GEMV_NW = 8;    // wavefronts per workgroup (split of K)
#ifndef GEMV_MAXC_DEF
#define GEMV_MAXC_DEF 3
#endif
#ifndef GEMV_AR_DEF
#define GEMV_AR_DEF 3
#endif
constexpr int GEMV_MAXC = GEMV_MAXC_DEF;  // 128-byte chunks per wave per pass (all loads in flight)
constexpr int GEMV_AR = GEMV_AR_DEF;      // activation chunks in flight (ring)
constexpr int CH_BYTES = 128; // chunk width per row
constexpr int CH_LD = CH_BYTES + 16;  // padded LDS row

static_assert(GEMV_NW * 64 >= 2 * 16 * 16, "epilogue maps one output per thread");

template <bool WI8, int T, int R, bool BT>
__global__ __launch_bounds__(GEMV_NW * 64) void gemv_kernel(GemvParams p) {
    constexpr int TA = BT ? 1 : T;            // A fragment sets per MFMA
    constexpr int KC = WI8 ? 128 : 64;        // k per 128-byte chunk
    constexpr int NF = KC / 32;               // MFMAs (k-slices of 32) per chunk
    constexpr int ESZ = WI8 ? 1 : 2;
    __shared__ f32x4 red[GEMV_NW][R][64];
    __shared__ float ssc[R][16];
    __shared__ __attribute__((aligned(16))) uint8_t wbuf[GEMV_NW][R][16][CH_LD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave index as a scalar: chunk counts and branches below are wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rr = lane & 15;
    const int lrow = lane >> 3, lcol = (lane & 7) * 16;  // load layout: 8 rows x 128 B
    const int NCH = p.K / KC;
    // A rows past the live ones re-read row 0: their MFMA output rows are
    // never read, and unconditional loads keep the memory counters exact
    const int arows = BT ? T * p.M : p.M;
    const uint16_t *abase = p.A + (size_t)(rr < arows ? rr : 0) * p.lda + g * (KC / 4);

    const uint8_t *wrow[R][2];
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int j = (blockIdx.x * R + t) * 16 + lrow + 8 * h;
            j = j < p.N ? j : p.N - 1;
            wrow[t][h] = p.W + (size_t)j * p.K * ESZ + lcol;
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

    for (int base = 0; base < NCH; base += GEMV_NW * GEMV_MAXC) {
        const int Cp = (NCH - base) < GEMV_NW * GEMV_MAXC ? (NCH - base) : GEMV_NW * GEMV_MAXC;
        const int c0 = base + (Cp * wave) / GEMV_NW;
        const int n = base + (Cp * (wave + 1)) / GEMV_NW - c0;
        // every load below is issued unconditionally (slots past this wave's
        // n chunks re-read a valid chunk and are not consumed): a load under
        // a branch makes the compiler drain the whole memory queue before the
        // next one, serialising the stream into one round trip per chunk
        auto chunk = [&](int i) {
            const int c = c0 + i;
            return c < NCH ? c : NCH - 1;
        };
        u32x4 av[GEMV_AR][TA][NF];
        auto load_a = [&](int i, u32x4 (&dst)[TA][NF]) {
            const uint16_t *ap = abase + (size_t)chunk(i) * KC;
#pragma unroll
            for (int tt = 0; tt < TA; ++tt)
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    dst[tt][f] = ldg16_cached(ap + (BT ? 0 : tt * p.tstride) + 8 * f);
        };
        // activation fragments of the first chunks go out first: the memory
        // counter retires in order, so they must not queue behind the weights
#pragma unroll
        for (int i = 0; i < GEMV_AR; ++i) load_a(i, av[i]);
        u32x4 wv[GEMV_MAXC][R][2];
#pragma unroll
        for (int i = 0; i < GEMV_MAXC; ++i)
#pragma unroll
            for (int t = 0; t < R; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    wv[i][t][h] = ldg16(wrow[t][h] + (size_t)chunk(i) * CH_BYTES);
#pragma unroll
        for (int i = 0; i < GEMV_MAXC; ++i) {
            u32x4 cur[TA][NF];
#pragma unroll
            for (int tt = 0; tt < TA; ++tt)
#pragma unroll
                for (int f = 0; f < NF; ++f) cur[tt][f] = av[i % GEMV_AR][tt][f];
            if (i + GEMV_AR < GEMV_MAXC) load_a(i + GEMV_AR, av[i % GEMV_AR]);
            if (i < n) {
#pragma unroll
                for (int t = 0; t < R; ++t) {
                    uint8_t(*buf)[CH_LD] = wbuf[wave][t];
                    *(u32x4 *)&buf[lrow][lcol] = wv[i][t][0];
                    *(u32x4 *)&buf[lrow + 8][lcol] = wv[i][t][1];
                    wave_lds_sync();
                    const u32x4 r0 = *(const u32x4 *)&buf[rr][g * 32];
                    const u32x4 r1 = *(const u32x4 *)&buf[rr][g * 32 + 16];
                    wave_lds_sync();
                    u32x4 bfr[NF];
                    if constexpr (WI8) {
                        i8x16_to_bf16(r0, bfr[0], bfr[1]);
                        i8x16_to_bf16(r1, bfr[2], bfr[3]);
                    } else {
                        bfr[0] = r0;
                        bfr[1] = r1;
                    }
#pragma unroll
                    for (int f = 0; f < NF; ++f)
#pragma unroll
                        for (int tt = 0; tt < TA; ++tt)
                            acc[t] = mfma_bf16(cur[tt][f], bfr[f], acc[t]);
                }
            }
        }
    }

    // ---- cross-wave reduction, fused with the epilogue: D[row = 4g+i][col =
    // rr] of tile t sits in red[*][t][(row / 4) * 16 + col][row % 4]; each
    // output sums its accumulator row over the waves, then (term, batch) rows
    // over the terms, in that fixed order
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = acc[t];
    // one output per thread (R * M * 16 <= 512): the residual operand is
    // fetched before the barrier so its latency overlaps the reduction
    const bool live = tid < (p.epi == EPI_SILU_MUL ? 1 : R) * p.M * 16;
    const int et = tid / (p.M * 16), eb = (tid >> 4) % p.M, ecol = tid & 15;
    const int ej = (blockIdx.x * R + et) * 16 + ecol;
    const bool ein = live && ej < p.N;
    float resid = 0.0f;
    if (ein && p.epi == EPI_RESIDUAL) resid = p.Rr[(size_t)eb * p.ldr + ej];
    __syncthreads();
    auto dsum = [&](int t, int row, int col) {
        const int ln = (row >> 2) * 16 + col, i = row & 3;
        float v = red[0][t][ln][i];
#pragma unroll
        for (int w = 1; w < GEMV_NW; ++w) v += red[w][t][ln][i];
        return v;
    };
    auto rowval = [&](int t, int b, int col) {
        if constexpr (BT) {
            float v = dsum(t, b, col);
#pragma unroll
            for (int tt = 1; tt < T; ++tt) v += dsum(t, tt * p.M + b, col);
            return v;
        } else {
            return dsum(t, b, col);
        }
    };
    if (!live) return;
    if (p.epi == EPI_SILU_MUL) {  // tile 0 = gate rows, tile 1 = up rows
        const int jo = blockIdx.x * 16 + ecol;
        const float gate = rowval(0, eb, ecol) * ssc[0][ecol];
        const float up = rowval(R - 1, eb, ecol) * ssc[R - 1][ecol];
        float a = (gate / (1.0f + exp_f(-gate))) * up;
        p.Y[(size_t)eb * p.ldy + jo] = a;
        for (int tt = 0; tt < p.Tout; ++tt) {
            const uint32_t h = bf16_rne_bits(a);
            a = a - bf16_bits_to_f32(h);
            p.Aout[((size_t)tt * p.M + eb) * p.ldaout + jo] = (uint16_t)h;
        }
        return;
    }
    float y = 0.0f;
    if (ein) {
        y = p.scale ? rowval(et, eb, ecol) * ssc[et][ecol] : rowval(et, eb, ecol);
        if (p.epi == EPI_RESIDUAL) y = resid + y;
        p.Y[(size_t)eb * p.ldy + ej] = y;
    }
    if (p.epi == EPI_ARGMAX) {
        // 16 consecutive threads hold the 16 columns of row eb: reduce keys
        unsigned long long k = 0;
        if (ein && y == y) k = argmax_key(y, (uint32_t)ej);
        if (ein && ej == 0 && y != y) k = ARGMAX_NAN0_KEY;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            unsigned long long ok = __shfl_xor(k, o, 64);
            k = ok > k ? ok : k;
        }
        if (ecol == 0 && k)
            atomicMax(p.keys + (size_t)eb * KEY_SLOTS + (blockIdx.x & (KEY_SLOTS - 1)), k);
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
    VMLM_GUARD(a.K > 0 && a.K % (a.w_int8 ? 128 : 64) == 0,
               "gemv: K=%d not a positive multiple of %d", a.K, a.w_int8 ? 128 : 64);
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

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
    int lda, M, N, K, ldy, ldr, ldaout, Tout, epi, ks;
    const float *X;  // wide kernel: f32 activation rows [M][ldx], split while staged
    int ldx;
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
constexpr int CH_BYTES = 128; // chunk width per row
constexpr int CH_LD = CH_BYTES + 16;  // padded LDS row

// MAXC: 128-byte chunks per wave per pass, all loads in flight; AR:
// activation chunks in flight (ring); R: 16-row tiles sharing the activation
// fragments (SiLU: R/2 gate/up pairs).
template <bool WI8, int T, int R, bool BT, int MAXC, int AR>
__global__ __launch_bounds__(GEMV_NW * 64) void gemv_kernel(GemvParams p) {
    constexpr int TA = BT ? 1 : T;            // A fragment sets per MFMA
    constexpr int KC = WI8 ? 128 : 64;        // k per 128-byte chunk
    constexpr int NF = KC / 32;               // MFMAs (k-slices of 32) per chunk
    constexpr int ESZ = WI8 ? 1 : 2;
    // one transpose buffer per wave (tiles pass through it in turn); the
    // cross-wave reduction reuses the same bytes after a barrier
    constexpr int WBUF_BYTES = GEMV_NW * 16 * CH_LD;
    constexpr int RED_BYTES = GEMV_NW * R * 64 * 16;
    __shared__ __attribute__((aligned(16)))
    uint8_t smem[WBUF_BYTES > RED_BYTES ? WBUF_BYTES : RED_BYTES];
    __shared__ float ssc[R][16];
    auto wbuf = reinterpret_cast<uint8_t(*)[16][CH_LD]>(smem);
    auto red = reinterpret_cast<f32x4(*)[R][64]>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave index as a scalar: chunk counts and branches below are wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rr = lane & 15;
    const int lrow = lane >> 3, lcol = (lane & 7) * 16;  // load layout: 8 rows x 128 B
    // split K: workgroup row blockIdx.y takes k-slice [ks * K / KS, ...)
    const int NCH = p.K / KC / gridDim.y;
    const int ch0 = blockIdx.y * NCH;
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

    for (int base = 0; base < NCH; base += GEMV_NW * MAXC) {
        const int Cp = (NCH - base) < GEMV_NW * MAXC ? (NCH - base) : GEMV_NW * MAXC;
        const int c0 = base + (Cp * wave) / GEMV_NW;
        const int n = base + (Cp * (wave + 1)) / GEMV_NW - c0;
        // every load below is issued unconditionally (slots past this wave's
        // n chunks re-read a valid chunk and are not consumed): a load under
        // a branch makes the compiler drain the whole memory queue before the
        // next one, serialising the stream into one round trip per chunk
        auto chunk = [&](int i) {
            const int c = c0 + i;
            return ch0 + (c < NCH ? c : NCH - 1);
        };
        u32x4 av[AR][TA][NF];
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
        for (int i = 0; i < AR; ++i) load_a(i, av[i]);
        u32x4 wv[MAXC][R][2];
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
#pragma unroll
            for (int t = 0; t < R; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    wv[i][t][h] = ldg16(wrow[t][h] + (size_t)chunk(i) * CH_BYTES);
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            u32x4 cur[TA][NF];
#pragma unroll
            for (int tt = 0; tt < TA; ++tt)
#pragma unroll
                for (int f = 0; f < NF; ++f) cur[tt][f] = av[i % AR][tt][f];
            if (i + AR < MAXC) load_a(i + AR, av[i % AR]);
            if (i < n) {
#pragma unroll
                for (int t = 0; t < R; ++t) {
                    uint8_t(*buf)[CH_LD] = wbuf[wave];
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
    __syncthreads();  // every wave is done with its transpose buffer
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = acc[t];
    // outputs (tile or pair, batch row, column); the first pass's residual
    // operand is fetched before the barrier so its latency overlaps the
    // reduction
    const bool silu = p.epi == EPI_SILU_MUL;
    const int nout = (silu ? R / 2 : R) * p.M * 16;
    auto coords = [&](int e, int &t, int &b, int &col) {
        t = e / (p.M * 16);
        b = (e >> 4) % p.M;
        col = e & 15;
    };
    float resid0 = 0.0f;
    if (p.epi == EPI_RESIDUAL && tid < nout) {
        int t, b, col;
        coords(tid, t, b, col);
        const int j = (blockIdx.x * R + t) * 16 + col;
        if (j < p.N) resid0 = p.Rr[(size_t)b * p.ldr + j];
    }
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
    for (int e = tid; e < nout; e += GEMV_NW * 64) {
        int t, b, col;
        coords(e, t, b, col);
        if (silu) {  // pair t: tile 2t = gate rows, tile 2t + 1 = up rows
            const int jo = (blockIdx.x * (R / 2) + t) * 16 + col;
            const float gate = rowval(2 * t, b, col) * ssc[2 * t][col];
            const float up = rowval(2 * t + 1, b, col) * ssc[2 * t + 1][col];
            float a = (gate / (1.0f + exp_f(-gate))) * up;
            p.Y[(size_t)b * p.ldy + jo] = a;
            for (int tt = 0; tt < p.Tout; ++tt) {
                const uint32_t h = bf16_rne_bits(a);
                a = term_rem(a, h);
                p.Aout[((size_t)tt * p.M + b) * p.ldaout + jo] = (uint16_t)h;
            }
            continue;
        }
        const int j = (blockIdx.x * R + t) * 16 + col;
        const bool in = j < p.N;
        if (p.epi == EPI_PARTIAL) {  // raw k-slice sums, reduced by the consumer
            if (in) p.Y[((size_t)blockIdx.y * p.M + b) * p.ldy + j] = rowval(t, b, col);
            continue;
        }
        float y = 0.0f;
        if (in) {
            y = p.scale ? rowval(t, b, col) * ssc[t][col] : rowval(t, b, col);
            if (p.epi == EPI_RESIDUAL)
                y = (e == tid ? resid0 : p.Rr[(size_t)b * p.ldr + j]) + y;
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
            if (col == 0 && k)
                atomicMax(p.keys + (size_t)b * KEY_SLOTS + (blockIdx.x & (KEY_SLOTS - 1)), k);
        }
    }
}

// ---------------------------------------------------------------------------
// Wide variant for int8 weights: the NWV (8 or 16) waves of a workgroup own
// NWV different 16-row tiles over one k-slice of NC chunks (blockIdx.y), and
// share that slice of the activation terms, loaded once into LDS. Activation
// bytes from L2 per weight byte drop from M*T*2/16 (one tile per workgroup)
// to M*T*2/(16*NWV). All weight chunks of a wave and the activation slice are in
// flight together (one memory round trip); the workgroup's k-slice sums go
// out raw (EPI_PARTIAL, reduced in a fixed order by the consumer) or, with a
// single slice, through the usual epilogues.
template <int T, bool BT, int NC, int NWV, bool XF32>
__global__ __launch_bounds__(NWV * 64) void gemv_wide_kernel(GemvParams p) {
    constexpr int NTH = NWV * 64;
    constexpr int TA = BT ? 1 : T;
    constexpr int KW = NC * 128;  // k of the slice
    constexpr int ALD = KW + 8;   // LDS row of the activation slice (+16 B)
    __shared__ __attribute__((aligned(16))) uint16_t as[TA][16][ALD];
    __shared__ __attribute__((aligned(16))) uint8_t wbuf[NWV][16][CH_LD];
    __shared__ float dwave[NWV][16][17];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rr = lane & 15;
    const int lrow = lane >> 3, lcol = (lane & 7) * 16;
    const int tile = blockIdx.x * NWV + wave;
    const int k0 = blockIdx.y * KW;

    // this wave's weight rows, every chunk of the slice (rows clamped),
    // issued after the activation loads below: those return first, so the
    // activation is split and staged while the weights are in flight
    u32x4 wv[NC][2];
    auto load_w = [&]() {
        int j0 = tile * 16 + lrow, j1 = j0 + 8;
        j0 = j0 < p.N ? j0 : p.N - 1;
        j1 = j1 < p.N ? j1 : p.N - 1;
        const uint8_t *w0 = p.W + (size_t)j0 * p.K + k0 + lcol;
        const uint8_t *w1 = p.W + (size_t)j1 * p.K + k0 + lcol;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            wv[c][0] = ldg16(w0 + c * CH_BYTES);
            wv[c][1] = ldg16(w1 + c * CH_BYTES);
        }
    };
    // the activation slice [TA][16 rows][KW] -> LDS in 16-byte pieces; rows
    // past the live ones repeat row 0 (their outputs are never read). From
    // f32 rows (p.X) each thread splits 8 values into the T terms.
    const int arows = BT ? T * p.M : p.M;
    if constexpr (XF32) {
        constexpr int UNITS = 16 * (KW / 8);
        constexpr int UPER = (UNITS + NTH - 1) / NTH;
        float4 xv[UPER][2];
#pragma unroll
        for (int i = 0; i < UPER; ++i) {
            int e = tid + i * NTH;
            e = e < UNITS ? e : UNITS - 1;
            const int r = e / (KW / 8), c8 = e % (KW / 8);
            const float *xr = p.X + (size_t)(r < p.M ? r : 0) * p.ldx + k0 + c8 * 8;
            xv[i][0] = *(const float4 *)xr;
            xv[i][1] = *(const float4 *)(xr + 4);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_w();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < UPER; ++i) {
            const int e = tid + i * NTH;
            const int r = e / (KW / 8), c8 = e % (KW / 8);
            float y[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                          xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                uint32_t hb[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    hb[q] = bf16_rne_bits(y[q]);
                    y[q] = term_rem(y[q], hb[q]);
                }
                const u32x4 pk = u32x4{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16),
                                       hb[4] | (hb[5] << 16), hb[6] | (hb[7] << 16)};
                if (e < UNITS && (!BT || r < p.M))
                    *(u32x4 *)&as[BT ? 0 : tt][BT ? tt * p.M + r : r][c8 * 8] = pk;
            }
        }
    } else {
        constexpr int PIECES = TA * 16 * (KW / 8);
        constexpr int PER = (PIECES + NTH - 1) / NTH;
        u32x4 ap[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int e = tid + i * NTH;
            e = e < PIECES ? e : PIECES - 1;
            const int tt = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
            const int rs = r < arows ? r : 0;
            ap[i] = ldg16_cached(p.A + (BT ? 0 : tt * p.tstride) + (size_t)rs * p.lda + k0 + c8 * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_w();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int e = tid + i * NTH;
            e = e < PIECES ? e : PIECES - 1;
            const int tt = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
            *(u32x4 *)&as[tt][r][c8 * 8] = ap[i];
        }
    }
    __syncthreads();

    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        uint8_t(*buf)[CH_LD] = wbuf[wave];
        *(u32x4 *)&buf[lrow][lcol] = wv[c][0];
        *(u32x4 *)&buf[lrow + 8][lcol] = wv[c][1];
        wave_lds_sync();
        const u32x4 r0 = *(const u32x4 *)&buf[rr][g * 32];
        const u32x4 r1 = *(const u32x4 *)&buf[rr][g * 32 + 16];
        wave_lds_sync();
        u32x4 bfr[4];
        i8x16_to_bf16(r0, bfr[0], bfr[1]);
        i8x16_to_bf16(r1, bfr[2], bfr[3]);
        // fragment f of lane (g, r): k = c*128 + 32g + 8f .. +7 (as the B side)
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int tt = 0; tt < TA; ++tt)
                acc = mfma_bf16(*(const u32x4 *)&as[tt][rr][c * 128 + g * 32 + 8 * f], bfr[f], acc);
    }

    // D[row = 4g + i][col = rr]: rows are (term, batch) or batch rows
#pragma unroll
    for (int i = 0; i < 4; ++i) dwave[wave][4 * g + i][rr] = acc[i];
    if (p.epi == EPI_SILU_MUL) __syncthreads();  // pairs read the partner wave's tile
    else wave_lds_sync();
    auto val = [&](int w, int b, int col) {
        float v = dwave[w][b][col];
        if constexpr (BT) {
#pragma unroll
            for (int tt = 1; tt < T; ++tt) v += dwave[w][tt * p.M + b][col];
        }
        return v;
    };
    if (p.epi == EPI_SILU_MUL) {  // wave 2q: gate tile, wave 2q + 1: up tile
        if (wave & 1) return;
        const int pt = blockIdx.x * (NWV / 2) + (wave >> 1);
        for (int e = lane; e < p.M * 16; e += 64) {
            const int b = e >> 4, col = e & 15;
            const int jg = tile * 16 + col, ju = jg + 16, jo = pt * 16 + col;
            const float gate = val(wave, b, col) * p.scale[jg];
            const float up = val(wave + 1, b, col) * p.scale[ju];
            float a = (gate / (1.0f + exp_f(-gate))) * up;
            p.Y[(size_t)b * p.ldy + jo] = a;
            for (int tt = 0; tt < p.Tout; ++tt) {
                const uint32_t h = bf16_rne_bits(a);
                a = term_rem(a, h);
                p.Aout[((size_t)tt * p.M + b) * p.ldaout + jo] = (uint16_t)h;
            }
        }
        return;
    }
    for (int e = lane; e < p.M * 16; e += 64) {
        const int b = e >> 4, col = e & 15;
        const int j = tile * 16 + col;
        if (j >= p.N) continue;
        const float v = val(wave, b, col);
        if (p.epi == EPI_PARTIAL) {
            p.Y[((size_t)blockIdx.y * p.M + b) * p.ldy + j] = v;
        } else {
            float y = p.scale ? v * p.scale[j] : v;
            if (p.epi == EPI_RESIDUAL) y = p.Rr[(size_t)b * p.ldr + j] + y;
            p.Y[(size_t)b * p.ldy + j] = y;
        }
    }
}

// Wide variant with a k-loop, for full-K workgroups (the LM head, and any
// projection whose k-slice spans more than three chunks): the 8 waves own 8
// row tiles; the k-range advances in steps of SC chunks. Per step the
// activation slice is staged through a double-buffered LDS area (loaded one
// step ahead), and each wave keeps the weight chunks of the next two steps
// in flight in a 3-slot register ring (the loop is unrolled by 3 so every
// slot is a fixed set of registers).
template <bool WI8, int T, bool BT, int SC>
__global__ __launch_bounds__(512) void gemv_wloop_kernel(GemvParams p) {
    constexpr int TA = BT ? 1 : T;
    constexpr int KC = WI8 ? 128 : 64;  // k per 128-byte chunk
    constexpr int NF = KC / 32;
    constexpr int ESZ = WI8 ? 1 : 2;
    constexpr int KW = SC * KC;         // k per step
    constexpr int ALD = KW + 8;
    __shared__ __attribute__((aligned(16))) uint16_t as[2][TA][16][ALD];
    __shared__ __attribute__((aligned(16))) uint8_t wbuf[8][16][CH_LD];
    __shared__ float dwave[8][16][17];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rr = lane & 15;
    const int lrow = lane >> 3, lcol = (lane & 7) * 16;
    const int tile = blockIdx.x * 8 + wave;
    const int nsteps = p.K / KW / (int)gridDim.y;
    const int kslice = blockIdx.y * nsteps * KW;

    int j0 = tile * 16 + lrow, j1 = j0 + 8;
    j0 = j0 < p.N ? j0 : p.N - 1;
    j1 = j1 < p.N ? j1 : p.N - 1;
    const uint8_t *w0 = p.W + ((size_t)j0 * p.K + kslice) * ESZ + lcol;
    const uint8_t *w1 = p.W + ((size_t)j1 * p.K + kslice) * ESZ + lcol;
    auto load_w = [&](int s, u32x4 (&dst)[SC][2]) {
        s = s < nsteps ? s : nsteps - 1;
#pragma unroll
        for (int c = 0; c < SC; ++c) {
            const size_t off = ((size_t)s * SC + c) * CH_BYTES;
            dst[c][0] = ldg16(w0 + off);
            dst[c][1] = ldg16(w1 + off);
        }
    };
    const int arows = BT ? T * p.M : p.M;
    constexpr int PIECES = TA * 16 * (KW / 8);
    constexpr int PER = (PIECES + 511) / 512;
    auto load_a = [&](int s, u32x4 (&dst)[PER]) {
        s = s < nsteps ? s : nsteps - 1;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int e = tid + i * 512;
            e = e < PIECES ? e : PIECES - 1;
            const int tt = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
            const int rs = r < arows ? r : 0;
            dst[i] = ldg16_cached(p.A + (BT ? 0 : tt * p.tstride) + (size_t)rs * p.lda + kslice +
                                  (size_t)s * KW + c8 * 8);
        }
    };
    auto store_a = [&](int buf, const u32x4 (&src)[PER]) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int e = tid + i * 512;
            e = e < PIECES ? e : PIECES - 1;
            const int tt = e / (16 * (KW / 8)), r = (e / (KW / 8)) % 16, c8 = e % (KW / 8);
            *(u32x4 *)&as[buf][tt][r][c8 * 8] = src[i];
        }
    };

    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const u32x4 (&w)[SC][2]) {
#pragma unroll
        for (int c = 0; c < SC; ++c) {
            uint8_t(*bw)[CH_LD] = wbuf[wave];
            *(u32x4 *)&bw[lrow][lcol] = w[c][0];
            *(u32x4 *)&bw[lrow + 8][lcol] = w[c][1];
            wave_lds_sync();
            const u32x4 r0 = *(const u32x4 *)&bw[rr][g * 32];
            const u32x4 r1 = *(const u32x4 *)&bw[rr][g * 32 + 16];
            wave_lds_sync();
            u32x4 bfr[NF];
            if constexpr (WI8) {
                i8x16_to_bf16(r0, bfr[0], bfr[1]);
                i8x16_to_bf16(r1, bfr[2], bfr[3]);
            } else {
                bfr[0] = r0;
                bfr[1] = r1;
            }
            // fragment f of lane (g, r): k = c*KC + (KC/4)*g + 8f .. +7
#pragma unroll
            for (int f = 0; f < NF; ++f)
#pragma unroll
                for (int tt = 0; tt < TA; ++tt)
                    acc = mfma_bf16(
                        *(const u32x4 *)&as[buf][tt][rr][c * KC + g * (KC / 4) + 8 * f], bfr[f],
                        acc);
        }
    };

    u32x4 wa[SC][2], wb[SC][2], wc[SC][2];
    u32x4 ap[PER];
    load_a(0, ap);
    load_w(0, wa);
    load_w(1, wb);
    store_a(0, ap);
    load_a(1, ap);
    __syncthreads();
    // step s: weights of s in the ring slot s % 3, activation of s in LDS
    // buffer s & 1, activation of s + 1 in registers
    auto step = [&](int s, u32x4 (&wcur)[SC][2], u32x4 (&wnext2)[SC][2]) {
        load_w(s + 2, wnext2);
        compute(s & 1, wcur);
        store_a((s + 1) & 1, ap);
        load_a(s + 2, ap);
        __syncthreads();
    };
    for (int s = 0; s < nsteps; s += 3) {
        step(s, wa, wc);
        if (s + 1 < nsteps) step(s + 1, wb, wa);
        if (s + 2 < nsteps) step(s + 2, wc, wb);
    }

    // D[row = 4g + i][col = rr]: rows are (term, batch) or batch rows
#pragma unroll
    for (int i = 0; i < 4; ++i) dwave[wave][4 * g + i][rr] = acc[i];
    if (p.epi == EPI_SILU_MUL) __syncthreads();
    else wave_lds_sync();
    auto val = [&](int w, int b, int col) {
        float v = dwave[w][b][col];
        if constexpr (BT) {
#pragma unroll
            for (int tt = 1; tt < T; ++tt) v += dwave[w][tt * p.M + b][col];
        }
        return v;
    };
    if (p.epi == EPI_SILU_MUL) {  // wave 2q: gate tile, wave 2q + 1: up tile
        if (wave & 1) return;
        const int pt = blockIdx.x * 4 + (wave >> 1);
        for (int e = lane; e < p.M * 16; e += 64) {
            const int b = e >> 4, col = e & 15;
            const int jg = tile * 16 + col, ju = jg + 16, jo = pt * 16 + col;
            const float gate = val(wave, b, col) * p.scale[jg];
            const float up = val(wave + 1, b, col) * p.scale[ju];
            float a = (gate / (1.0f + exp_f(-gate))) * up;
            p.Y[(size_t)b * p.ldy + jo] = a;
            for (int tt = 0; tt < p.Tout; ++tt) {
                const uint32_t h = bf16_rne_bits(a);
                a = term_rem(a, h);
                p.Aout[((size_t)tt * p.M + b) * p.ldaout + jo] = (uint16_t)h;
            }
        }
        return;
    }
    for (int e = lane; e < p.M * 16; e += 64) {
        const int b = e >> 4, col = e & 15;
        const int j = tile * 16 + col;
        const bool in = j < p.N;
        const float v = val(wave, b, col);
        if (p.epi == EPI_PARTIAL) {
            if (in) p.Y[((size_t)blockIdx.y * p.M + b) * p.ldy + j] = v;
            continue;
        }
        float y = p.scale ? v * p.scale[in ? j : 0] : v;
        if (in && p.epi == EPI_RESIDUAL) y = p.Rr[(size_t)b * p.ldr + j] + y;
        if (in) p.Y[(size_t)b * p.ldy + j] = y;
        if (p.epi == EPI_ARGMAX) {
            // 16 consecutive lanes hold the 16 columns of row b
            unsigned long long k = 0;
            if (in && y == y) k = argmax_key(y, (uint32_t)j);
            if (in && j == 0 && y != y) k = ARGMAX_NAN0_KEY;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const unsigned long long ok = __shfl_xor(k, o, 64);
                k = ok > k ? ok : k;
            }
            if (col == 0 && k)
                atomicMax(p.keys + (size_t)b * KEY_SLOTS + (tile & (KEY_SLOTS - 1)), k);
        }
    }
}

template <bool WI8, int T, bool BT>
static int launch_wloop_t(const GemvParams &p, hipStream_t st) {
    const dim3 grid((p.N + 127) / 128, p.ks);
    gemv_wloop_kernel<WI8, T, BT, 1><<<grid, 512, 0, st>>>(p);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Workgroups of one wide-kernel variant resident on the device at once.
template <int T, bool BT, int NC, int NWV>
static int wide_slots() {
    static int slots = -1;
    if (slots < 0) {
        int per_cu = 0, dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, (const void *)gemv_wide_kernel<T, BT, NC, NWV, false>, NWV * 64, 0) !=
                hipSuccess)
            return 0;
        slots = per_cu * cus;
    }
    return slots;
}

template <int T, bool BT, int NC, bool XF32>
static void launch_wide_x(const GemvParams &p, bool wide16, hipStream_t st) {
    if (wide16)
        gemv_wide_kernel<T, BT, NC, 16, XF32><<<dim3(p.N / 256, p.ks), 1024, 0, st>>>(p);
    else
        gemv_wide_kernel<T, BT, NC, 8, XF32><<<dim3((p.N + 127) / 128, p.ks), 512, 0, st>>>(p);
}

// 8 waves (128 rows) per workgroup while the grid fits on the device in one
// round; 16 waves (256 rows, half the workgroups) when it would spill into a
// second round and the rows split evenly.
template <int T, bool BT, int NC>
static int launch_wide_nc(const GemvParams &p, hipStream_t st) {
    const int wgs8 = (p.N + 127) / 128 * p.ks;
    const bool wide16 = p.N % 256 == 0 && wgs8 > wide_slots<T, BT, NC, 8>();
    if (p.X)
        launch_wide_x<T, BT, NC, true>(p, wide16, st);
    else
        launch_wide_x<T, BT, NC, false>(p, wide16, st);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

template <int T, bool BT>
static int launch_wide_t(const GemvParams &p, int nc, hipStream_t st) {
    switch (nc) {
    case 1: return launch_wide_nc<T, BT, 1>(p, st);
    case 2: return launch_wide_nc<T, BT, 2>(p, st);
    case 3: return launch_wide_nc<T, BT, 3>(p, st);
    default: return fail(VMLM_ERR_UNIMPL, "gemv wide: %d chunks per slice", nc);
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
        v = term_rem(v, h);
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
    // chunk depth / activation ring per tile count, from measurements: one
    // tile keeps three chunks and their activation fragments in flight; more
    // tiles share one activation chunk at a time (register budget)
    constexpr int MAXC = 3, AR = R == 1 ? 3 : 1;
    int wgs = (p.N + 16 * R - 1) / (16 * R);
    if (p.epi == EPI_SILU_MUL) wgs = p.N / (16 * R);
    gemv_kernel<WI8, T, R, BT, MAXC, AR><<<dim3(wgs, p.ks), GEMV_NW * 64, 0, st>>>(p);
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

// C[b][j] = (sum over the ks k-slices of part[s][b][j], in slice order) * scale[j];
// every slice of an output is loaded up front (index clamped).
constexpr int RED_KS_MAX = 16;
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float *__restrict__ part, int ks,
                                                          int M, int N,
                                                          const float *__restrict__ scale,
                                                          float *__restrict__ C, int ldc) {
    const int n = M * N;
    int i = blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;
    i = live ? i : n - 1;
    float v[RED_KS_MAX];
#pragma unroll
    for (int s = 0; s < RED_KS_MAX; ++s) v[s] = part[(size_t)(s < ks ? s : ks - 1) * n + i];
    float acc = v[0];
#pragma unroll
    for (int s = 1; s < RED_KS_MAX; ++s)
        if (s < ks) acc += v[s];
    if (!live) return;
    const int b = i / N, j = i % N;
    C[(size_t)b * ldc + j] = scale ? acc * scale[j] : acc;
}

int launch_gemv_reduce(const float *part, int ks, int M, int N, const float *scale, float *C,
                       int ldc, hipStream_t st) {
    VMLM_GUARD(ks >= 1 && ks <= RED_KS_MAX && M >= 1 && N >= 1,
               "gemv reduce: 1 <= ks <= %d k-slices", RED_KS_MAX);
    const size_t n = (size_t)M * N;
    gemv_reduce_kernel<<<cdiv(n, 256), 256, 0, st>>>(part, ks, M, N, scale, C, ldc);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_gemv(const GemvArgs &a, hipStream_t st) {
    VMLM_GUARD(a.M >= 1 && a.M <= 16, "gemv: M=%d outside 1..16", a.M);
    VMLM_GUARD(a.K > 0 && a.K % (a.w_int8 ? 128 : 64) == 0,
               "gemv: K=%d not a positive multiple of %d", a.K, a.w_int8 ? 128 : 64);
    VMLM_GUARD(a.N > 0, "gemv: N=%d", a.N);
    VMLM_GUARD(((uintptr_t)a.W & 15) == 0 && ((uintptr_t)a.A & 15) == 0 && a.lda % 64 == 0,
               "gemv: operands must be 16-byte aligned with lda %% 64 == 0");
    VMLM_GUARD(!a.X || (a.tiles == 8 && ((uintptr_t)a.X & 15) == 0 && a.ldx % 4 == 0),
               "gemv: f32 activation rows need the wide kernel and 16-byte aligned rows");
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
    p.ks = a.ksplit > 0 ? a.ksplit : 1;
    p.X = a.X;
    p.ldx = a.ldx;
    VMLM_GUARD(p.ks == 1 || (a.epi == EPI_PARTIAL && (a.K / (a.w_int8 ? 128 : 64)) % p.ks == 0) ||
                   (a.tiles >= 8 && a.epi == EPI_PARTIAL),
               "gemv: k-split %d needs EPI_PARTIAL and whole chunks per slice", p.ks);
    // (term, batch) rows need the planes contiguous: row r = buffer row r
    const bool bt = a.T > 1 && a.T * a.M <= 16 && p.tstride == (size_t)a.M * a.lda;
    // Tiles per workgroup: the activation fragments a wave loads serve R
    // tiles, so R trades activation traffic (M * T * 2 bytes per k per
    // workgroup) against workgroup count. One tile while the activation is a
    // few (term, batch) rows; with a full 16-row batch, 4 tiles where that
    // still leaves a workgroup for most CUs.
    int R = a.tiles;
    if (R == 9) {  // wide with a k-loop: 128 rows per workgroup, any k-slice length
        const int kstep = 128;  // int8: one chunk per step; bf16: two
        VMLM_GUARD(a.K % kstep == 0 && (a.K / kstep) % p.ks == 0,
                   "gemv wide loop: K %% 128 and whole steps per k-slice");
        VMLM_GUARD(p.ks == 1 || a.epi == EPI_PARTIAL, "gemv wide loop: k-slices need EPI_PARTIAL");
        VMLM_GUARD(a.epi != EPI_SILU_MUL || (a.N % 128 == 0 && a.scale && a.Aout && a.w_int8),
                   "gemv wide loop silu: int8, N %% 128, scale, Aout");
        if (a.w_int8) {
            switch (a.T) {
            case 1: return launch_wloop_t<true, 1, false>(p, st);
            case 2: return bt ? launch_wloop_t<true, 2, true>(p, st) : launch_wloop_t<true, 2, false>(p, st);
            case 3: return bt ? launch_wloop_t<true, 3, true>(p, st) : launch_wloop_t<true, 3, false>(p, st);
            default: return fail(VMLM_ERR_UNIMPL, "gemv: %d activation terms unsupported", a.T);
            }
        }
        switch (a.T) {
        case 1: return launch_wloop_t<false, 1, false>(p, st);
        case 2: return bt ? launch_wloop_t<false, 2, true>(p, st) : launch_wloop_t<false, 2, false>(p, st);
        case 3: return bt ? launch_wloop_t<false, 3, true>(p, st) : launch_wloop_t<false, 3, false>(p, st);
        default: return fail(VMLM_ERR_UNIMPL, "gemv: %d activation terms unsupported", a.T);
        }
    }
    if (R == 8) {  // wide: 128 rows per workgroup, activation slice in LDS
        const int nch = a.K / 128;
        VMLM_GUARD(a.w_int8 && nch % p.ks == 0 && nch / p.ks <= 3,
                   "gemv wide: int8, k-slices of 1..3 whole chunks");
        VMLM_GUARD(a.epi != EPI_ARGMAX, "gemv wide: no argmax epilogue");
        VMLM_GUARD(a.epi != EPI_SILU_MUL || (p.ks == 1 && a.N % 128 == 0 && a.scale && a.Aout),
                   "gemv wide silu: one k-slice, N %% 128, scale, Aout");
        const int nc = nch / p.ks;
        switch (a.T) {
        case 1: return launch_wide_t<1, false>(p, nc, st);
        case 2: return bt ? launch_wide_t<2, true>(p, nc, st) : launch_wide_t<2, false>(p, nc, st);
        case 3: return bt ? launch_wide_t<3, true>(p, nc, st) : launch_wide_t<3, false>(p, nc, st);
        default: return fail(VMLM_ERR_UNIMPL, "gemv: %d activation terms unsupported", a.T);
        }
    }
    if (R == 0) {
        const int tiles16 = a.N / 16;
        if (a.epi == EPI_SILU_MUL) R = (!bt && tiles16 / 4 >= 128) ? 4 : 2;
        else R = (a.w_int8 && !bt && tiles16 / 4 >= 96) ? 4 : 1;
    }
    if (a.epi == EPI_SILU_MUL) {
        VMLM_GUARD(a.w_int8 && a.scale && a.Aout && (R == 2 || R == 4) && a.N % (16 * R) == 0,
                   "gemv silu: int8 weights, scale, Aout, 2 or 4 tiles dividing N");
        return R == 4 ? launch_r<true, 4>(p, a.T, bt, st) : launch_r<true, 2>(p, a.T, bt, st);
    }
    VMLM_GUARD(R == 1 || R == 2 || R == 4, "gemv: %d tiles per workgroup unsupported", R);
    if (!a.w_int8) {
        VMLM_GUARD(R == 1, "gemv bf16: one tile per workgroup");
        return launch_r<false, 1>(p, a.T, bt, st);
    }
    switch (R) {
    case 1: return launch_r<true, 1>(p, a.T, bt, st);
    case 2: return launch_r<true, 2>(p, a.T, bt, st);
    default: return launch_r<true, 4>(p, a.T, bt, st);
    }
}

}  // namespace vmlm

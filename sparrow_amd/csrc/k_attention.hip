// k_attention.hip -- attention as the VM program composes it, fused.
//
// Prefill (tools/p12_build_minicpm.py:770-781): per head SLICE -> ROPE(pos0)
// -> GEMM NT q.k -> SCALE -> SOFTMAX(causal) -> GEMM NN p.v -> WRITECOL.
// Here: RoPE is applied once to Q and K (bit-exact port), then one kernel
// per (head, 64-query block) streams 64-key tiles through LDS with an
// online softmax (exp_f of the reference, scores scaled exactly as OP_SCALE
// does) -- the [S,S] score matrix never reaches HBM.
//
// Decode (tools/p12_build_minicpm.py:941-967): per (sequence, head) one
// workgroup rotates q and the new k at `pos` and appends the rotated k and
// raw v to the f32 cache; its waves score 16-position sub-chunks (16 lanes
// per 256-byte K row, four rows per coalesced load instruction, the next
// sub-chunk's rows in flight) and leave a (max, sum, p.V) partial for each;
// the partials are merged in position order, in LDS or, with the positions
// split over several workgroups, by a second kernel (flash-decoding).
//
// Both change the order of the reference's sums (E contract: 1e-4 of the
// output RMS); RoPE, the scale multiply and every exp_f are bitwise.
#include "internal.hpp"

namespace vmlm {

// ---------------------------------------------------------------- f32 GEMM
// C[m,n] (+)= A[m,k] . op(B), op(B) = B[n,k]^T (nt) or B[k,n], on the f32
// matrix cores: v_mfma_f32_16x16x4f32 multiplies f32 operands exactly and
// accumulates in f32 (only the summation order differs from the reference's
// FMA chains, inside the 1e-4 * RMS contract of the attention composition).
// 32 x 32 tiles, four waves of 16 x 16 (lane (g, r) = (lane / 16, lane % 16)
// gives A[row r][k g] and op(B)[k g][col r] and holds rows 4g..4g+3 of column
// r). 64-deep k-steps through LDS: A as [row][k], an NT B as [col][k], an NN
// B as [k][col]; the next step's tiles are loaded into registers while the
// current one is consumed. With VEC the rows are read as float4 (k, or n for
// an NN B, a multiple of 4 and 16-byte aligned operands). A grid of few tiles
// is split over k (grid z): each slice writes its partial tile to `part`
// [ks][m][n] and gemm_f32_reduce_kernel sums the slices in order
// (deterministic).
constexpr int GF_T = 32, GF_K = 64;
constexpr int GF_LDA = GF_K + 4;   // [row][k] pitch (floats)
constexpr int GF_LDB = GF_T + 16;  // [k][col] pitch: lanes (g, r) two-way at most

template <bool NT, bool VEC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float *__restrict__ A,
                                                       const float *__restrict__ B,
                                                       float *__restrict__ C, int m, int n, int k,
                                                       int acc, int kslice,
                                                       float *__restrict__ part) {
    __shared__ __attribute__((aligned(16))) float As[GF_T][GF_LDA];
    __shared__ __attribute__((aligned(16))) float Bs[NT ? GF_T : GF_K][NT ? GF_LDA : GF_LDB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 4, r = lane & 15;
    const int row0 = blockIdx.y * GF_T, col0 = blockIdx.x * GF_T;
    const int kb = blockIdx.z * kslice;
    const int ke = kb + kslice < k ? kb + kslice : k;
    auto ld4 = [&](const float *p, bool ok, int left) {
        if constexpr (VEC) {
            return ok && left >= 4 ? *(const float4 *)p : make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            return make_float4(ok && left > 0 ? p[0] : 0.f, ok && left > 1 ? p[1] : 0.f,
                               ok && left > 2 ? p[2] : 0.f, ok && left > 3 ? p[3] : 0.f);
        }
    };
    // loader roles (two float4 per thread and operand): A and an NT B as 32
    // rows x 16 float4 of k; an NN B as 64 k-rows x 8 float4 of n
    float4 ra[2], rb[2];
    auto load = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = tid + q * 256, rr = e >> 4, c4 = (e & 15) * 4, gk = k0 + c4;
            const int gr = row0 + rr;
            ra[q] = ld4(A + (size_t)(gr < m ? gr : 0) * k + (gk < ke ? gk : kb), gr < m, ke - gk);
            if constexpr (NT) {
                const int gc = col0 + rr;
                rb[q] = ld4(B + (size_t)(gc < n ? gc : 0) * k + (gk < ke ? gk : kb), gc < n, ke - gk);
            } else {
                const int kr = e >> 3, n4 = (e & 7) * 4, gkr = k0 + kr, gc = col0 + n4;
                rb[q] = ld4(B + (size_t)(gkr < ke ? gkr : kb) * n + (gc < n ? gc : 0), gkr < ke,
                            n - gc);
            }
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = tid + q * 256, rr = e >> 4, c4 = (e & 15) * 4;
            *(float4 *)&As[rr][c4] = ra[q];
            if constexpr (NT) *(float4 *)&Bs[rr][c4] = rb[q];
            else *(float4 *)&Bs[e >> 3][(e & 7) * 4] = rb[q];
        }
    };
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    load(kb);
    for (int k0 = kb; k0 < ke; k0 += GF_K) {
        __syncthreads();
        store();
        __syncthreads();
        if (k0 + GF_K < ke) load(k0 + GF_K);
#pragma unroll
        for (int kk = 0; kk < GF_K; kk += 4) {
            const float a = As[wm * 16 + r][kk + g];
            const float b = NT ? Bs[wn * 16 + r][kk + g] : Bs[kk + g][wn * 16 + r];
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, d, 0, 0, 0);
        }
    }
    const int gc = col0 + wn * 16 + r;
    if (gc >= n) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int gr = row0 + wm * 16 + 4 * g + q;
        if (gr >= m) continue;
        if (part) {
            part[((size_t)blockIdx.z * m + gr) * n + gc] = d[q];
        } else {
            float *o = C + (size_t)gr * n + gc;
            *o = acc ? *o + d[q] : d[q];
        }
    }
}

__global__ __launch_bounds__(256) void gemm_f32_reduce_kernel(const float *__restrict__ part,
                                                              int ks, size_t mn,
                                                              float *__restrict__ C, int acc) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float v = part[i];
    for (int z = 1; z < ks; ++z) v += part[(size_t)z * mn + i];
    C[i] = acc ? C[i] + v : v;
}

size_t gemm_f32_work_floats(size_t m, size_t n, size_t k) {
    const size_t tiles = cdiv(m, (size_t)GF_T) * cdiv(n, (size_t)GF_T);
    if (tiles >= 128 || k < 2 * GF_K) return 0;
    size_t ks = cdiv((size_t)256, tiles);
    const size_t steps = cdiv(k, (size_t)GF_K);
    ks = ks < steps ? ks : steps;
    return ks > 1 ? ks * m * n : 0;
}

int launch_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                    bool acc, bool b_is_nt, hipStream_t st, float *work) {
    if (m == 0 || n == 0) return VMLM_OK;
    if (k == 0) {
        if (!acc) return launch_fill_zero(c, m * n * sizeof(float), st);
        return VMLM_OK;
    }
    VMLM_GUARD(m <= 0x7fffffffu && n <= 0x7fffffffu && k <= 0x7fffffffu, "gemm f32: shape too large");
    // split k when the output is narrow (and the caller gave the workspace)
    const size_t wf = gemm_f32_work_floats(m, n, k);
    int ks = 1;
    if (wf && work) ks = (int)(wf / (m * n));
    const size_t steps = cdiv(k, (size_t)GF_K);
    const int kslice = (int)(cdiv(steps, (size_t)ks) * GF_K);
    ks = (int)cdiv(k, (size_t)kslice);
    const bool vec = k % 4 == 0 && (b_is_nt || n % 4 == 0) && ((uintptr_t)a & 15) == 0 &&
                     ((uintptr_t)b & 15) == 0;
    float *part = ks > 1 ? work : nullptr;
    dim3 grid(cdiv(n, (size_t)GF_T), cdiv(m, (size_t)GF_T), ks);
    const int ia = acc ? 1 : 0, ik = (int)k;
    if (b_is_nt) {
        if (vec) gemm_f32_kernel<true, true><<<grid, 256, 0, st>>>(a, b, c, (int)m, (int)n, ik, ia, kslice, part);
        else gemm_f32_kernel<true, false><<<grid, 256, 0, st>>>(a, b, c, (int)m, (int)n, ik, ia, kslice, part);
    } else {
        if (vec) gemm_f32_kernel<false, true><<<grid, 256, 0, st>>>(a, b, c, (int)m, (int)n, ik, ia, kslice, part);
        else gemm_f32_kernel<false, false><<<grid, 256, 0, st>>>(a, b, c, (int)m, (int)n, ik, ia, kslice, part);
    }
    VMLM_HIP_CHECK(hipGetLastError());
    if (part) {
        gemm_f32_reduce_kernel<<<cdiv(m * n, (size_t)256), 256, 0, st>>>(part, ks, m * n, c, ia);
        VMLM_HIP_CHECK(hipGetLastError());
    }
    return VMLM_OK;
}

// ---------------------------------------------------------------- prefill
// Q, K already rotated; all [S][ld] with head h at columns h*64.
//
// Flash attention on the bf16 matrix cores. Q, K and the probabilities are
// carried as two bf16 terms x0 = bf16(x), x1 = bf16(x - x0) (|x - x0 - x1|
// <= 2^-17 |x|), V as three (exact); a product is the sum of the term
// products (q0k0 + q0k1 + q1k0 + q1k1; v0p0 + v1p0 + v2p0 + v0p1 + v1p1),
// each exact, accumulated in f32 by v_mfma_f32_16x16x32_bf16: relative error
// ~2^-16, well inside the 1e-4 * RMS contract of the attention composition,
// and a one-key softmax row returns its V row exactly. A workgroup owns 64
// queries of one head (wave w: queries 16w..16w+15) and walks the key blocks
// of 64 up to the diagonal: K is staged as [key][dim] terms, V transposed as
// [dim][key] terms.
//
// Both products are computed transposed, S^T = K Q^T and O^T += V^T P^T, so
// that the accumulator layout (lane (g, r): rows 4g..4g+3 of column r) puts
// one query (column r) in each lane: its scores for keys 16j + 4g + i are
// exactly the B-operand fragment of the next product once the key slots of a
// 32-key step are taken in the order (32m + 4g + i, 32m + 16 + 4g + i), and V
// is read in the same order. The probabilities never leave registers; the
// running max / sum of a query live in its lane (the four lanes g of a query
// exchange partial max / sum with permlane swaps).
constexpr int AT_B = 64;   // query / key block
constexpr int AT_LD = 72;  // bf16 elements per LDS row (64 + 8)

// DPP lane moves inside a row of 16 lanes (row_mirror: lane i <- 15 - i;
// row_half_mirror: i <- 7 - i within each 8; quad_perm [3,2,1,0] and
// [1,0,3,2]): partners that differ in bit 3, 2, 1, 0 of the lane index.
constexpr int DPP_ROW_MIRROR = 0x140, DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_QUAD_REV = 0x1B, DPP_QUAD_SWAP = 0xB1;
// row_ror:n (the row's 16 lanes rotated by n) and row_newbcast:n (every
// lane of the row <- lane n of the row)
constexpr int DPP_ROW_ROR1 = 0x121, DPP_ROW_ROR2 = 0x122, DPP_ROW_ROR4 = 0x124,
              DPP_ROW_ROR8 = 0x128, DPP_ROW_BCAST0 = 0x150;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_REV>(v));
    return fmaxf(v, dpp_f<DPP_QUAD_SWAP>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<DPP_ROW_MIRROR>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f<DPP_QUAD_REV>(v);
    return v + dpp_f<DPP_QUAD_SWAP>(v);
}

// value of the same register in lane l ^ 16 / l ^ 32 (v_permlane16_swap pairs
// rows 0-1 and 2-3 of 16 lanes; v_permlane32_swap pairs the two halves)
__device__ __forceinline__ float lane_xor16(float v) {
    const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float((__lane_id() & 16) ? t[0] : t[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float((__lane_id() & 32) ? t[0] : t[1]);
}

__device__ __forceinline__ f32x4 mfma_b(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 8 f32 -> two bf16 term fragments
__device__ __forceinline__ float bf16_lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

__device__ __forceinline__ void split8(const float (&x)[8], u32x4 &t0, u32x4 &t1) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float a = x[2 * q], b = x[2 * q + 1];
        const uint32_t h = bf16x2_rne_bits(a, b);
        t0[q] = h;
        t1[q] = bf16x2_rne_bits(a - bf16_lo_f32(h), b - bf16_hi_f32(h));
    }
}

// 8 f32 -> three bf16 term fragments (their sum is x exactly)
__device__ __forceinline__ void split8x3(const float (&x)[8], u32x4 &t0, u32x4 &t1, u32x4 &t2) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float a = x[2 * q], b = x[2 * q + 1];
        const uint32_t h = bf16x2_rne_bits(a, b);
        const float ra = a - bf16_lo_f32(h), rb = b - bf16_hi_f32(h);
        const uint32_t m = bf16x2_rne_bits(ra, rb);
        t0[q] = h;
        t1[q] = m;
        t2[q] = bf16x2_rne_bits(ra - bf16_lo_f32(m), rb - bf16_hi_f32(m));
    }
}

// One workgroup per (query block, head, sequence); sequences at strides
// sin / sout (elements) along grid z. The longest causal rows go first.
struct PrefillParams {
    const uint16_t *Qt, *Kt, *Vt;  // bf16 term planes written by attn_qkv_prep_kernel
    float *O;
    size_t sout;
    int S, Sp, ldo, causal, nqb, H;
    int o_vec;  // O rows 16-byte aligned: float4 stores
    float scale;
};

// Q, K and V of every (sequence, head) as bf16 term planes, rows padded to Sp
// (a multiple of 64) with zeros:
//   Qt[z][t][h][row][64], Kt[z][t][h][row][64]  (t < 2; rotated here when
//                                               rope is set)
//   Vt[z][t][h][dim][Sp]                        (t < 3; V transposed)
// so that the attention kernel loads its Q fragments and stages each key
// block with 16-byte copies. One workgroup per (64-row block, head,
// sequence); thread (row, c) rotates RoPE pairs 2c and 2c + 1 of its Q and K
// rows with one angle evaluation per pair (Q and K share the position).
// With kc / vc the rotated K rows and the raw V rows also go to a KV cache
// [sequence][head][hs][64] f32 at positions 0 .. S-1 (the decoder's prefill).
// With pks > 0, Q, K and V point into slice 0 of pks k-slices pst floats
// apart: each value is the slices summed in order times its column scale
// (sq, sk, sv), as the slice reduction would have written it.
struct QKVPrepParams {
    const float *Q, *K, *V;
    uint16_t *Qt, *Kt, *Vt;
    float *kc, *vc;
    size_t sin;
    int S, Sp, ld, H, rope, hs;
    float rope_step, pos0;
    int pks;
    size_t pst;
    const float *sq, *sk, *sv;
};
__global__ __launch_bounds__(1024) void attn_qkv_prep_kernel(QKVPrepParams p) {
    const int h = blockIdx.y, z = blockIdx.z, tid = threadIdx.x;
    const int k0 = blockIdx.x * AT_B;
    const size_t plane = (size_t)p.H * p.Sp * 64;
    {
        const int row = k0 + (tid >> 4), c = tid & 15, rr = min(row, p.S - 1);
        const size_t src = z * p.sin + (size_t)rr * p.ld + h * 64 + 2 * c;
        auto ld2 = [&](const float *b, const float *sc, int off) {
            float2 v = *(const float2 *)(b + src + off);
            if (p.pks) {
                for (int s = 1; s < p.pks; ++s) {
                    const float2 t = *(const float2 *)(b + (size_t)s * p.pst + src + off);
                    v.x += t.x;
                    v.y += t.y;
                }
                const int j = h * 64 + 2 * c + off;
                v = make_float2(v.x * sc[j], v.y * sc[j + 1]);
            }
            return v;
        };
        float2 q1 = ld2(p.Q, p.sq, 0), q2 = ld2(p.Q, p.sq, 32);
        float2 k1 = ld2(p.K, p.sk, 0), k2 = ld2(p.K, p.sk, 32);
        if (p.rope) {
            const float fpos = p.pos0 + (float)rr;
            float si, co, a, b;
            rope_angle(fpos, 2 * c, p.rope_step, &si, &co);
            a = q1.x * co - q2.x * si, b = q1.x * si + q2.x * co, q1.x = a, q2.x = b;
            a = k1.x * co - k2.x * si, b = k1.x * si + k2.x * co, k1.x = a, k2.x = b;
            rope_angle(fpos, 2 * c + 1, p.rope_step, &si, &co);
            a = q1.y * co - q2.y * si, b = q1.y * si + q2.y * co, q1.y = a, q2.y = b;
            a = k1.y * co - k2.y * si, b = k1.y * si + k2.y * co, k1.y = a, k2.y = b;
        }
        if (row >= p.S) q1 = q2 = k1 = k2 = make_float2(0.0f, 0.0f);
        else if (p.kc) {
            float *kr = p.kc + (((size_t)z * p.H + h) * p.hs + row) * 64 + 2 * c;
            *(float2 *)kr = k1;
            *(float2 *)(kr + 32) = k2;
        }
        const size_t dst = ((size_t)z * 2 * p.H + h) * p.Sp * 64 + (size_t)row * 64 + 2 * c;
        auto put = [&](uint16_t *base, float2 lo, float2 hi) {
            const uint32_t l0 = bf16x2_rne_bits(lo.x, lo.y), h0 = bf16x2_rne_bits(hi.x, hi.y);
            *(uint32_t *)(base + dst) = l0;
            *(uint32_t *)(base + dst + 32) = h0;
            *(uint32_t *)(base + dst + plane) =
                bf16x2_rne_bits(lo.x - bf16_lo_f32(l0), lo.y - bf16_hi_f32(l0));
            *(uint32_t *)(base + dst + plane + 32) =
                bf16x2_rne_bits(hi.x - bf16_lo_f32(h0), hi.y - bf16_hi_f32(h0));
        };
        put(p.Qt, q1, q2);
        put(p.Kt, k1, k2);
    }
    {
        // V transposed through LDS: rows read as float4 (thread: row tid / 16,
        // dims 4 (tid % 16) ..), then thread (dim, key octet) of the first 512
        // splits 8 consecutive keys and writes each term as one 16-byte piece
        __shared__ float vs[AT_B][AT_B + 1];
        {
            const int row = k0 + (tid >> 4), d0 = 4 * (tid & 15);
            const size_t vsrc = z * p.sin + (size_t)min(row, p.S - 1) * p.ld + h * 64 + d0;
            float4 x = *(const float4 *)(p.V + vsrc);
            if (p.pks) {
                for (int s = 1; s < p.pks; ++s) {
                    const float4 t = *(const float4 *)(p.V + (size_t)s * p.pst + vsrc);
                    x = make_float4(x.x + t.x, x.y + t.y, x.z + t.z, x.w + t.w);
                }
                const float4 sc = *(const float4 *)(p.sv + h * 64 + d0);
                x = make_float4(x.x * sc.x, x.y * sc.y, x.z * sc.z, x.w * sc.w);
            }
            const bool ok = row < p.S;
            if (ok && p.vc) *(float4 *)(p.vc + (((size_t)z * p.H + h) * p.hs + row) * 64 + d0) = x;
            vs[tid >> 4][d0] = ok ? x.x : 0.0f;
            vs[tid >> 4][d0 + 1] = ok ? x.y : 0.0f;
            vs[tid >> 4][d0 + 2] = ok ? x.z : 0.0f;
            vs[tid >> 4][d0 + 3] = ok ? x.w : 0.0f;
        }
        __syncthreads();
        if (tid < 512) {
            const int dim = tid >> 3, kg = tid & 7;
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = vs[8 * kg + i][dim];
            u32x4 t0, t1, t2;
            split8x3(x, t0, t1, t2);
            uint16_t *vt =
                p.Vt + ((size_t)z * 3 * p.H + h) * 64 * p.Sp + (size_t)dim * p.Sp + k0 + 8 * kg;
            *(u32x4 *)vt = t0;
            *(u32x4 *)(vt + plane) = t1;
            *(u32x4 *)(vt + 2 * plane) = t2;
        }
    }
}

// One key block of the prefill attention for the wave's 16 queries: S^T =
// K Q^T over the block's 64 keys (two bf16 terms of K and of Q), the online
// softmax update of (m, l, o), then O^T += V^T P^T (three terms of V, two of
// P). Ks / Vt hold the block's terms in LDS; lane (g, r) owns query qa.
__device__ __forceinline__ void prefill_block(const uint16_t (*Ks)[AT_B][AT_LD],
                                              const uint16_t (*Vt)[64][AT_LD],
                                              const u32x4 (&aq)[2][2], int k0, int qa, int S,
                                              int causal, float scale, float &m, float &l,
                                              f32x4 (&o)[4]) {
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    // S^T: block j = keys 16j..16j+15; lane (g, r): keys 16j + 4g + i of
    // query q0 + r. The four blocks' MFMA chains are interleaved.
    f32x4 sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
        u32x4 b0[4], b1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b0[j] = *(const u32x4 *)&Ks[0][16 * j + r][sl * 32 + g * 8];
            b1[j] = *(const u32x4 *)&Ks[1][16 * j + r][sl * 32 + g * 8];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = mfma_b(b0[j], aq[sl][0], sc[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = mfma_b(b1[j], aq[sl][0], sc[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = mfma_b(b0[j], aq[sl][1], sc[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = mfma_b(b1[j], aq[sl][1], sc[j]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ka = k0 + 16 * j + 4 * g + i;
            const bool valid = ka < S && (!causal || ka <= qa);
            sc[j][i] = valid ? sc[j][i] * scale : -INFINITY;
            mx = fmaxf(mx, sc[j][i]);
        }
    mx = fmaxf(mx, lane_xor16(mx));
    mx = fmaxf(mx, lane_xor32(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = m == -INFINITY ? 0.0f : __expf(m - mn);
    float pv[4][4], rs = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pv[j][i] = sc[j][i] == -INFINITY ? 0.0f : __expf(sc[j][i] - mn);
            rs += pv[j][i];
        }
    rs += lane_xor16(rs);
    rs += lane_xor32(rs);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[jd][i] *= alpha;
    // P^T fragments of the two 32-key steps: slots 8g..8g+7 hold keys
    // 32 st + 4g + i and 32 st + 16 + 4g + i
    u32x4 pb[2][2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        const float x[8] = {pv[2 * st][0],     pv[2 * st][1],     pv[2 * st][2],
                            pv[2 * st][3],     pv[2 * st + 1][0], pv[2 * st + 1][1],
                            pv[2 * st + 1][2], pv[2 * st + 1][3]};
        split8(x, pb[st][0], pb[st][1]);
    }
    // O^T[d][q] += V^T[d][key] P^T[key][q]: A = V^T rows (dim 16 jd + r)
    // at the same key slots; the four dim blocks' chains interleaved
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        u32x4 va[3][4];
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) {
                const uint16_t *row = &Vt[t][16 * jd + r][32 * st + 4 * g];
                const uint2 lo = *(const uint2 *)row, hi = *(const uint2 *)(row + 16);
                va[t][jd] = u32x4{lo.x, lo.y, hi.x, hi.y};
            }
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(va[0][jd], pb[st][0], o[jd]);
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(va[1][jd], pb[st][0], o[jd]);
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(va[2][jd], pb[st][0], o[jd]);
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(va[0][jd], pb[st][1], o[jd]);
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(va[1][jd], pb[st][1], o[jd]);
    }
}

// lane (g, r): query qa, dims 16 jd + 4g .. +3
__device__ __forceinline__ void prefill_store(const f32x4 (&o)[4], float l, int qa, int S,
                                              float *O, size_t sout, int ldo, int o_vec, int h) {
    const int g = (threadIdx.x & 63) >> 4;
    if (qa >= S) return;
    const float inv = 1.0f / l;
    float *orow = O + blockIdx.z * sout + (size_t)qa * ldo + h * 64 + 4 * g;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
        const float4 v = make_float4(o[jd][0] * inv, o[jd][1] * inv, o[jd][2] * inv, o[jd][3] * inv);
        if (o_vec) {
            *(float4 *)(orow + 16 * jd) = v;
        } else {
            orow[16 * jd] = v.x;
            orow[16 * jd + 1] = v.y;
            orow[16 * jd + 2] = v.z;
            orow[16 * jd + 3] = v.w;
        }
    }
}

__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(PrefillParams P) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AT_B][AT_LD];   // [term][key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t Vt[3][64][AT_LD];     // [term][dim][key]
    const int S = P.S, causal = P.causal;
    const int h = blockIdx.y, z = blockIdx.z;
    const int qb = causal ? P.nqb - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int kb0 = 0, kb1 = causal ? qb + 1 : (S + AT_B - 1) / AT_B;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int q0 = qb * AT_B + wave * 16;
    const size_t kplane = (size_t)P.H * P.Sp * 64;
    const uint16_t *Kth = P.Kt + ((size_t)z * 2 * P.H + h) * P.Sp * 64;
    const uint16_t *Vth = P.Vt + ((size_t)z * 3 * P.H + h) * 64 * P.Sp;

    // this lane's query fragments: row q0 + r, dims 32 sl + 8g .. +7, two terms
    u32x4 aq[2][2];  // [slice][term]
    {
        const uint16_t *Qth = P.Qt + ((size_t)z * 2 * P.H + h) * P.Sp * 64 + (size_t)(q0 + r) * 64;
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
            for (int t = 0; t < 2; ++t)
                aq[sl][t] = *(const u32x4 *)(Qth + t * (size_t)P.H * P.Sp * 64 + sl * 32 + g * 8);
    }
    float m = -INFINITY, l = 0.0f;  // query q0 + r
    f32x4 o[4];                      // o[jd][i]: dim 16 jd + 4g + i of query q0 + r
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    // staging: 16-byte pieces, 4 of K (term, key, eighth) and 6 of V^T
    // (term, dim, eighth) per thread; the next key block's pieces are loaded
    // into registers while the current one is consumed (the last block
    // reloads itself)
    u32x4 stg[10];
    auto load_kv = [&](int kb) {
        const int k0 = kb * AT_B;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int idx = tid + 256 * k, t = idx >> 9, key = (idx >> 3) & 63, pc = idx & 7;
            stg[k] = *(const u32x4 *)(Kth + t * kplane + (size_t)(k0 + key) * 64 + 8 * pc);
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const int idx = tid + 256 * k, t = idx >> 9, dim = (idx >> 3) & 63, pc = idx & 7;
            stg[4 + k] = *(const u32x4 *)(Vth + t * kplane + (size_t)dim * P.Sp + k0 + 8 * pc);
        }
    };
    const int qa = q0 + r;
    load_kv(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        __syncthreads();  // the previous block's K / V are no longer read
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int idx = tid + 256 * k, t = idx >> 9, key = (idx >> 3) & 63, pc = idx & 7;
            *(u32x4 *)&Ks[t][key][8 * pc] = stg[k];
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const int idx = tid + 256 * k, t = idx >> 9, dim = (idx >> 3) & 63, pc = idx & 7;
            *(u32x4 *)&Vt[t][dim][8 * pc] = stg[4 + k];
        }
        __syncthreads();
        load_kv(kb + 1 < kb1 ? kb + 1 : kb);
        __builtin_amdgcn_sched_barrier(0);
        prefill_block(Ks, Vt, aq, kb * AT_B, qa, S, causal, P.scale, m, l, o);
    }
    prefill_store(o, l, qa, S, P.O, P.sout, P.ldo, P.o_vec, h);
}

// The same attention straight from the f32 Q, K and V rows (no term planes
// in HBM and no second launch): each workgroup forms its queries' fragments
// and, per key block, the block's K and V^T terms in LDS with the operations
// of attn_qkv_prep_kernel (rotation, bf16 splits), so the scores, weights
// and output are the two-kernel path's bits. The workgroup whose query block
// is the key block (every key block has one) writes the block's rotated K
// rows and raw V rows to the KV cache. K blocks are rotated by every query
// block that reads them, so the launcher takes this form for up to four
// query blocks (S <= 256).
struct QKVPrefillParams {
    const float *Q, *K, *V;  // rows of `ld` floats; sequence z at z * sin
    float *O;
    float *kc, *vc;          // KV cache [sequence][head][hs][64], or null
    size_t sin, sout;
    int S, ld, ldo, causal, nqb, H, hs, rope, o_vec;
    float scale, rope_step, pos0;
    const float2 *tab;       // (sin, cos) of [row][pair index], or null
};

// tab[row][i] = the (sin, cos) that rope_angle gives at position pos0 + row
__global__ __launch_bounds__(256) void rope_table_kernel(float2 *tab, int S, float pos0, float step) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= S * 32) return;
    float si, co;
    rope_angle(pos0 + (float)(e >> 5), e & 31, step, &si, &co);
    tab[e] = make_float2(si, co);
}

__global__ __launch_bounds__(256, 2) void attn_prefill_qkv_kernel(QKVPrefillParams P) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AT_B][AT_LD];   // [term][key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t Vt[3][64][AT_LD];     // [term][dim][key]
    const int S = P.S, causal = P.causal;
    const int h = blockIdx.y, z = blockIdx.z;
    const int qb = causal ? P.nqb - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int kb1 = causal ? qb + 1 : P.nqb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int q0 = qb * AT_B + wave * 16;
    const size_t base = (size_t)z * P.sin + h * 64;
    // 4 values of row `row` from dim d
    auto ld4 = [&](const float *b, int row, int d) {
        return *(const float4 *)(b + base + (size_t)row * P.ld + d);
    };
    // RoPE of a row's dims d0 .. d0 + 7 (x1) with their partners d0 + 32 ..
    // (x2) at position pos0 + row, the prep kernel's arithmetic
    // (sin, cos) of a row's pairs d0 .. d0 + 7 from the table (P.tab), or
    // from rope_angle when there is none
    auto load_tab = [&](float2 (&t)[8], int row, int d0) {
        if (!P.rope || !P.tab) return;
        const float4 *tp = (const float4 *)(P.tab + (size_t)row * 32 + d0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 u = tp[i];
            t[2 * i] = make_float2(u.x, u.y);
            t[2 * i + 1] = make_float2(u.z, u.w);
        }
    };
    auto rotate = [&](float (&x1)[8], float (&x2)[8], int row, int d0, const float2 (&t)[8]) {
        if (!P.rope) return;
        const float fpos = P.pos0 + (float)row;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float si, co;
            if (P.tab) {
                si = t[i].x;
                co = t[i].y;
            } else {
                rope_angle(fpos, d0 + i, P.rope_step, &si, &co);
            }
            const float a = x1[i] * co - x2[i] * si, b = x1[i] * si + x2[i] * co;
            x1[i] = a;
            x2[i] = b;
        }
    };
    auto unpack8 = [](float4 a, float4 b, float (&x)[8]) {
        x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w;
        x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
    };

    // the block's raw rows in registers, loaded one block ahead: thread (key
    // kt, quarter kq) holds K dims 8 kq .. +7 and 32 + 8 kq .. +7 with their
    // rotation angles, and for the V^T items tid and tid + 256 (dim vd, keys
    // 8 kg .. 8 kg + 7 with kg = tid / 64 + 4 j) the eight V values (each
    // load instruction reads 64 consecutive dims of one row)
    const int kt = tid >> 2, kq = tid & 3, vd = tid & 63;
    float4 kr[4];
    float2 ktab[8];
    float vv[2][8];
    auto load_kv = [&](int kb) {
        const int row = min(kb * AT_B + kt, S - 1);
        kr[0] = ld4(P.K, row, 8 * kq);
        kr[1] = ld4(P.K, row, 8 * kq + 4);
        kr[2] = ld4(P.K, row, 32 + 8 * kq);
        kr[3] = ld4(P.K, row, 32 + 8 * kq + 4);
        load_tab(ktab, row, 8 * kq);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int vrow = min(kb * AT_B + 8 * ((tid >> 6) + 4 * j) + i, S - 1);
                vv[j][i] = P.V[base + (size_t)vrow * P.ld + vd];
            }
    };
    load_kv(0);

    // this lane's query fragments: row q0 + r, dims 8g .. +7 and 32 + 8g ..
    // (a RoPE pair per dim), two terms each; zero past the last row
    const int qa = q0 + r;
    u32x4 aq[2][2];  // [slice][term]
    {
        const int row = min(qa, S - 1);
        float x1[8], x2[8];
        float2 qtab[8];
        unpack8(ld4(P.Q, row, 8 * g), ld4(P.Q, row, 8 * g + 4), x1);
        unpack8(ld4(P.Q, row, 32 + 8 * g), ld4(P.Q, row, 32 + 8 * g + 4), x2);
        load_tab(qtab, row, 8 * g);
        rotate(x1, x2, row, 8 * g, qtab);
        if (qa >= S)
#pragma unroll
            for (int i = 0; i < 8; ++i) x1[i] = x2[i] = 0.0f;
        split8(x1, aq[0][0], aq[0][1]);
        split8(x2, aq[1][0], aq[1][1]);
    }
    float m = -INFINITY, l = 0.0f;
    f32x4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = 0; kb < kb1; ++kb) {
        const int key = kb * AT_B + kt, row = min(key, S - 1);
        const bool ok = key < S, diag = kb == qb && ok;
        __syncthreads();  // the previous block's Ks and Vt are no longer read
        {
            float x1[8], x2[8];
            unpack8(kr[0], kr[1], x1);
            unpack8(kr[2], kr[3], x2);
            rotate(x1, x2, row, 8 * kq, ktab);
            if (!ok)
#pragma unroll
                for (int i = 0; i < 8; ++i) x1[i] = x2[i] = 0.0f;
            if (diag && P.kc) {
                float *kcr = P.kc + (((size_t)z * P.H + h) * P.hs + key) * 64;
                *(float4 *)(kcr + 8 * kq) = make_float4(x1[0], x1[1], x1[2], x1[3]);
                *(float4 *)(kcr + 8 * kq + 4) = make_float4(x1[4], x1[5], x1[6], x1[7]);
                *(float4 *)(kcr + 32 + 8 * kq) = make_float4(x2[0], x2[1], x2[2], x2[3]);
                *(float4 *)(kcr + 32 + 8 * kq + 4) = make_float4(x2[4], x2[5], x2[6], x2[7]);
            }
            u32x4 t0, t1;
            split8(x1, t0, t1);
            *(u32x4 *)&Ks[0][kt][8 * kq] = t0;
            *(u32x4 *)&Ks[1][kt][8 * kq] = t1;
            split8(x2, t0, t1);
            *(u32x4 *)&Ks[0][kt][32 + 8 * kq] = t0;
            *(u32x4 *)&Ks[1][kt][32 + 8 * kq] = t1;
            // V^T terms: item (dim vd, key octet kg) splits 8 consecutive keys
            // (zero past the last row); the diagonal block's raw rows go to
            // the cache, 64 consecutive dims per store instruction
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int kg = (tid >> 6) + 4 * j;
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int vkey = kb * AT_B + 8 * kg + i;
                    x[i] = vkey < S ? vv[j][i] : 0.0f;
                    if (kb == qb && vkey < S && P.vc)
                        P.vc[(((size_t)z * P.H + h) * P.hs + vkey) * 64 + vd] = vv[j][i];
                }
                u32x4 t0, t1, t2;
                split8x3(x, t0, t1, t2);
                *(u32x4 *)&Vt[0][vd][8 * kg] = t0;
                *(u32x4 *)&Vt[1][vd][8 * kg] = t1;
                *(u32x4 *)&Vt[2][vd][8 * kg] = t2;
            }
        }
        __syncthreads();
        if (kb + 1 < kb1) load_kv(kb + 1);
        __builtin_amdgcn_sched_barrier(0);
        prefill_block(Ks, Vt, aq, kb * AT_B, qa, S, causal, P.scale, m, l, o);
    }
    prefill_store(o, l, qa, S, P.O, P.sout, P.ldo, P.o_vec, h);
}

// One launch when the K blocks are rotated by few query blocks and the grid
// fills the CUs: with fewer workgroups (one 128-token sequence: 72) the
// separate prep launch spreads the rotation and splitting over 4x the
// threads, 5 % faster over the batch-1 prefill; at 16 sequences the one
// launch is 2.4 % faster over the batch-16 prefill.
bool attention_prefill_one_launch(int S, int H, int nseq) {
    const int nqb = (S + AT_B - 1) / AT_B;
    return S >= 1 && nqb <= 4 && (size_t)nqb * H * nseq >= 256;
}

int launch_rope_table(float2 *tab, int S, float pos0, float rope_step, hipStream_t st) {
    if (S <= 0) return VMLM_OK;
    rope_table_kernel<<<(S * 32 + 255) / 256, 256, 0, st>>>(tab, S, pos0, rope_step);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

size_t attention_prefill_work_bytes(int S, int H, int nseq) {
    const size_t Sp = (size_t)(S + AT_B - 1) / AT_B * AT_B;
    return (size_t)nseq * H * Sp * 64 * 7 * sizeof(uint16_t);
}

int launch_attention_prefill(const float *q, const float *k, const float *v, float *out, int S,
                             int H, int ld, int ldo, float scale, bool causal, void *work,
                             hipStream_t st, bool rope, float rope_step, float pos0, int nseq,
                             size_t sin, size_t sout, float *kc, float *vc, int hs,
                             const Slices &qs, const float2 *rope_tab) {
    VMLM_GUARD(ld % 4 == 0 && ((uintptr_t)q & 7) == 0 && ((uintptr_t)k & 7) == 0 &&
                   ((uintptr_t)v & 15) == 0 && (nseq == 1 || sin % 4 == 0),
               "attention prefill: 16-byte aligned V rows and 8-byte aligned Q / K rows "
               "required");
    VMLM_GUARD(!kc == !vc && (!kc || (hs >= S && pos0 == 0.0f && ((uintptr_t)kc & 15) == 0 &&
                                      ((uintptr_t)vc & 15) == 0)),
               "attention prefill: a KV cache needs both rows, hs >= S, position 0 and "
               "16-byte alignment");
    VMLM_GUARD(!qs.part || (qs.ks >= 1 && qs.pst % 4 == 0 && qs.scale &&
                            ((uintptr_t)qs.scale & 15) == 0 && (k - q) % 4 == 0 && (v - q) % 4 == 0),
               "attention prefill: k-slice q/k/v need ks >= 1, a slice stride that is a "
               "multiple of 4 and 16-byte aligned column scales");
    VMLM_GUARD(nseq >= 1 && nseq <= 65535 && H <= 65535, "attention prefill: grid too large");
    if (S <= 0) return VMLM_OK;
    const int Sp = (S + AT_B - 1) / AT_B * AT_B;
    // up to four query blocks over a full grid: one launch from the f32 rows
    // (16-byte rows, no k-slices)
    if (attention_prefill_one_launch(S, H, nseq) && !qs.part && ((uintptr_t)q & 15) == 0 &&
        ((uintptr_t)k & 15) == 0 && (nseq == 1 || sin % 4 == 0)) {
        QKVPrefillParams F;
        F.Q = q;
        F.K = k;
        F.V = v;
        F.O = out;
        F.kc = kc;
        F.vc = vc;
        F.sin = sin;
        F.sout = sout;
        F.S = S;
        F.ld = ld;
        F.ldo = ldo;
        F.causal = causal ? 1 : 0;
        F.nqb = Sp / AT_B;
        F.H = H;
        F.hs = hs;
        F.rope = rope ? 1 : 0;
        F.o_vec = ((uintptr_t)out & 15) == 0 && ldo % 4 == 0 && (nseq == 1 || sout % 4 == 0);
        F.scale = scale;
        F.rope_step = rope_step;
        F.pos0 = pos0;
        F.tab = rope && ((uintptr_t)rope_tab & 15) == 0 ? rope_tab : nullptr;  // 16-byte table loads
        attn_prefill_qkv_kernel<<<dim3(F.nqb, H, nseq), 256, 0, st>>>(F);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    const size_t plane = (size_t)nseq * 2 * H * Sp * 64;
    QKVPrepParams kp;
    kp.Q = q;
    kp.K = k;
    kp.V = v;
    kp.Qt = (uint16_t *)work;
    kp.Kt = kp.Qt + plane;
    kp.Vt = kp.Kt + plane;
    kp.sin = sin;
    kp.S = S;
    kp.Sp = Sp;
    kp.ld = ld;
    kp.H = H;
    kp.rope = rope ? 1 : 0;
    kp.rope_step = rope_step;
    kp.pos0 = pos0;
    kp.kc = kc;
    kp.vc = vc;
    kp.hs = hs;
    kp.pks = qs.part ? qs.ks : 0;
    kp.pst = qs.pst;
    kp.sq = qs.scale;
    kp.sk = qs.part ? qs.scale + (k - q) : nullptr;
    kp.sv = qs.part ? qs.scale + (v - q) : nullptr;
    attn_qkv_prep_kernel<<<dim3(Sp / AT_B, H, nseq), 1024, 0, st>>>(kp);
    VMLM_HIP_CHECK(hipGetLastError());
    PrefillParams P;
    P.Qt = kp.Qt;
    P.Kt = kp.Kt;
    P.Vt = kp.Vt;
    P.O = out;
    P.sout = sout;
    P.S = S;
    P.Sp = Sp;
    P.ldo = ldo;
    P.causal = causal ? 1 : 0;
    P.nqb = Sp / AT_B;
    P.H = H;
    P.o_vec = ((uintptr_t)out & 15) == 0 && ldo % 4 == 0 && (nseq == 1 || sout % 4 == 0);
    P.scale = scale;
    attn_prefill_kernel<<<dim3(P.nqb, H, nseq), 256, 0, st>>>(P);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- decode
// Decode attention over sub-chunks of 16 cached positions. A wave takes one
// sub-chunk s at a time (rows 16 s .. 16 s + 15) and leaves its partial
//   (m_s, l_s, o_s) = (max score, sum e^{x - m_s}, sum e^{x - m_s} v)
// then the partials are merged in sub-chunk order,
//   out = sum_s o_s e^{m_s - M} / sum_s l_s e^{m_s - M},  M = max_s m_s,
// either by the workgroup itself (one workgroup per (head, sequence), the
// partials in LDS) or, with the positions split over several workgroups, by
// attn_decode_merge_kernel from partials in global memory. Both merges are
// the same arithmetic over the same partials, so the result does not depend
// on how the positions are split. A third form (DecodeArgs::frac, the
// batch-1 decoder) splits a head's positions into a few ranges of about
// equal size, merges each range in its workgroup and leaves one (max, sum,
// O) partial per range, which the o projection merges in range order: a
// two-level merge, within 1e-4 of the output RMS of the one-level result
// but not the same bits.
// Lane (grp, q) of a wave holds dims 4q..4q+3 of rows 16 s + 4 it + grp
// (it = 0..3): one load instruction covers 4 consecutive 256-byte rows. Dot
// products are summed over the 16 lanes of a row group with DPP and over
// the four groups with lane swaps (v_permlane16/32_swap), so every sum runs
// in VALU registers and each lane ends with the values it consumes. The
// next sub-chunk's rows are loaded while the current one is consumed (small
// loads in flight on many waves stream faster than one large batch per wave).
// The workgroup that holds sub-chunk 0 rotates the new query and key once
// and appends the new key/value row to the cache.
constexpr int BUF_RSRC_WORD3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format
constexpr int BUF_NT = 2;  // buffer load cache policy: nontemporal (streamed once)

// One stage of the transposing butterfly: N values per lane become N/2 sums;
// the lane with `up` keeps the upper half and sends the lower.
template <int N, int CTRL, int SZ>
__device__ __forceinline__ void bfly_stage(float (&d)[SZ], bool up) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const float send = up ? d[j] : d[j + N / 2];
        const float keep = up ? d[j + N / 2] : d[j];
        d[j] = keep + dpp_f<CTRL>(send);
    }
}

// Max and sum over the 64 lanes as wave-uniform values: DPP inside each
// row, then the four row results read out in a fixed order.
__device__ __forceinline__ float rows_to_uniform_max(float v) {
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_REV>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_SWAP>(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float rows_to_uniform_sum(float v) {
    v += dpp_f<DPP_ROW_MIRROR>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f<DPP_QUAD_REV>(v);
    v += dpp_f<DPP_QUAD_SWAP>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}
constexpr int AD_PART = 68;             // floats per sub-chunk partial: m, l, f, pad, o[64]
static_assert(AD_PART == ATTN_PART, "the range partials the o projection reads");
constexpr int AD_SUB = 16;              // cached positions per sub-chunk (16, 32 or 64)
constexpr int AD_NV = AD_SUB / 4;       // rows of a sub-chunk per lane
constexpr int AD_RSH = AD_NV == 4 ? 2 : AD_NV == 8 ? 1 : 0;  // lane q holds row q >> AD_RSH
constexpr int AD_LDS_MAX = 64 * 1024;   // partials of one workgroup's positions in LDS
constexpr int PART_KS_MAX = 16;         // k-slices of partial q/k/v read up front

// The output row: y = O / L, written as f32 and, with T > 0, as T bf16
// terms (y0 = bf16(y), y1 = bf16(y - y0), ...).
__device__ __forceinline__ void decode_store(float y, int col, int b, float *out, int ldo,
                                             uint16_t *terms, int T, int ldt, int B) {
    out[(size_t)b * ldo + col] = y;
    if (terms) {
        for (int t = 0; t < T; ++t) {
            const uint32_t hb = bf16_rne_bits(y);
            y = term_rem(y, hb);
            terms[((size_t)t * B + b) * ldt + col] = (uint16_t)hb;
        }
    }
}

// w[it] = lane it << RSH of the lane's row (row_newbcast), it = 0..NV-1.
template <int NV, int RSH>
__device__ __forceinline__ void bcast_rows(float e, float (&w)[NV]) {
    w[0] = dpp_f<DPP_ROW_BCAST0>(e);
    if constexpr (NV > 1) w[1] = dpp_f<DPP_ROW_BCAST0 + (1 << RSH)>(e);
    if constexpr (NV > 2) w[2] = dpp_f<DPP_ROW_BCAST0 + (2 << RSH)>(e);
    if constexpr (NV > 3) w[3] = dpp_f<DPP_ROW_BCAST0 + (3 << RSH)>(e);
    if constexpr (NV > 4) {
        w[4] = dpp_f<DPP_ROW_BCAST0 + (4 << RSH)>(e);
        w[5] = dpp_f<DPP_ROW_BCAST0 + (5 << RSH)>(e);
        w[6] = dpp_f<DPP_ROW_BCAST0 + (6 << RSH)>(e);
        w[7] = dpp_f<DPP_ROW_BCAST0 + (7 << RSH)>(e);
    }
    if constexpr (NV > 8) {
        w[8] = dpp_f<DPP_ROW_BCAST0 + 8>(e);
        w[9] = dpp_f<DPP_ROW_BCAST0 + 9>(e);
        w[10] = dpp_f<DPP_ROW_BCAST0 + 10>(e);
        w[11] = dpp_f<DPP_ROW_BCAST0 + 11>(e);
        w[12] = dpp_f<DPP_ROW_BCAST0 + 12>(e);
        w[13] = dpp_f<DPP_ROW_BCAST0 + 13>(e);
        w[14] = dpp_f<DPP_ROW_BCAST0 + 14>(e);
        w[15] = dpp_f<DPP_ROW_BCAST0 + 15>(e);
    }
}

// M = max_s m_s, as a wave-uniform value (lane j takes s = j, j + 64, ...;
// a max is exact, so the grouping does not change it).
__device__ __forceinline__ float partial_max(const float *pp, int n) {
    const int lane = threadIdx.x & 63;
    float M = pp[(lane < n ? lane : 0) * AD_PART];
    for (int c = lane + 64; c < n; c += 64) M = fmaxf(M, pp[c * AD_PART]);
    M = row16_max(M);
    M = fmaxf(M, lane_xor16(M));
    return fmaxf(M, lane_xor32(M));
}
// L += sum_s l_s f_s and O += sum_s o_s[d] f_s over n partials in order,
// the weights f_s = e^{m_s - M} in slot 2; the loads of four sub-chunks are
// issued before their FMAs.
__device__ __forceinline__ void merge_partials(const float *pp, int n, int d, float &L, float &O) {
    int c = 0;
    for (; c + 16 <= n; c += 16) {
        float f[16], l[16], o[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            f[j] = pp[(c + j) * AD_PART + 2];
            l[j] = pp[(c + j) * AD_PART + 1];
            o[j] = pp[(c + j) * AD_PART + 4 + d];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            L = __builtin_fmaf(l[j], f[j], L);
            O = __builtin_fmaf(o[j], f[j], O);
        }
    }
    for (; c + 4 <= n; c += 4) {
        float f[4], l[4], o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[j] = pp[(c + j) * AD_PART + 2];
            l[j] = pp[(c + j) * AD_PART + 1];
            o[j] = pp[(c + j) * AD_PART + 4 + d];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            L = __builtin_fmaf(l[j], f[j], L);
            O = __builtin_fmaf(o[j], f[j], O);
        }
    }
    for (; c < n; ++c) {
        const float f = pp[c * AD_PART + 2];
        L = __builtin_fmaf(pp[c * AD_PART + 1], f, L);
        O = __builtin_fmaf(pp[c * AD_PART + 4 + d], f, O);
    }
}

// grid (H, B, partitions); partition z takes sub-chunks [z spp, z spp + spp)
// (spp = 0: all of them, merged here). gsub: sub-chunk slots per (head,
// sequence) in gpart.
template <int NW, bool PART, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void attn_decode_kernel(DecodeArgs a, float *out, int ldo,
                                                              uint16_t *terms, int T, int ldt,
                                                              int B, int spp, float *gpart,
                                                              int gsub) {
    extern __shared__ float spart[];  // [nsub][AD_PART] when this workgroup merges
    __shared__ float qs[64], kn[64], vn[64];
    // the cache rows are streamed once per step: nontemporal loads
    constexpr int KV_POLICY = BUF_NT;
    const int h = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 4, q = lane & 15;
    const int pos = a.posp ? *a.posp : a.pos;
    const int nsub = pos / AD_SUB + 1;
    const int z = (int)blockIdx.z, nf = SPLIT ? 0 : a.frac;
    // spp: fixed partitions of spp sub-chunks; nf: nf ranges of about equal
    // size, [ceil(z nsub / nf), ceil((z + 1) nsub / nf)) -- range 0 is never
    // empty, so its workgroup always appends the new row
    const int s0 = nf ? (z * nsub + nf - 1) / nf : spp ? z * spp : 0;
    const int s1 = nf ? ((z + 1) * nsub + nf - 1) / nf : spp ? min(s0 + spp, nsub) : nsub;
    if (s0 >= s1) {  // a partition past the cached positions (never z = 0)
        if (nf && tid < 64) {  // an empty range: max -inf, sum 0, O 0
            float *fp = a.fpart + (((size_t)b * a.H + h) * nf + z) * AD_PART;
            if (tid == 0) *(float2 *)fp = make_float2(-INFINITY, 0.0f);
            fp[4 + tid] = 0.0f;
        }
        return;
    }
    const size_t head = ((size_t)b * a.H + h) * (a.hs ? a.hs : a.cap) * 64;

    // Cache rows through buffer loads whose range ends at row `pos`: rows at
    // or past it (the new row, rows of a sub-chunk past the last) read as
    // zero without a memory access, so every load is issued unconditionally
    // and the memory counter waits stay exact.
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.kc + head), 0, pos * 256, BUF_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + head), 0, pos * 256, BUF_RSRC_WORD3);
    auto load = [&](float4 (&kk)[AD_NV], float4 (&vv)[AD_NV], int s) {
#pragma unroll
        for (int it = 0; it < AD_NV; ++it) {
            const int off = (s * AD_SUB + it * 4 + grp) * 256 + 16 * q;
            kk[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, KV_POLICY));
            vv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, KV_POLICY));
        }
    };
    // a sub-chunk this workgroup owns, else one wholly past `pos` (zeros)
    auto live = [&](int s) { return s < s1 ? s : nsub + wave; };

    // the new q/k/v values first (every lane, unconditionally), then the
    // first rows; the scheduling barriers keep that issue order so the
    // rotation below waits only for the former
    const int l32 = lane & 31;
    float q1 = 0.f, q2 = 0.f, k1 = 0.f, k2 = 0.f, vnew = 0.f;
    float pv[PART ? PART_KS_MAX : 1];
    float wsc = 0.f;
    if constexpr (PART) {
        // threads 0..191 (waves 0-2) each own one of the head's q/k/v
        // columns and load every k-slice partial of it before the cache
        // rows; the branches on the wave and the slice count are uniform
#pragma unroll
        for (int k = 0; k < PART_KS_MAX; ++k) pv[k] = 0.0f;
        if (tid < 192) {
            const int pcol = (tid >> 6) * a.H * 64 + h * 64 + (tid & 63);
            const float *pp = a.part + (size_t)b * a.ldp + pcol;
            wsc = a.wscale[pcol];
            const size_t pst = (size_t)B * a.ldp;
#pragma unroll
            for (int k = 0; k < PART_KS_MAX; ++k)
                if (k < a.ks) pv[k] = pp[k * pst];
        }
    } else {
        const float *qr = a.q + (size_t)b * a.ldq + h * 64;
        const float *kr = a.k_new + (size_t)b * a.ldq + h * 64;
        q1 = qr[l32], q2 = qr[l32 + 32], k1 = kr[l32], k2 = kr[l32 + 32];
        vnew = a.v_new[(size_t)b * a.ldq + h * 64 + lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 ka[AD_NV], va[AD_NV], kb[AD_NV], vb[AD_NV];
    int s = s0 + wave;
    load(ka, va, live(s));
    __builtin_amdgcn_sched_barrier(0);
    const float fpos = (float)pos;
    if constexpr (PART) {
        // slices summed in order, then the column scale; wave 0 holds q, wave
        // 1 k, wave 2 v, one column per lane: each lane of waves 0 and 1
        // takes its RoPE partner (column l ^ 32) by a lane swap and keeps its
        // own half of the rotated pair (l32, l32 + 32)
        if (tid < 192) {
            float v = pv[0];
#pragma unroll
            for (int k = 1; k < PART_KS_MAX; ++k)
                if (k < a.ks) v += pv[k];
            v = v * wsc;
            if (wave < 2) {
                const float o = lane_xor32(v);
                const bool lo = lane < 32;
                float y1, y2;
                rope_pair(lo ? v : o, lo ? o : v, fpos, l32, a.step, &y1, &y2);
                (wave == 0 ? qs : kn)[lane] = lo ? y1 : y2;
            } else {
                vn[lane] = v;
            }
        }
    } else {  // q rotated by wave 0, k by wave 1
        if (wave < 2 && lane < 32) {
            float y1, y2;
            rope_pair(wave == 0 ? q1 : k1, wave == 0 ? q2 : k2, fpos, lane, a.step, &y1, &y2);
            float *dst = wave == 0 ? qs : kn;
            dst[lane] = y1;
            dst[lane + 32] = y2;
        }
        if (wave == 0) vn[lane] = vnew;
    }
    __syncthreads();
    if (tid < 64 && blockIdx.z == 0) {  // append the new row (no wave reads row `pos` from the cache)
        a.kc[head + (size_t)pos * 64 + tid] = kn[tid];
        a.vc[head + (size_t)pos * 64 + tid] = vn[tid];
    }
    const float4 qv = make_float4(qs[4 * q], qs[4 * q + 1], qs[4 * q + 2], qs[4 * q + 3]);
    const float4 kq = make_float4(kn[4 * q], kn[4 * q + 1], kn[4 * q + 2], kn[4 * q + 3]);
    const float4 vq = make_float4(vn[4 * q], vn[4 * q + 1], vn[4 * q + 2], vn[4 * q + 3]);

    auto consume = [&](const float4 (&kk)[AD_NV], const float4 (&vv)[AD_NV], int sc_) {
        const int p0 = sc_ * AD_SUB;
        // partial dots (4 dims per lane), then a transposing butterfly over
        // the 16 lanes of a row group: lane (grp, q) ends with row
        // p0 + 4 (q >> AD_RSH) + grp, the same value on the lanes that
        // differ only in the low AD_RSH bits of q
        float d[AD_NV];
#pragma unroll
        for (int it = 0; it < AD_NV; ++it) {
            const int p = p0 + it * 4 + grp;
            const float4 k4 = p == pos ? kq : kk[it];
            float t = qv.x * k4.x;
            t = __builtin_fmaf(qv.y, k4.y, t);
            t = __builtin_fmaf(qv.z, k4.z, t);
            d[it] = __builtin_fmaf(qv.w, k4.w, t);
        }
        bfly_stage<AD_NV, DPP_ROW_MIRROR>(d, (q & 8) != 0);
        bfly_stage<AD_NV / 2, DPP_ROW_HALF_MIRROR>(d, (q & 4) != 0);
        if constexpr (AD_NV >= 8) bfly_stage<AD_NV / 4, DPP_QUAD_REV>(d, (q & 2) != 0);
        if constexpr (AD_NV >= 16) bfly_stage<AD_NV / 8, DPP_QUAD_SWAP>(d, (q & 1) != 0);
        float dd = d[0];
        if constexpr (AD_NV < 8) dd = dd + dpp_f<DPP_QUAD_REV>(dd);
        if constexpr (AD_NV < 16) dd = dd + dpp_f<DPP_QUAD_SWAP>(dd);
        const float sc = p0 + 4 * (q >> AD_RSH) + grp <= pos ? dd * a.scale : -INFINITY;
        // the sub-chunk's max and sum: the rows of the group (lanes rotated
        // by 8, 4, ... within the row, each row once), then the four groups
        // (lanes l ^ 16, l ^ 32)
        float mc = fmaxf(sc, dpp_f<DPP_ROW_ROR8>(sc));
        mc = fmaxf(mc, dpp_f<DPP_ROW_ROR4>(mc));
        if constexpr (AD_NV >= 8) mc = fmaxf(mc, dpp_f<DPP_ROW_ROR2>(mc));
        if constexpr (AD_NV >= 16) mc = fmaxf(mc, dpp_f<DPP_ROW_ROR1>(mc));
        mc = fmaxf(mc, lane_xor16(mc));
        mc = fmaxf(mc, lane_xor32(mc));  // row p0 <= pos: finite
        const float e = sc == -INFINITY ? 0.0f : exp_f(sc - mc);
        float lc = e + dpp_f<DPP_ROW_ROR8>(e);
        lc = lc + dpp_f<DPP_ROW_ROR4>(lc);
        if constexpr (AD_NV >= 8) lc = lc + dpp_f<DPP_ROW_ROR2>(lc);
        if constexpr (AD_NV >= 16) lc = lc + dpp_f<DPP_ROW_ROR1>(lc);
        lc = lc + lane_xor16(lc);
        lc = lc + lane_xor32(lc);
        // weights of rows (it, grp): lane it << AD_RSH of the row, broadcast
        float w[AD_NV];
        bcast_rows<AD_NV, AD_RSH>(e, w);
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int it = 0; it < AD_NV; ++it) {
            const float4 v4 = p0 + it * 4 + grp == pos ? vq : vv[it];
            o.x = __builtin_fmaf(w[it], v4.x, o.x);
            o.y = __builtin_fmaf(w[it], v4.y, o.y);
            o.z = __builtin_fmaf(w[it], v4.z, o.z);
            o.w = __builtin_fmaf(w[it], v4.w, o.w);
        }
        o.x = o.x + lane_xor16(o.x);
        o.y = o.y + lane_xor16(o.y);
        o.z = o.z + lane_xor16(o.z);
        o.w = o.w + lane_xor16(o.w);
        o.x = o.x + lane_xor32(o.x);
        o.y = o.y + lane_xor32(o.y);
        o.z = o.z + lane_xor32(o.z);
        o.w = o.w + lane_xor32(o.w);
        if constexpr (SPLIT) {
            float *pc = gpart + (((size_t)b * a.H + h) * gsub + sc_) * AD_PART;
            if (lane == 0) *(float2 *)pc = make_float2(mc, lc);
            if (grp == 0) *(float4 *)&pc[4 + 4 * q] = o;
        } else {
            float *pc = spart + (sc_ - s0) * AD_PART;
            if (lane == 0) *(float2 *)pc = make_float2(mc, lc);
            if (grp == 0) *(float4 *)&pc[4 + 4 * q] = o;
        }
    };
    while (s < s1) {
        load(kb, vb, live(s + NW));
        consume(ka, va, s);
        s += NW;
        if (s >= s1) break;
        load(ka, va, live(s + NW));
        consume(kb, vb, s);
        s += NW;
    }
    if constexpr (SPLIT) return;  // merged by attn_decode_merge_kernel
    __syncthreads();
    const int nloc = s1 - s0;  // this workgroup's sub-chunks (all of them unless nf)
    const float M = partial_max(spart, nloc);  // every wave, the same value
    for (int c = tid; c < nloc; c += NW * 64) spart[c * AD_PART + 2] = exp_f(spart[c * AD_PART] - M);
    __syncthreads();
    if (tid >= 64) return;
    float L = 0.0f, O = 0.0f;
    merge_partials(spart, nloc, tid, L, O);
    if (nf) {  // the range's partial, merged with the others by the consumer
        float *fp = a.fpart + (((size_t)b * a.H + h) * nf + z) * AD_PART;
        if (tid == 0) *(float2 *)fp = make_float2(M, L);
        fp[4 + tid] = O;
        return;
    }
    decode_store(O / L, h * 64 + tid, b, out, ldo, terms, T, ldt, B);
}

// The same merge over the partials of every partition, in sub-chunk order:
// blocks of AD_MBLK sub-chunks copied to LDS (one coalesced pass by the 256
// threads) and folded into the running sums in order; M from the copy when
// one block holds them all, else from a first pass over the m_s.
constexpr int AD_MBLK = AD_LDS_MAX / (AD_PART * sizeof(float));
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(const float *__restrict__ gpart,
                                                                int gsub, const int *posp, int pos,
                                                                int H, float *out, int ldo,
                                                                uint16_t *terms, int T, int ldt,
                                                                int B) {
    extern __shared__ float sm[];  // [min(nsub, AD_MBLK)][AD_PART]
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int nsub = (posp ? *posp : pos) / AD_SUB + 1;
    const float *pp = gpart + ((size_t)b * H + h) * gsub * AD_PART;
    float M = nsub > AD_MBLK ? partial_max(pp, nsub) : 0.0f;
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nsub; c0 += AD_MBLK) {
        const int n = min(AD_MBLK, nsub - c0);
        const float4 *src = (const float4 *)(pp + (size_t)c0 * AD_PART);
        for (int i = tid; i < n * (AD_PART / 4); i += 256) ((float4 *)sm)[i] = src[i];
        __syncthreads();
        if (nsub <= AD_MBLK) M = partial_max(sm, n);
        for (int c = tid; c < n; c += 256) sm[c * AD_PART + 2] = exp_f(sm[c * AD_PART] - M);
        __syncthreads();
        if (tid < 64) merge_partials(sm, n, tid, L, O);
        __syncthreads();
    }
    if (tid < 64) decode_store(O / L, h * 64 + tid, b, out, ldo, terms, T, ldt, B);
}

// Sub-chunks per partition, or 0 for one workgroup per (head, sequence):
// the caller's choice (a.split >= 0), else partitions when one workgroup's
// partials would not fit in LDS, or with a host position when the pairs are
// fewer than the CUs and the rows long (512 positions or more; 64 positions
// per workgroup: 8.30 us at 36 heads x 1024 positions, against 8.53 with 128
// positions, 10.7 with 16 and 9.7 with 256).
static int decode_spp(const DecodeArgs &a, int B) {
    if (a.split >= 0) return a.split;
    const int gsub = (a.cap + AD_SUB - 1) / AD_SUB;
    if ((size_t)gsub * AD_PART * sizeof(float) > AD_LDS_MAX) return 4;
    if (a.posp || a.part || a.H * B >= 256) return 0;
    return a.pos + 1 >= 512 ? 64 / AD_SUB : 0;
}

size_t attention_decode_work_floats(const DecodeArgs &a, int B) {
    return decode_spp(a, B) ? (size_t)B * a.H * ((a.cap + AD_SUB - 1) / AD_SUB) * AD_PART : 0;
}

template <int NW>
static void launch_decode_nw(const DecodeArgs &a, int B, float *out, int ldo, uint16_t *terms,
                             int T, int ldt, hipStream_t st, dim3 grid, size_t lds, int spp,
                             float *work, int gsub) {
    if (spp) {
        if (a.part)
            attn_decode_kernel<NW, true, true><<<grid, NW * 64, lds, st>>>(a, out, ldo, terms, T,
                                                                           ldt, B, spp, work, gsub);
        else
            attn_decode_kernel<NW, false, true><<<grid, NW * 64, lds, st>>>(a, out, ldo, terms, T,
                                                                            ldt, B, spp, work, gsub);
    } else {
        if (a.part)
            attn_decode_kernel<NW, true, false><<<grid, NW * 64, lds, st>>>(a, out, ldo, terms, T,
                                                                            ldt, B, 0, work, gsub);
        else
            attn_decode_kernel<NW, false, false><<<grid, NW * 64, lds, st>>>(a, out, ldo, terms, T,
                                                                             ldt, B, 0, work, gsub);
    }
}

int launch_attention_decode(const DecodeArgs &a, int B, float *out, int ldo, uint16_t *terms,
                            int T, int ldt, hipStream_t st, float *work) {
    VMLM_GUARD(a.cap >= 1 && a.H >= 1 && B >= 1 && (a.hs == 0 || a.hs >= a.cap),
               "attention decode: empty shape, or head stride below the capacity");
    VMLM_GUARD((size_t)(a.cap + 16 * AD_SUB) * 256 <= 0x7fffffffu,
               "attention decode: cache row range too large");
    VMLM_GUARD(!a.part || (a.ks >= 1 && a.ks <= PART_KS_MAX && a.wscale && a.ldp >= 3 * a.H * 64),
               "attention decode: partial q/k/v need ks, ldp and scales");
    const int gsub = (a.cap + AD_SUB - 1) / AD_SUB;
    const int spp = a.frac > 0 ? 0 : decode_spp(a, B);
    if (a.frac > 0) {
        VMLM_GUARD(a.fpart && !a.part && a.frac <= 64 && (size_t)gsub * AD_PART * sizeof(float) <= AD_LDS_MAX,
                   "attention decode: position ranges need the partial buffer, rows (not slices) "
                   "of q/k/v, at most 64 ranges and a capacity within one workgroup's LDS");
        const dim3 grid(a.H, B, a.frac);
        launch_decode_nw<4>(a, B, out, ldo, terms, T, ldt, st, grid,
                            (size_t)gsub * AD_PART * sizeof(float), 0, nullptr, gsub);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    if (spp > 0) {
        VMLM_GUARD(work, "attention decode: split positions need a work buffer of %zu floats",
                   attention_decode_work_floats(a, B));
        // grid from the capacity for a device position, else from `pos`
        const int nsub = a.posp ? gsub : a.pos / AD_SUB + 1;
        const dim3 grid(a.H, B, (nsub + spp - 1) / spp);
        launch_decode_nw<4>(a, B, out, ldo, terms, T, ldt, st, grid, 0, spp, work, gsub);
        VMLM_HIP_CHECK(hipGetLastError());
        const size_t mlds = (size_t)(gsub < AD_MBLK ? gsub : AD_MBLK) * AD_PART * sizeof(float);
        attn_decode_merge_kernel<<<dim3(a.H, B), 256, mlds, st>>>(
            work, gsub, a.posp, a.pos, a.H, out, ldo, terms, T, ldt, B);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    const size_t lds = (size_t)gsub * AD_PART * sizeof(float);
    VMLM_GUARD(lds <= AD_LDS_MAX, "attention decode: cache capacity %d needs split positions",
               a.cap);
    const dim3 grid(a.H, B);
    // (at 36 heads x 16 sequences, 8 and 16 waves per workgroup, 2 waves,
    // 32-position sub-chunks, or two and three sub-chunks in flight per wave
    // while one is consumed (one now) measured 1 to 34 % slower than 4 waves)
    if (a.H * B < 256)
        launch_decode_nw<8>(a, B, out, ldo, terms, T, ldt, st, grid, lds, 0, nullptr, gsub);
    else
        launch_decode_nw<4>(a, B, out, ldo, terms, T, ldt, st, grid, lds, 0, nullptr, gsub);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

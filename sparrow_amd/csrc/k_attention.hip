// k_attention.hip -- attention as the VM program composes it, fused.
//
// Prefill (tools/p12_build_minicpm.py:770-781): per head SLICE -> ROPE(pos0)
// -> GEMM NT q.k -> SCALE -> SOFTMAX(causal) -> GEMM NN p.v -> WRITECOL.
// Here: RoPE is applied once to Q and K (bit-exact port), then one kernel
// per (head, 64-query block) streams 64-key tiles through LDS with an
// online softmax (exp_f of the reference, scores scaled exactly as OP_SCALE
// does) -- the [S,S] score matrix never reaches HBM.
//
// Decode (tools/p12_build_minicpm.py:941-967): per (sequence, head, 64-
// position split) one wavefront rotates q and the new k at `pos`, appends the
// rotated k and raw v to the f32 cache, scores its positions (16 lanes per
// 256-byte K row, four rows per coalesced load instruction, all loads of
// the split in flight together), and accumulates its share of p.V; a
// combine kernel merges the splits (flash-decoding).
//
// Both change the order of the reference's sums (E contract: 1e-4 of the
// output RMS); RoPE, the scale multiply and every exp_f are bitwise.
#include "internal.hpp"

namespace vmlm {

// ---------------------------------------------------------------- f32 GEMM
// C[m,n] (+)= A[m,k] . op(B), op(B) = B[n,k]^T (nt) or B[k,n].
// 64x64 tiles, 256 threads of 4x4 outputs, 64-deep k-steps through LDS
// (As[k][row], Bs[k][col]); the next step's tiles are loaded into registers
// while the current one is consumed. With VEC the rows are read as float4
// (k, or n for an NN B, a multiple of 4 and 16-byte aligned operands).
// A narrow output is split over k (grid z): each slice writes its partial
// tile to `part` [ks][m][n] and gemm_f32_reduce_kernel sums the slices in
// order (deterministic).
constexpr int GF_T = 64, GF_K = 64, GF_LD = 68;

template <bool NT, bool VEC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float *__restrict__ A,
                                                       const float *__restrict__ B,
                                                       float *__restrict__ C, int m, int n, int k,
                                                       int acc, int kslice,
                                                       float *__restrict__ part) {
    __shared__ __attribute__((aligned(16))) float As[GF_K][GF_LD];
    __shared__ __attribute__((aligned(16))) float Bs[GF_K][GF_LD];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int row0 = blockIdx.y * GF_T, col0 = blockIdx.x * GF_T;
    const int kb = blockIdx.z * kslice;
    const int ke = kb + kslice < k ? kb + kslice : k;
    // loader roles: A (and an NT B) as 64 rows x 16 float4 of k; an NN B as
    // 64 k-rows x 16 float4 of n; 4 pieces per thread
    float4 ra[4], rb[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = tid + q * 256, r = e >> 4, c4 = (e & 15) * 4;
            const int gk = k0 + c4;
            {
                const int gr = row0 + r;
                const float *pa = A + (size_t)(gr < m ? gr : 0) * k + gk;
                if constexpr (VEC) {
                    ra[q] = gr < m && gk < ke ? *(const float4 *)pa : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    ra[q].x = gr < m && gk < ke ? pa[0] : 0.f;
                    ra[q].y = gr < m && gk + 1 < ke ? pa[1] : 0.f;
                    ra[q].z = gr < m && gk + 2 < ke ? pa[2] : 0.f;
                    ra[q].w = gr < m && gk + 3 < ke ? pa[3] : 0.f;
                }
            }
            if constexpr (NT) {
                const int gc = col0 + r;
                const float *pb = B + (size_t)(gc < n ? gc : 0) * k + gk;
                if constexpr (VEC) {
                    rb[q] = gc < n && gk < ke ? *(const float4 *)pb : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    rb[q].x = gc < n && gk < ke ? pb[0] : 0.f;
                    rb[q].y = gc < n && gk + 1 < ke ? pb[1] : 0.f;
                    rb[q].z = gc < n && gk + 2 < ke ? pb[2] : 0.f;
                    rb[q].w = gc < n && gk + 3 < ke ? pb[3] : 0.f;
                }
            } else {
                const int gkr = k0 + r, gc = col0 + c4;
                const float *pb = B + (size_t)(gkr < ke ? gkr : kb) * n + gc;
                if constexpr (VEC) {
                    rb[q] = gkr < ke && gc < n ? *(const float4 *)pb : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    rb[q].x = gkr < ke && gc < n ? pb[0] : 0.f;
                    rb[q].y = gkr < ke && gc + 1 < n ? pb[1] : 0.f;
                    rb[q].z = gkr < ke && gc + 2 < n ? pb[2] : 0.f;
                    rb[q].w = gkr < ke && gc + 3 < n ? pb[3] : 0.f;
                }
            }
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = tid + q * 256, r = e >> 4, c4 = (e & 15) * 4;
            As[c4][r] = ra[q].x;
            As[c4 + 1][r] = ra[q].y;
            As[c4 + 2][r] = ra[q].z;
            As[c4 + 3][r] = ra[q].w;
            if constexpr (NT) {
                Bs[c4][r] = rb[q].x;
                Bs[c4 + 1][r] = rb[q].y;
                Bs[c4 + 2][r] = rb[q].z;
                Bs[c4 + 3][r] = rb[q].w;
            } else {
                *(float4 *)&Bs[r][c4] = rb[q];
            }
        }
    };
    float c[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[i][j] = 0.0f;
    load(kb);
    for (int k0 = kb; k0 < ke; k0 += GF_K) {
        __syncthreads();
        store();
        __syncthreads();
        if (k0 + GF_K < ke) load(k0 + GF_K);
#pragma unroll 16
        for (int kk = 0; kk < GF_K; ++kk) {
            const float4 a = *(const float4 *)&As[kk][ty * 4];
            const float4 b = *(const float4 *)&Bs[kk][tx * 4];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[i][j] = __builtin_fmaf(av[i], bv[j], c[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gr = row0 + ty * 4 + i;
        if (gr >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gc = col0 + tx * 4 + j;
            if (gc >= n) continue;
            if (part) {
                part[((size_t)blockIdx.z * m + gr) * n + gc] = c[i][j];
            } else {
                float *o = C + (size_t)gr * n + gc;
                *o = acc ? *o + c[i][j] : c[i][j];
            }
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
        if (!acc) VMLM_HIP_CHECK(hipMemsetAsync(c, 0, m * n * sizeof(float), st));
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
// products (q0k0 + q0k1 + q1k0 + q1k1; p0v0 + p0v1 + p0v2 + p1v0 + p1v1),
// each exact, accumulated in f32 by v_mfma_f32_16x16x32_bf16: relative error
// ~2^-16, well inside the 1e-4 * RMS contract of the attention composition,
// and a one-key softmax row returns its V row exactly. A workgroup owns 64
// queries of one head (wave w: queries 16w..16w+15) and walks the key blocks
// of 64 up to the diagonal: K is staged as [key][dim] terms, V transposed as
// [dim][key] terms, the probabilities go back through LDS as terms, and the
// running max / sum are per query row (rows 4g..4g+3 of lane (g, r), reduced
// over the 16 lanes r of a DPP row).
constexpr int AT_B = 64;   // query / key block
constexpr int AT_LD = 72;  // bf16 elements per LDS row (64 + 8)

// DPP lane moves inside a row of 16 lanes (row_mirror: lane i <- 15 - i;
// row_half_mirror: i <- 7 - i within each 8; quad_perm [3,2,1,0] and
// [1,0,3,2]): partners that differ in bit 3, 2, 1, 0 of the lane index.
constexpr int DPP_ROW_MIRROR = 0x140, DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_QUAD_REV = 0x1B, DPP_QUAD_SWAP = 0xB1;

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
    const float *Q, *K, *V;
    float *O;
    size_t sin, sout;
    int S, ld, ldo, causal, rope_q, nqb;
    float scale, rope_step, pos0;
};

__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(PrefillParams P) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AT_B][AT_LD];   // [term][key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t Vt[3][64][AT_LD];     // [term][dim][key]
    __shared__ __attribute__((aligned(16))) uint16_t Ps[4][2][16][AT_LD];  // [wave][term][q][key]
    const int S = P.S, ld = P.ld, causal = P.causal;
    const int h = blockIdx.y, z = blockIdx.z;
    const int qb = causal ? P.nqb - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int kb0 = 0, kb1 = causal ? qb + 1 : (S + AT_B - 1) / AT_B;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int q0 = qb * AT_B + wave * 16;
    const float *Qh = P.Q + z * P.sin + h * 64, *Kh = P.K + z * P.sin + h * 64,
                *Vh = P.V + z * P.sin + h * 64;

    // this lane's query fragments: row q0 + r, dims 32s + 8g .. +7, two terms;
    // the lane holds both members (i, i + 32) of its RoPE pairs, so an
    // unrotated Q is rotated here (position pos0 + row)
    u32x4 aq[2][2];  // [slice][term]
    {
        const int qr = q0 + r < S ? q0 + r : S - 1;
        float x[2][8];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            const float4 *src = (const float4 *)(Qh + (size_t)qr * ld + sl * 32 + g * 8);
            const float4 x0 = src[0], x1 = src[1];
            x[sl][0] = x0.x, x[sl][1] = x0.y, x[sl][2] = x0.z, x[sl][3] = x0.w;
            x[sl][4] = x1.x, x[sl][5] = x1.y, x[sl][6] = x1.z, x[sl][7] = x1.w;
        }
        if (P.rope_q) {
            const float fpos = P.pos0 + (float)qr;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                rope_pair(x[0][e], x[1][e], fpos, g * 8 + e, P.rope_step, &x[0][e], &x[1][e]);
        }
        split8(x[0], aq[0][0], aq[0][1]);
        split8(x[1], aq[1][0], aq[1][1]);
    }
    float m[4], l[4];
    f32x4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
        o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // staging roles: K rows (key tid/4, dims 16*(tid%4) ..), V columns (dim
    // tid%64, keys 16*(tid/64) ..)
    const int kkey = tid >> 2, kd0 = (tid & 3) * 16;
    const int vd = tid & 63, vk0 = (tid >> 6) * 16;
    // the next key block's K / V are loaded into registers while the current
    // one is consumed (the last block reloads itself)
    float kx[16], vx[16];
    auto load_kv = [&](int kb) {
        const int k0 = kb * AT_B;
        const int kr = k0 + kkey < S ? k0 + kkey : S - 1;
        const float4 *src = (const float4 *)(Kh + (size_t)kr * ld + kd0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = src[i];
            kx[4 * i] = v.x;
            kx[4 * i + 1] = v.y;
            kx[4 * i + 2] = v.z;
            kx[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int vr = k0 + vk0 + i < S ? k0 + vk0 + i : S - 1;
            vx[i] = Vh[(size_t)vr * ld + vd];
        }
    };
    load_kv(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        const int k0 = kb * AT_B;
        __syncthreads();  // the previous block's K / V are no longer read
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float x[8], y[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[i] = k0 + kkey < S ? kx[8 * half + i] : 0.0f;
                y[i] = k0 + vk0 + 8 * half + i < S ? vx[8 * half + i] : 0.0f;
            }
            u32x4 t0, t1, t2;
            split8(x, t0, t1);
            *(u32x4 *)&Ks[0][kkey][kd0 + 8 * half] = t0;
            *(u32x4 *)&Ks[1][kkey][kd0 + 8 * half] = t1;
            split8x3(y, t0, t1, t2);
            *(u32x4 *)&Vt[0][vd][vk0 + 8 * half] = t0;
            *(u32x4 *)&Vt[1][vd][vk0 + 8 * half] = t1;
            *(u32x4 *)&Vt[2][vd][vk0 + 8 * half] = t2;
        }
        __syncthreads();
        load_kv(kb + 1 < kb1 ? kb + 1 : kb);
        __builtin_amdgcn_sched_barrier(0);

        // scores: block j = keys 16j..16j+15; lane (g, r): queries 4g+i, key
        // 16j+r. The four blocks' MFMA chains are interleaved (each block's
        // own term order is q0k0, q0k1, q1k0, q1k1 per 32-dim slice).
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
            for (int j = 0; j < 4; ++j) sc[j] = mfma_b(aq[sl][0], b0[j], sc[j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) sc[j] = mfma_b(aq[sl][0], b1[j], sc[j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) sc[j] = mfma_b(aq[sl][1], b0[j], sc[j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) sc[j] = mfma_b(aq[sl][1], b1[j], sc[j]);
        }
        float rmax[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qa = q0 + 4 * g + i;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ka = k0 + 16 * j + r;
                const bool valid = ka < S && (!causal || ka <= qa);
                sc[j][i] = valid ? sc[j][i] * P.scale : -INFINITY;
                mx = fmaxf(mx, sc[j][i]);
            }
            rmax[i] = row16_max(mx);
        }
        float p[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float mn = fmaxf(m[i], rmax[i]);
            const float alpha = m[i] == -INFINITY ? 0.0f : __expf(m[i] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                p[j][i] = sc[j][i] == -INFINITY ? 0.0f : __expf(sc[j][i] - mn);
                rs += p[j][i];
            }
            rs = row16_sum(rs);
            l[i] = l[i] * alpha + rs;
            m[i] = mn;
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd][i] *= alpha;
        }
        // P terms -> LDS as [q][key] rows of this wave
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t hb = bf16_rne_bits(p[j][i]);
                const uint32_t lb = bf16_rne_bits(p[j][i] - bf16_bits_to_f32(hb));
                Ps[wave][0][4 * g + i][16 * j + r] = (uint16_t)hb;
                Ps[wave][1][4 * g + i][16 * j + r] = (uint16_t)lb;
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O[q][d] += P[q][key] V[key][d]: A = P rows, B = V^T rows (dims);
        // the four dim blocks' chains interleaved, each in the term order
        // p0v0, p0v1, p0v2, p1v0, p1v1
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            const u32x4 p0 = *(const u32x4 *)&Ps[wave][0][r][sl * 32 + g * 8];
            const u32x4 p1 = *(const u32x4 *)&Ps[wave][1][r][sl * 32 + g * 8];
            u32x4 v0[4], v1[4], v2[4];
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) {
                v0[jd] = *(const u32x4 *)&Vt[0][16 * jd + r][sl * 32 + g * 8];
                v1[jd] = *(const u32x4 *)&Vt[1][16 * jd + r][sl * 32 + g * 8];
                v2[jd] = *(const u32x4 *)&Vt[2][16 * jd + r][sl * 32 + g * 8];
            }
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(p0, v0[jd], o[jd]);
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(p0, v1[jd], o[jd]);
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(p0, v2[jd], o[jd]);
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(p1, v0[jd], o[jd]);
#pragma unroll
            for (int jd = 0; jd < 4; ++jd) o[jd] = mfma_b(p1, v1[jd], o[jd]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // lane (g, r) of block jd: queries 4g+i, dim 16jd + r
    float *Oz = P.O + z * P.sout;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qa = q0 + 4 * g + i;
        if (qa >= S) continue;
        const float inv = 1.0f / l[i];
#pragma unroll
        for (int jd = 0; jd < 4; ++jd)
            Oz[(size_t)qa * P.ldo + h * 64 + 16 * jd + r] = o[jd][i] * inv;
    }
}

int launch_attention_prefill(const float *q, const float *krot, const float *v, float *out,
                             int S, int H, int ld, int ldo, float scale, bool causal,
                             hipStream_t st, bool rope_q, float rope_step, float pos0, int nseq,
                             size_t sin, size_t sout) {
    VMLM_GUARD(ld % 4 == 0 && ((uintptr_t)q & 15) == 0 && ((uintptr_t)krot & 15) == 0 &&
                   (nseq == 1 || sin % 4 == 0),
               "attention prefill: 16-byte aligned rows required");
    VMLM_GUARD(nseq >= 1 && nseq <= 65535 && H <= 65535, "attention prefill: grid too large");
    if (S <= 0) return VMLM_OK;
    PrefillParams P;
    P.Q = q;
    P.K = krot;
    P.V = v;
    P.O = out;
    P.sin = sin;
    P.sout = sout;
    P.S = S;
    P.ld = ld;
    P.ldo = ldo;
    P.causal = causal ? 1 : 0;
    P.rope_q = rope_q ? 1 : 0;
    P.nqb = cdiv(S, AT_B);
    P.scale = scale;
    P.rope_step = rope_step;
    P.pos0 = pos0;
    attn_prefill_kernel<<<dim3(P.nqb, H, nseq), 256, 0, st>>>(P);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- decode
// Decode attention, one workgroup per (head, sequence): the new query and key
// are rotated once, the new key/value row is appended to the cache, and the
// AD_NW waves stride over the positions in chunks of 64 (wave w takes chunks
// w, w + AD_NW, ...). Each chunk leaves (m_c, l_c, o_c) = (max score,
// sum e^{s - m_c}, sum e^{s - m_c} v) in LDS; after a barrier they are merged
// in chunk order,
//   out = sum_c o_c e^{m_c - M} / sum_c l_c e^{m_c - M},
// so the result does not depend on the wave count.
// Lane (grp, q) of a wave holds dims 4q..4q+3 of positions p0 + 4*it + grp
// (it = 0..15): one load instruction covers 4 consecutive 256-byte rows.
// All 32 row loads of a chunk are issued together, unconditionally.
// AD_NW is 8 when the (head, sequence) pairs are fewer than the CUs (one
// workgroup per CU), else 4 with a register budget for three workgroups per
// CU so that all of them are resident at once.
constexpr int BUF_RSRC_WORD3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format


// One stage of the transposing butterfly: N values per lane become N/2 sums;
// the lane with `up` keeps the upper half and sends the lower.
template <int N, int CTRL>
__device__ __forceinline__ void bfly_stage(float (&d)[16], bool up) {
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
constexpr int AD_PART = 68;                 // floats per chunk partial: m, l, pad, o[64]
constexpr int PART_KS_MAX = 16;             // k-slices of partial q/k/v read up front

template <int AD_NW, bool PART>
__global__ __launch_bounds__(AD_NW * 64) __attribute__((amdgpu_waves_per_eu(AD_NW == 4 ? 3 : 2)))
void attn_decode_kernel(DecodeArgs a, float *out, int ldo, uint16_t *terms, int T, int ldt,
                        int B) {
    extern __shared__ float cpart[];  // [ceil(cap / 64)][AD_PART]
    __shared__ float qs[64], kn[64], vn[64];
    __shared__ float es[AD_NW][64];
    __shared__ float qkv_s[PART ? 192 : 1];
    const int h = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 4, q = lane & 15;
    const int pos = a.posp ? *a.posp : a.pos;
    const int nch = (pos + 1 + 63) / 64;
    const size_t head = ((size_t)b * a.H + h) * a.cap * 64;

    // Cache rows through buffer loads whose range ends at row `pos`: rows at
    // or past it (the new row, unused rows, chunks past the last) read as
    // zero without a memory access, so every wave issues its first chunk
    // unconditionally and the memory counter waits stay exact.
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.kc + head), 0, pos * 256, BUF_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + head), 0, pos * 256, BUF_RSRC_WORD3);
    float4 kv[16], vv[16];
    auto load_chunk = [&](int c) {
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int off = (c * 64 + it * 4 + grp) * 256 + 16 * q;
            kv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
            vv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
        }
    };
    // a wave's next chunk: its keys as soon as the scores are out of kv, its
    // values once the weighted sum is out of vv (chunks past the last read as 0)
    auto load_k = [&](int c) {
#pragma unroll
        for (int it = 0; it < 16; ++it)
            kv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    krs, (c * 64 + it * 4 + grp) * 256 + 16 * q, 0, 0));
    };
    auto load_v = [&](int c) {
#pragma unroll
        for (int it = 0; it < 16; ++it)
            vv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    vrs, (c * 64 + it * 4 + grp) * 256 + 16 * q, 0, 0));
    };
    // the new q/k/v values first (every lane, unconditionally), then the
    // chunk rows; the scheduling barriers keep that issue order so the
    // rotation below waits only for the former
    const int l32 = lane & 31;
    float q1 = 0.f, q2 = 0.f, k1 = 0.f, k2 = 0.f, vnew = 0.f;
    float pv[PART ? PART_KS_MAX : 1];
    float wsc = 0.f;
    if constexpr (PART) {
        // threads 0..191 each own one of the head's q/k/v columns and load
        // every k-slice partial of it (index clamped) before the chunk rows
        const int c = tid < 192 ? tid : 191;
        const int pcol = (c >> 6) * a.H * 64 + h * 64 + (c & 63);
        const float *pp = a.part + (size_t)b * a.ldp + pcol;
        wsc = a.wscale[pcol];
        const size_t pst = (size_t)B * a.ldp;
#pragma unroll
        for (int k = 0; k < PART_KS_MAX; ++k) pv[k] = pp[(k < a.ks ? k : a.ks - 1) * pst];
    } else {
        const float *qr = a.q + (size_t)b * a.ldq + h * 64;
        const float *kr = a.k_new + (size_t)b * a.ldq + h * 64;
        q1 = qr[l32], q2 = qr[l32 + 32], k1 = kr[l32], k2 = kr[l32 + 32];
        vnew = a.v_new[(size_t)b * a.ldq + h * 64 + lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_chunk(wave);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PART) {  // slices summed in order, then the row scale
        float v = pv[0];
#pragma unroll
        for (int k = 1; k < PART_KS_MAX; ++k)
            if (k < a.ks) v += pv[k];
        if (tid < 192) qkv_s[tid] = v * wsc;
        __syncthreads();
        q1 = qkv_s[l32];
        q2 = qkv_s[l32 + 32];
        k1 = qkv_s[64 + l32];
        k2 = qkv_s[96 + l32];
        vnew = qkv_s[128 + lane];
    }
    if (wave == 0) {
        if (lane < 32) {
            const float fpos = (float)pos;
            float y1, y2;
            rope_pair(q1, q2, fpos, lane, a.step, &y1, &y2);
            qs[lane] = y1;
            qs[lane + 32] = y2;
            rope_pair(k1, k2, fpos, lane, a.step, &y1, &y2);
            kn[lane] = y1;
            kn[lane + 32] = y2;
        }
        vn[lane] = vnew;
    }
    __syncthreads();
    if (tid < 64) {  // append the new row (no wave reads row `pos` from the cache)
        a.kc[head + (size_t)pos * 64 + tid] = kn[tid];
        a.vc[head + (size_t)pos * 64 + tid] = vn[tid];
    }
    const float4 qv = make_float4(qs[4 * q], qs[4 * q + 1], qs[4 * q + 2], qs[4 * q + 3]);
    const float4 kq = make_float4(kn[4 * q], kn[4 * q + 1], kn[4 * q + 2], kn[4 * q + 3]);
    const float4 vq = make_float4(vn[4 * q], vn[4 * q + 1], vn[4 * q + 2], vn[4 * q + 3]);

    // 8 waves (few workgroups, long rows per wave): a wave's next chunk is
    // loaded while the current one is consumed; 4 waves: loaded at the top
    constexpr bool PIPE = AD_NW == 8;
    for (int c = wave; c < nch; c += AD_NW) {
        if (!PIPE && c != wave) load_chunk(c);
        const int p0 = c * 64;
        // partial dots (4 dims per lane), then a transposing butterfly over
        // the 16 lanes of a group: lane (grp, q) ends with position
        // p0 + 4q + grp (15 DPP exchanges for 16 sums)
        float d[16];
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int p = p0 + it * 4 + grp;
            const float4 k4 = p == pos ? kq : kv[it];
            float t = qv.x * k4.x;
            t = __builtin_fmaf(qv.y, k4.y, t);
            t = __builtin_fmaf(qv.z, k4.z, t);
            d[it] = __builtin_fmaf(qv.w, k4.w, t);
        }
        bfly_stage<16, DPP_ROW_MIRROR>(d, (q & 8) != 0);
        bfly_stage<8, DPP_ROW_HALF_MIRROR>(d, (q & 4) != 0);
        bfly_stage<4, DPP_QUAD_REV>(d, (q & 2) != 0);
        bfly_stage<2, DPP_QUAD_SWAP>(d, (q & 1) != 0);
        if constexpr (PIPE) load_k(c + AD_NW);
        const float sc = p0 + 4 * q + grp <= pos ? d[0] * a.scale : -INFINITY;
        const float mc = rows_to_uniform_max(sc);  // chunk c holds position p0 <= pos: finite
        const float e = sc == -INFINITY ? 0.0f : exp_f(sc - mc);
        const float lc = rows_to_uniform_sum(e);
        es[wave][4 * q + grp] = e;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const float w = es[wave][it * 4 + grp];
            const float4 v4 = p0 + it * 4 + grp == pos ? vq : vv[it];
            o.x = __builtin_fmaf(w, v4.x, o.x);
            o.y = __builtin_fmaf(w, v4.y, o.y);
            o.z = __builtin_fmaf(w, v4.z, o.z);
            o.w = __builtin_fmaf(w, v4.w, o.w);
        }
        if constexpr (PIPE) load_v(c + AD_NW);
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
            o.x += __shfl_xor(o.x, off, 64);
            o.y += __shfl_xor(o.y, off, 64);
            o.z += __shfl_xor(o.z, off, 64);
            o.w += __shfl_xor(o.w, off, 64);
        }
        float *pc = cpart + (size_t)c * AD_PART;
        if (lane == 0) {
            pc[0] = mc;
            pc[1] = lc;
        }
        if (grp == 0) *(float4 *)&pc[4 + 4 * q] = o;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();
    // each chunk's weight e^{m_c - M} once (into the chunk's spare slot),
    // then every output dim sums over the chunks in order
    float M = cpart[0];
    for (int c = 1; c < nch; ++c) M = fmaxf(M, cpart[c * AD_PART]);
    for (int c = tid; c < nch; c += AD_NW * 64) cpart[c * AD_PART + 2] = exp_f(cpart[c * AD_PART] - M);
    __syncthreads();
    if (tid >= 64) return;
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < nch; ++c) {
        const float f = cpart[c * AD_PART + 2];
        L = __builtin_fmaf(cpart[c * AD_PART + 1], f, L);
        O = __builtin_fmaf(cpart[c * AD_PART + 4 + tid], f, O);
    }
    float y = O / L;
    const int col = h * 64 + tid;
    out[(size_t)b * ldo + col] = y;
    if (terms) {
        for (int t = 0; t < T; ++t) {
            const uint32_t hb = bf16_rne_bits(y);
            y = y - bf16_bits_to_f32(hb);
            terms[((size_t)t * B + b) * ldt + col] = (uint16_t)hb;
        }
    }
}

int launch_attention_decode(const DecodeArgs &a, int B, float *out, int ldo, uint16_t *terms,
                            int T, int ldt, hipStream_t st) {
    VMLM_GUARD(a.cap >= 1 && a.H >= 1 && B >= 1, "attention decode: empty shape");
    const size_t lds = (size_t)((a.cap + 63) / 64) * AD_PART * sizeof(float);
    VMLM_GUARD(lds <= 96 * 1024, "attention decode: cache capacity %d beyond %d positions",
               a.cap, 96 * 1024 / (AD_PART * 4) * 64);
    VMLM_GUARD((size_t)a.cap * 256 <= 0x7fffffffu, "attention decode: cache row range too large");
    VMLM_GUARD(!a.part || (a.ks >= 1 && a.ks <= PART_KS_MAX && a.wscale && a.ldp >= 3 * a.H * 64),
               "attention decode: partial q/k/v need ks, ldp and scales");
    const dim3 grid(a.H, B);
    if (a.H * B < 256) {
        if (a.part)
            attn_decode_kernel<8, true><<<grid, 8 * 64, lds, st>>>(a, out, ldo, terms, T, ldt, B);
        else
            attn_decode_kernel<8, false><<<grid, 8 * 64, lds, st>>>(a, out, ldo, terms, T, ldt, B);
    } else {
        if (a.part)
            attn_decode_kernel<4, true><<<grid, 4 * 64, lds, st>>>(a, out, ldo, terms, T, ldt, B);
        else
            attn_decode_kernel<4, false><<<grid, 4 * 64, lds, st>>>(a, out, ldo, terms, T, ldt, B);
    }
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

// k_b1.hip -- B1 sparse-connection forward (ops/src/b1_pure.rs, ops/src/kernels.rs).
//
// Activations are kept source-major, xt[d][t8] (transpose_t8_avx2's layout,
// ops/src/kernels.rs:1881): a wavefront's 64 lanes are 64 consecutive tokens
// of one neuron, so for a connection (i, j) every lane reads the same source
// row src[i][j] at consecutive addresses -- the gather becomes one coalesced
// 256-byte read, and w[i][j] / src[i][j] are wave-uniform scalar loads.
//
// Two accumulation contracts, both reproduced bit for bit:
//  * T8: ops/src/kernels.rs:2163-2188 -- j ascending, first term assigned,
//    multiply then add (the contract of b1_forward_t8).
//  * FOLD: ops/src/kernels.rs:1773-1804 -- 8 partial sums (lane l takes
//    j = l mod 8 over the full 8-blocks, each starting at +0.0), the fixed
//    fold ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)), then the ascending tail; the
//    small-k0 packed groupings of b1_forward_packed_avx2 (:2720-2800) for
//    k0 in {1, 4, 8} (the contract of b1_forward).
// An optional activation (VMLM_ACT_*) is applied to each output (tanh_f for
// the layer stack), bitwise like act_scalar.
#include <algorithm>
#include <vector>

#include "internal.hpp"

namespace vmlm {

enum { B1_T8 = 0, B1_FOLD = 1 };

__device__ __forceinline__ float b1_fold(const float *__restrict__ w,
                                         const uint32_t *__restrict__ src,
                                         const float *__restrict__ xt, size_t t8, int t,
                                         int k0) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    int j = 0;
    for (; j + 8 <= k0; j += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + w[j + l] * xt[(size_t)src[j + l] * t8 + t];
    }
    float s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
    for (; j < k0; ++j) s += w[j] * xt[(size_t)src[j] * t8 + t];
    return s;
}

__device__ __forceinline__ float hsum4(float v0, float v1, float v2, float v3) {
    return (v0 + v2) + (v1 + v3);
}

// grid: (ceil(n_tokens/64), n); block 64 (one neuron, 64 tokens)
__global__ __launch_bounds__(64) void b1_forward_kernel(const float *__restrict__ w,
                                                        const uint32_t *__restrict__ src,
                                                        int n, int k0,
                                                        const float *__restrict__ xt,
                                                        size_t t8, int n_tokens,
                                                        float *__restrict__ yt, int mode,
                                                        int act) {
    const int i = blockIdx.y;
    const int t = blockIdx.x * 64 + threadIdx.x;
    if (t >= n_tokens) return;
    const float *wi = w + (size_t)i * k0;
    const uint32_t *si = src + (size_t)i * k0;
    float y;
    if (k0 == 0) {
        y = 0.0f;
    } else if (mode == B1_T8) {
        float acc = wi[0] * xt[(size_t)si[0] * t8 + t];
        for (int j = 1; j < k0; ++j) acc = acc + wi[j] * xt[(size_t)si[j] * t8 + t];
        y = acc;
    } else {
        // b1_forward: packed rows for k0 in {1,2,4,8}. At k0 == 2 the
        // reference reduces a 128-bit half that holds two rows' products, so
        // rows 2r and 2r + 1 (r < n / 4 * 2) both get the sum of the pair's
        // four products, (p0+p2)+(p1+p3) and (p2+p0)+(p3+p1) for the odd row
        // (ops/src/kernels.rs:2748-2766).
        if (k0 == 1 && i < (n / 8) * 8) {
            y = wi[0] * xt[(size_t)si[0] * t8 + t];
        } else if (k0 == 2 && i < (n / 4) * 4) {
            const float *wp = w + (size_t)(i & ~1) * 2;
            const uint32_t *sp = src + (size_t)(i & ~1) * 2;
            float p[4];
#pragma unroll
            for (int l = 0; l < 4; ++l) p[l] = wp[l] * xt[(size_t)sp[l] * t8 + t];
            y = (i & 1) ? hsum4(p[2], p[3], p[0], p[1]) : hsum4(p[0], p[1], p[2], p[3]);
        } else if (k0 == 4 && i < (n / 2) * 2) {
            float p[4];
#pragma unroll
            for (int l = 0; l < 4; ++l) p[l] = wi[l] * xt[(size_t)si[l] * t8 + t];
            y = hsum4(p[0], p[1], p[2], p[3]);
        } else if (k0 == 8) {
            float p[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) p[l] = wi[l] * xt[(size_t)si[l] * t8 + t];
            y = hsum4(p[0] + p[4], p[1] + p[5], p[2] + p[6], p[3] + p[7]);
        } else {
            y = b1_fold(wi, si, xt, t8, t, k0);
        }
    }
    if (act >= 0) y = act_scalar(y, act);
    yt[(size_t)i * t8 + t] = y;
}

int launch_b1_forward(const float *w, const uint32_t *src, int n, int k0, const float *xt,
                      size_t t8, int n_tokens, float *yt, int mode, int act, hipStream_t st) {
    if (n == 0 || n_tokens == 0) return VMLM_OK;
    dim3 grid(cdiv(n_tokens, 64), n);
    b1_forward_kernel<<<grid, 64, 0, st>>>(w, src, n, k0, xt, t8, n_tokens, yt, mode, act);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- T8 layers
// A T8 layer runs in two kernels.
//
// b1_plan_kernel rewrites a layer's connections (src[n][k0], w[n][k0]) into a
// plan: for every group of four connections g and neuron i, a uint4 of LDS
// byte offsets (the staged row of each source, index clamped to d - 1) at
// off[g][i] and the four weights at wp[g][i]. Connections past k0 in the last
// group point at an all-zero row with weight -0.0f: p = -0.0f * +0.0f = -0.0f
// and acc + (-0.0f) == acc bit for bit for every acc (signed zeros, infinities
// and NaNs included), so padded steps leave the T8 sum unchanged.
//
// b1_t8_layer_kernel: a workgroup owns one 16-token block and 32 * NW
// neurons. The 16-token slice of every source row is staged once into LDS
// (B1_ROW bytes per row: 64 bytes of data and 16 of padding, so row starts
// fall on all 16 bank groups), with rows permuted inside aligned groups of 16
// by b1_row_slot so that block-aligned topologies (sources 8b .. 8b + 7) do
// not map every lane of a step to the same banks. Lane l of a wave computes
// neuron (l & 31) for tokens 8 h .. 8 h + 7 of the block, h = l >> 5: each
// step is two 16-byte LDS reads, eight multiplies and eight adds, in the T8
// order (j ascending, first product assigned, no FMA). The two lanes of a
// neuron each load half of its plan and exchange the halves across the wave
// halves (v_permlane32_swap).
//
// Activations are addressed by strides: element (row s, token t) lives at
// (t / 16) * bs + s * rs + t % 16. The reference layout xt[s][t8] is
// bs = 16, rs = t8; the layer stack keeps its intermediate activations in
// 16-token blocks, bs = 16 d, rs = 16, so each block is contiguous.
constexpr int B1_ROW = 80;
constexpr int B1_KMAX = 32;          // connections per neuron on the planned path
constexpr int B1_GMAX = B1_KMAX / 4;
constexpr int B1_DMAX = 2032;        // (d16 + 1) * B1_ROW bytes of LDS <= 160 KiB
constexpr int B1_NW = 12;            // waves per workgroup

__host__ __device__ inline uint32_t b1_row_slot(uint32_t r) {
    return r ^ (((r >> 4) ^ (r >> 8)) & 15u);
}

bool b1_plan_ok(int n, int k0, int d) {
    return n > 0 && k0 >= 1 && k0 <= B1_KMAX && d >= 1 && d <= B1_DMAX;
}
size_t b1_plan_bytes(int n, int k0) { return (size_t)((k0 + 3) / 4) * n * 32; }

// grid: (ceil(n / 64), jobs). A workgroup copies the connection rows of 64
// neurons into LDS with coalesced loads, then writes their plan entries
// (group-major, so consecutive threads write consecutive neurons).
__global__ __launch_bounds__(256) void b1_plan_kernel(B1PlanJobs jobs, int n, int d, int row_bytes,
                                                      int g_pad) {
    __shared__ uint32_t ss[64][B1_KMAX + 1];
    __shared__ float sw[64][B1_KMAX + 1];
    const B1PlanJob &jb = jobs.job[blockIdx.y];
    const int k0 = jb.k0, G = g_pad > 0 ? g_pad : (k0 + 3) / 4;
    const int i0 = (int)blockIdx.x * 64, rows = n - i0 < 64 ? n - i0 : 64;
    {
        // thread (tid >> 5, tid & 31) takes rows tid >> 5, + 8, ..., + 56 at
        // column tid & 31; all 16 loads are issued before any store (rows and
        // columns clamped, so the loads do not branch)
        const int j = threadIdx.x & 31, jc = j < k0 ? j : k0 - 1;
        uint32_t vs[8];
        float vw[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = min((int)(threadIdx.x >> 5) + 8 * k, rows - 1);
            vs[k] = jb.src[(size_t)(i0 + r) * k0 + jc];
            vw[k] = jb.w[(size_t)(i0 + r) * k0 + jc];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = min((int)(threadIdx.x >> 5) + 8 * k, rows - 1);
            ss[r][jc] = vs[k];
            sw[r][jc] = vw[k];
        }
    }
    __syncthreads();
    const uint32_t zero_row = jb.base + (uint32_t)((d + 15) & ~15) * (uint32_t)row_bytes;
    uint4 *off = (uint4 *)jb.plan;
    float4 *wp = (float4 *)(off + (size_t)G * n);
    for (int q = threadIdx.x; q < 64 * G; q += 256) {
        const int r = q & 63, g = q >> 6;
        if (r >= rows) continue;
        uint32_t o[4];
        float w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 4 * g + e;
            if (j < k0) {
                const uint32_t s = ss[r][j] < (uint32_t)d ? ss[r][j] : (uint32_t)(d - 1);
                o[e] = jb.base + b1_row_slot(s) * (uint32_t)row_bytes;
                w[e] = sw[r][j];
            } else {
                o[e] = zero_row;
                w[e] = -0.0f;
            }
        }
        off[(size_t)g * n + i0 + r] = make_uint4(o[0], o[1], o[2], o[3]);
        wp[(size_t)g * n + i0 + r] = make_float4(w[0], w[1], w[2], w[3]);
    }
}

int launch_b1_plan(const B1PlanJobs &jobs, int njobs, int n, int d, hipStream_t st) {
    if (njobs <= 0 || n <= 0) return VMLM_OK;
    for (int b = 0; b < njobs; ++b)
        if (!b1_plan_ok(n, jobs.job[b].k0, d)) return fail(VMLM_ERR_DEVICE, "b1 plan: bad shape");
    b1_plan_kernel<<<dim3(cdiv((size_t)n, 64), njobs), 256, 0, st>>>(jobs, n, d, B1_ROW, 0);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

__device__ __forceinline__ uint32_t u4c(const uint4 &v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}
__device__ __forceinline__ float f4c(const float4 &v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}
// value of the same register in lane l ^ 32
__device__ __forceinline__ uint32_t swap_halves(uint32_t v, bool upper) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return upper ? r[0] : r[1];
}

template <int G>
__global__ __launch_bounds__(64 * B1_NW) void b1_t8_layer_kernel(
    const uint4 *__restrict__ off, const float4 *__restrict__ wp, int n, int d,
    const float *__restrict__ x, size_t xbs, size_t xrs, int n_tokens, float *__restrict__ y,
    size_t ybs, size_t yrs, int act) {
    extern __shared__ float4 b1_lds[];
    char *lds = (char *)b1_lds;
    constexpr int GH = (G + 1) / 2;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5;
    const int i = (int)blockIdx.y * (int)(blockDim.x / 2) + (tid >> 6) * 32 + (lane & 31);
    const int ic = i < n ? i : n - 1;
    // this lane's half of the plan: groups h * GH .. h * GH + GH - 1 (clamped)
    uint4 po[GH];
    float4 pw[GH];
#pragma unroll
    for (int k = 0; k < GH; ++k) {
        const int g = h * GH + k < G ? h * GH + k : G - 1;
        po[k] = off[(size_t)g * n + ic];
        pw[k] = wp[(size_t)g * n + ic];
    }
    // stage the block: 16-byte pieces (row, quarter), all loads before any store
    const float *xb = x + (size_t)blockIdx.x * xbs;
    const int npc = d * 4, nthr = (int)blockDim.x;
    for (int pc0 = 0; pc0 < npc; pc0 += nthr * 8) {
        float4 v[8];
        int pcs[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int pc = pc0 + tid + k * nthr;
            pcs[k] = pc < npc ? pc : npc - 1;
            v[k] = *(const float4 *)(xb + (size_t)(pcs[k] >> 2) * xrs + (pcs[k] & 3) * 4);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            *(float4 *)(lds + b1_row_slot((uint32_t)(pcs[k] >> 2)) * B1_ROW + (pcs[k] & 3) * 16) =
                v[k];
    }
    if (tid < 4)
        *(float4 *)(lds + (size_t)((d + 15) & ~15) * B1_ROW + tid * 16) =
            make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // the full plan: groups below GH come from the lower half-wave's loads
    uint4 o[G];
    float4 w[G];
#pragma unroll
    for (int k = 0; k < GH; ++k) {
        uint4 so;
        float4 sw;
        so.x = swap_halves(po[k].x, h);
        so.y = swap_halves(po[k].y, h);
        so.z = swap_halves(po[k].z, h);
        so.w = swap_halves(po[k].w, h);
        sw.x = __uint_as_float(swap_halves(__float_as_uint(pw[k].x), h));
        sw.y = __uint_as_float(swap_halves(__float_as_uint(pw[k].y), h));
        sw.z = __uint_as_float(swap_halves(__float_as_uint(pw[k].z), h));
        sw.w = __uint_as_float(swap_halves(__float_as_uint(pw[k].w), h));
        o[k] = h ? so : po[k];
        w[k] = h ? sw : pw[k];
        if (GH + k < G) {
            o[GH + k] = h ? po[k] : so;
            w[GH + k] = h ? pw[k] : sw;
        }
    }
    __syncthreads();
    const char *lh = lds + 32 * h;
    float acc[8];
    float4 ca, cb, na, nb, ma, mb;
    auto get = [&](int j, float4 &a, float4 &b) {
        const uint32_t oo = u4c(o[j / 4], j % 4);
        a = *(const float4 *)(lh + oo);
        b = *(const float4 *)(lh + oo + 16);
    };
    // two steps of LDS reads in flight ahead of the one being summed
    get(0, ca, cb);
    get(1, na, nb);
#pragma unroll
    for (int j = 0; j < 4 * G; ++j) {
        if (j + 2 < 4 * G) get(j + 2, ma, mb);
        const float wj = f4c(w[j / 4], j % 4);
        const float xv[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float p = wj * xv[t];
            acc[t] = j == 0 ? p : acc[t] + p;
        }
        ca = na;
        cb = nb;
        na = ma;
        nb = mb;
    }
    if (act >= 0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] = act_scalar(acc[t], act);
    }
    if (i >= n) return;
    const int t0 = (int)blockIdx.x * 16 + 8 * h;
    float *yo = y + (size_t)blockIdx.x * ybs + (size_t)i * yrs + 8 * h;
    if (t0 + 8 <= n_tokens) {
        ((float4 *)yo)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        ((float4 *)yo)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t)
            if (t0 + t < n_tokens) yo[t] = acc[t];
    }
}

template <int G>
static int launch_layer_g(const void *plan, int n, int d, const float *x, size_t xbs, size_t xrs,
                          int n_tokens, float *y, size_t ybs, size_t yrs, int act, hipStream_t st) {
    const size_t lds = (size_t)(((d + 15) & ~15) + 1) * B1_ROW;
    static bool attr = false;
    if (!attr) {
        VMLM_HIP_CHECK(hipFuncSetAttribute((const void *)b1_t8_layer_kernel<G>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(((B1_DMAX + 15) / 16 * 16 + 1) * B1_ROW)));
        attr = true;
    }
    const uint4 *off = (const uint4 *)plan;
    const float4 *wp = (const float4 *)(off + (size_t)G * n);
    const int per = 32 * B1_NW;
    dim3 grid(cdiv((size_t)n_tokens, 16), cdiv((size_t)n, (size_t)per));
    b1_t8_layer_kernel<G><<<grid, 64 * B1_NW, lds, st>>>(off, wp, n, d, x, xbs, xrs, n_tokens, y,
                                                         ybs, yrs, act);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_b1_t8_plan_layer(const void *plan, int n, int k0, int d, const float *x, size_t xbs,
                            size_t xrs, int n_tokens, float *y, size_t ybs, size_t yrs, int act,
                            hipStream_t st) {
    if (n == 0 || n_tokens == 0) return VMLM_OK;
    if (!b1_plan_ok(n, k0, d)) return fail(VMLM_ERR_DEVICE, "b1 layer: bad shape");
    switch ((k0 + 3) / 4) {
    case 1: return launch_layer_g<1>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 2: return launch_layer_g<2>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 3: return launch_layer_g<3>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 4: return launch_layer_g<4>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 5: return launch_layer_g<5>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 6: return launch_layer_g<6>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    case 7: return launch_layer_g<7>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    default: return launch_layer_g<8>(plan, n, d, x, xbs, xrs, n_tokens, y, ybs, yrs, act, st);
    }
}

// Source-major copy of x[T][d]: element (s, t) at (t / 16) * bs + s * rs + t % 16
// for t < tp (zero for T <= t < tp), 32x32 LDS tiles.
__global__ __launch_bounds__(256) void transpose_t8_kernel(const float *__restrict__ x, int T,
                                                           int d, float *__restrict__ xt,
                                                           size_t tp, size_t bs, size_t rs) {
    __shared__ float tile[32][33];
    const int t0 = blockIdx.x * 32, s0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        int t = t0 + r, s = s0 + tx;
        tile[r][tx] = (t < T && s < d) ? x[(size_t)t * d + s] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int s = s0 + r, t = t0 + tx;
        if (s < d && (size_t)t < tp) xt[(size_t)(t >> 4) * bs + (size_t)s * rs + (t & 15)] = tile[tx][r];
    }
}

int launch_transpose_t8(const float *x, size_t T, size_t d, float *xt, size_t t8,
                        hipStream_t st) {
    if (d == 0 || t8 == 0) return VMLM_OK;
    dim3 grid(cdiv(t8, 32), cdiv(d, 32));
    transpose_t8_kernel<<<grid, 256, 0, st>>>(x, (int)T, (int)d, xt, t8, 16, t8);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ------------------------------------------------------------- whole stack
// b1_stack_kernel runs every layer of a stack (n = d in all layers) for 4
// tokens per workgroup. Layer l + 1 of a token needs only layer l of the same
// token, so the activations never leave LDS: two buffers of d rows x 16 bytes
// (4 tokens), the layer input and output, swap after each layer. Lane = neuron
// (passes of 64 * B1_SNW neurons); a step is one 16-byte LDS read at the
// planned offset, four multiplies and four adds in the T8 order. Plans of all
// layers are padded to the same number of groups with no-op steps; the plan
// of the next pass is loaded while the current one is summed. x is read and y
// written in [T][d] directly.
constexpr int B1_SNW = 12;                  // waves per workgroup
constexpr int B1_SROW = 16;                 // LDS bytes per row (4 tokens)
constexpr int B1_SDMAX = 5104;              // 2 * (d16 + 1) * 16 bytes <= 160 KiB
constexpr int B1_SPD = 8;                   // LDS reads in flight per lane
constexpr bool B1_SPF = false;              // next pass's plan loaded during the current one

template <int G>
__global__ __launch_bounds__(64 * B1_SNW) void b1_stack_kernel(const char *__restrict__ plan,
                                                               size_t plan_stride, int n_layers,
                                                               int d, const float *__restrict__ x,
                                                               float *__restrict__ y, int T,
                                                               int act) {
    extern __shared__ float4 b1s_lds[];
    const int tid = threadIdx.x, nthr = (int)blockDim.x;
    const int d16 = (d + 15) & ~15;
    // buffer k at lds + k * bufb (addressed from the shared base, so every
    // access stays an LDS access)
    char *lds = (char *)b1s_lds;
    const int bufb = (d16 + 1) * B1_SROW;
    const int tok0 = (int)blockIdx.x * 4;
    // layer input: x[tok0 + t][s] -> row slot(s), column t (tokens past T are
    // 0); every load of a sweep (2 sources x 4 tokens per thread) is issued
    // before its stores, source indices clamped so that nothing branches
    for (int s0 = 0; s0 < d; s0 += 2 * nthr) {
        float v[2][4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int s = min(s0 + k * nthr + tid, d - 1);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                v[k][t] = x[(size_t)min(tok0 + t, T - 1) * d + s];
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int s = min(s0 + k * nthr + tid, d - 1);
            *(float4 *)(lds + b1_row_slot((uint32_t)s) * B1_SROW) =
                make_float4(v[k][0], tok0 + 1 < T ? v[k][1] : 0.0f, tok0 + 2 < T ? v[k][2] : 0.0f,
                            tok0 + 3 < T ? v[k][3] : 0.0f);
        }
    }
    if (tid < 2)
        *(float4 *)(lds + tid * bufb + d16 * B1_SROW) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int npass = (d + nthr - 1) / nthr, units = n_layers * npass;
    auto load = [&](int u, uint4 (&o)[G], float4 (&w)[G]) {
        const int l = u / npass, i = (u - l * npass) * nthr + tid, ic = i < d ? i : d - 1;
        const uint4 *off = (const uint4 *)(plan + (size_t)l * plan_stride);
        const float4 *wp = (const float4 *)(off + (size_t)G * d);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            o[g] = off[(size_t)g * d + ic];
            w[g] = wp[(size_t)g * d + ic];
        }
    };
    uint4 o[G], on[G];
    float4 w[G], wn[G];
    if (B1_SPF) load(0, o, w);
    __syncthreads();
    for (int u = 0; u < units; ++u) {
        const int l = u / npass, pass = u - l * npass;
        if (B1_SPF)
            load(u + 1 < units ? u + 1 : u, on, wn);  // unconditional: no branch around the loads
        else
            load(u, o, w);
        const char *in = lds;  // the plan's offsets include buffer l & 1
        float acc[4];
        // ring of LDS reads B1_SPD steps ahead of the step being summed
        float4 ring[B1_SPD];
#pragma unroll
        for (int j = 0; j < B1_SPD && j < 4 * G; ++j)
            ring[j] = *(const float4 *)(in + u4c(o[j / 4], j % 4));
#pragma unroll
        for (int j = 0; j < 4 * G; ++j) {
            const float4 c = ring[j % B1_SPD];
            if (j + B1_SPD < 4 * G)
                ring[j % B1_SPD] = *(const float4 *)(in + u4c(o[(j + B1_SPD) / 4], (j + B1_SPD) % 4));
            const float wj = f4c(w[j / 4], j % 4);
            const float xv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float p = wj * xv[t];
                acc[t] = j == 0 ? p : acc[t] + p;
            }
        }
        if (act >= 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = act_scalar(acc[t], act);
        }
        const int i = pass * nthr + tid;
        if (i < d) {
            if (l + 1 < n_layers) {
                *(float4 *)(lds + ((l + 1) & 1) * bufb + b1_row_slot((uint32_t)i) * B1_SROW) =
                    make_float4(acc[0], acc[1], acc[2], acc[3]);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (tok0 + t < T) y[(size_t)(tok0 + t) * d + i] = acc[t];
            }
        }
        if (pass == npass - 1) __syncthreads();  // layer l complete before l + 1 reads it
        if (B1_SPF) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                o[g] = on[g];
                w[g] = wn[g];
            }
        }
    }
}

bool b1_stack_ok(int d, const int *k0, int n_layers) {
    if (d < 1 || d > B1_SDMAX || n_layers < 1) return false;
    for (int l = 0; l < n_layers; ++l)
        if (k0[l] < 1 || k0[l] > B1_KMAX) return false;
    return true;
}
static int stack_groups(const int *k0, int n_layers) {
    int g = 1;
    for (int l = 0; l < n_layers; ++l) g = std::max(g, (k0[l] + 3) / 4);
    return g;
}
static size_t stack_plan_stride(int d, int G) { return ((size_t)G * d * 32 + 255) / 256 * 256; }
size_t b1_stack_plan_bytes(int d, const int *k0, int n_layers) {
    return stack_plan_stride(d, stack_groups(k0, n_layers)) * (size_t)n_layers;
}

template <int G>
static int launch_stack_g(const char *plan, size_t stride, int n_layers, int d, const float *x,
                          float *y, int T, int act, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        VMLM_HIP_CHECK(hipFuncSetAttribute((const void *)b1_stack_kernel<G>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           2 * ((B1_SDMAX + 15) / 16 * 16 + 1) * B1_SROW));
        attr = true;
    }
    const size_t lds = 2 * (size_t)(((d + 15) & ~15) + 1) * B1_SROW;
    b1_stack_kernel<G><<<cdiv((size_t)T, 4), 64 * B1_SNW, lds, st>>>(plan, stride, n_layers, d, x,
                                                                      y, T, act);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int launch_b1_stack(const B1PlanJob *layers, int n_layers, int d, const float *x, float *y, int T,
                    int act, void *plan, hipStream_t st) {
    if (T == 0) return VMLM_OK;
    int rc = launch_b1_stack_plan(layers, n_layers, d, plan, st);
    if (rc) return rc;
    std::vector<int> k0(n_layers);
    for (int l = 0; l < n_layers; ++l) k0[l] = layers[l].k0;
    return launch_b1_stack_run(plan, k0.data(), n_layers, d, x, y, T, act, st);
}

// The plan of every layer (connection words in the stack kernel's layout),
// a function of the topology and weights only.
int launch_b1_stack_plan(const B1PlanJob *layers, int n_layers, int d, void *plan,
                         hipStream_t st) {
    std::vector<int> k0(n_layers);
    for (int l = 0; l < n_layers; ++l) k0[l] = layers[l].k0;
    if (!b1_stack_ok(d, k0.data(), n_layers)) return fail(VMLM_ERR_DEVICE, "b1 stack: bad shape");
    const int G = stack_groups(k0.data(), n_layers);
    const size_t stride = stack_plan_stride(d, G);
    for (int l0 = 0; l0 < n_layers; l0 += B1_PLAN_JOBS) {
        B1PlanJobs jobs{};
        const int nj = std::min(B1_PLAN_JOBS, n_layers - l0);
        // layer l reads LDS buffer l & 1: its offsets carry that buffer's base
        const uint32_t bufb = (uint32_t)(((d + 15) & ~15) + 1) * B1_SROW;
        for (int k = 0; k < nj; ++k) {
            jobs.job[k] = layers[l0 + k];
            jobs.job[k].plan = (char *)plan + (size_t)(l0 + k) * stride;
            jobs.job[k].base = ((l0 + k) & 1) * bufb;
        }
        b1_plan_kernel<<<dim3(cdiv((size_t)d, 64), nj), 256, 0, st>>>(jobs, d, d, B1_SROW, G);
        VMLM_HIP_CHECK(hipGetLastError());
    }
    return VMLM_OK;
}

// The stack kernel over a prepared plan (one launch, no allocation).
int launch_b1_stack_run(const void *plan, const int *k0, int n_layers, int d, const float *x,
                        float *y, int T, int act, hipStream_t st) {
    if (T == 0) return VMLM_OK;
    if (!b1_stack_ok(d, k0, n_layers)) return fail(VMLM_ERR_DEVICE, "b1 stack: bad shape");
    const int G = stack_groups(k0, n_layers);
    const size_t stride = stack_plan_stride(d, G);
    const char *p = (const char *)plan;
    switch (G) {
    case 1: return launch_stack_g<1>(p, stride, n_layers, d, x, y, T, act, st);
    case 2: return launch_stack_g<2>(p, stride, n_layers, d, x, y, T, act, st);
    case 3: return launch_stack_g<3>(p, stride, n_layers, d, x, y, T, act, st);
    case 4: return launch_stack_g<4>(p, stride, n_layers, d, x, y, T, act, st);
    case 5: return launch_stack_g<5>(p, stride, n_layers, d, x, y, T, act, st);
    case 6: return launch_stack_g<6>(p, stride, n_layers, d, x, y, T, act, st);
    case 7: return launch_stack_g<7>(p, stride, n_layers, d, x, y, T, act, st);
    default: return launch_stack_g<8>(p, stride, n_layers, d, x, y, T, act, st);
    }
}

// out[i*os + s] = a(s, i), s < rows, i < cols (ops/src/kernels.rs:3307), where
// a(s, i) is at (i / 16) * bs + s * rs + i % 16 (the reference layout:
// bs = 16, rs = in_stride).
__global__ __launch_bounds__(256) void transpose_back_kernel(const float *__restrict__ a,
                                                             int rows, int cols,
                                                             float *__restrict__ out,
                                                             size_t os, size_t bs, size_t rs) {
    __shared__ float tile[32][33];
    const int i0 = blockIdx.x * 32, s0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        int s = s0 + r, i = i0 + tx;
        tile[r][tx] = (s < rows && i < cols) ? a[(size_t)(i >> 4) * bs + (size_t)s * rs + (i & 15)]
                                             : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int i = i0 + r, s = s0 + tx;
        if (i < cols && s < rows) out[(size_t)i * os + s] = tile[tx][r];
    }
}

int launch_transpose_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                          size_t in_stride, hipStream_t st) {
    if (rows == 0 || cols == 0) return VMLM_OK;
    dim3 grid(cdiv(cols, 32), cdiv(rows, 32));
    transpose_back_kernel<<<grid, 256, 0, st>>>(a, (int)rows, (int)cols, out, os, 16, in_stride);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

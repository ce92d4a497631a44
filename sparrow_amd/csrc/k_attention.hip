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
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float *__restrict__ A,
                                                       const float *__restrict__ B,
                                                       float *__restrict__ C, int m, int n,
                                                       int k, int acc, int nt) {
    __shared__ float As[16][68];
    __shared__ float Bs[16][68];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
    float c[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[i][j] = 0.0f;
    for (int k0 = 0; k0 < k; k0 += 16) {
        for (int e = threadIdx.x; e < 1024; e += 256) {
            int r = e >> 4, kk = e & 15;
            int gr = row0 + r, gk = k0 + kk;
            As[kk][r] = (gr < m && gk < k) ? A[(size_t)gr * k + gk] : 0.0f;
            if (nt) {
                int gc = col0 + r;
                Bs[kk][r] = (gc < n && gk < k) ? B[(size_t)gc * k + gk] : 0.0f;
            } else {
                int kk2 = e >> 6, cc = e & 63;
                int gk2 = k0 + kk2, gc = col0 + cc;
                Bs[kk2][cc] = (gc < n && gk2 < k) ? B[(size_t)gk2 * n + gc] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[i][j] = __builtin_fmaf(a[i], b[j], c[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int gr = row0 + ty * 4 + i;
        if (gr >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int gc = col0 + tx * 4 + j;
            if (gc >= n) continue;
            float *o = C + (size_t)gr * n + gc;
            *o = acc ? *o + c[i][j] : c[i][j];
        }
    }
}

int launch_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                    bool acc, bool b_is_nt, hipStream_t st) {
    if (m == 0 || n == 0) return VMLM_OK;
    if (k == 0) {
        if (!acc) VMLM_HIP_CHECK(hipMemsetAsync(c, 0, m * n * sizeof(float), st));
        return VMLM_OK;
    }
    dim3 grid(cdiv(n, 64), cdiv(m, 64));
    gemm_f32_kernel<<<grid, 256, 0, st>>>(a, b, c, (int)m, (int)n, (int)k, acc ? 1 : 0,
                                          b_is_nt ? 1 : 0);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// ---------------------------------------------------------------- prefill
// Q, K already rotated; all [S][ld] with head h at columns h*64.
constexpr int AT_B = 64;  // query / key block

__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, int S, int ld, int ldo, float scale, int causal) {
    __shared__ float Qs[64][AT_B + 1];   // [d][q]
    __shared__ float KPs[AT_B][AT_B + 1];  // K as [d][key], then P as [q][key]
    __shared__ float Vs[AT_B][64 + 4];   // [key][d]
    const int h = blockIdx.y, qb = blockIdx.x;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int q0 = qb * AT_B;
    const float *Qh = Q + h * 64, *Kh = K + h * 64, *Vh = V + h * 64;

    for (int e = threadIdx.x; e < AT_B * 64; e += 256) {
        int q = e >> 6, d = e & 63;
        Qs[d][q] = (q0 + q < S) ? Qh[(size_t)(q0 + q) * ld + d] : 0.0f;
    }
    float m[4], l[4], o[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[i][j] = 0.0f;
    }
    const int nkb = causal ? qb + 1 : (S + AT_B - 1) / AT_B;
    for (int kb = 0; kb < nkb; ++kb) {
        const int k0 = kb * AT_B;
        __syncthreads();
        for (int e = threadIdx.x; e < AT_B * 64; e += 256) {
            int kk = e >> 6, d = e & 63;
            bool in = k0 + kk < S;
            KPs[d][kk] = in ? Kh[(size_t)(k0 + kk) * ld + d] : 0.0f;
            Vs[kk][d] = in ? Vh[(size_t)(k0 + kk) * ld + d] : 0.0f;
        }
        __syncthreads();
        float s[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) s[i][j] = 0.0f;
        for (int d = 0; d < 64; ++d) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = Qs[d][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = KPs[d][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[i][j] = __builtin_fmaf(a[i], b[j], s[i][j]);
        }
        float pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = q0 + ty * 4 + i;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int kk = k0 + tx * 4 + j;
                bool valid = kk < S && (!causal || kk <= q);
                s[i][j] = valid ? s[i][j] * scale : -INFINITY;
                mx = fmaxf(mx, s[i][j]);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            pm[i] = fmaxf(m[i], mx);
        }
        __syncthreads();  // K no longer needed; reuse its LDS for P
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float corr = (m[i] == -INFINITY) ? 0.0f : exp_f(m[i] - pm[i]);
            float rs = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float p = (s[i][j] == -INFINITY) ? 0.0f : exp_f(s[i][j] - pm[i]);
                KPs[ty * 4 + i][tx * 4 + j] = p;
                rs += p;
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) rs += __shfl_xor(rs, off, 64);
            l[i] = l[i] * corr + rs;
            m[i] = pm[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) o[i][j] *= corr;
        }
        __syncthreads();
        for (int kk = 0; kk < AT_B; ++kk) {
            float p[4], v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = KPs[ty * 4 + i][kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = Vs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) o[i][j] = __builtin_fmaf(p[i], v[j], o[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = q0 + ty * 4 + i;
        if (q >= S) continue;
        const float inv = 1.0f / l[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) O[(size_t)q * ldo + h * 64 + tx * 4 + j] = o[i][j] * inv;
    }
}

int launch_attention_prefill(const float *qrot, const float *krot, const float *v, float *out,
                             int S, int H, int ld, int ldo, float scale, bool causal,
                             hipStream_t st) {
    dim3 grid(cdiv(S, AT_B), H);
    attn_prefill_kernel<<<grid, 256, 0, st>>>(qrot, krot, v, out, S, ld, ldo, scale,
                                              causal ? 1 : 0);
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

    for (int c = wave; c < nch; c += AD_NW) {
        if (c != wave) load_chunk(c);
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
    if (tid >= 64) return;
    float M = cpart[0];
    for (int c = 1; c < nch; ++c) M = fmaxf(M, cpart[c * AD_PART]);
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < nch; ++c) {
        const float f = exp_f(cpart[c * AD_PART] - M);
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

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
// One wavefront per (sequence b, head h, split s of 64 positions). Lane =
// (group grp = lane/16, dim quad q = lane%16): a K or V row (64 f32 = 256 B)
// is read by the 16 lanes of a group as float4s, four rows per load
// instruction; the 16 row loads of the split are issued before use.
__global__ __launch_bounds__(64) void attn_decode_split_kernel(DecodeArgs a) {
    __shared__ float qs[64], kn[64], vn[64];
    __shared__ float es[64];
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x, grp = lane >> 4, q = lane & 15;
    const int pos = a.posp ? *a.posp : a.pos;
    const int live = pos + 1;
    float *part = a.part + (((size_t)b * a.H + h) * a.NS + s) * 66;
    const int p0 = s * 64;
    if (p0 >= live) {
        if (lane == 0) {
            part[0] = -INFINITY;
            part[1] = 0.0f;
        }
        return;
    }
    const float *kc = a.kc + ((size_t)b * a.H + h) * a.cap * 64;
    const float *vc = a.vc + ((size_t)b * a.H + h) * a.cap * 64;
    // K rows of this split (positions < pos come from the cache)
    float4 kv[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const int p = p0 + it * 4 + grp;
        kv[it] = p < pos ? *(const float4 *)(kc + (size_t)p * 64 + 4 * q)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float *qr = a.q + (size_t)b * a.ldq + h * 64;
    const float *kr = a.k_new + (size_t)b * a.ldq + h * 64;
    const float *vr = a.v_new + (size_t)b * a.ldq + h * 64;
    const float fpos = (float)pos;
    if (lane < 32) {
        float y1, y2;
        rope_pair(qr[lane], qr[lane + 32], fpos, lane, a.step, &y1, &y2);
        qs[lane] = y1;
        qs[lane + 32] = y2;
        rope_pair(kr[lane], kr[lane + 32], fpos, lane, a.step, &y1, &y2);
        kn[lane] = y1;
        kn[lane + 32] = y2;
    }
    vn[lane] = vr[lane];
    __syncthreads();
    if (pos >= p0 && pos < p0 + 64) {  // this split owns the new position
        float *kw = a.kc + ((size_t)b * a.H + h) * a.cap * 64;
        float *vw = a.vc + ((size_t)b * a.H + h) * a.cap * 64;
        kw[(size_t)pos * 64 + lane] = kn[lane];
        vw[(size_t)pos * 64 + lane] = vn[lane];
    }
    // V rows, issued before the scores are reduced
    float4 vv[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const int p = p0 + it * 4 + grp;
        vv[it] = p < pos ? *(const float4 *)(vc + (size_t)p * 64 + 4 * q)
                         : (p == pos ? make_float4(vn[4 * q], vn[4 * q + 1], vn[4 * q + 2],
                                                   vn[4 * q + 3])
                                     : make_float4(0.f, 0.f, 0.f, 0.f));
    }
    const float4 qv = make_float4(qs[4 * q], qs[4 * q + 1], qs[4 * q + 2], qs[4 * q + 3]);
    const float4 kq = make_float4(kn[4 * q], kn[4 * q + 1], kn[4 * q + 2], kn[4 * q + 3]);
    float myscore = -INFINITY;
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const int p = p0 + it * 4 + grp;
        const float4 k4 = p == pos ? kq : kv[it];
        float d = qv.x * k4.x;
        d = __builtin_fmaf(qv.y, k4.y, d);
        d = __builtin_fmaf(qv.z, k4.z, d);
        d = __builtin_fmaf(qv.w, k4.w, d);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) d += __shfl_xor(d, o, 64);
        if (q == it) myscore = p <= pos ? d * a.scale : -INFINITY;  // lane (grp, it) keeps row it*4+grp
    }
    // lane (grp, q) now holds the score of position p0 + q*4 + grp
    const float mx = wave_max(myscore);
    const float e = (myscore == -INFINITY) ? 0.0f : exp_f(myscore - mx);
    const float l = wave_sum(e);
    es[q * 4 + grp] = e;
    __syncthreads();
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const float w = es[it * 4 + grp];
        o.x = __builtin_fmaf(w, vv[it].x, o.x);
        o.y = __builtin_fmaf(w, vv[it].y, o.y);
        o.z = __builtin_fmaf(w, vv[it].z, o.z);
        o.w = __builtin_fmaf(w, vv[it].w, o.w);
    }
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        o.x += __shfl_xor(o.x, off, 64);
        o.y += __shfl_xor(o.y, off, 64);
        o.z += __shfl_xor(o.z, off, 64);
        o.w += __shfl_xor(o.w, off, 64);
    }
    if (lane == 0) {
        part[0] = mx;
        part[1] = l;
    }
    if (grp == 0) {
        part[2 + 4 * q + 0] = o.x;
        part[2 + 4 * q + 1] = o.y;
        part[2 + 4 * q + 2] = o.z;
        part[2 + 4 * q + 3] = o.w;
    }
}

// Merge the splits of (b, h): out = sum_s o_s e^{m_s-M} / sum_s l_s e^{m_s-M};
// also writes the bf16 terms of the output row (operand of the o-projection).
// The partials of up to 16 splits are loaded in one batch.
__global__ __launch_bounds__(64) void attn_decode_combine_kernel(
    const float *__restrict__ part, int NS, int H, float *__restrict__ out, int ldo,
    uint16_t *__restrict__ terms, int T, int ldt, int B) {
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const float *pb = part + ((size_t)b * H + h) * NS * 66;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < NS; s0 += 16) {
        float ms[16], ls[16], os[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int s = s0 + i;
            ms[i] = s < NS ? pb[s * 66] : -INFINITY;
            ls[i] = s < NS ? pb[s * 66 + 1] : 0.0f;
            os[i] = s < NS ? pb[s * 66 + 2 + lane] : 0.0f;
        }
        float Mn = M;
#pragma unroll
        for (int i = 0; i < 16; ++i) Mn = fmaxf(Mn, ms[i]);
        if (Mn == -INFINITY) continue;
        const float c = (M == -INFINITY) ? 0.0f : exp_f(M - Mn);
        L *= c;
        O *= c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (ms[i] == -INFINITY) continue;
            const float w = exp_f(ms[i] - Mn);
            L = __builtin_fmaf(ls[i], w, L);
            O = __builtin_fmaf(os[i], w, O);
        }
        M = Mn;
    }
    float y = O / L;
    const int col = h * 64 + lane;
    out[(size_t)b * ldo + col] = y;
    if (terms) {
        for (int t = 0; t < T; ++t) {
            uint32_t hb = bf16_rne_bits(y);
            y = y - bf16_bits_to_f32(hb);
            terms[((size_t)t * B + b) * ldt + col] = (uint16_t)hb;
        }
    }
}

int launch_attention_decode(const DecodeArgs &a, int B, float *out, int ldo, uint16_t *terms,
                            int T, int ldt, hipStream_t st) {
    dim3 grid(a.NS, a.H, B);
    attn_decode_split_kernel<<<grid, 64, 0, st>>>(a);
    VMLM_HIP_CHECK(hipGetLastError());
    attn_decode_combine_kernel<<<dim3(a.H, B), 64, 0, st>>>(a.part, a.NS, a.H, out, ldo,
                                                            terms, T, ldt, B);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

}  // namespace vmlm

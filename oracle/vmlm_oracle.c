/*
 * vmlm_oracle.c -- CPU restatement of the reference VMLM inference kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see vmlm_oracle.h). Built with
 *   gcc -O3 -fPIC -shared -ffp-contract=off -fopenmp [-mavx2 -mfma]
 * by oracle/Makefile into oracle/_build/libvmlm_oracle.so.
 *
 * Restatement rules followed throughout:
 *  - `_mm256_fmadd_ps(a, b, c)` of the reference becomes fmaf(a, b, c) per lane;
 *    every other multiply-add stays a separate multiply then add (Rust never
 *    contracts; this file is compiled with -ffp-contract=off).
 *  - 8-lane AVX2 accumulators become float[8] arrays updated lane by lane;
 *    horizontal folds are written out in the reference's fixed order.
 *  - Loop order over independent output elements may differ from the
 *    reference (j-outer for cache reuse, OpenMP over rows); the arithmetic of
 *    each element does not.
 *
 * Parity pins (tests/test_oracle.py): the reference's own known-answer tests
 * (tests/src/main.rs, tools/p13_q8_check.py, tools/p13_kv_probe.py,
 * examples/p17_infer/ref_L2_d16.txt), closed forms, and brute-force float64
 * references chosen so that a dropped term, a wrong sign/index or a
 * transposed operand fails at least one of them.
 */
#include "vmlm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* reference constants: core/src/format.rs:98-103, tensor/src/act_op.rs:9-12 */
#define ACT_RELU 0
#define ACT_GELU 1
#define ACT_SILU 2
#define ACT_SIGMOID 3
#define ACT_TANH 4
#define ACT_RELU2 5
#define OP_EWADD 20
#define OP_EWMUL 21
#define OP_EWSUB 22
#define OP_EWDIV 23

static int g_threads = 1;

void vo_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int vo_get_threads(void) { return g_threads; }

static inline float f_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* ====================================================================== */
/* scalar math                                                             */
/* ====================================================================== */

/* sys/src/math/mod.rs:68-71 -- magic-number round to nearest even (|v| < 2^22). */
float vo_round_f32(float v) {
    const float MAGIC = 12582912.0f; /* 1.5 * 2^23 */
    return (v + MAGIC) - MAGIC;
}

/* Rust's `f as i32` (saturating; NaN -> 0). The callers convert values that
 * are integral and small after their clamps, or NaN; C's (int) cast of NaN is
 * undefined (x86 yields INT_MIN, which would send exp_f(NaN) to the
 * underflow branch instead of the reference's NaN). */
static inline int rust_as_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int)-2147483647 - 1;
    return (int)v;
}

/* sys/src/math/mod.rs:74-140 -- clamp, Cody-Waite ln2 split, degree-7
 * polynomial in Horner form, normal / subnormal / underflow 2^n. */
float vo_exp_f(float x) {
    if (x < -88.0f)
        x = -88.0f;
    else if (x > 88.0f)
        x = 88.0f;
    const float LOG2E = 1.4426950f;
    const float LN2_HI = 0.69314575f;
    const float LN2_LO = 1.4286068e-6f;
    float n = vo_round_f32(x * LOG2E);
    float r = (x - n * LN2_HI) - n * LN2_LO;
    float r2 = r * r;
    float p = 1.9875691e-4f;
    p = p * r + 1.3981999e-3f;
    p = p * r + 8.333452e-3f;
    p = p * r + 4.1665797e-2f;
    p = p * r + 1.6666665e-1f;
    p = p * r + 0.5f;
    p = p * r2 + r + 1.0f;
    int ni = rust_as_i32(n);
    if (ni >= -126) return p * f_from_bits((uint32_t)(ni + 127) << 23);
    if (ni >= -149) return p * f_from_bits(1u << (ni + 149));
    return 0.0f;
}

/* ops/src/kernels.rs:240-255 -- ln via exponent split and an atanh series. */
float vo_ln_f(float x) {
    if (x <= 0.0f) return -88.0f;
    uint32_t bits = f_to_bits(x);
    int e = (int)((bits >> 23) & 0xffu) - 127;
    float m = f_from_bits((bits & 0x007fffffu) | 0x3f800000u);
    if (m > 1.4142136f) {
        m *= 0.5f;
        e += 1;
    }
    float t = (m - 1.0f) / (m + 1.0f);
    float t2 = t * t;
    float p = 2.0f * t * (1.0f + t2 * (0.33333334f + t2 * (0.2f + t2 * 0.14285715f)));
    return p + (float)e * 0.69314718f;
}

/* ops/src/kernels.rs:113-130 -- three-part pi/2 Cody-Waite reduction. */
static inline void sin_cos_reduce(float x, float *r_out, float *r2_out, int *n_out) {
    const float PI2_HI = 1.57079637f;
    const float PI2_MID = -4.3711388e-8f;
    const float PI2_LO = -1.7151245e-15f;
    const float TWO_OVER_PI = 0.6366198f;
    if (x > 1.0e7f)
        x = 1.0e7f;
    else if (x < -1.0e7f)
        x = -1.0e7f;
    float n = vo_round_f32(x * TWO_OVER_PI);
    float r = ((x - n * PI2_HI) - n * PI2_MID) - n * PI2_LO;
    *r_out = r;
    *r2_out = r * r;
    *n_out = rust_as_i32(n);
}

/* ops/src/kernels.rs:194-200 */
static inline float sin_poly(float r, float r2) {
    float q = 2.7269829e-6f;
    q = q * r2 - 1.9840246e-4f;
    q = q * r2 + 8.3333322e-3f;
    q = q * r2 - 1.6666667e-1f;
    return r * (1.0f + r2 * q);
}

/* ops/src/kernels.rs:226-232 */
static inline float cos_poly(float r, float r2) {
    float p = 2.4410573e-5f;
    p = p * r2 - 1.3886977e-3f;
    p = p * r2 + 4.1666630e-2f;
    p = p * r2 - 5.0e-1f;
    return r2 * p + 1.0f;
}

/* ops/src/kernels.rs:144-152 */
float vo_sin_f(float x) {
    float r, r2;
    int n;
    sin_cos_reduce(x, &r, &r2, &n);
    switch (n & 3) {
    case 0: return sin_poly(r, r2);
    case 1: return cos_poly(r, r2);
    case 2: return -sin_poly(r, r2);
    default: return -cos_poly(r, r2);
    }
}

/* ops/src/kernels.rs:160-168 */
float vo_cos_f(float x) {
    float r, r2;
    int n;
    sin_cos_reduce(x, &r, &r2, &n);
    switch (n & 3) {
    case 0: return cos_poly(r, r2);
    case 1: return -sin_poly(r, r2);
    case 2: return -cos_poly(r, r2);
    default: return sin_poly(r, r2);
    }
}

/* ops/src/kernels.rs:216-223 -- truncate through i64, minus one if above. */
float vo_floor_f(float x) {
    float t = (float)(int64_t)x;
    return t > x ? t - 1.0f : t;
}

/* ops/src/kernels.rs:58-67 */
float vo_tanh_f(float x) {
    if (x > 15.0f) return 1.0f;
    if (x < -15.0f) return -1.0f;
    float e = vo_exp_f(2.0f * x);
    return (e - 1.0f) / (e + 1.0f);
}

/* ops/src/kernels.rs:1371-1375 -- sqrtss, correctly rounded. */
float vo_sqrt_f(float x) { return sqrtf(x); }

/* ops/src/kernels.rs:27-52 */
float vo_act_scalar(float x, uint16_t kind) {
    switch (kind) {
    case ACT_RELU: return x > 0.0f ? x : 0.0f;
    case ACT_GELU:
        return 0.5f * x * (1.0f + vo_tanh_f(0.7978846f * (x + 0.044715f * x * x * x)));
    case ACT_SILU: return x / (1.0f + vo_exp_f(-x));
    case ACT_SIGMOID: return 1.0f / (1.0f + vo_exp_f(-x));
    case ACT_TANH: return vo_tanh_f(x);
    case ACT_RELU2: {
        float r = x > 0.0f ? x : 0.0f;
        return r * r;
    }
    default: return x;
    }
}

/* tensor/src/dtype.rs:40-51 */
uint16_t vo_f32_to_bf16(float v) {
    uint32_t u = f_to_bits(v);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}
float vo_bf16_to_f32(uint16_t h) { return f_from_bits((uint32_t)h << 16); }

void vo_map(int which, const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        switch (which) {
        case 0: y[i] = vo_exp_f(v); break;
        case 1: y[i] = vo_ln_f(v); break;
        case 2: y[i] = vo_sin_f(v); break;
        case 3: y[i] = vo_cos_f(v); break;
        case 4: y[i] = vo_tanh_f(v); break;
        case 5: y[i] = vo_floor_f(v); break;
        case 6: y[i] = vo_round_f32(v); break;
        default: y[i] = vo_act_scalar(v, (uint16_t)(which - 100)); break;
        }
    }
}

/* tensor/src/dtype.rs:27-36 (hsum_ps) and sys/src/x86_avx2/simd.rs:17-26:
 * the 8-lane fold ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). */
static inline float fold8(const float l[8]) {
    float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
    return (s0 + s2) + (s1 + s3);
}

/* ====================================================================== */
/* GEMM family                                                             */
/* ====================================================================== */

/* ops/src/kernels.rs:1256-1287 -- per (i,j): 8 FMA lanes over k step 8,
 * fold, ascending scalar tail (mul then add), one multiply by scale[j]. */
static inline float dot_int8(const float *ar, const int8_t *qr, size_t k) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t kk = 0;
    for (; kk + 8 <= k; kk += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(ar[kk + l], (float)qr[kk + l], acc[l]);
    float s = fold8(acc);
    for (; kk < k; ++kk) s += ar[kk] * (float)qr[kk];
    return s;
}

/* Same per-element arithmetic as dot_int8 with the weight row converted to
 * f32 once ((float)q is exact) and four activation rows sharing it. */
static inline void dot_rowf_x4(const float *a0, const float *a1, const float *a2,
                               const float *a3, const float *wf, size_t k, float out[4]) {
    float c0[8] = {0}, c1[8] = {0}, c2[8] = {0}, c3[8] = {0};
    size_t kk = 0;
    for (; kk + 8 <= k; kk += 8)
        for (int l = 0; l < 8; ++l) {
            float w = wf[kk + l];
            c0[l] = fmaf(a0[kk + l], w, c0[l]);
            c1[l] = fmaf(a1[kk + l], w, c1[l]);
            c2[l] = fmaf(a2[kk + l], w, c2[l]);
            c3[l] = fmaf(a3[kk + l], w, c3[l]);
        }
    float s0 = fold8(c0), s1 = fold8(c1), s2 = fold8(c2), s3 = fold8(c3);
    for (; kk < k; ++kk) {
        s0 += a0[kk] * wf[kk];
        s1 += a1[kk] * wf[kk];
        s2 += a2[kk] * wf[kk];
        s3 += a3[kk] * wf[kk];
    }
    out[0] = s0;
    out[1] = s1;
    out[2] = s2;
    out[3] = s3;
}

void vo_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c,
                     size_t m, size_t n, size_t k) {
    long nn = (long)n;
    if (m < 4) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (long j = 0; j < nn; ++j) {
            const int8_t *qr = q + (size_t)j * k;
            for (size_t i = 0; i < m; ++i) c[i * n + j] = dot_int8(a + i * k, qr, k) * scale[j];
        }
        return;
    }
#pragma omp parallel num_threads(g_threads)
    {
        float *wf = malloc(k * sizeof(float));
#pragma omp for schedule(static)
        for (long j = 0; j < nn; ++j) {
            const int8_t *qr = q + (size_t)j * k;
            for (size_t p = 0; p < k; ++p) wf[p] = (float)qr[p];
            size_t i = 0;
            for (; i + 4 <= m; i += 4) {
                float o[4];
                dot_rowf_x4(a + i * k, a + (i + 1) * k, a + (i + 2) * k, a + (i + 3) * k, wf, k, o);
                for (int r = 0; r < 4; ++r) c[(i + r) * n + j] = o[r] * scale[j];
            }
            for (; i < m; ++i) c[i * n + j] = dot_int8(a + i * k, qr, k) * scale[j];
        }
        free(wf);
    }
}

/* ops/src/kernels.rs:1199-1227 -- two 8-lane FMA accumulators (k, k+8 per
 * 16-step), hsum(acc0)+hsum(acc1), ascending scalar tail. */
static inline float dot_bf16(const float *ar, const uint16_t *br, size_t k) {
    float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t kk = 0;
    for (; kk + 16 <= k; kk += 16) {
        for (int l = 0; l < 8; ++l) a0[l] = fmaf(ar[kk + l], vo_bf16_to_f32(br[kk + l]), a0[l]);
        for (int l = 0; l < 8; ++l)
            a1[l] = fmaf(ar[kk + 8 + l], vo_bf16_to_f32(br[kk + 8 + l]), a1[l]);
    }
    float s = fold8(a0) + fold8(a1);
    for (; kk < k; ++kk) s += ar[kk] * vo_bf16_to_f32(br[kk]);
    return s;
}

void vo_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                     size_t k) {
    long nn = (long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long j = 0; j < nn; ++j) {
        const uint16_t *br = b + (size_t)j * k;
        for (size_t i = 0; i < m; ++i) c[i * n + j] = dot_bf16(a + i * k, br, k);
    }
}

/* ops/src/kernels.rs:986-1015 dispatch. Per element the reference computes
 * either an FMA chain over p (the 8x8 AVX2 micro-kernel :436-546 and the packed
 * kernel :758-835 both broadcast a[i][p] against an 8-column B vector and fmadd
 * into one accumulator per element, p ascending) or a mul+add chain (scalar
 * paths :947-967 and the edge tail :924-945). `acc` adds the old C afterwards. */
enum { GEMM_SCALAR, GEMM_AVX2, GEMM_PACKED };

static inline int gemm_nt_path(size_t m, size_t n, size_t k) {
    if (n >= 8 && m >= 8) {
        if (k >= 8 && m >= 16 && (uint64_t)m * n * k >= 1000000ull) return GEMM_PACKED;
        return GEMM_AVX2;
    }
    return GEMM_SCALAR;
}

void vo_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                int acc) {
    int path = gemm_nt_path(m, n, k);
    size_t i8 = (m / 8) * 8, j8 = (n / 8) * 8;
    long mm = (long)m;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long ii = 0; ii < mm; ++ii) {
        size_t i = (size_t)ii;
        const float *ar = a + i * k;
        for (size_t j = 0; j < n; ++j) {
            const float *br = b + j * k;
            int use_fma = (path == GEMM_PACKED && i < i8) ||
                          (path == GEMM_AVX2 && i < i8 && j < j8);
            float s = 0.0f;
            if (use_fma) {
                for (size_t p = 0; p < k; ++p) s = fmaf(ar[p], br[p], s);
            } else {
                for (size_t p = 0; p < k; ++p) s += ar[p] * br[p];
            }
            if (acc) s += c[i * n + j];
            c[i * n + j] = s;
        }
    }
}

/* ops/src/kernels.rs:383-419 -- NN layout, scalar mul+add, p ascending. */
void vo_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
             int acc) {
    long mm = (long)m;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long ii = 0; ii < mm; ++ii) {
        size_t i = (size_t)ii;
        for (size_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (size_t p = 0; p < k; ++p) s += a[i * k + p] * b[p * n + j];
            if (acc) s += c[i * n + j];
            c[i * n + j] = s;
        }
    }
}

/* ====================================================================== */
/* row / elementwise ops                                                   */
/* ====================================================================== */

/* ops/src/kernels.rs:1346-1368 */
void vo_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *p = src + r * cols;
        float *q = dst + r * cols;
        float ss = 0.0f;
        for (size_t i = 0; i < cols; ++i) ss += p[i] * p[i];
        ss /= (float)cols;
        float inv = 1.0f / vo_sqrt_f(ss + eps);
        for (size_t i = 0; i < cols; ++i) q[i] = p[i] * inv * g[i];
    }
}

/* ops/src/kernels.rs:1388-1414 */
void vo_softmax(float *p, size_t rows, size_t cols, int causal) {
    for (size_t r = 0; r < rows; ++r) {
        float *row = p + r * cols;
        size_t lim = causal ? r + 1 : cols;
        if (lim > cols) lim = cols;
        float mx = -INFINITY;
        for (size_t i = 0; i < lim; ++i)
            if (row[i] > mx) mx = row[i];
        float sum = 0.0f;
        for (size_t i = 0; i < lim; ++i) {
            float e = vo_exp_f(row[i] - mx);
            row[i] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        for (size_t i = 0; i < lim; ++i) row[i] *= inv;
        for (size_t i = lim; i < cols; ++i) row[i] = 0.0f;
    }
}

/* ops/src/kernels.rs:1144-1167 -- RELU vector body is maxps(v, 0) (returns
 * the second operand unless v > 0), its scalar tail is `if x < 0 { 0 }`;
 * every other kind goes through act_scalar. */
void vo_act(float *dst, size_t n, uint16_t kind) {
    if (kind == ACT_RELU) {
        size_t n8 = (n / 8) * 8, i = 0;
        for (; i < n8; ++i)
            if (!(dst[i] > 0.0f)) dst[i] = 0.0f;
        for (; i < n; ++i)
            if (dst[i] < 0.0f) dst[i] = 0.0f;
        return;
    }
    for (size_t i = 0; i < n; ++i) dst[i] = vo_act_scalar(dst[i], kind);
}

/* ops/src/kernels.rs:1115-1142 */
void vo_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op) {
    for (size_t i = 0; i < n; ++i) {
        float a = x[i], b = y[i];
        switch (op) {
        case OP_EWADD: dst[i] = a + b; break;
        case OP_EWMUL: dst[i] = a * b; break;
        case OP_EWSUB: dst[i] = a - b; break;
        default: dst[i] = a / b; break;
        }
    }
}

/* core/src/interp.rs:1225-1235 (OP_SCALE) */
void vo_scale(float *dst, const float *src, size_t n, float s) {
    for (size_t i = 0; i < n; ++i) dst[i] = src[i] * s;
}

/* core/src/interp.rs:1159-1223 (OP_ROPE): half-split rotation, inverse
 * frequency exp_f(i*step) with step = (-2/hd)*ln_f(theta), position reduced
 * modulo the component's period unless the period is >= 1e6. */
int vo_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
            uint32_t pos0) {
    if (hd < 2 || (hd & 1)) return 9;
    if (!(theta > 0.0f)) return 9;
    const float TWO_PI = 6.2831855f;
    size_t half = hd / 2;
    float step = -2.0f / (float)hd * vo_ln_f(theta);
    float p0 = (float)pos0;
    for (size_t row = 0; row < rows; ++row) {
        float pos = p0 + (float)row;
        const float *sr = src + row * hd;
        float *dr = dst + row * hd;
        for (size_t i = 0; i < half; ++i) {
            float inv = vo_exp_f((float)i * step);
            float period = TWO_PI / inv;
            float pr = period >= 1.0e6f ? pos : pos - period * vo_floor_f(pos / period);
            float ang = pr * inv;
            float co = vo_cos_f(ang), si = vo_sin_f(ang);
            float x1 = sr[i], x2 = sr[i + half];
            dr[i] = x1 * co - x2 * si;
            dr[i + half] = x1 * si + x2 * co;
        }
    }
    return 0;
}

/* core/src/interp.rs:1351-1436 (OP_EMB): NaN/negative/out-of-range and
 * non-integral row indices are guard failures (exit 9); bf16 rows widen
 * exactly by a 16-bit shift. */
static int emb_row(float rowf, size_t rows, size_t *row_out) {
    if (!(rowf >= 0.0f) || rowf >= (float)rows) return 9;
    size_t row = (size_t)rowf;
    if ((float)row != rowf) return 9;
    *row_out = row;
    return 0;
}
int vo_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols, float rowf) {
    size_t row;
    int st = emb_row(rowf, rows, &row);
    if (st) return st;
    for (size_t i = 0; i < cols; ++i) dst[i] = vo_bf16_to_f32(table[row * cols + i]);
    return 0;
}
int vo_emb_f32(float *dst, const float *table, size_t rows, size_t cols, float rowf) {
    size_t row;
    int st = emb_row(rowf, rows, &row);
    if (st) return st;
    for (size_t i = 0; i < cols; ++i) dst[i] = table[row * cols + i];
    return 0;
}

/* core/src/interp.rs:1649-1681 (OP_TOPK_IDX): argmax of row 0, strict `>`
 * so the lowest index wins ties; the index is written as f32. */
int vo_topk_idx(const float *src, size_t rows, size_t cols, float *dst) {
    if (rows == 0 || cols == 0) return 9;
    size_t best = 0;
    float mv = src[0];
    for (size_t j = 1; j < cols; ++j)
        if (src[j] > mv) {
            mv = src[j];
            best = j;
        }
    *dst = (float)best;
    return 0;
}

/* ====================================================================== */
/* B1 sparse connections                                                   */
/* ====================================================================== */

/* core/src/conn_sparse.rs:157-214 -- stateless splitmix32 PRNG. */
#define SPLITMIX_GOLDEN 0x9E3779B9u
static inline uint32_t mix32(uint32_t z) {
    z = (z ^ (z >> 16)) * 0x7FEB352Du;
    z = (z ^ (z >> 15)) * 0x846CA68Bu;
    return z ^ (z >> 16);
}
uint32_t vo_neuron_seed(uint32_t layer, uint32_t i) {
    uint32_t a = SPLITMIX_GOLDEN * (layer + 1u);
    uint32_t b = 0x85EBCA6Bu * (i + 1u);
    return mix32(a ^ b);
}
uint32_t vo_neuron_rand(uint32_t seed, uint32_t j) {
    return mix32(seed ^ (SPLITMIX_GOLDEN * (j + 1u)));
}
uint32_t vo_neuron_conn_src(uint32_t layer, uint32_t i, uint32_t j, uint32_t n_neurons,
                            uint32_t k0) {
    if (n_neurons == 0 || k0 == 0) return 0;
    uint32_t seed = vo_neuron_seed(layer, i);
    uint32_t r = j == 0 ? vo_neuron_rand(seed, 0xFFFFFFFFu) : vo_neuron_rand(seed, j);
    return r % n_neurons;
}

/* ops/src/kernels.rs:1773-1804 -- 8 gather lanes starting at +0.0, each
 * lane acc + (w*x) (no FMA), fixed fold, ascending scalar tail. */
float vo_b1_dot_row_u32(const float *wrow, const uint32_t *srcrow, const float *x,
                        size_t k0) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t j = 0;
    for (; j + 8 <= k0; j += 8)
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + wrow[j + l] * x[srcrow[j + l]];
    float s = fold8(acc);
    for (; j < k0; ++j) s += wrow[j] * x[srcrow[j]];
    return s;
}

/* ops/src/kernels.rs:2720-2800 hsum128: (v0+v2)+(v1+v3). */
static inline float hsum4(float v0, float v1, float v2, float v3) {
    return (v0 + v2) + (v1 + v3);
}

/* ops/src/b1_pure.rs:151-226 (AVX2 branch) -> b1_forward_packed_avx2
 * (ops/src/kernels.rs:2720-2800) for k0 in {1,2,4,8}, then
 * b1_dot_row_u32_avx2 for the rows it left. Restated exactly, including the
 * k0==2 branch, which sums the two rows that share a 128-bit half
 * (rows i and i+1 both receive row_i + row_{i+1}). */
size_t vo_b1_forward(size_t n, size_t k0, const float *w, const uint32_t *src,
                     const float *x, float *y) {
    size_t done = 0;
    if (k0 == 1) {
        for (; done + 8 <= n; done += 8)
            for (int l = 0; l < 8; ++l) y[done + l] = w[done + l] * x[src[done + l]];
    } else if (k0 == 2) {
        for (; done + 4 <= n; done += 4) {
            float p[8];
            for (int l = 0; l < 8; ++l) p[l] = w[done * 2 + l] * x[src[done * 2 + l]];
            y[done] = hsum4(p[0], p[1], p[2], p[3]);
            y[done + 1] = hsum4(p[2], p[3], p[0], p[1]);
            y[done + 2] = hsum4(p[4], p[5], p[6], p[7]);
            y[done + 3] = hsum4(p[6], p[7], p[4], p[5]);
        }
    } else if (k0 == 4) {
        for (; done + 2 <= n; done += 2) {
            float p[8];
            for (int l = 0; l < 8; ++l) p[l] = w[done * 4 + l] * x[src[done * 4 + l]];
            y[done] = hsum4(p[0], p[1], p[2], p[3]);
            y[done + 1] = hsum4(p[4], p[5], p[6], p[7]);
        }
    } else if (k0 == 8) {
        for (; done < n; ++done) {
            float p[8];
            for (int l = 0; l < 8; ++l) p[l] = w[done * 8 + l] * x[src[done * 8 + l]];
            y[done] = hsum4(p[0] + p[4], p[1] + p[5], p[2] + p[6], p[3] + p[7]);
        }
    }
    for (size_t i = done; i < n; ++i) y[i] = vo_b1_dot_row_u32(w + i * k0, src + i * k0, x, k0);
    return n * k0;
}

/* ops/src/kernels.rs:2163-2188 -- the token-lane bitwise contract: j
 * ascending, first term assigned, mul then add. The AVX2 t8x4 kernel
 * (:2064-2155) is bitwise equal to this by construction. */
size_t vo_b1_forward_t8_scalar(const float *w, const uint32_t *src, size_t n, size_t k0,
                               const float *xt, size_t t8, size_t n_tokens, float *yt) {
    long nn = (long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long ii = 0; ii < nn; ++ii) {
        size_t i = (size_t)ii, base = i * k0;
        for (size_t t = 0; t < n_tokens; ++t) {
            float acc = 0.0f;
            for (size_t j = 0; j < k0; ++j) {
                float term = w[base + j] * xt[(size_t)src[base + j] * t8 + t];
                acc = j == 0 ? term : acc + term;
            }
            yt[i * t8 + t] = acc;
        }
    }
    return n * k0;
}

/* ops/src/kernels.rs:1875-1960 -- xt[s*t8 + t] = x[t*d + s]; pad columns
 * t in [t, t8) are written 0. */
void vo_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8) {
    for (size_t s = 0; s < d; ++s) {
        for (size_t tt = 0; tt < t; ++tt) xt[s * t8 + tt] = x[tt * d + s];
        for (size_t tt = t; tt < t8; ++tt) xt[s * t8 + tt] = 0.0f;
    }
}

/* ops/src/kernels.rs:3307-3370 -- out[i*os + s] = a[s*in_stride + i]. */
void vo_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                          size_t in_stride) {
    for (size_t s = 0; s < rows; ++s)
        for (size_t i = 0; i < cols; ++i) out[i * os + s] = a[s * in_stride + i];
}

/* ====================================================================== */
/* attention as the VM program composes it                                 */
/* ====================================================================== */

/* tools/p12_build_minicpm.py:770-781: per head SLICE -> ROPE(dt=pos0) ->
 * GEMM NT (dispatch of ops/src/kernels.rs:986) -> SCALE -> SOFTMAX(causal)
 * -> GEMM NN (scalar) -> WRITECOL. */
void vo_attention_prefill(const float *q, const float *k, const float *v, float *out,
                          size_t S, size_t H, size_t hd, float theta, uint32_t pos0,
                          float scale, int causal) {
    size_t W = H * hd;
    long hh = (long)H;
    int saved = g_threads;
    int outer = g_threads;
    g_threads = 1; /* heads in parallel, each head's GEMMs single-threaded */
#pragma omp parallel for schedule(dynamic) num_threads(outer)
    for (long h = 0; h < hh; ++h) {
        float *qh = malloc(S * hd * 4), *kh = malloc(S * hd * 4), *vh = malloc(S * hd * 4);
        float *sc = malloc(S * S * 4), *ctx = malloc(S * hd * 4);
        for (size_t r = 0; r < S; ++r) {
            memcpy(qh + r * hd, q + r * W + h * hd, hd * 4);
            memcpy(kh + r * hd, k + r * W + h * hd, hd * 4);
            memcpy(vh + r * hd, v + r * W + h * hd, hd * 4);
        }
        vo_rope(qh, qh, S, hd, theta, pos0);
        vo_rope(kh, kh, S, hd, theta, pos0);
        vo_gemm_nt(qh, kh, sc, S, S, hd, 0);
        vo_scale(sc, sc, S * S, scale);
        vo_softmax(sc, S, S, causal);
        vo_gemm(sc, vh, ctx, S, hd, S, 0);
        for (size_t r = 0; r < S; ++r) memcpy(out + r * W + h * hd, ctx + r * hd, hd * 4);
        free(qh);
        free(kh);
        free(vh);
        free(sc);
        free(ctx);
    }
    g_threads = saved;
}

/* tools/p12_build_minicpm.py:941-967: append ROPE(k, pos) and raw v at column
 * pos; per head ROPE(q, pos) -> GEMM NN over the live range (scalar, d
 * ascending) -> SCALE -> SOFTMAX (non-causal) -> GEMM NT with m=1 (scalar
 * path, positions ascending). */
void vo_attention_decode(const float *q, const float *k_new, const float *v_new,
                         float *kcache, float *vcache, float *out, size_t H, size_t hd,
                         size_t cap, size_t pos, float theta, float scale) {
    size_t live = pos + 1;
    float *qr = malloc(hd * 4), *sc = malloc(live * 4);
    for (size_t h = 0; h < H; ++h) {
        vo_rope(kcache + (h * cap + pos) * hd, k_new + h * hd, 1, hd, theta, (uint32_t)pos);
        memcpy(vcache + (h * cap + pos) * hd, v_new + h * hd, hd * 4);
    }
    for (size_t h = 0; h < H; ++h) {
        vo_rope(qr, q + h * hd, 1, hd, theta, (uint32_t)pos);
        const float *kc = kcache + h * cap * hd, *vc = vcache + h * cap * hd;
        for (size_t p = 0; p < live; ++p) {
            float s = 0.0f;
            for (size_t d = 0; d < hd; ++d) s += qr[d] * kc[p * hd + d];
            sc[p] = s;
        }
        vo_scale(sc, sc, live, scale);
        vo_softmax(sc, 1, live, 0);
        for (size_t d = 0; d < hd; ++d) {
            float s = 0.0f;
            for (size_t p = 0; p < live; ++p) s += sc[p] * vc[p * hd + d];
            out[h * hd + d] = s;
        }
    }
    free(qr);
    free(sc);
}

/* ====================================================================== */
/* MiniCPM-shaped decoder (tools/p12_build_minicpm.py, tools/p14_gen_build.py) */
/* ====================================================================== */

static float *xalloc(size_t n) {
    float *p = malloc(n * sizeof(float));
    return p;
}

/* One layer of the program body (p12_build_minicpm.py:766-792) over M rows at
 * positions pos0..pos0+M-1. For the prefill (cache empty before the layer) the
 * attention is the causal per-head composition; the rotated K / raw V of the
 * M rows are then written to the cache (:800-835). */
static void layer_prefill(const vo_model *md, const vo_layer *L, size_t li, float *h,
                          size_t M, float *kcache, float *vcache, size_t cap) {
    size_t H = md->hidden, I = md->inter, NH = md->n_heads, HD = md->head_dim;
    float *xn = xalloc(M * H), *q = xalloc(M * H), *k = xalloc(M * H), *v = xalloc(M * H);
    float *att = xalloc(M * H), *o = xalloc(M * H), *h2 = xalloc(M * H);
    float *g = xalloc(M * I), *u = xalloc(M * I), *dn = xalloc(M * H);
    vo_rmsnorm(xn, h, L->in_ln, M, H, md->eps);
    vo_gemm_nt_int8(xn, L->wq, L->sq, q, M, H, H);
    vo_gemm_nt_int8(xn, L->wk, L->sk, k, M, H, H);
    vo_gemm_nt_int8(xn, L->wv, L->sv, v, M, H, H);
    vo_attention_prefill(q, k, v, att, M, NH, HD, md->theta, 0, md->attn_scale, 1);
    vo_gemm_nt_int8(att, L->wo, L->so, o, M, H, H);
    vo_ew_op(h2, h, o, M * H, OP_EWADD);
    vo_rmsnorm(xn, h2, L->post_ln, M, H, md->eps);
    vo_gemm_nt_int8(xn, L->wg, L->sg, g, M, I, H);
    vo_gemm_nt_int8(xn, L->wu, L->su, u, M, I, H);
    vo_act(g, M * I, ACT_SILU);
    vo_ew_op(g, g, u, M * I, OP_EWMUL);
    vo_gemm_nt_int8(g, L->wd, L->sd, dn, M, H, I);
    vo_ew_op(h, h2, dn, M * H, OP_EWADD);
    /* cache rotated K and raw V for positions 0..M-1 */
    float *kr = xalloc(M * HD);
    for (size_t hh = 0; hh < NH; ++hh) {
        float *kc = kcache + ((li * NH + hh) * cap) * HD;
        float *vc = vcache + ((li * NH + hh) * cap) * HD;
        for (size_t r = 0; r < M; ++r) memcpy(kr + r * HD, k + r * H + hh * HD, HD * 4);
        vo_rope(kr, kr, M, HD, md->theta, 0);
        for (size_t r = 0; r < M; ++r) {
            memcpy(kc + r * HD, kr + r * HD, HD * 4);
            memcpy(vc + r * HD, v + r * H + hh * HD, HD * 4);
        }
    }
    free(kr);
    free(xn); free(q); free(k); free(v); free(att); free(o); free(h2);
    free(g); free(u); free(dn);
}

int vo_decoder_prefill(const vo_model *md, float *kcache, float *vcache, size_t cap,
                       const int32_t *tokens, size_t S, float *logits_last,
                       float *hidden_last) {
    size_t H = md->hidden;
    if (S == 0 || S > cap) return 9;
    float *h = xalloc(S * H);
    for (size_t r = 0; r < S; ++r) {
        int st = vo_emb_bf16(h + r * H, md->embed, md->vocab, H, (float)tokens[r]);
        if (st) {
            free(h);
            return st;
        }
    }
    for (size_t li = 0; li < md->n_layers; ++li)
        layer_prefill(md, &md->layers[li], li, h, S, kcache, vcache, cap);
    float *xn = xalloc(H);
    vo_rmsnorm(xn, h + (S - 1) * H, md->final_norm, 1, H, md->eps);
    if (hidden_last) memcpy(hidden_last, xn, H * 4);
    if (logits_last) vo_gemm_nt_bf16(xn, md->lm_head, logits_last, 1, md->vocab, H);
    free(xn);
    free(h);
    return 0;
}

/* p12_build_minicpm.py:917-981 -- one decode token through every layer, then
 * the final norm and the LM head. */
int vo_decoder_step(const vo_model *md, float *kcache, float *vcache, size_t cap,
                    int32_t token, size_t pos, float *logits, float *hidden) {
    size_t H = md->hidden, I = md->inter, NH = md->n_heads, HD = md->head_dim;
    if (pos >= cap) return 9;
    float *h = xalloc(H), *xn = xalloc(H), *q = xalloc(H), *k = xalloc(H), *v = xalloc(H);
    float *att = xalloc(H), *o = xalloc(H), *h2 = xalloc(H), *g = xalloc(I), *u = xalloc(I),
          *dn = xalloc(H);
    int st = vo_emb_bf16(h, md->embed, md->vocab, H, (float)token);
    if (st) goto out;
    for (size_t li = 0; li < md->n_layers; ++li) {
        const vo_layer *L = &md->layers[li];
        vo_rmsnorm(xn, h, L->in_ln, 1, H, md->eps);
        vo_gemm_nt_int8(xn, L->wq, L->sq, q, 1, H, H);
        vo_gemm_nt_int8(xn, L->wk, L->sk, k, 1, H, H);
        vo_gemm_nt_int8(xn, L->wv, L->sv, v, 1, H, H);
        vo_attention_decode(q, k, v, kcache + li * NH * cap * HD, vcache + li * NH * cap * HD,
                            att, NH, HD, cap, pos, md->theta, md->attn_scale);
        vo_gemm_nt_int8(att, L->wo, L->so, o, 1, H, H);
        vo_ew_op(h2, h, o, H, OP_EWADD);
        vo_rmsnorm(xn, h2, L->post_ln, 1, H, md->eps);
        vo_gemm_nt_int8(xn, L->wg, L->sg, g, 1, I, H);
        vo_gemm_nt_int8(xn, L->wu, L->su, u, 1, I, H);
        vo_act(g, I, ACT_SILU);
        vo_ew_op(g, g, u, I, OP_EWMUL);
        vo_gemm_nt_int8(g, L->wd, L->sd, dn, 1, H, I);
        vo_ew_op(h, h2, dn, H, OP_EWADD);
    }
    vo_rmsnorm(xn, h, md->final_norm, 1, H, md->eps);
    if (hidden) memcpy(hidden, xn, H * 4);
    if (logits) vo_gemm_nt_bf16(xn, md->lm_head, logits, 1, md->vocab, H);
out:
    free(h); free(xn); free(q); free(k); free(v); free(att); free(o); free(h2);
    free(g); free(u); free(dn);
    return st;
}

static void argmax_margin(const float *x, size_t n, int32_t *idx, float *margin) {
    float top = -INFINITY, second = -INFINITY;
    size_t best = 0;
    float mv = x[0];
    for (size_t j = 1; j < n; ++j)
        if (x[j] > mv) {
            mv = x[j];
            best = j;
        }
    top = mv;
    for (size_t j = 0; j < n; ++j)
        if (j != best && x[j] > second) second = x[j];
    *idx = (int32_t)best;
    if (margin) *margin = top - second;
}

/* p14_gen_build.py:470-560 -- TOPK_IDX feeds st_gen[k+1]; the chain starts
 * from the argmax of the prefill's last row. */
int vo_decoder_generate(const vo_model *md, float *kcache, float *vcache, size_t cap,
                        const int32_t *prompt, size_t S, size_t n_steps,
                        int32_t *out_tokens, float *margins) {
    if (S + n_steps > cap) return 9;
    float *logits = xalloc(md->vocab);
    int st = vo_decoder_prefill(md, kcache, vcache, cap, prompt, S, logits, NULL);
    if (st) goto out;
    argmax_margin(logits, md->vocab, &out_tokens[0], margins ? &margins[0] : NULL);
    for (size_t s = 0; s < n_steps; ++s) {
        st = vo_decoder_step(md, kcache, vcache, cap, out_tokens[s], S + s, logits, NULL);
        if (st) goto out;
        argmax_margin(logits, md->vocab, &out_tokens[s + 1], margins ? &margins[s + 1] : NULL);
    }
out:
    free(logits);
    return st;
}

/* ====================================================================== */
/* Backend primitives and the jit_* helpers                                */
/* ====================================================================== */

/* sys/src/x86_avx2/simd.rs:17-26 hsum256: lo + hi, then two hadds, i.e.
 * ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) -- not the hsum_ps order of fold8. */
static inline float hsum256(const float l[8]) {
    float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
    return (s0 + s1) + (s2 + s3);
}

/* sys/src/x86_avx2/simd.rs:27-57 dot256_f32: four 8-lane FMA chains over
 * 32-blocks, 8-blocks into chain 0, (a0+a1)+(a2+a3), hsum256, scalar tail. */
float vo_dot256(const float *a, const float *b, size_t n) {
    float c[4][8] = {{0}};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int r = 0; r < 4; ++r)
            for (int l = 0; l < 8; ++l) c[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], c[r][l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) c[0][l] = fmaf(a[i + l], b[i + l], c[0][l]);
    float s[8];
    for (int l = 0; l < 8; ++l) s[l] = (c[0][l] + c[1][l]) + (c[2][l] + c[3][l]);
    float acc = hsum256(s);
    for (; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

/* sys/src/x86_avx2/simd.rs:70-95 axpy256_f32: y = fma(a, x, y) on 8-blocks,
 * y += a * x (no FMA) on the tail. */
void vo_axpy256(float *y, const float *x, float a, size_t n) {
    size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < n8; ++i) y[i] = fmaf(a, x[i], y[i]);
    for (size_t i = n8; i < n; ++i) y[i] += a * x[i];
}

/* sys/src/x86_avx2/simd.rs:170-193 add256_f32. */
void vo_add256(float *y, const float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] += x[i];
}

/* _mm256_max_ps(a, b) per lane: a > b ? a : b (b on NaN or equal). */
static inline float maxps(float a, float b) { return a > b ? a : b; }

/* sys/src/x86_avx2/simd.rs:203-235 max256_f32: 8 lanes from -inf over the
 * 8-blocks, fold max(lo,hi), max(s, movehl), max(s, s1), then the tail with
 * a strict `>`. Empty input gives -inf. */
float vo_max256(const float *x, size_t n) {
    float m[8];
    for (int l = 0; l < 8; ++l) m[l] = -INFINITY;
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) m[l] = maxps(m[l], x[i + l]);
    float s[4];
    for (int l = 0; l < 4; ++l) s[l] = maxps(m[l], m[l + 4]);
    float t0 = maxps(s[0], s[2]), t1 = maxps(s[1], s[3]);
    float r = maxps(t0, t1);
    for (; i < n; ++i)
        if (x[i] > r) r = x[i];
    return r;
}

/* sys/src/x86_avx2/simd.rs:380-405 sum256_f32: two chains (s0 takes blocks
 * i and i+16, s1 blocks i+8 and i+24), 8-blocks into s0, hsum256(s0+s1),
 * scalar tail. */
float vo_sum256(const float *x, size_t n) {
    float s0[8] = {0}, s1[8] = {0};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int l = 0; l < 8; ++l) {
            s0[l] = s0[l] + x[i + l];
            s1[l] = s1[l] + x[i + 8 + l];
            s0[l] = s0[l] + x[i + 16 + l];
            s1[l] = s1[l] + x[i + 24 + l];
        }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) s0[l] = s0[l] + x[i + l];
    float s[8];
    for (int l = 0; l < 8; ++l) s[l] = s0[l] + s1[l];
    float acc = hsum256(s);
    for (; i < n; ++i) acc += x[i];
    return acc;
}

/* sys/src/x86_avx2/simd.rs:349-372 scale_mul_avx2: dst = a * src. */
void vo_scale_mul(float *dst, const float *src, float a, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = a * src[i];
}

/* ops/src/kernels.rs:1308-1333 layernorm (in place): sequential mean and
 * variance sums, inv = 1/sqrt_f(var + eps), y = (x - mean) * inv * g + b. */
void vo_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                  float eps) {
    for (size_t r = 0; r < rows; ++r) {
        float *p = x + r * cols;
        float mean = 0.0f;
        for (size_t i = 0; i < cols; ++i) mean += p[i];
        mean /= (float)cols;
        float var = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float d = p[i] - mean;
            var += d * d;
        }
        var /= (float)cols;
        float inv = 1.0f / vo_sqrt_f(var + eps);
        for (size_t i = 0; i < cols; ++i) p[i] = (p[i] - mean) * inv * g[i] + b[i];
    }
}

/* ops/src/kernels.rs:1058-1065 jit_bias: d[i, j] += b[j]. */
void vo_bias(float *d, const float *b, size_t rows, size_t cols) {
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j) d[i * cols + j] += b[j];
}

/* ops/src/kernels.rs:1416-1448 outer (AVX2 path outer_avx2): vi = v[i] * sc,
 * s = fma(vi, k, s) on 8-blocks of j, s += v[i] * sc * k[j] on the tail. */
void vo_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc) {
    size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < m; ++i) {
        float vi = v[i] * sc;
        for (size_t j = 0; j < n8; ++j) s[i * n + j] = fmaf(vi, k[j], s[i * n + j]);
        for (size_t j = n8; j < n; ++j) s[i * n + j] += v[i] * sc * k[j];
    }
}

/* ====================================================================== */
/* B1 backward                                                             */
/* ====================================================================== */

/* ops/src/b1_pure.rs:642-656 b1_backward: dw[i*k0+j] += dy[i] * x[src[i*k0+j]]
 * with the f32 source ids (`sc.src`, cast as usize). */
size_t vo_b1_backward(size_t n, size_t k0, const float *srcf, const float *dy, const float *x,
                      float *dw) {
    for (size_t i = 0; i < n; ++i) {
        float g = dy[i];
        for (size_t j = 0; j < k0; ++j) {
            float f = srcf[i * k0 + j];
            size_t s = f > 0.0f ? (size_t)f : 0;
            dw[i * k0 + j] += g * x[s];
        }
    }
    return n * k0;
}

/* ops/src/b1_pure.rs:410-428 b1_backward_dx: dx[src[i*k0+j]] += dy[i] * w[i*k0+j],
 * i ascending, j ascending. */
size_t vo_b1_backward_dx(size_t n, size_t k0, const float *w, const uint32_t *src,
                         const float *dy, float *dx) {
    for (size_t i = 0; i < n; ++i) {
        float g = dy[i];
        for (size_t j = 0; j < k0; ++j) dx[src[i * k0 + j]] += g * w[i * k0 + j];
    }
    return n * k0;
}

/* ops/src/kernels.rs:2458-2478 b1_backward_fused_dwdx_scalar, the contract of
 * the AVX2 fused kernel (:2401-2456): per connection dw first, then dx, i and
 * j ascending, mul then add. */
size_t vo_b1_backward_fused(size_t n, size_t k0, const float *w, const uint32_t *src,
                            const float *dy, const float *x, float *dw, float *dx) {
    for (size_t i = 0; i < n; ++i) {
        float g = dy[i];
        for (size_t j = 0; j < k0; ++j) {
            size_t s = src[i * k0 + j];
            dw[i * k0 + j] += g * x[s];
            dx[s] += g * w[i * k0 + j];
        }
    }
    return n * k0;
}

/* ops/src/kernels.rs:3229-3275 b1_backward_t8_avx2 over source-major
 * activations (t8 a multiple of 8): per connection (i, j), s = src: the
 * token dot product in eight FMA lanes (lane l takes p = l, l+8, ...),
 * reduced by hsum256 and added to dw; dxt[s][p] = fma(dyt[i][p], w, dxt[s][p]). */
void vo_b1_backward_t8(const float *w, const uint32_t *src, const float *xt, const float *dyt,
                       size_t t8, size_t n, size_t k0, float *dxt, float *dw) {
    for (size_t i = 0; i < n; ++i) {
        const float *dy = dyt + i * t8;
        for (size_t j = 0; j < k0; ++j) {
            size_t s = src[i * k0 + j];
            float wij = w[i * k0 + j];
            const float *xr = xt + s * t8;
            float *dr = dxt + s * t8;
            float acc[8] = {0};
            for (size_t p = 0; p + 8 <= t8; p += 8)
                for (int l = 0; l < 8; ++l) {
                    acc[l] = fmaf(dy[p + l], xr[p + l], acc[l]);
                    dr[p + l] = fmaf(dy[p + l], wij, dr[p + l]);
                }
            dw[i * k0 + j] += hsum256(acc);
        }
    }
}

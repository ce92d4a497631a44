// common.hpp -- shared definitions of libvmlm_hip.so (gfx950 only).
//
// Everything here compiles with -ffp-contract=off: device float expressions
// round after every operation exactly like the reference's Rust code, and
// FMAs appear only where written as __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/vmlm_hip.h"

namespace vmlm {

// ------------------------------------------------------------------ status
// Sets the thread's last-error message and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char *what);

#define VMLM_HIP_CHECK(expr)                                   \
    do {                                                       \
        hipError_t _e = (expr);                                \
        if (_e != hipSuccess) return ::vmlm::hip_fail(_e, #expr); \
    } while (0)

#define VMLM_GUARD(cond, ...)                                  \
    do {                                                       \
        if (!(cond)) return ::vmlm::fail(VMLM_ERR_GUARD, __VA_ARGS__); \
    } while (0)

// Library stream (created on first use, default priority) and device init.
int ensure_init();
hipStream_t lib_stream();
inline hipStream_t as_stream(void *s) { return s ? (hipStream_t)s : lib_stream(); }

// Device-side guard flag (set by kernels that validate indices on the GPU).
int *guard_flag_ptr();

// ------------------------------------------------------------------ types
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

// ------------------------------------------------------------------ bf16
// bf16 bits of f32, round to nearest even (tensor/src/dtype.rs:40-46).
// f32 -> bf16 bits, round to nearest even: v_cvt_pk_bf16_f32, which equals
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 on every non-NaN input (checked on
// all 2^28 strided f32 patterns) and keeps NaNs NaN.
typedef __bf16 hw_bf16x2 __attribute__((ext_vector_type(2)));
typedef float hw_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_rne_bits(float v) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v);
}
// two values packed (lo = a, hi = b) in one conversion
__device__ __forceinline__ uint32_t bf16x2_rne_bits(float a, float b) {
    const hw_f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, hw_bf16x2));
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// What is left of y after its bf16 term h: y - h, or 0 when y is not
// finite (inf - inf would be NaN), so an infinite value sits in its first
// term alone and its products stay +-inf (NaN against a zero weight).
__device__ __forceinline__ float term_rem(float y, uint32_t h) {
    const float r = y - bf16_bits_to_f32(h);
    return r == r ? r : 0.0f;
}

// Splits f32 x into up to three bf16 terms hi + mid + lo whose sum equals x
// to within 2^-24 |x| (each residual is exact in f32). Products of a bf16
// term with a bf16 (or small-integer) weight are exact in f32, so an MFMA
// over the terms reproduces f32 x . w up to the order of f32 accumulation.
// A non-finite x keeps its value in the first term and zeros in the others
// (inf - inf would make the residual NaN), so the products of an infinite
// activation are +-inf, or NaN against a zero weight, as in the f32 product.
template <int T>
__device__ __forceinline__ void split_bf16(float x, uint32_t (&t)[T]) {
    float r = x;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        t[i] = bf16_rne_bits(r);
        r = term_rem(r, t[i]);
    }
}

// 16 int8 (one 16-byte load) -> 16 bf16 in two 16-byte vectors, element order
// kept. Exact: |q| <= 128 has at most 8 significant bits; the bf16 is the high
// half of the f32 conversion, packed two per dword with v_perm_b32.
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
__device__ __forceinline__ void i8x16_to_bf16(u32x4 w, u32x4 &lo, u32x4 &hi) {
    uint32_t d[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t x = w[q];
        const float f0 = (float)(int)(int8_t)(x & 0xffu);
        const float f1 = (float)(int)(int8_t)((x >> 8) & 0xffu);
        const float f2 = (float)(int)(int8_t)((x >> 16) & 0xffu);
        const float f3 = (float)(int)(int8_t)(x >> 24);
        d[2 * q] = pack_hi16(f0, f1);
        d[2 * q + 1] = pack_hi16(f2, f3);
    }
    lo = u32x4{d[0], d[1], d[2], d[3]};
    hi = u32x4{d[4], d[5], d[6], d[7]};
}

// ------------------------------------------------------------------ int8 rows
// An f32 row y enters the int8 MFMA as Q8_T = 3 int8 terms with one
// power-of-two scale 2^k per row: the largest k with m * 2^k <= 127,
// m = max|y| or a bound on it within a few ulps. With u = y * 2^k (exact),
// a0 = rint(u), then each further term is rint of the remainder times 128, so
// u = a0 + a1/2^7 + a2/2^14 + e with |e| <= 2^-15: every value to within
// 2^-21 of the row maximum. |a0| <= 127, |a1|, |a2| <= 64; every step is
// exact in f32. k is clamped to [-126, 126] (rows whose maximum is below
// 2^-120 keep fewer bits). The error this adds to a dot product over K
// values is about 2^-21 * max|y| * sqrt(K) * rms(w), against the
// 1e-4 * RMS(C) contract of gemm_nt_int8: a row's maximum would have to be
// some 400 times its RMS to reach it. A fourth term (28 bits) gave the same
// greedy tokens and costs a third more MFMAs and row bytes.
//
// Non-finite rows: the magnitude used for the maximum maps NaN to +inf
// (q8_mag; fmaxf alone would drop a NaN), a non-finite maximum gives
// k = Q8_NONFINITE, whose factor is NaN and whose terms are 0. Every output
// of such a row is then NaN, never a finite value. (The standalone GEMM
// recomputes those rows in f32 to give the exact +-inf / NaN pattern.)
constexpr int Q8_T = 3;
constexpr int Q8_NONFINITE = 0x4000;
__device__ __forceinline__ float q8_mag(float y) {
    const float a = fabsf(y);
    return a == a ? a : __builtin_inff();
}
__device__ __forceinline__ int q8_row_k(float mx) {
    if (!(mx <= 3.40282347e38f)) return Q8_NONFINITE;
    if (!(mx > 0.0f)) return 0;
    int k = 6 - ilogbf(mx);
    if (ldexpf(mx, k) > 127.0f) --k;
    return k < -126 ? -126 : k > 126 ? 126 : k;
}
// the factor a consumer multiplies the term sums by: 2^-k, NaN for a
// non-finite row
__device__ __forceinline__ float q8_factor(int k) {
    return k == Q8_NONFINITE ? __builtin_nanf("") : ldexpf(1.0f, -k);
}
__device__ __forceinline__ void q8_split(float y, int k, int (&a)[Q8_T]) {
    float u = k == Q8_NONFINITE ? 0.0f : ldexpf(y, k);
    if (!(u == u)) u = 0.0f;
    // the scale keeps |u| <= 127 up to a few ulps of a bounding estimate;
    // 127.25 still rounds to 127 and leaves the excess to the next term
    u = fminf(fmaxf(u, -127.25f), 127.25f);
#pragma unroll
    for (int t = 0; t < Q8_T; ++t) {
        const float r = rintf(u);
        a[t] = (int)r;
        u = (u - r) * 128.0f;
    }
}
// the weight 2^-7t of term t's sum when the terms are combined in f32
__device__ __forceinline__ constexpr float q8_term_weight(int t) {
    return t == 1 ? 0.0078125f : t == 2 ? 6.103515625e-05f : 4.76837158203125e-07f;
}
// packs the bytes of four ints (low bytes) into one dword
__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// ------------------------------------------------------------------ math
// Device ports of the reference's scalar math, operation for operation, so
// that elementwise kernels are bitwise equal to the CPU kernels.

// sys/src/math/mod.rs:68-71
__device__ __forceinline__ float round_f32(float v) {
    const float MAGIC = 12582912.0f;
    return (v + MAGIC) - MAGIC;
}

// Rust's `f as i32` for the values these routines convert: NaN becomes 0
// (the others are integral and within +-2^24 after the clamps). The explicit
// test keeps C++ from treating the NaN conversion as undefined.
__device__ __forceinline__ int as_i32(float n) { return n == n ? (int)n : 0; }

// sys/src/math/mod.rs:74-140. exp_f_poly is the reduction and polynomial,
// e^x = p * 2^n; exp_f clamps x to [-88, 88] first and scales by 2^n, a
// normal or (n < -126) a subnormal float.
__device__ __forceinline__ float exp_f_poly(float x, float &n_out) {
    const float LOG2E = 1.4426950f;
    const float LN2_HI = 0.69314575f;
    const float LN2_LO = 1.4286068e-6f;
    float n = round_f32(x * LOG2E);
    float r = (x - n * LN2_HI) - n * LN2_LO;
    float r2 = r * r;
    float p = 1.9875691e-4f;
    p = p * r + 1.3981999e-3f;
    p = p * r + 8.333452e-3f;
    p = p * r + 4.1665797e-2f;
    p = p * r + 1.6666665e-1f;
    p = p * r + 0.5f;
    p = p * r2 + r + 1.0f;
    n_out = n;
    return p;
}
__device__ __forceinline__ float exp_f(float x) {
    x = x < -88.0f ? -88.0f : (x > 88.0f ? 88.0f : x);
    float n;
    const float p = exp_f_poly(x, n);
    // p * 2^n, 2^n a normal or (n < -126) a subnormal float; the two cases
    // as one select so the function has no branch (n >= -127 after the clamp)
    const int ni = as_i32(n);
    const float sc = ni >= -126 ? __uint_as_float((uint32_t)(ni + 127) << 23)
                     : ni >= -149 ? __uint_as_float(1u << ((ni + 149) & 31))
                                  : 0.0f;
    return p * sc;
}

// ops/src/kernels.rs:240-255
__device__ __forceinline__ float ln_f(float x) {
    if (x <= 0.0f) return -88.0f;
    uint32_t bits = __float_as_uint(x);
    int e = (int)((bits >> 23) & 0xffu) - 127;
    float m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
    if (m > 1.4142136f) {
        m *= 0.5f;
        e += 1;
    }
    float t = (m - 1.0f) / (m + 1.0f);
    float t2 = t * t;
    float p = 2.0f * t * (1.0f + t2 * (0.33333334f + t2 * (0.2f + t2 * 0.14285715f)));
    return p + (float)e * 0.69314718f;
}

// ops/src/kernels.rs:113-232 (reduction, quadrant select, polynomials)
__device__ __forceinline__ void sincos_f(float x, float *s_out, float *c_out) {
    const float PI2_HI = 1.57079637f;
    const float PI2_MID = -4.3711388e-8f;
    const float PI2_LO = -1.7151245e-15f;
    const float TWO_OVER_PI = 0.6366198f;
    x = x > 1.0e7f ? 1.0e7f : (x < -1.0e7f ? -1.0e7f : x);
    float n = round_f32(x * TWO_OVER_PI);
    float r = ((x - n * PI2_HI) - n * PI2_MID) - n * PI2_LO;
    float r2 = r * r;
    float q = 2.7269829e-6f;
    q = q * r2 - 1.9840246e-4f;
    q = q * r2 + 8.3333322e-3f;
    q = q * r2 - 1.6666667e-1f;
    float sp = r * (1.0f + r2 * q);
    float p = 2.4410573e-5f;
    p = p * r2 - 1.3886977e-3f;
    p = p * r2 + 4.1666630e-2f;
    p = p * r2 - 5.0e-1f;
    float cp = r2 * p + 1.0f;
    switch (as_i32(n) & 3) {
    case 0: *s_out = sp; *c_out = cp; break;
    case 1: *s_out = cp; *c_out = -sp; break;
    case 2: *s_out = -sp; *c_out = -cp; break;
    default: *s_out = -cp; *c_out = sp; break;
    }
}

// ops/src/kernels.rs:216-223
__device__ __forceinline__ float floor_f(float x) {
    float t = (float)(long long)x;
    return t > x ? t - 1.0f : t;
}

// ops/src/kernels.rs:58-67. Past the clamps 2x is within [-30, 30] (or NaN),
// where exp_f's own clamp does nothing and 2^n (|n| <= 44, or n NaN -> 0) is
// a normal float: exp_f's operations without those two selects.
__device__ __forceinline__ float tanh_f(float x) {
    if (x > 15.0f) return 1.0f;
    if (x < -15.0f) return -1.0f;
    float n;
    const float p = exp_f_poly(2.0f * x, n);
    const float e = p * __uint_as_float((uint32_t)(as_i32(n) + 127) << 23);
    return (e - 1.0f) / (e + 1.0f);
}

// ops/src/kernels.rs:27-52
__device__ __forceinline__ float act_scalar(float x, int kind) {
    switch (kind) {
    case VMLM_ACT_RELU: return x > 0.0f ? x : 0.0f;
    case VMLM_ACT_GELU:
        return 0.5f * x * (1.0f + tanh_f(0.7978846f * (x + 0.044715f * x * x * x)));
    case VMLM_ACT_SILU: return x / (1.0f + exp_f(-x));
    case VMLM_ACT_SIGMOID: return 1.0f / (1.0f + exp_f(-x));
    case VMLM_ACT_TANH: return tanh_f(x);
    case VMLM_ACT_RELU2: {
        float r = x > 0.0f ? x : 0.0f;
        return r * r;
    }
    default: return x;
    }
}

// core/src/interp.rs:1183-1221: the rotation of RoPE component i at position
// `pos` (a function of (pos, i) only, so rows at one position share it) ...
__device__ __forceinline__ void rope_angle(float pos, int i, float step, float *si, float *co) {
    const float TWO_PI = 6.2831855f;
    float inv = exp_f((float)i * step);
    float period = TWO_PI / inv;
    float pr = period >= 1.0e6f ? pos : pos - period * floor_f(pos / period);
    float ang = pr * inv;
    sincos_f(ang, si, co);
}
// ... and one rotated pair
__device__ __forceinline__ void rope_pair(float x1, float x2, float pos, int i, float step,
                                          float *y1, float *y2) {
    float si, co;
    rope_angle(pos, i, step, &si, &co);
    *y1 = x1 * co - x2 * si;
    *y2 = x1 * si + x2 * co;
}

// ------------------------------------------------------------------ wave ops
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// DPP forms of the wave reductions: no LDS round trip per step (each
// __shfl_xor above is a ds_bpermute). Inside a row of 16 lanes: quad swaps
// (quad_perm 1,0,3,2 and 2,3,0,1), then rotations of the row by 4 and 8.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL,
                                                      0xF, 0xF, false));
}
// Maximum of a non-negative v over each row of 16 lanes, in every lane of
// the row (exact in any order).
__device__ __forceinline__ float row16_max_nonneg(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x124>(v));
    return fmaxf(v, dpp_mov<0x128>(v));
}
// Maximum of a non-negative v over the wave, the same in every lane: the
// four row maxima read as scalars.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = row16_max_nonneg(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}
// Sum over the wave in a fixed order, the same in every lane: lane 16r
// holds row r's sum ((quad pairs), then the rotations), and the four row
// sums are read as scalars and added as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = v + dpp_mov<0xB1>(v);
    v = v + dpp_mov<0x4E>(v);
    v = v + dpp_mov<0x124>(v);
    v = v + dpp_mov<0x128>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace vmlm

// internal.hpp -- launchers shared between translation units of libvmlm_hip.so.
#pragma once

#include "common.hpp"

namespace vmlm {

// Host restatement of ln_f (ops/src/kernels.rs:240-255) for RoPE's step
// constant -2/hd * ln_f(theta), computed once per launch.
float host_ln_f(float x);

// Activation operand of the MFMA GEMV / GEMM: T planes of bf16 bits
// [T][rows][ld] (ld a multiple of 64, zero padded) whose sum is the f32
// activation (see split_bf16).
int launch_split_terms(const float *x, size_t ldx, int rows, int K, int T, uint16_t *out,
                       int ld_out, hipStream_t st);

enum GemvEpi {
    EPI_STORE = 0,    // Y = acc * scale
    EPI_RESIDUAL = 1, // Y = R + acc * scale              (OP_GEMM then OP_EWADD)
    EPI_SILU_MUL = 2, // pairs of 16-row tiles (gate, up): Y = silu(g) * u and its terms
    EPI_ARGMAX = 3,   // Y = acc (* scale), plus the row argmax folded into keys[M]
    EPI_PARTIAL = 4,  // Y[ks][M][ldy] = raw sums of k-slice ks (no scale); consumer reduces
};

// Argmax keys: (order-preserving bits of the value << 32) | (0xffffffff - index),
// combined with 64-bit atomicMax -> the largest value, lowest index on ties
// (the strict `>` scan of OP_TOPK_IDX). 0 = empty.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal under `>`: one key, lowest index wins
    uint32_t u = __float_as_uint(v);
    uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xffffffffu - idx);
}
__device__ __forceinline__ int32_t argmax_key_index(unsigned long long k) {
    return (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
}
constexpr unsigned long long ARGMAX_NAN0_KEY = 0xffffffffffffffffull;  // NaN at index 0
constexpr int KEY_SLOTS = 64;  // argmax slots per row (spreads the atomics)

struct GemvArgs {
    const void *W = nullptr; // [N][K] int8 or bf16 bits, rows 16-byte aligned
    bool w_int8 = true;
    const float *scale = nullptr; // [N] per-row scale (int8) or null
    const uint16_t *A = nullptr;  // terms [T][.][lda], plane stride a_tstride
    int T = 3;
    int lda = 0;
    size_t a_tstride = 0;    // elements between term planes (0: M * lda)
    int M = 1, N = 0, K = 0; // K % 64 == 0, M <= 16
    float *Y = nullptr;
    int ldy = 0;
    const float *R = nullptr; // residual (EPI_RESIDUAL), [M][ldr]
    int ldr = 0;
    int epi = EPI_STORE;
    uint16_t *Aout = nullptr; // EPI_SILU_MUL: terms of Y, [T][M][ldaout]
    int ldaout = 0;
    int Tout = 3;
    unsigned long long *keys = nullptr; // EPI_ARGMAX: [M], zeroed before the launch
    int tiles = 0; // 16-row tiles per workgroup (1, 2, 4; SiLU: 2, 4); 0 = chosen by shape
    int ksplit = 1; // k-slices (workgroup rows) for EPI_PARTIAL
    const float *X = nullptr; // tiles == 8: f32 activation rows [M][ldx] instead of A
    int ldx = 0;
};
int launch_gemv(const GemvArgs &a, hipStream_t st);
// C = (in-order sum of ks k-slice partials [ks][M][N]) * scale (per column, or none).
int launch_gemv_reduce(const float *part, int ks, int M, int N, const float *scale, float *C,
                       int ldc, hipStream_t st);

// Full-K GEMV for decode batches of M <= 5 rows with fused row ops. Input:
// bf16 term planes A [3][M][lda]; with ssp, the rows are RMSNorm inputs
// given as terms of x * g, and the dot products are multiplied by
// inv = 1 / sqrt(sum(ssp[.][b]) / K + eps). Output: Y = acc * scale[j]
// (FK_STORE), Y = R + acc * scale[j] (FK_RESID; with ssp_out also the terms
// of Y * gout into Aout and sum Y^2 per 16 columns into ssp_out [N/16][M]),
// or over 16-row gate/up tile pairs Y[.][16p + r] = silu(gate) * up
// (FK_SILU; Y and/or its terms in Aout). W is the copy made by
// launch_swizzle_w.
enum FkEpi { FK_STORE = 0, FK_RESID = 1, FK_SILU = 2 };
struct FkArgs {
    const int8_t *W = nullptr;
    const float *scale = nullptr;
    const uint16_t *A = nullptr;
    int lda = 0;
    const float *ssp = nullptr;
    int nssp = 0;
    float eps = 0.0f;
    float *Y = nullptr;
    int ldy = 0;
    const float *R = nullptr;
    int ldr = 0;
    uint16_t *Aout = nullptr;
    const float *gout = nullptr;
    float *ssp_out = nullptr;
    int M = 1, N = 0, K = 0;
    int epi = FK_STORE;
    int kb = 0;  // 64-wide k-blocks per wave (2, 3, 4, 6, 8); 0 = chosen by shape
    // optional (M = 1, K = heads x 64): the input row as the attention's
    // FK_APART position-range partials per head [K/64][FK_APART][68]
    // (DecodeArgs::frac), merged in order here instead of term planes
    const float *apart = nullptr;
};
constexpr int FK_APART = 4;  // position ranges per head of the attention partials
constexpr int ATTN_PART = 68;  // floats per attention partial: max, sum, 2 unused, O[64]
bool fk_gemv_ok(int M, int N, int K, int epi);
// an o projection of input width K can take the attention's range partials
bool fk_apart_ok(int K);
int launch_fk_gemv(const FkArgs &a, hipStream_t st);
// Rows h [M][ldh] entering the fused path: terms of h * g into [3][M][ldt]
// and the partial sums of squares [N/16][M].
int launch_fk_norm_prep(const float *h, int ldh, const float *g, int M, int N, uint16_t *terms,
                        int ldt, float *ssp, hipStream_t st);
// k-slice GEMV for decode batches up to 16 over the swizzled weights: raw
// slice sums Y[ks][M][ldy] of A . W^T, with ks = ks_gemv_slices(K) slices of
// ks_gemv_window(K) columns; the consumer reduces the slices in order and
// applies the row scales. A is given as bf16 term planes [3][M][lda], or as
// int8 rows from launch_resid_q8 (segments = the slices): the int8 terms
// [Q8_T][M][lda] of x * g, each slice's row factors a8s[ks][M] and the
// segment sums of squares ssp[ks][M]; slice s of row m is then multiplied by
// a8s[s][m] / sqrt(sum_s ssp[s][m] / K + eps).
struct KsArgs {
    const int8_t *W = nullptr;
    const uint16_t *A = nullptr;
    const int8_t *A8 = nullptr;
    const float *a8s = nullptr;
    const float *ssp = nullptr;
    float eps = 0.0f;
    int lda = 0;
    float *Y = nullptr;
    int ldy = 0;
    int M = 1, N = 0, K = 0;
    int tw = 0, nwv = 0;  // tiles per wave, waves per workgroup; 0 = 2, 4
    const float *X = nullptr;  // f32 rows [M][lda], quantized per slice while staged
};
int ks_gemv_slices(int K);
// (with X instead of A / A8: f32 rows [M][lda], each slice's rows split into
// int8 terms while staged, with the factor of the slice's own maximum.)
inline int ks_gemv_window(int K) { return K / ks_gemv_slices(K); }
int launch_ks_gemv(const KsArgs &a, hipStream_t st);
// Full-K int8 GEMV for decode batches up to 16 rows (k_fullk.hip): one
// launch per projection, no k-slice partials. Input: int8 rows in blocked
// layout [Q8_T][K/64][1 KiB] (launch_resid_q8 with `blocked`), segment
// factors a8s[K/64/seg_kb][M] and, for an RMSNorm input, segment sums of
// squares ssp (same shape). FQ_STORE: Y[m][j] = acc * scale[j] * inv[m];
// FQ_SILU over the gate/up tile pairs of the swizzled Wgu:
// Y[m][16p + r] = silu(gate) * up.
enum FqEpi { FQ_STORE = 0, FQ_SILU = 1 };
struct FqArgs {
    const int8_t *W = nullptr;
    const float *scale = nullptr;
    const int8_t *A8 = nullptr;
    const float *a8s = nullptr;
    const float *ssp = nullptr;
    float eps = 0.0f;
    int seg_kb = 4;
    float *Y = nullptr;
    int ldy = 0;
    int M = 1, N = 0, K = 0;
    int epi = FQ_STORE;
    int tw = 1;  // 16-row tiles per workgroup (1, 2 or 4; FQ_SILU: 2 or 4)
};
bool fq_gemv_ok(int M, int N, int K, int epi, int tw);
int launch_fq_gemv(const FqArgs &a, hipStream_t st);

// The standalone q8 GEMM at M <= FX_ROWS f32 rows in one launch
// (k_q8gemv.hip): C[m][j] = (X[m] . W[j]) * scale[j], int8 weights
// row-major [N][ldw] or swizzled (launch_swizzle_w's layout, N % 16 == 0).
// fx_run_blocks(K) != 0 says a kernel exists for K.
constexpr int FX_ROWS = 4;
int fx_run_blocks(int K);
struct FxArgs {
    const void *W = nullptr;
    bool swizzled = false;
    int ldw = 0;
    const float *scale = nullptr;
    const float *X = nullptr;
    int ldx = 0;
    float *C = nullptr;
    int ldc = 0;
    int M = 0, N = 0, K = 0;
    int kb = 0, tw = 0;  // blocks per wave run, 16-row tiles per workgroup (0: by shape)
};
int launch_fx_gemv(const FxArgs &a, hipStream_t st);
// Up to three projections of the same rows in one launch (each output what
// its own launch_fx_gemv gives), or, with `act`, a gate/up pair (two
// segments of one width) that also writes act = silu(gate) * up.
struct FxSegArgs {
    const void *W = nullptr;
    const float *scale = nullptr;
    float *C = nullptr;
    int N = 0, ldc = 0;
};
struct FxMultiArgs {
    FxSegArgs seg[3];
    int nseg = 0;
    bool swizzled = false;
    int ldw = 0;
    const float *X = nullptr;
    int ldx = 0;
    int M = 0, K = 0;
    float *act = nullptr;
    int ldact = 0;
    // one segment: also zadd = radd + C elementwise ([M][ldc], the EWADD
    // after the GEMM; f32 addition, as the separate opcode)
    const float *radd = nullptr;
    float *zadd = nullptr;
    // with norm_g: the GEMMs read the RMSNorm of the row X (M = 1), y = (x *
    // inv) * g with inv = 1 / sqrt(mean(x^2) + eps) summed as launch_rmsnorm's
    // one-pass kernel sums it (the same bits as that launch), and y is also
    // written to norm_out [K] (swizzled weights, K % 4 == 0, K <= 4096)
    const float *norm_g = nullptr;
    float *norm_out = nullptr;
    float norm_eps = 0.0f;
};
int launch_fx_multi(const FxMultiArgs &a, hipStream_t st);
// a normalizing launch_fx_multi kernel exists for rows of K values
bool fx_norm_ok(int K);
// The int8 GEMM C[m][n] = (A[m] . Q[n]) * scale[n] (vmlm_hip_gemm_nt_int8) with
// a swizzled copy wsw of Q (launch_swizzle_w, N % 16 == 0) that the caller
// keeps, read instead of Q where a kernel takes that layout; wsw may be null.
int q8_gemm_vm(const float *a, const int8_t *q, const int8_t *wsw, const float *scale, float *c,
               size_t m, size_t n, size_t k, hipStream_t st);

// int8 [N][K] row-major -> [N/16][K/64][64 lanes][16 B] MFMA-operand order.
int launch_swizzle_w(const int8_t *src, int8_t *dst, int N, int K, hipStream_t st);

// Tiled MFMA GEMM for M > 16: C[M,N] = A[M,K] . W[N,K]^T (* scale[n]).
struct GemmArgs {
    const void *W = nullptr;
    bool w_int8 = true;
    const float *scale = nullptr;
    const uint16_t *A = nullptr; // terms [T][M][lda]
    int T = 3;
    int lda = 0;
    int M = 0, N = 0, K = 0; // K % 64 == 0
    float *C = nullptr;
    int ldc = 0;
    int bm = 0;      // tile rows (64, 128); 0 = chosen by shape
    int stages = 0;  // LDS stages of the copy pipeline (2..4); 0 = chosen by shape
    int group = -1;  // tile order: 0 as dispatched, g > 0 grouped per XCD; -1 = default
    // or int8 rows (with int8 weights): the blocked term planes and row
    // factors [M] of launch_rows_q8 (A, T and lda unused)
    const int8_t *A8 = nullptr;
    const float *a8s = nullptr;
    // int8 rows: W is the swizzled copy (launch_swizzle_w) instead of row-major
    bool w_blocked = false;
    // int8 rows, optional: gemm_i8_work_floats() floats for the k-slices of
    // a grid that would leave most CUs idle (null: one slice); work_floats is
    // its size, checked against the slices the launch would write
    float *work = nullptr;
    size_t work_floats = 0;
    // int8 rows with k-slices: leave the slices in `work` for the consumer
    // (Slices below) instead of reducing them into C
    bool keep_slices = false;
    // int8 rows: the N weight rows are (gate, up) pairs interleaved in blocks
    // of 16 (rows 32t .. 32t + 15 gate, 32t + 16 .. 32t + 31 up); C receives
    // act = SiLU(gate) * up [M][N / 2] (column 16t + j from rows 32t + j and
    // 32t + 16 + j), formed in the epilogue from the scaled results (one
    // slice; N % 32 == 0)
    bool silu_pairs = false;
};
int launch_gemm(const GemmArgs &a, hipStream_t st);
// An [M][N] matrix left as ks ordered k-slices [ks][M][N] (row factors
// applied) by launch_gemm with keep_slices: element (i, j) is
// (part[0][i][j] + part[1][i][j] + ...) * scale[j], the arithmetic of the
// slice reduction (launch_gemv_reduce).
struct Slices {
    const float *part = nullptr;
    int ks = 0;
    size_t pst = 0;  // floats from one slice to the next (M * N)
    const float *scale = nullptr;
};
// Recomputes in f32 the rows of an int8-row GEMM whose factor a8s[i] is NaN
// (non-finite inputs), giving the reference's +-inf / NaN pattern.
int launch_gemm_i8_nonfinite_rows(const float *a, int lda, const int8_t *q, int ldq,
                                  const float *scale, const float *a8s, float *c, int ldc, int M,
                                  int N, int K, hipStream_t st);
// Backend-table primitives and jit helpers (k_backend.hip). `part` holds
// bk_reduce_work_floats() floats, `work` bk_max_work_bytes() bytes; the
// scalar result goes to out[0] on the device.
int bk_reduce_work_floats();
size_t bk_max_work_bytes();
int launch_bk_reduce(const float *a, const float *b, size_t n, bool dot, float *part, float *out,
                     hipStream_t st);
int launch_bk_max(const float *x, size_t n, void *work, float *out, hipStream_t st);
int launch_bk_axpy(float *y, const float *x, float a, size_t n, hipStream_t st);
int launch_bk_add(float *y, const float *x, size_t n, hipStream_t st);
int launch_bk_scale_mul(float *d, const float *s, float a, size_t n, hipStream_t st);
int launch_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                     float eps, hipStream_t st);
int launch_bias(float *d, const float *b, size_t rows, size_t cols, hipStream_t st);
int launch_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc,
                 hipStream_t st);
// B1 backward (k_b1_bwd.hip). dw / dx / dxt accumulate; `work` holds
// b1_rev_work_bytes(n * k0, n) bytes (the reverse index of the sources).
// srcf (f32 ids) feeds dw when given, else src (u32 ids).
size_t b1_rev_work_bytes(size_t E, size_t d);
int launch_b1_backward(const float *w, const float *srcf, const uint32_t *src, size_t n,
                       size_t k0, const float *dy, const float *x, float *dw, float *dx,
                       void *work, hipStream_t st);
int launch_b1_backward_t8(const float *w, const uint32_t *src, const float *xt, const float *dyt,
                          size_t t8, size_t n, size_t k0, float *dxt, float *dw, void *work,
                          hipStream_t st);
// Zero-fills `bytes` bytes with a kernel (capturable, unlike hipMemsetAsync).
int launch_fill_zero(void *p, size_t bytes, hipStream_t st);
int gemm_i8_kslices(int M, int N, int K);
inline size_t gemm_i8_work_floats(int M, int N, int K) {
    const int ks = gemm_i8_kslices(M, N, K);
    return ks > 1 ? (size_t)ks * M * N : 0;
}

// f32 GEMMs (NT and NN) with optional accumulate.
// work: gemm_f32_work_floats() floats (narrow outputs are split over k; null: no split).
int launch_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                    bool acc, bool b_is_nt, hipStream_t st, float *work = nullptr);
size_t gemm_f32_work_floats(size_t m, size_t n, size_t k);

// Row / elementwise ops.
int launch_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                   float eps, uint16_t *terms, int T, int ld_terms, hipStream_t st);
// x = base + (sum of ks k-slice partials [ks][rows][ldp]) * scale -> resid;
// RMSNorm(x) * g -> T bf16 terms [T][rows][cols].
int launch_rmsnorm_resid(const float *base, const float *part, int ks, int ldp,
                         const float *scale, float *resid, size_t rows, size_t cols,
                         const float *g, float eps, uint16_t *terms, int T, int ld_terms,
                         hipStream_t st);
// The residual add of a k-split projection and the int8 input of the next
// k-slice GEMVs, by segments of `seg` columns (the consumers' k window):
//   x = base + (sum_ks part[ks]) * scale   (ks == 0: x = base, nothing stored)
//   resid = x;  q8/q8s = int8 terms of x * g with each segment's power-of-two
//   factor [cols/seg][rows];  ssp = each segment's sum of x^2 [cols/seg][rows].
// The consumer applies 1/sqrt(sum(ssp)/cols + eps) (the RMSNorm) to its dot
// products. With `blocked` (rows <= 16) q8 takes the layout of the full-K
// GEMV's input instead of row-major planes: [Q8_T][cols/64][1 KiB], lane
// (g, n) of a block = row n, k 8g .. +7 and 32 + 8g .. +7 (rows past `rows`
// are left as they are: zero from the owner's initialisation).
int launch_resid_q8(const float *base, const float *part, int ks, int ldp, const float *scale,
                    float *resid, const float *g, size_t rows, size_t cols, int seg, int8_t *q8,
                    float *q8s, float *ssp, hipStream_t st, bool blocked = false);
// Rows x [rows][ldx] (with g: RMSNorm(x) * g) as Q8_T int8 terms with
// per-row power-of-two factors q8s [rows]: the input of launch_gemm's
// int8-row path. Layout (q8_rows_bytes(rows, cols) bytes): Q8_T planes of
// q8_rows_tiles(rows) x (cols / 64) blocks of 1 KiB; block (row tile rt,
// k-block kb) holds rows 16 rt .. 16 rt + 15, k 64 kb .. 64 kb + 63, lane
// (g, r) = 16 bytes at (16 g + r) * 16: row r, k 8g .. 8g + 7 and 32 + 8g ..
// 32 + 8g + 7 (the order of the swizzled weights, launch_swizzle_w); then
// one float per row tile row, used between the two launches. Rows past
// `rows` in the last 16-row tile are zero terms; later tiles may be left
// unwritten. cols % 64 == 0, cols <= 8192. With ra and rb (same ldx) the
// rows are first formed as x = ra + rb and written to x (a residual add).
size_t q8_rows_tiles(size_t rows);
size_t q8_rows_bytes(size_t rows, size_t cols);
int launch_rows_q8(const float *x, size_t ldx, const float *g, float eps, size_t rows, size_t cols,
                   int8_t *q8, float *q8s, hipStream_t st, const float *ra = nullptr,
                   const float *rb = nullptr, const Slices &rbs = Slices{});
// SiLU(gate) * up from the partials of the interleaved gate/up projection,
// as int8 terms [Q8_T][rows][I] with a power-of-two
// factor per segment of `seg` columns, q8s [I/seg][rows] (the input of a
// k-slice GEMV whose slices are the segments).
int launch_silu_q8(const float *part, int ks, int ldp, const float *sgu, int rows, int I, int seg,
                   int8_t *q8, float *q8s, hipStream_t st);
int launch_softmax(float *p, size_t rows, size_t cols, bool causal, hipStream_t st);
int launch_act(float *dst, size_t n, int kind, hipStream_t st);
int launch_ew(float *dst, const float *x, const float *y, size_t n, int op, hipStream_t st);
int launch_scale(float *dst, const float *src, size_t n, float s, hipStream_t st);
// RoPE over `rows` positions (pos0 + row) x `heads` heads of width hd,
// head h at column h*hd of a row of stride ld.
int launch_rope(float *dst, const float *src, size_t rows, size_t hd, size_t ld, float theta,
                float pos0, int heads, hipStream_t st);
// `guard` (null: the library's flag) is raised for a bad row index.
int launch_emb_bf16(float *dst, size_t ldd, const uint16_t *table, size_t rows, size_t cols,
                    const float *rowf, const int32_t *rowi, int n, hipStream_t st,
                    int *guard = nullptr);
// OP_TOPK_IDX over one row of cols values: index of the largest non-NaN value,
// lowest index on ties, 0 when x[0] is NaN or every value is; keys:
// ARGMAX_KEYS 64-bit device words of workspace.
constexpr int ARGMAX_KEYS = 4096;
int launch_argmax(const float *src, size_t cols, float *dst_f, int32_t *dst_i,
                  unsigned long long *keys, hipStream_t st);

// Attention (head_dim 64). Prefill takes rotated K, and Q rotated (rope_q
// false) or raw (rope_q: rotated on load with the step -2/64*ln_f(theta),
// row positions pos0 + row).
// nseq sequences (one launch, grid z) at strides sin (q/k/v) and sout (out)
// elements.
// Causal / full attention over [S][ld] rows (head h at columns 64 h), for
// nseq sequences at strides sin / sout. `work` holds
// attention_prefill_work_bytes(S, H, nseq) bytes (bf16 term planes of K and
// V); with rope, K is rotated there and Q as it is loaded (positions pos0 + row).
// With kc and vc (pos0 = 0) the rotated K rows and raw V rows are also written
// to a KV cache [nseq][H][hs][64] at positions 0 .. S-1. With qs.part, q, k and
// v point into slice 0 of k-slices (qs.ks slices qs.pst floats apart) and
// qs.scale holds the column scales of q's columns (k's and v's follow at
// k - q and v - q).
// Prompts of up to four 64-row blocks over a grid that fills the CUs
// (attention_prefill_one_launch) run as one launch from the f32 rows; `rope_tab`, if given, holds the rotation's
// (sin, cos) for positions pos0 + 0 .. S-1 and pair indices 0..31
// (launch_rope_table), read instead of evaluating the angles.
size_t attention_prefill_work_bytes(int S, int H, int nseq);
bool attention_prefill_one_launch(int S, int H, int nseq);
int launch_rope_table(float2 *tab, int S, float pos0, float rope_step, hipStream_t st);
int launch_attention_prefill(const float *q, const float *k, const float *v, float *out, int S,
                             int H, int ld, int ldo, float scale, bool causal, void *work,
                             hipStream_t st, bool rope = false, float rope_step = 0.0f,
                             float pos0 = 0.0f, int nseq = 1, size_t sin = 0, size_t sout = 0,
                             float *kc = nullptr, float *vc = nullptr, int hs = 0,
                             const Slices &qs = Slices{}, const float2 *rope_tab = nullptr);
struct DecodeArgs {
    const float *q, *k_new, *v_new;  // raw (unrotated) rows [B][ldq]
    int ldq;
    float *kc, *vc;  // [B][H][hs][64]
    int cap, H;
    int hs = 0;      // rows from one head's cache to the next (0: cap)
    const int *posp;  // device position (graph replay) or null -> `pos`
    int pos;
    float step, scale;  // RoPE step -2/64*ln_f(theta); score scale
    // optional: q/k/v as ks k-slice partials [ks][B][ldp] of the q/k/v
    // projection (q at column 0, k at H*64, v at 2*H*64) times wscale
    const float *part = nullptr;
    int ks = 0, ldp = 0;
    const float *wscale = nullptr;
    // 16-position sub-chunks per workgroup when the positions are split over
    // several workgroups per pair (then merged by a second kernel); 0: one
    // workgroup per pair; -1: chosen by the launcher. The result is the same
    // bits for every choice.
    int split = -1;
    // optional (one sequence, device or host position): the cached positions
    // split into `frac` ranges of about equal size, one workgroup each, which
    // merges its range in LDS and writes (max, sum, O[64]) as one partial
    // [B][H][frac][68] to fpart instead of the output; the consumer merges
    // the frac partials of a head in order (launch_fk_gemv's apart)
    int frac = 0;
    float *fpart = nullptr;
};
// `work` (attention_decode_work_floats() floats, 0 when the positions are
// not split) holds the sub-chunk partials of a split launch.
size_t attention_decode_work_floats(const DecodeArgs &a, int B);
int launch_attention_decode(const DecodeArgs &a, int B, float *out, int ldo, uint16_t *terms,
                            int T, int ldt, hipStream_t st, float *work = nullptr);

// B1 gather forward over source-major activations.
int launch_b1_forward(const float *w, const uint32_t *src, int n, int k0, const float *xt,
                      size_t t8, int n_tokens, float *yt, int mode, int act, hipStream_t st);
// T8 layers with a prepared plan (k0 <= 32, d <= 2032). A plan job rewrites
// one layer's (src, w) into b1_plan_bytes(n, k0) bytes at `plan`; the layer
// kernel reads activations addressed as (t / 16) * bs + s * rs + t % 16.
struct B1PlanJob {
    const float *w;
    const uint32_t *src;
    void *plan;
    int k0;
    uint32_t base = 0;  // added to every LDS offset of the plan (the stack's buffer)
};
constexpr int B1_PLAN_JOBS = 16;
struct B1PlanJobs {
    B1PlanJob job[B1_PLAN_JOBS];
};
bool b1_plan_ok(int n, int k0, int d);
size_t b1_plan_bytes(int n, int k0);
int launch_b1_plan(const B1PlanJobs &jobs, int njobs, int n, int d, hipStream_t st);
// Whole layer stack in one kernel (every layer n = d, k0 <= 32, d <= 5104):
// a workgroup carries 4 tokens through all layers with the activations in
// LDS. x and y are [T][d]; plans are prepared by launch_b1_stack.
bool b1_stack_ok(int d, const int *k0, int n_layers);
size_t b1_stack_plan_bytes(int d, const int *k0, int n_layers);
int launch_b1_stack(const B1PlanJob *layers, int n_layers, int d, const float *x, float *y,
                    int T, int act, void *plan, hipStream_t st);
// launch_b1_stack in two parts: the plan (once per topology) and the stack
// kernel over it.
int launch_b1_stack_plan(const B1PlanJob *layers, int n_layers, int d, void *plan, hipStream_t st);
int launch_b1_stack_run(const void *plan, const int *k0, int n_layers, int d, const float *x,
                        float *y, int T, int act, hipStream_t st);
int launch_b1_t8_plan_layer(const void *plan, int n, int k0, int d, const float *x, size_t xbs,
                            size_t xrs, int n_tokens, float *y, size_t ybs, size_t yrs, int act,
                            hipStream_t st);
int launch_transpose_t8(const float *x, size_t T, size_t d, float *xt, size_t t8,
                        hipStream_t st);
int launch_transpose_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                          size_t in_stride, hipStream_t st);

}  // namespace vmlm

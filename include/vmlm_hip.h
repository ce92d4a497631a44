/*
 * vmlm_hip.h -- C ABI of libvmlm_hip.so, the MI355X (gfx950) backend for the
 * inference hot path of VMLM (shouzugzs-AI/Sparrow).
 *
 * Plain C: pointers, sizes, status codes. No HIP or torch types cross this
 * boundary (streams travel as `void *`, a hipStream_t; NULL = the library's
 * own stream).
 *
 * Three layers:
 *  1. vmlm_*        Host-pointer kernels with the exact parameter lists of the
 *                   reference's vmlm-ops functions (cited per entry). They
 *                   copy in, run on the GPU, copy out and synchronise: a
 *                   drop-in for the Rust FFI crate that replaces
 *                   `vmlm_ops::kernels::*`.
 *  2. vmlm_hip_*    Device-pointer variants (same arguments + stream), async.
 *  3. vmlm_decoder_*, vmlm_b1_stack_*
 *                   Device-resident sessions for the MiniCPM-shaped decoder
 *                   program (tools/p12_build_minicpm.py, p14_gen_build.py)
 *                   and the B1 layer stack (models/src/b1.rs:108-150).
 *
 * Error convention. The reference kernels never validate; the interpreter
 * validates and exits the process (core/src/interp.rs:2357-2376). Here every
 * entry point validates and returns a status code equal to the reference's
 * exit code, with a message from vmlm_hip_last_error():
 *   0 ok, 2 device/runtime failure, 5 unimplemented, 9 guard violation.
 * All entry points are thread-safe; host-pointer calls serialise.
 */
#ifndef VMLM_HIP_H
#define VMLM_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VMLM_OK 0
#define VMLM_ERR_DEVICE 2
#define VMLM_ERR_UNIMPL 5
#define VMLM_ERR_GUARD 9

/* Activation kinds and elementwise opcodes: core/src/format.rs:98-103,
 * tensor/src/act_op.rs:9-12 (same numeric values). */
#define VMLM_ACT_RELU 0
#define VMLM_ACT_GELU 1
#define VMLM_ACT_SILU 2
#define VMLM_ACT_SIGMOID 3
#define VMLM_ACT_TANH 4
#define VMLM_ACT_RELU2 5
#define VMLM_OP_EWADD 20
#define VMLM_OP_EWMUL 21
#define VMLM_OP_EWSUB 22
#define VMLM_OP_EWDIV 23

/* ---------------------------------------------------------------- library */
int vmlm_hip_init(int device);         /* optional; first call does it */
const char *vmlm_hip_last_error(void); /* message of the last non-zero status */
const char *vmlm_hip_version(void);
int vmlm_hip_sync(void);               /* wait for the library stream */
int vmlm_hip_malloc(void **dptr, size_t bytes);
int vmlm_hip_free(void *dptr);
int vmlm_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int vmlm_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
/* device -> device on the library stream (synchronous); also the plain copy
 * of known size that calibrates the HBM traffic counters */
int vmlm_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int vmlm_hip_memset(void *dptr, int value, size_t bytes);
/* Event timing on a stream (NULL = library stream): returns an opaque id. */
int vmlm_hip_event_record(void *stream, int *event_id);
int vmlm_hip_event_elapsed_ms(int start_id, int end_id, float *ms);
int vmlm_hip_event_release_all(void);
/* Stream capture of device-API calls into a HIP graph (for replaying a fixed
 * sequence of ops without host launch cost). capture_end fails, with the
 * capture discarded, when the captured work holds anything but kernel
 * launches (a memset, a copy or an allocation), so only kernel-only
 * sequences are ever replayed. The calls must have run once on the stream
 * before (their workspace is then in place). (No reference counterpart: the
 * reference dispatches each op from its interpreter loop.) */
int vmlm_hip_capture_begin(void *stream);
int vmlm_hip_capture_end(void *stream, void **graph);
int vmlm_hip_graph_launch(void *graph, void *stream);
int vmlm_hip_graph_destroy(void *graph);

/* B1 connection block, field for field ops/src/conn.rs:8-53 SparseConnW
 * (the Rust struct is not repr(C); the FFI shim fills this one). The GPU
 * kernels read `w` and `src_u32`; `src` / `act` are not read. */
typedef struct vmlm_sparse_conn_w {
    size_t e;
    size_t k0;
    uint32_t layer;
    uint32_t n_neurons;
    float *w;
    float *src;
    uint32_t *src_u32;
    float *act;
} vmlm_sparse_conn_w;

/* ================================================================ layer 1
 * Host pointers, synchronous. Each replaces the vmlm-ops function cited. */

/* ops/src/kernels.rs:1258 gemm_nt_int8(a,q,scale,c,m,n,k):
 * C[m,n] = (A[m,k] . Q[n,k]^T) * scale[n], overwrite. */
int vmlm_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c,
                      size_t m, size_t n, size_t k);
/* ops/src/kernels.rs:1202 gemm_nt_bf16(a,b,c,m,n,k): C = A . B^T, B bf16 [n,k]. */
int vmlm_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                      size_t k);
/* ops/src/kernels.rs:987 gemm_nt(a,b,c,m,n,k,acc): C (+)= A[m,k] . B[n,k]^T. */
int vmlm_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                 bool acc);
/* ops/src/kernels.rs:407 gemm(a,b,c,m,n,k,acc): C (+)= A[m,k] . B[k,n]. */
int vmlm_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
              bool acc);
/* ops/src/kernels.rs:1346 rmsnorm(dst,src,g,rows,cols,eps). */
int vmlm_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                 float eps);
/* ops/src/kernels.rs:1389 softmax(p,rows,cols,causal), in place. */
int vmlm_softmax(float *p, size_t rows, size_t cols, bool causal);
/* ops/src/kernels.rs:1146 act_avx2(dst,n,kind), in place. */
int vmlm_act(float *dst, size_t n, uint16_t kind);
/* ops/src/kernels.rs:1117 ew_op(dst,x,y,n,op). */
int vmlm_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op);
/* core/src/interp.rs:1225-1235 OP_SCALE: dst = src * s. */
int vmlm_scale(float *dst, const float *src, size_t n, float s);
/* core/src/interp.rs:1159-1223 OP_ROPE over [rows, hd], positions pos0+row;
 * dst may equal src. */
int vmlm_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
              uint16_t pos0);
/* core/src/interp.rs:1351-1436 OP_EMB: one row of a bf16 / f32 table. */
int vmlm_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols, float rowf);
int vmlm_emb_f32(float *dst, const float *table, size_t rows, size_t cols, float rowf);
/* core/src/interp.rs:1649-1681 OP_TOPK_IDX: argmax of row 0 as f32. */
int vmlm_topk_idx(const float *src, size_t rows, size_t cols, float *dst);
/* ops/src/b1_pure.rs:151 b1_forward(sc,x,y) -> macs. */
int vmlm_b1_forward(const vmlm_sparse_conn_w *sc, const float *x, float *y, size_t *macs);
/* ops/src/b1_pure.rs:271 b1_forward_t8(sc,xt,t8,n_tokens,yt) -> macs. */
int vmlm_b1_forward_t8(const vmlm_sparse_conn_w *sc, const float *xt, size_t t8,
                       size_t n_tokens, float *yt, size_t *macs);
/* ops/src/b1_pure.rs:642 b1_backward(sc,dy,x,dw) -> macs: dw[i,j] +=
 * dy[i] * x[src[i,j]] over the f32 ids `sc->src`. */
int vmlm_b1_backward(const vmlm_sparse_conn_w *sc, const float *dy, const float *x, float *dw,
                     size_t *macs);
/* ops/src/b1_pure.rs:410 b1_backward_dx(sc,dy,dx) -> accs: dx[src[i,j]] +=
 * dy[i] * w[i,j], i and j ascending (bitwise). */
int vmlm_b1_backward_dx(const vmlm_sparse_conn_w *sc, const float *dy, float *dx, size_t *accs);
/* ops/src/b1_pure.rs:466 b1_backward_fused(sc,dy,x,dw,dx) -> n*k0: both of
 * the above over `src_u32` (ops/src/kernels.rs:2401 fused kernel). */
int vmlm_b1_backward_fused(const vmlm_sparse_conn_w *sc, const float *dy, const float *x,
                           float *dw, float *dx, size_t *conns);
/* ops/src/kernels.rs:3229 b1_backward_t8_avx2(w,src_u32,xt,dyt,t8,n,k0,dxt,dw):
 * source-major activations [n][t8] (t8 % 8 == 0); dxt and dw accumulate. */
int vmlm_b1_backward_t8(const float *w, const uint32_t *src_u32, const float *xt,
                        const float *dyt, size_t t8, size_t n, size_t k0, float *dxt,
                        float *dw);
/* ops/src/kernels.rs:1881 transpose_t8_avx2(x,t,d,xt,t8). */
int vmlm_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8);
/* ops/src/kernels.rs:3307 transpose_t8_back_avx2(a,rows,cols,out,os,in_stride). */
int vmlm_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                           size_t in_stride);
/* ops/src/kernels.rs:1308 layernorm(x,g,b,rows,cols,eps), in place. */
int vmlm_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                   float eps);
/* ops/src/kernels.rs:1436 outer(s,v,k,m,n,sc): S[i,j] += v[i] * sc * k[j]. */
int vmlm_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc);
/* ops/src/kernels.rs:1058-1065 jit_bias's body: d[i,j] += b[j]. */
int vmlm_bias(float *d, const float *b, size_t rows, size_t cols);

/* The JIT glue's entry points (ops/src/kernels.rs:1017-1113), host pointers,
 * with the reference's packed dims; they return the status the reference's
 * extern "system" functions cannot. jit_print / jit_unimpl / jit_memcpy are
 * host utilities (stdout, abort, memcpy), not kernels, and are not here. */
/* :1017-1033 jit_gemm_nt(a,b,c,dims), dims = m | n<<16 | k<<32 | acc<<48. */
int vmlm_jit_gemm_nt(const float *a, const float *b, float *c, uint64_t dims);
/* :1036 jit_act(p,n,kind). */
int vmlm_jit_act(float *p, size_t n, uint64_t kind);
/* :1041-1056 jit_ewadd / ewmul / ewsub / ewdiv(d,x,y,n). */
int vmlm_jit_ewadd(float *d, const float *x, const float *y, size_t n);
int vmlm_jit_ewmul(float *d, const float *x, const float *y, size_t n);
int vmlm_jit_ewsub(float *d, const float *x, const float *y, size_t n);
int vmlm_jit_ewdiv(float *d, const float *x, const float *y, size_t n);
/* :1058 jit_bias(d,b,rows,cols). */
int vmlm_jit_bias(float *d, const float *b, size_t rows, size_t cols);
/* :1068 jit_ln(x,g,b,dims,pad), dims = m | c<<32, eps 1e-5, in place. */
int vmlm_jit_ln(float *x, const float *g, const float *b, uint64_t dims, uint64_t pad);
/* :1081 jit_softmax(p,dims,causal), dims = m | c<<32. */
int vmlm_jit_softmax(float *p, uint64_t dims, uint64_t causal);
/* :1088 jit_outer(s,v,k,dims), dims = m | n<<32, scale 1. */
int vmlm_jit_outer(float *s, const float *v, const float *k, uint64_t dims);

/* Attention as tools/p12_build_minicpm.py:770-781 composes it (SLICE, ROPE,
 * GEMM NT, SCALE, SOFTMAX causal, GEMM NN, WRITECOL), fused.
 * q,k,v,out: [S, n_heads*head_dim] f32. */
int vmlm_attention_prefill(const float *q, const float *k, const float *v, float *out,
                           size_t S, size_t n_heads, size_t head_dim, float theta,
                           uint16_t pos0, float scale, bool causal);
/* One decode token (tools/p12_build_minicpm.py:941-967): rotate k_new at
 * `pos` and append it with v_new to the caches ([n_heads][cap][head_dim]
 * f32, updated in place), then attend q (rotated at pos) over [0, pos]. */
int vmlm_attention_decode(const float *q, const float *k_new, const float *v_new,
                          float *kcache, float *vcache, float *out, size_t n_heads,
                          size_t head_dim, size_t cap, size_t pos, float theta,
                          float scale);
/* The same decode with the cached positions split over workgroups of
 * `split` 16-position sub-chunks (0: one workgroup per head; -1: chosen by
 * the library). No counterpart in the reference (a tuning choice); every
 * split gives the same bits, since the sub-chunk partials are merged in
 * position order whichever workgroup computed them. */
int vmlm_attention_decode_split(const float *q, const float *k_new, const float *v_new,
                                float *kcache, float *vcache, float *out, size_t n_heads,
                                size_t head_dim, size_t cap, size_t pos, float theta,
                                float scale, int split);

/* ================================================================ layer 2
 * Device pointers, asynchronous on `stream`. Same semantics as layer 1. */
int vmlm_hip_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c,
                          size_t m, size_t n, size_t k, void *stream);
/* The same GEMM with no device allocation: no counterpart in the
 * reference. For callers that cannot allocate (HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Its temporaries (k-slice
 * partials, int8 rows, a padded weight copy) live in one fixed 16 MiB
 * array per GPU, set up by vmlm_hip_init (which must have run; this call
 * never initialises the library). A shape whose temporaries exceed it
 * returns 9 before launching anything (M <= 16 at the decoder's shapes and
 * small prefills fit; M = 16 over N = 5760, K = 2304 needs 3.3 MB). All
 * calls on one GPU share the array: calls that overlap in time (two
 * streams, two threads) race and must be serialised by the caller. */
int vmlm_hip_gemm_nt_int8_noalloc(const float *a, const int8_t *q, const float *scale, float *c,
                                  size_t m, size_t n, size_t k, void *stream);
int vmlm_hip_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                          size_t k, void *stream);
/* bf16 x bf16 -> f32 (the dense training shape): C = A[m,k] . B[n,k]^T. */
int vmlm_hip_gemm_nt_bf16bf16(const uint16_t *a, const uint16_t *b, float *c, size_t m,
                              size_t n, size_t k, void *stream);
int vmlm_hip_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n,
                     size_t k, bool acc, void *stream);
int vmlm_hip_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                  bool acc, void *stream);
int vmlm_hip_rmsnorm(float *dst, const float *src, const float *g, size_t rows,
                     size_t cols, float eps, void *stream);
int vmlm_hip_softmax(float *p, size_t rows, size_t cols, bool causal, void *stream);
int vmlm_hip_act(float *dst, size_t n, uint16_t kind, void *stream);
int vmlm_hip_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op,
                   void *stream);
int vmlm_hip_scale(float *dst, const float *src, size_t n, float s, void *stream);
int vmlm_hip_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
                  uint16_t pos0, void *stream);
/* Row index guards are checked on the device; a violation is reported by
 * the next vmlm_hip_check_guards() as status 9. */
int vmlm_hip_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols,
                      const float *rowf, void *stream);
int vmlm_hip_topk_idx(const float *src, size_t rows, size_t cols, float *dst, void *stream);
int vmlm_hip_check_guards(void);
int vmlm_hip_b1_forward(const vmlm_sparse_conn_w *sc, const float *x, float *y,
                        size_t n_tokens, void *stream);
int vmlm_hip_b1_forward_t8(const vmlm_sparse_conn_w *sc, const float *xt, size_t t8,
                           size_t n_tokens, float *yt, void *stream);
int vmlm_hip_b1_backward_fused(const vmlm_sparse_conn_w *sc, const float *dy, const float *x,
                               float *dw, float *dx, void *stream);
int vmlm_hip_b1_backward_t8(const float *w, const uint32_t *src_u32, const float *xt,
                            const float *dyt, size_t t8, size_t n, size_t k0, float *dxt,
                            float *dw, void *stream);
int vmlm_hip_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8,
                          void *stream);
int vmlm_hip_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out,
                               size_t os, size_t in_stride, void *stream);
int vmlm_hip_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                       float eps, void *stream);
int vmlm_hip_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc,
                   void *stream);
int vmlm_hip_bias(float *d, const float *b, size_t rows, size_t cols, void *stream);
int vmlm_hip_attention_prefill(const float *q, const float *k, const float *v, float *out,
                               size_t S, size_t n_heads, size_t head_dim, float theta,
                               uint16_t pos0, float scale, bool causal, void *stream);
int vmlm_hip_attention_decode(const float *q, const float *k_new, const float *v_new,
                              float *kcache, float *vcache, float *out, size_t n_heads,
                              size_t head_dim, size_t cap, size_t pos, float theta,
                              float scale, void *stream);
int vmlm_hip_attention_decode_split(const float *q, const float *k_new, const float *v_new,
                                    float *kcache, float *vcache, float *out, size_t n_heads,
                                    size_t head_dim, size_t cap, size_t pos, float theta,
                                    float scale, int split, void *stream);

/* ================================================================ layer 3 */

/* MiniCPM-shaped decoder session (config: MHA, SiLU-gated MLP, int8 weights
 * with per-output-row f32 scales, bf16 embedding and LM head). Weights and
 * the f32 KV cache ([layer][seq][head][cap][head_dim]) live in HBM. */
typedef struct vmlm_decoder_cfg {
    uint32_t n_layers, hidden, n_heads, head_dim, inter, vocab;
    uint32_t batch; /* independent sequences decoded together */
    uint32_t cap;   /* KV capacity in positions */
    float eps, theta, attn_scale;
} vmlm_decoder_cfg;
typedef struct vmlm_decoder vmlm_decoder;

int vmlm_decoder_create(const vmlm_decoder_cfg *cfg, vmlm_decoder **out);
int vmlm_decoder_destroy(vmlm_decoder *dec);
/* Host weights of one layer, [N,K] row-major, as the program's constants
 * L{l}_{q,k,v,o,gate,up,down} with their _sc scales and the two norms. */
int vmlm_decoder_load_layer(vmlm_decoder *dec, uint32_t layer, const int8_t *wq,
                            const float *sq, const int8_t *wk, const float *sk,
                            const int8_t *wv, const float *sv, const int8_t *wo,
                            const float *so, const int8_t *wg, const float *sg,
                            const int8_t *wu, const float *su, const int8_t *wd,
                            const float *sd, const float *in_ln, const float *post_ln);
int vmlm_decoder_load_globals(vmlm_decoder *dec, const uint16_t *embed,
                              const uint16_t *lm_head, const float *final_norm);
/* Prefill `S` prompt tokens per sequence (tokens [batch][S]); writes the
 * greedy first token of each sequence (argmax of row S-1) and optionally the
 * row-(S-1) logits [batch][vocab]. Resets the session position to S. */
int vmlm_decoder_prefill(vmlm_decoder *dec, const int32_t *tokens, uint32_t S,
                         int32_t *first_tokens, float *logits_last);
/* `n_steps` greedy decode steps (p14_gen_build.py:470-560): each step feeds
 * the previous argmax, appends to the KV cache and takes the argmax of the
 * new logits. tokens_out [n_steps][batch] (optional), logits_last
 * [batch][vocab] of the final step (optional). */
int vmlm_decoder_decode(vmlm_decoder *dec, uint32_t n_steps, int32_t *tokens_out,
                        float *logits_last);
int vmlm_decoder_position(const vmlm_decoder *dec, uint32_t *pos);
/* 1 = replay one captured HIP graph per step (default), 0 = launch eagerly. */
int vmlm_decoder_set_graph(vmlm_decoder *dec, int enable);
void *vmlm_decoder_stream(vmlm_decoder *dec);
/* Layer program of the decode step. Batches of at most 5 sequences default
 * to the fused layer (five launches: RMSNorm fused into the q/k/v and
 * gate/up projections, the residual adds into o and down, SiLU * up into
 * gate/up; full-K GEMVs over weights kept a second time in MFMA-operand
 * order); larger batches use k-slice GEMVs with separate reduction kernels
 * (eight launches). 0 selects the k-slice program at any batch. (No
 * reference counterpart: the reference runs one opcode per instruction.) */
int vmlm_decoder_set_fused(vmlm_decoder *dec, int enable);
int vmlm_decoder_fused(const vmlm_decoder *dec);
/* The layer program by number: VMLM_DECODER_KSLICE (k-slice GEMVs, eight
 * launches per layer), VMLM_DECODER_FUSED (batch <= 5, five launches) or
 * VMLM_DECODER_FULLK (batch <= 16, hidden 768, 1536 or 2304: q/k/v and gate/up over the
 * whole K in one launch each, SiLU * up in the gate/up epilogue, seven
 * launches). A new session takes the fused program where it fits, else the
 * full-K one, else the k-slice one. All give the same greedy tokens within
 * the 1e-4 x RMS contract of their logits. (No reference counterpart.) */
#define VMLM_DECODER_KSLICE 0
#define VMLM_DECODER_FUSED 1
#define VMLM_DECODER_FULLK 2
int vmlm_decoder_set_program(vmlm_decoder *dec, int program);
int vmlm_decoder_program(const vmlm_decoder *dec);
/* Times `iters` launches of one decode-step GEMV of every layer in turn
 * (which: 0 qkv, 1 o, 2 gate/up, 3 down, 4 LM head; on the k-slice and
 * full-K programs also 5, 6, 7: the o, gate/up or down projection followed
 * by the kernel that reduces its k-slice partials (the full-K gate/up needs
 * none); 8..11: a plain streaming read of the q/k/v, o, gate/up or down
 * weights, the single-launch floor of those bytes; 12: the decode
 * attention; 13: an empty kernel; 14, 15 (full-K program): the q/k/v
 * projection at four tiles per workgroup, the gate/up projection at one
 * tile pair per workgroup) captured into
 * one HIP graph on the session stream; writes the mean per-launch (or
 * per-pair) duration of a replay (HIP events, launch gaps included) and the
 * algorithmic HBM bytes (weights + scales + activations in + outputs; on the
 * fused path also the norm gain or the residual rows; 8..11 the weight
 * bytes; 12 the K and V rows read). */
int vmlm_decoder_time_gemv(vmlm_decoder *dec, int which, uint32_t iters, float *avg_us,
                           double *bytes_per_launch);

/* B1 layer stack (models/src/b1.rs:108-150 with the t8 contract of
 * ops/src/b1_pure.rs:271): y = act(gather-dot) per layer over source-major
 * activations. act: VMLM_ACT_* or 0xFFFF for none. */
int vmlm_b1_stack_forward(const vmlm_sparse_conn_w *layers, uint32_t n_layers,
                          const float *x, float *y, size_t n_tokens, uint16_t act,
                          void *stream);
/* The same stack with its connection plan built once (no reference
 * counterpart: the reference re-reads the SparseConnW arrays on every
 * forward). create validates the layers as vmlm_b1_stack_forward does,
 * prepares the plan from the current weights and indices on `stream` and
 * waits for it (later changes to the arrays need a new plan; stacks the
 * one-kernel path does not cover return 5). run is one kernel launch with
 * no allocation, so it can be captured into a graph. */
typedef struct vmlm_b1_stack vmlm_b1_stack;
int vmlm_b1_stack_create(const vmlm_sparse_conn_w *layers, uint32_t n_layers, void *stream,
                         vmlm_b1_stack **out);
int vmlm_b1_stack_run(vmlm_b1_stack *stack, const float *x, float *y, size_t n_tokens,
                      uint16_t act, void *stream);
int vmlm_b1_stack_destroy(vmlm_b1_stack *stack);

/* ================================================================ VM
 * Device-resident executor of .vmb programs: core/src/interp.rs Vm::load /
 * load_weights_mapped (:108-236) and Vm::run (:720-2370), with the constant
 * pool uploaded to the GPU once (read-only there), the activation / state /
 * gradient arenas in HBM (64-byte aligned, zeroed) and every opcode
 * dispatched to this library's kernels by slot address. Status codes are
 * the interpreter's exit codes (9 guard, 5 unimplemented op, 6 training op,
 * 3 bad magic, 7 slot not found, 8 EW shape mismatch, 2 device failure).
 * Extensions (no reference counterpart): bit 6 of `fl` reads the ROPE
 * position and the WRITECOL column from slot `dt`, and the SOFTMAX live
 * width from slot `b`, at run time. */
typedef struct vmlm_vm vmlm_vm;
/* Loads `image` (.vmb bytes). `weights` (optional) is the constant region
 * of a mapped weights file (load_weights_mapped): VMs loaded over the same
 * (weights, weights_len) share one device copy, uploaded once; the caller
 * keeps that memory unchanged while they live. Without it the image's own
 * CONST region is uploaded for this VM. The audit of audit_const_dtypes
 * (:241-348) runs here (9). */
int vmlm_vm_load(const void *image, size_t len, const void *weights, size_t weights_len,
                 vmlm_vm **out);
int vmlm_vm_destroy(vmlm_vm *vm);
/* Runs TEXT from instruction 0 to HALT (or its end); synchronous. */
int vmlm_vm_run(vmlm_vm *vm);
/* Slot lookup by name (FNV-1a hash, core/src/interp.rs:410-418 find_slot). */
int vmlm_vm_find_slot(const vmlm_vm *vm, const char *name, uint32_t *slot);
/* Device address (layer base applied), shape and dtype of a slot. */
int vmlm_vm_slot_info(vmlm_vm *vm, uint32_t slot, void **dptr, uint32_t *rows, uint32_t *cols,
                      uint8_t *dtype);
/* Copies f32 values into / out of an activation, state or gradient slot
 * (the runtime's token files: st_tok, st_gen). */
int vmlm_vm_write_slot(vmlm_vm *vm, uint32_t slot, const float *host, size_t count);
int vmlm_vm_read_slot(vmlm_vm *vm, uint32_t slot, float *host, size_t count);
/* Values PRINTed so far (all runs): *count of them, the first `cap` copied. */
int vmlm_vm_output(vmlm_vm *vm, float *host, size_t cap, size_t *count);
int vmlm_vm_clear_output(vmlm_vm *vm);
void *vmlm_vm_stream(vmlm_vm *vm);
/* Constant pools uploaded by this process so far (shared pools count once). */
int vmlm_vm_pool_uploads(size_t *n);
/* int8 constants this VM also holds in the swizzled MFMA layout (made once
 * per pool at load, read by OP_GEMM instead of the row-major bytes). No
 * counterpart in the reference (a layout of this build); for diagnostics
 * and tests. */
int vmlm_vm_swizzled_consts(const vmlm_vm *vm, size_t *n);
/* Opcode runs that this VM executes as one launch each (or, for a
 * prompt's column-by-column cache writes, two strided copies per stream),
 * found at load: the decode loop's per-head cache append and attention of
 * all heads of a layer, int8 GEMMs of one input at decode rows (with the
 * RMSNORM before them, the ACT and EWMUL of a gate/up pair, or the residual
 * EWADD after one GEMM), and column-by-column cache writes. No counterpart
 * in the reference (an execution strategy of this build: the interpreter
 * runs them opcode by opcode with the same results); for diagnostics and
 * tests. vmlm_vm_fused_opcodes gives the number of opcodes those runs
 * cover. */
int vmlm_vm_fused_runs(const vmlm_vm *vm, size_t *n);
int vmlm_vm_fused_opcodes(const vmlm_vm *vm, size_t *n);
/* LOOP_CNT bodies, from the jump target up to the first opcode that needs
 * the host between steps (PRINT, the counter, jumps, LAYERB, LN_EPS), run
 * opcode by opcode on their first visit, are captured into a HIP graph on
 * the second and replayed after (at the layer base they were captured at).
 * on = 0 runs every body opcode by opcode; the results are the same bits.
 * graph_segments counts the bodies replayed as graphs. No counterpart in the
 * reference (an execution strategy of this build). */
int vmlm_vm_set_graphs(vmlm_vm *vm, int on);
int vmlm_vm_graph_segments(const vmlm_vm *vm, size_t *n);

/* ================================================================ tables */

/* sys/src/lib.rs:29-38 `#[repr(C)] struct Backend`, field for field: the
 * reference's cross-language backend form. The functions keep the
 * reference's signatures (no status return): pointers may be device memory
 * (used in place) or host memory (staged through the library's workspace);
 * each call is synchronous. On failure the value-returning functions return
 * NaN, the others leave their output untouched, and vmlm_hip_last_error()
 * holds the message. dot256 / sum256 are tree sums within f32 rounding of
 * the reference's 8-lane chains; the others are bitwise
 * (sys/src/x86_avx2/simd.rs:27-405). */
typedef struct vmlm_backend_t {
    const char *name; /* "hip_gfx950" */
    float (*dot256)(const float *a, const float *b, size_t n);
    void (*axpy256)(float *y, const float *x, float a, size_t n);
    void (*add256)(float *y, const float *x, size_t n);
    float (*max256)(const float *x, size_t n);
    float (*sum256)(const float *x, size_t n);
    void (*scale_mul)(float *dst, const float *src, float a, size_t n);
} vmlm_backend_t;
const vmlm_backend_t *vmlm_hip_backend(void);
/* sys/src/x86_avx2/simd.rs:32 dot256_f32: sum of a[i] * b[i]. */
float vmlm_backend_dot256(const float *a, const float *b, size_t n);
/* :76 axpy256_f32: y[i] += a * x[i] (fused on 8-blocks, mul + add on the tail). */
void vmlm_backend_axpy256(float *y, const float *x, float a, size_t n);
/* :175 add256_f32: y[i] += x[i]. */
void vmlm_backend_add256(float *y, const float *x, size_t n);
/* :207 max256_f32: max over x (MAXPS lanes, -inf when empty). */
float vmlm_backend_max256(const float *x, size_t n);
/* :386 sum256_f32: sum of x. */
float vmlm_backend_sum256(const float *x, size_t n);
/* :353 scale_mul_avx2: dst[i] = a * src[i]. */
void vmlm_backend_scale_mul(float *dst, const float *src, float a, size_t n);

/* The kernel-level table of this library (host-pointer entry points of
 * layer 1); no reference counterpart. */
typedef struct vmlm_hip_kernel_table_t {
    const char *name;
    int (*gemm_nt_int8)(const float *, const int8_t *, const float *, float *, size_t,
                        size_t, size_t);
    int (*gemm_nt_bf16)(const float *, const uint16_t *, float *, size_t, size_t, size_t);
    int (*gemm_nt)(const float *, const float *, float *, size_t, size_t, size_t, bool);
    int (*gemm)(const float *, const float *, float *, size_t, size_t, size_t, bool);
    int (*rmsnorm)(float *, const float *, const float *, size_t, size_t, float);
    int (*softmax)(float *, size_t, size_t, bool);
    int (*act)(float *, size_t, uint16_t);
    int (*ew_op)(float *, const float *, const float *, size_t, uint8_t);
    int (*b1_forward)(const vmlm_sparse_conn_w *, const float *, float *, size_t *);
    int (*b1_forward_t8)(const vmlm_sparse_conn_w *, const float *, size_t, size_t, float *,
                         size_t *);
} vmlm_hip_kernel_table_t;
const vmlm_hip_kernel_table_t *vmlm_hip_kernel_table(void);

#ifdef __cplusplus
}
#endif
#endif

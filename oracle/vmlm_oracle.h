/*
 * vmlm_oracle.h -- CPU restatement of the reference (shouzugzs-AI/Sparrow, "VMLM")
 * inference kernels, used ONLY as the parity checker of the HIP library.
 *
 * TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library. The product path (sparrow_amd,
 * libvmlm_hip.so) never calls it and fails loudly without its HIP build.
 *
 * Every function restates one reference function (file:line cited at its
 * definition in vmlm_oracle.c) with the SAME floating-point operation order:
 * the same lane structure, fold order, FMA-vs-mul+add choice and tails, so
 * that on identical inputs it returns the reference's bits. The library is
 * compiled with -ffp-contract=off; FMAs appear only as explicit fmaf() where
 * the reference uses _mm256_fmadd_ps.
 *
 * Row-parallel entry points use OpenMP over output rows/columns; each output
 * element's arithmetic is unchanged, so any thread count gives the bits of one
 * thread (the reference's par_for row split, ops/src/par.rs:30-64).
 */
#ifndef VMLM_ORACLE_H
#define VMLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- configuration ---- */
void vo_set_threads(int n);
int vo_get_threads(void);

/* ---- scalar math (sys/src/math/mod.rs, ops/src/kernels.rs) ---- */
float vo_round_f32(float v);
float vo_exp_f(float x);
float vo_ln_f(float x);
float vo_sin_f(float x);
float vo_cos_f(float x);
float vo_floor_f(float x);
float vo_tanh_f(float x);
float vo_sqrt_f(float x);
float vo_act_scalar(float x, uint16_t kind);
uint16_t vo_f32_to_bf16(float v);
float vo_bf16_to_f32(uint16_t h);
/* y[i] = f(x[i]) for f = 0 exp_f, 1 ln_f, 2 sin_f, 3 cos_f, 4 tanh_f,
 * 5 floor_f, 6 round_f32, 100+kind act_scalar(kind) -- sweep helper. */
void vo_map(int which, const float *x, float *y, size_t n);

/* ---- GEMM family (ops/src/kernels.rs) ---- */
void vo_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c,
                     size_t m, size_t n, size_t k);
void vo_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                     size_t k);
void vo_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                int acc);
void vo_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
             int acc);

/* ---- Backend primitives (sys/src/x86_avx2/simd.rs) and jit helpers ---- */
float vo_dot256(const float *a, const float *b, size_t n);
void vo_axpy256(float *y, const float *x, float a, size_t n);
void vo_add256(float *y, const float *x, size_t n);
float vo_max256(const float *x, size_t n);
float vo_sum256(const float *x, size_t n);
void vo_scale_mul(float *dst, const float *src, float a, size_t n);
void vo_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                  float eps);
void vo_bias(float *d, const float *b, size_t rows, size_t cols);
void vo_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc);

/* ---- row / elementwise ops ---- */
void vo_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                float eps);
void vo_softmax(float *p, size_t rows, size_t cols, int causal);
void vo_act(float *dst, size_t n, uint16_t kind);
void vo_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op);
void vo_scale(float *dst, const float *src, size_t n, float s);
/* returns 0, or 9 (the reference's guard exit code) */
int vo_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
            uint32_t pos0);
int vo_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols, float rowf);
int vo_emb_f32(float *dst, const float *table, size_t rows, size_t cols, float rowf);
int vo_topk_idx(const float *src, size_t rows, size_t cols, float *dst);

/* ---- B1 sparse connections (core/src/conn_sparse.rs, ops/src/kernels.rs, ops/src/b1_pure.rs) ---- */
uint32_t vo_neuron_seed(uint32_t layer, uint32_t i);
uint32_t vo_neuron_rand(uint32_t seed, uint32_t j);
uint32_t vo_neuron_conn_src(uint32_t layer, uint32_t i, uint32_t j, uint32_t n_neurons,
                            uint32_t k0);
float vo_b1_dot_row_u32(const float *wrow, const uint32_t *srcrow, const float *x,
                        size_t k0);
size_t vo_b1_forward(size_t n, size_t k0, const float *w, const uint32_t *src,
                     const float *x, float *y);
size_t vo_b1_forward_t8_scalar(const float *w, const uint32_t *src, size_t n, size_t k0,
                               const float *xt, size_t t8, size_t n_tokens, float *yt);
void vo_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8);
void vo_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                          size_t in_stride);

/* ---- attention as the VM program composes it (tools/p12_build_minicpm.py) ---- */
/* q,k,v,out: [S, H*hd] token-major, head h at columns h*hd..h*hd+hd. */
void vo_attention_prefill(const float *q, const float *k, const float *v, float *out,
                          size_t S, size_t H, size_t hd, float theta, uint32_t pos0,
                          float scale, int causal);
/* One decode token at absolute position `pos`: rotates k_new and appends it
 * (and raw v_new) to the caches at `pos`, then attends q (rotated at pos) over
 * positions [0, pos]. Caches: [H][cap][hd] f32. q,k_new,v_new,out: [H*hd]. */
void vo_attention_decode(const float *q, const float *k_new, const float *v_new,
                         float *kcache, float *vcache, float *out, size_t H, size_t hd,
                         size_t cap, size_t pos, float theta, float scale);

/* ---- MiniCPM-shaped decoder program (p12_build_minicpm.py / p14_gen_build.py) ---- */
typedef struct vo_layer {
    const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd; /* [N,K] row-major */
    const float *sq, *sk, *sv, *so, *sg, *su, *sd;  /* per-output-row scale [N] */
    const float *in_ln, *post_ln;                   /* [hidden] */
} vo_layer;

typedef struct vo_model {
    size_t n_layers, hidden, n_heads, head_dim, inter, vocab;
    float eps, theta, attn_scale;
    const vo_layer *layers;
    const uint16_t *embed;   /* [vocab, hidden] bf16 */
    const uint16_t *lm_head; /* [vocab, hidden] bf16 */
    const float *final_norm; /* [hidden] */
} vo_model;

/* KV caches: [n_layers][n_heads][cap][head_dim] f32, rotated K and raw V.
 * Prefill of S tokens at positions 0..S-1; logits_last: [vocab] (row S-1),
 * hidden_last (optional): final-normed hidden state of row S-1. */
int vo_decoder_prefill(const vo_model *md, float *kcache, float *vcache, size_t cap,
                       const int32_t *tokens, size_t S, float *logits_last,
                       float *hidden_last);
/* One decode step for `token` at absolute position `pos`. */
int vo_decoder_step(const vo_model *md, float *kcache, float *vcache, size_t cap,
                    int32_t token, size_t pos, float *logits, float *hidden);
/* Greedy chain: prefill, t0 = argmax(logits[S-1]), then n_steps steps; writes
 * n_steps+1 tokens [t0..t_n] and per-token top1-top2 logit margins. */
int vo_decoder_generate(const vo_model *md, float *kcache, float *vcache, size_t cap,
                        const int32_t *prompt, size_t S, size_t n_steps,
                        int32_t *out_tokens, float *margins);

/* ---- B1 backward (ops/src/b1_pure.rs, ops/src/kernels.rs) ---- */
size_t vo_b1_backward(size_t n, size_t k0, const float *srcf, const float *dy, const float *x,
                      float *dw);
size_t vo_b1_backward_dx(size_t n, size_t k0, const float *w, const uint32_t *src,
                         const float *dy, float *dx);
size_t vo_b1_backward_fused(size_t n, size_t k0, const float *w, const uint32_t *src,
                            const float *dy, const float *x, float *dw, float *dx);
void vo_b1_backward_t8(const float *w, const uint32_t *src, const float *xt, const float *dyt,
                       size_t t8, size_t n, size_t k0, float *dxt, float *dw);

/* ---- the VM (vmlm_vm_oracle.c): core/src/interp.rs load + run ---- */
typedef struct vo_vm vo_vm;
int vo_vm_load(const uint8_t *image, size_t len, vo_vm **out); /* exit code */
int vo_vm_run(vo_vm *vm);                                      /* exit code */
void vo_vm_free(vo_vm *vm);
int vo_vm_find(const vo_vm *vm, uint32_t hash, uint32_t *slot);
int vo_vm_slot(vo_vm *vm, uint32_t slot, float **p, uint32_t *rows, uint32_t *cols,
               uint8_t *dtype);
size_t vo_vm_output(const vo_vm *vm, float *dst, size_t cap);
const char *vo_vm_message(const vo_vm *vm);
const char *vo_vm_last_load_error(void);
void vo_vm_last_load_error_set(const char *m);

#ifdef __cplusplus
}
#endif
#endif

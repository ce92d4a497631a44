// sessions.hip -- device-resident sessions: the MiniCPM-shaped decoder program
// (tools/p12_build_minicpm.py:766-981 + tools/p14_gen_build.py:470-560) and
// the B1 layer stack (models/src/b1.rs:108-150).
//
// Decoder layout in HBM (one allocation each):
//   weights per layer  [Wqkv 3H x H | Wo H x H | Wgu 2I x H | Wd H x I] int8
//                      Wqkv = rows of q, k, v concatenated; Wgu interleaves
//                      16-row blocks of gate and up so one GEMV workgroup owns
//                      the gate and up rows of the same 16 outputs. Held once,
//                      swizzled into 1 KiB blocks of 16 rows x 64 k in MFMA
//                      operand order (launch_swizzle_w), which the decode
//                      GEMVs and the prefill GEMMs both read; the row-major
//                      form passes through a one-layer staging buffer at load.
//   scales per layer   [sqkv 3H | so H | sgu 2I (same interleave) | sd H] f32
//   norms per layer    [in_ln H | post_ln H] f32
//   KV cache           [layer][seq][head][cap][64] f32, rotated K and raw V
//                      (the program's [HD, PMAX] state slots, position-major so
//                      one lane streams one 256-byte row)
// A decode step is captured once as a HIP graph; the position and the greedy
// tokens live in device memory, so replays need no host round trip -- the
// same closed loop the reference runs inside one Vm::run.
#include <cstring>
#include <type_traits>
#include <utility>
#include <vector>

#include "internal.hpp"

namespace vmlm {

enum { PROG_KSLICE = 0, PROG_FUSED = 1, PROG_FULLK = 2 };

// Folds the LM head's argmax slots of each sequence into tok[b] (the
// TOPK_IDX result fed to the next step's EMB), clears the slots for the next
// step, and -- when `out` is given -- records tok into tokens_out[step] and
// advances step and position. One wavefront per sequence.
__global__ __launch_bounds__(64) void argmax_advance_kernel(
    unsigned long long *__restrict__ keys, int32_t *__restrict__ tok, int32_t *__restrict__ out,
    int B, int max_steps, int *step, int *pos, int *guard) {
    const int b = blockIdx.x, lane = threadIdx.x;
    unsigned long long k = keys[(size_t)b * KEY_SLOTS + lane];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long ok = __shfl_xor(k, o, 64);
        k = ok > k ? ok : k;
    }
    keys[(size_t)b * KEY_SLOTS + lane] = 0ull;
    if (lane != 0) return;
    const int32_t t = k ? argmax_key_index(k) : 0;  // all-NaN row: the scan keeps index 0
    tok[b] = t;
    if (!out) return;
    const int s = *step;
    if (s < max_steps) out[(size_t)s * B + b] = t;
    else atomicOr(guard, 2);
}

// Reads n16 16-byte pieces with nontemporal loads, eight per thread, all
// issued before any is used: the load pattern of the decode GEMVs without
// their arithmetic, i.e. the floor of one launch that streams the same
// bytes. The xor of the data goes to `sink` only if it hits a constant, so
// the loads stay and nothing is written in practice.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *__restrict__ src, size_t n16,
                                                          uint32_t *__restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * 2048 + threadIdx.x;
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const size_t idx = base + (size_t)i * 256;
        v[i] = idx < n16 ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    if (x == 0x9e3779b9u) sink[0] = x;
}

// An empty kernel: back to back in a graph, its launches measure the fixed
// cost every launch of the step pays before any work.
__global__ void empty_kernel() {}

__global__ void step_advance_kernel(int *step, int *pos) {
    *step = *step + 1;
    *pos = *pos + 1;
}

}  // namespace vmlm

using namespace vmlm;

struct vmlm_decoder {
    vmlm_decoder_cfg c{};
    hipStream_t st = nullptr;
    size_t H = 0, I = 0, NH = 0, V = 0, B = 0, cap = 0, L = 0;
    size_t w_layer = 0, s_layer = 0;  // per-layer element counts
    int8_t *wstage = nullptr;  // one layer's row-major weights, swizzled into wsw at load
    int8_t *wsw = nullptr;     // the weights in MFMA-operand order (every projection)
    float *ssp = nullptr;   // fused path: RMSNorm partial sums of squares [H/16][B]
    // layer program of the decode step: PROG_KSLICE (k-slice GEMVs and
    // reduction kernels, eight launches per layer), PROG_FUSED (batch <= 5:
    // five launches of full-K fused GEMVs) or PROG_FULLK (batch <= 16: full-K
    // int8 GEMVs for q/k/v and gate/up, seven launches)
    int prog = PROG_KSLICE;
    bool fused = false;     // prog == PROG_FUSED
    // full-K program: the normed rows as blocked int8 terms [Q8_T][H/64][1 KiB]
    int8_t *x8b = nullptr;
    int fq_tw = 2;     // 16-row tiles per workgroup of the full-K q/k/v projection
    int fq_tw_gu = 4;  // and of the gate/up projection (two gate/up tile pairs)
    float *s = nullptr, *norms = nullptr;
    uint16_t *embed = nullptr, *lm_head = nullptr;
    float *final_norm = nullptr;
    float *kc = nullptr, *vc = nullptr;
    // decode activations
    float *h = nullptr, *h2 = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr;
    float *logits = nullptr;
    uint16_t *t_x = nullptr, *t_att = nullptr, *t_act = nullptr;
    // k-slice program: the normed input as int8 terms of h * g [Q8_T][B][H],
    // by segments of the GEMVs' k window: factors and sums of squares [H/seg][B]
    int8_t *x8 = nullptr;
    float *x8s = nullptr, *x8ssp = nullptr;
    int seg = 0;
    // and the down projection's input silu(gate) * up: [Q8_T][B][I], factors
    // [I/seg_i][B]
    int8_t *act8 = nullptr;
    float *act8s = nullptr;
    int seg_i = 0;
    // fused program at batch 1: the attention's position-range partials per
    // head [NH][FK_APART][68], merged by the o projection
    float *apart = nullptr;
    int32_t *tok = nullptr, *tokens_out = nullptr;
    unsigned long long *keys = nullptr;  // [B][KEY_SLOTS] argmax slots
    float *part = nullptr;               // k-slice partial sums of the decode GEMVs
    int ks_h = 1, ks_i = 1;              // k-slices of the K=H and K=I projections
    int *pos = nullptr, *step = nullptr;
    float rope_step = 0.0f;
    uint32_t pos_host = 0, step_host = 0;
    // the prefill's workspace, kept between calls (grown for a longer prompt)
    void *pf = nullptr;
    size_t pf_bytes = 0;
    // host sources of the step / position reset copies (live as long as the session)
    int32_t reset_step = 0, reset_pos = 0;
    bool loaded_globals = false;
    std::vector<bool> loaded;
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
    std::vector<void *> allocs;

    // layer l's projections in the swizzled copy ([N/16][K/64][1 KiB] blocks)
    const int8_t *Wqkv(size_t l) const { return wsw + l * w_layer; }
    const int8_t *Wo(size_t l) const { return Wqkv(l) + 3 * H * H; }
    const int8_t *Wgu(size_t l) const { return Wo(l) + H * H; }
    const int8_t *Wd(size_t l) const { return Wgu(l) + 2 * I * H; }
    const float *Sqkv(size_t l) const { return s + l * s_layer; }
    const float *So(size_t l) const { return Sqkv(l) + 3 * H; }
    const float *Sgu(size_t l) const { return So(l) + H; }
    const float *Sd(size_t l) const { return Sgu(l) + 2 * I; }
    const float *InLn(size_t l) const { return norms + l * 2 * H; }
    const float *PostLn(size_t l) const { return InLn(l) + H; }
    // cache rows [L][B][NH][hs][64], hs = cap + 1: one spare row per head
    // staggers the heads' starting addresses over the HBM channels (a
    // 256 KiB-aligned head stride streamed 3-8 % slower in a probe)
    size_t hs = 0;
    float *Kc(size_t l) const { return kc + l * B * NH * hs * 64; }
    float *Vc(size_t l) const { return vc + l * B * NH * hs * 64; }
};

namespace {

template <typename T>
int dalloc(vmlm_decoder *d, T **p, size_t count) {
    void *q = nullptr;
    VMLM_HIP_CHECK(hipMalloc(&q, (count ? count : 1) * sizeof(T)));
    d->allocs.push_back(q);
    *p = (T *)q;
    return VMLM_OK;
}

// LM head over the final-normed terms in d->t_x with the argmax folded into
// its epilogue, then the argmax slots -> d->tok (and tokens_out when recording).
int enqueue_head(vmlm_decoder *d, bool record) {
    GemvArgs lm;
    lm.W = d->lm_head;
    lm.w_int8 = false;
    lm.A = d->t_x;
    lm.T = 3;
    lm.lda = (int)d->H;
    lm.M = (int)d->B;
    lm.N = (int)d->V;
    lm.K = (int)d->H;
    lm.Y = d->logits;
    lm.ldy = (int)d->V;
    lm.epi = EPI_ARGMAX;
    lm.keys = d->keys;
    lm.tiles = 9;  // 128 rows per workgroup over the full K, activation through LDS
    int rc = launch_gemv(lm, d->st);
    if (rc) return rc;
    argmax_advance_kernel<<<(unsigned)d->B, 64, 0, d->st>>>(
        d->keys, d->tok, record ? d->tokens_out : nullptr, (int)d->B, (int)d->cap, d->step,
        d->pos, guard_flag_ptr());
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// Decode GEMV of the step (k-slice program): raw slice sums to d->part from
// the swizzled weights; the consumer (attention, residual RMSNorm, SiLU)
// reduces them in slice order and applies the row scales.
KsArgs step_gemv(vmlm_decoder *d, const int8_t *W, const uint16_t *A, int N, int K) {
    KsArgs g;
    g.W = W;
    if (A == d->t_x) {  // the normed rows enter as int8 rows
        g.A8 = d->x8;
        g.a8s = d->x8s;
        g.ssp = d->x8ssp;
        g.eps = d->c.eps;
    } else if (A == d->t_act) {
        g.A8 = d->act8;
        g.a8s = d->act8s;
    } else {
        g.A = A;
    }
    g.lda = K;
    g.M = (int)d->B;
    g.N = N;
    g.K = K;
    g.Y = d->part;
    g.ldy = N;
    // launch shape (16-row tiles per wave, waves per workgroup), from a sweep
    // of 1..6 tiles x 2, 4, 8 waves at the MiniCPM-2B shapes, batch 16 (graph
    // replay over 40 layers' weights): q/k/v 2 x 8 (5.40 us; 2 x 4 5.36,
    // 4 x 4 5.64), gate/up 4 x 4 (7.90; 2 x 8 8.19), down 3 x 4 (5.46; 2 x 8
    // 6.08, 4 x 4 5.86), o 2 x 4. Swept again with the tiles stored one at a
    // time: q/k/v 4 x 4 5.07-5.09 (2 x 8 5.18-5.20, 2 x 4 5.20, 1 x 8 5.58),
    // gate/up 4 x 4 7.79-7.99 (2 x 8 8.00, 3 x 4 8.47), down 3 x 4 4.72
    // (2 x 8 5.26, 4 x 4 5.25)
    if (g.A8) {
        const bool wide = N >= 4 * K, deep = K > N;
        g.tw = wide ? 4 : deep ? 3 : 4;
        g.nwv = 4;
    } else {
        g.tw = 2;
        g.nwv = K > (int)d->H ? 8 : 4;
    }
    return g;
}

// Decode attention of layer l at the device position: q/k/v as the q/k/v
// projection's k-slice partials (k-slice program) or as final rows (fused
// and full-K programs).
DecodeArgs attn_args(vmlm_decoder *d, size_t l) {
    const int H = (int)d->H;
    DecodeArgs a;
    a.q = a.k_new = a.v_new = nullptr;
    if (d->prog != PROG_KSLICE) {
        a.q = d->qkv;
        a.k_new = d->qkv + H;
        a.v_new = d->qkv + 2 * H;
        if (d->fused && d->B == 1 && fk_apart_ok(H)) {  // FK_APART workgroups per head, merged by the o projection
            a.frac = FK_APART;
            a.fpart = d->apart;
        }
    } else {
        a.part = d->part;
        a.ks = d->ks_h;
        a.ldp = 3 * H;
        a.wscale = d->Sqkv(l);
    }
    a.ldq = 3 * H;
    a.kc = d->Kc(l);
    a.vc = d->Vc(l);
    a.hs = (int)d->hs;
    a.cap = (int)d->cap;
    a.H = (int)d->NH;
    a.posp = d->pos;
    a.pos = 0;
    a.step = d->rope_step;
    a.scale = d->c.attn_scale;
    return a;
}

// One decode step over the B sequences (all launches on d->st). Layer l's
// input norm is produced by the previous layer's closing residual RMSNorm.
int enqueue_step(vmlm_decoder *d) {
    hipStream_t st = d->st;
    const int B = (int)d->B, H = (int)d->H, I = (int)d->I;
    const int T = 3;
    int rc = launch_emb_bf16(d->h, H, d->embed, d->V, H, nullptr, d->tok, B, st);
    if (rc) return rc;
    if ((rc = launch_resid_q8(d->h, nullptr, 0, 0, nullptr, nullptr, d->InLn(0), B, H, d->seg,
                              d->x8, d->x8s, d->x8ssp, st)))
        return rc;
    for (size_t l = 0; l < d->L; ++l) {
        if ((rc = launch_ks_gemv(step_gemv(d, d->Wqkv(l), d->t_x, 3 * H, H), st))) return rc;
        if ((rc = launch_attention_decode(attn_args(d, l), B, d->att, H, d->t_att, T, H, st)))
            return rc;
        if ((rc = launch_ks_gemv(step_gemv(d, d->Wo(l), d->t_att, H, H), st))) return rc;
        if ((rc = launch_resid_q8(d->h, d->part, d->ks_h, H, d->So(l), d->h2, d->PostLn(l), B, H,
                                  d->seg, d->x8, d->x8s, d->x8ssp, st)))
            return rc;
        if ((rc = launch_ks_gemv(step_gemv(d, d->Wgu(l), d->t_x, 2 * I, H), st))) return rc;
        if ((rc = launch_silu_q8(d->part, d->ks_h, 2 * I, d->Sgu(l), B, I, d->seg_i, d->act8,
                                 d->act8s, st)))
            return rc;
        if ((rc = launch_ks_gemv(step_gemv(d, d->Wd(l), d->t_act, H, I), st))) return rc;
        // the next layer's input as int8 rows; after the last layer the final
        // norm's bf16 terms for the LM head
        if (l + 1 < d->L)
            rc = launch_resid_q8(d->h2, d->part, d->ks_i, H, d->Sd(l), d->h, d->InLn(l + 1), B, H,
                                 d->seg, d->x8, d->x8s, d->x8ssp, st);
        else
            rc = launch_rmsnorm_resid(d->h2, d->part, d->ks_i, H, d->Sd(l), d->h, B, H,
                                      d->final_norm, d->c.eps, d->t_x, T, H, st);
        if (rc) return rc;
    }
    if ((rc = enqueue_head(d, true))) return rc;
    step_advance_kernel<<<1, 1, 0, st>>>(d->step, d->pos);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// The fused path's four projections of layer l (which: 0 q/k/v, 1 o, 2
// gate/up, 3 down). Residual rows stay f32 (h, h2); every projection input
// is a set of bf16 term planes: t_x (terms of x * g of the next RMSNorm, with
// the partial sums of squares in ssp), t_att (attention output) and t_act
// (SiLU(gate) * up).
FkArgs fk_args(vmlm_decoder *d, size_t l, int which) {
    const int H = (int)d->H, I = (int)d->I;
    FkArgs f;
    f.eps = d->c.eps;
    f.M = (int)d->B;
    f.nssp = H / 16;
    switch (which) {
    case 0:
        f.W = d->Wqkv(l), f.scale = d->Sqkv(l), f.N = 3 * H, f.K = H;
        f.A = d->t_x, f.ssp = d->ssp;
        f.Y = d->qkv, f.ldy = 3 * H, f.epi = FK_STORE;
        break;
    case 1:
        f.W = d->Wo(l), f.scale = d->So(l), f.N = H, f.K = H;
        f.A = d->t_att;
        if (d->B == 1 && fk_apart_ok(H)) f.apart = d->apart;  // the attention's range partials (attn_args)
        f.Y = d->h2, f.ldy = H, f.epi = FK_RESID, f.R = d->h, f.ldr = H;
        f.Aout = d->t_x, f.gout = d->PostLn(l), f.ssp_out = d->ssp;
        break;
    case 2:
        f.W = d->Wgu(l), f.scale = d->Sgu(l), f.N = 2 * I, f.K = H;
        f.A = d->t_x, f.ssp = d->ssp;
        f.ldy = I, f.epi = FK_SILU, f.Aout = d->t_act;
        break;
    default:
        f.W = d->Wd(l), f.scale = d->Sd(l), f.N = H, f.K = I;
        f.A = d->t_act;
        f.Y = d->h, f.ldy = H, f.epi = FK_RESID, f.R = d->h2, f.ldr = H;
        f.Aout = d->t_x, f.gout = l + 1 < d->L ? d->InLn(l + 1) : d->final_norm;
        f.ssp_out = d->ssp;
        break;
    }
    f.lda = f.K;
    return f;
}

// The same step with five launches per layer (batch <= 5): RMSNorm split
// between the residual epilogues and the q/k/v and gate/up projections,
// the residual adds in the o and down projections, SiLU * up in the gate/up
// epilogue; q, k, v reach the attention kernel as final rows.
int enqueue_step_fused(vmlm_decoder *d) {
    hipStream_t st = d->st;
    const int B = (int)d->B, H = (int)d->H;
    int rc = launch_emb_bf16(d->h, H, d->embed, d->V, H, nullptr, d->tok, B, st);
    if (rc) return rc;
    if ((rc = launch_fk_norm_prep(d->h, H, d->InLn(0), B, H, d->t_x, H, d->ssp, st))) return rc;
    for (size_t l = 0; l < d->L; ++l) {
        if ((rc = launch_fk_gemv(fk_args(d, l, 0), st))) return rc;
        if ((rc = launch_attention_decode(attn_args(d, l), B, d->att, H, d->t_att, 3, H, st)))
            return rc;
        for (int which = 1; which < 4; ++which)
            if ((rc = launch_fk_gemv(fk_args(d, l, which), st))) return rc;
    }
    if ((rc = launch_rmsnorm(nullptr, d->h, d->final_norm, B, H, d->c.eps, d->t_x, 3, H, st)))
        return rc;
    if ((rc = enqueue_head(d, true))) return rc;
    step_advance_kernel<<<1, 1, 0, st>>>(d->step, d->pos);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// The full-K projections of layer l (which: 0 q/k/v rows, 2 gate/up with
// SiLU * up) over the blocked int8 rows of the input norm.
FqArgs fq_args(vmlm_decoder *d, size_t l, int which) {
    const int H = (int)d->H, I = (int)d->I;
    FqArgs f;
    f.A8 = d->x8b;
    f.a8s = d->x8s;
    f.ssp = d->x8ssp;
    f.eps = d->c.eps;
    f.seg_kb = d->seg / 64;
    f.M = (int)d->B;
    f.K = H;
    if (which == 0) {
        f.W = d->Wqkv(l), f.scale = d->Sqkv(l), f.N = 3 * H;
        f.Y = d->qkv, f.ldy = 3 * H, f.epi = FQ_STORE, f.tw = d->fq_tw;
    } else {
        f.W = d->Wgu(l), f.scale = d->Sgu(l), f.N = 2 * I;
        f.Y = d->act, f.ldy = I, f.epi = FQ_SILU, f.tw = d->fq_tw_gu;
    }
    return f;
}

// The down projection of the full-K program: k-slice GEMV over the f32
// SiLU * up rows, each slice split into int8 terms while staged.
KsArgs fq_down(vmlm_decoder *d, size_t l) {
    KsArgs g;
    g.W = d->Wd(l);
    g.X = d->act;
    g.lda = (int)d->I;
    g.M = (int)d->B;
    g.N = (int)d->H;
    g.K = (int)d->I;
    g.Y = d->part;
    g.ldy = (int)d->H;
    g.tw = 3;
    g.nwv = 4;
    return g;
}

// Seven launches per layer (batch <= 16): the q/k/v and gate/up projections
// over the whole K in one launch each (q/k/v rows for the attention; SiLU *
// up in the gate/up epilogue), o and down as k-slice GEMVs whose partials the
// residual kernels reduce; the residual kernels write the next projection's
// input as blocked int8 rows.
int enqueue_step_fullk(vmlm_decoder *d) {
    hipStream_t st = d->st;
    const int B = (int)d->B, H = (int)d->H;
    int rc = launch_emb_bf16(d->h, H, d->embed, d->V, H, nullptr, d->tok, B, st);
    if (rc) return rc;
    if ((rc = launch_resid_q8(d->h, nullptr, 0, 0, nullptr, nullptr, d->InLn(0), B, H, d->seg,
                              d->x8b, d->x8s, d->x8ssp, st, true)))
        return rc;
    for (size_t l = 0; l < d->L; ++l) {
        if ((rc = launch_fq_gemv(fq_args(d, l, 0), st))) return rc;
        if ((rc = launch_attention_decode(attn_args(d, l), B, d->att, H, d->t_att, 3, H, st)))
            return rc;
        if ((rc = launch_ks_gemv(step_gemv(d, d->Wo(l), d->t_att, H, H), st))) return rc;
        if ((rc = launch_resid_q8(d->h, d->part, d->ks_h, H, d->So(l), d->h2, d->PostLn(l), B, H,
                                  d->seg, d->x8b, d->x8s, d->x8ssp, st, true)))
            return rc;
        if ((rc = launch_fq_gemv(fq_args(d, l, 2), st))) return rc;
        if ((rc = launch_ks_gemv(fq_down(d, l), st))) return rc;
        if (l + 1 < d->L)
            rc = launch_resid_q8(d->h2, d->part, d->ks_i, H, d->Sd(l), d->h, d->InLn(l + 1), B, H,
                                 d->seg, d->x8b, d->x8s, d->x8ssp, st, true);
        else
            rc = launch_rmsnorm_resid(d->h2, d->part, d->ks_i, H, d->Sd(l), d->h, B, H,
                                      d->final_norm, d->c.eps, d->t_x, 3, H, st);
        if (rc) return rc;
    }
    if ((rc = enqueue_head(d, true))) return rc;
    step_advance_kernel<<<1, 1, 0, st>>>(d->step, d->pos);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

int enqueue_any_step(vmlm_decoder *d) {
    return d->prog == PROG_FUSED   ? enqueue_step_fused(d)
           : d->prog == PROG_FULLK ? enqueue_step_fullk(d)
                                   : enqueue_step(d);
}

int ensure_graph(vmlm_decoder *d) {
    if (d->graph) return VMLM_OK;
    hipGraph_t g = nullptr;
    VMLM_HIP_CHECK(hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_any_step(d);
    hipError_t e = hipStreamEndCapture(d->st, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&d->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    return VMLM_OK;
}

// Batches of up to five sequences run the five-launch layer when every
// projection shape fits the fused kernel.
bool fused_ok(const vmlm_decoder *d) {
    const int B = (int)d->B, H = (int)d->H, I = (int)d->I;
    return H / 16 * B <= 768 && fk_gemv_ok(B, 3 * H, H, FK_STORE) && fk_gemv_ok(B, H, H, FK_RESID) &&
           fk_gemv_ok(B, 2 * I, H, FK_SILU) && fk_gemv_ok(B, H, I, FK_RESID);
}

// The full-K program: the q/k/v and gate/up shapes fit the full-K kernel,
// the down projection's slices are whole 64-column blocks staged by 4 waves.
bool fullk_ok(const vmlm_decoder *d) {
    const int B = (int)d->B, H = (int)d->H, I = (int)d->I;
    return fq_gemv_ok(B, 3 * H, H, FQ_STORE, d->fq_tw) &&
           fq_gemv_ok(B, 2 * I, H, FQ_SILU, d->fq_tw_gu) &&
           d->seg % 64 == 0 && d->seg_i % 64 == 0 && d->seg_i / 64 <= 6;
}

// Sets the layer program (the graph of the old one is dropped).
int set_program(vmlm_decoder *d, int prog) {
    if (d->prog == prog) return VMLM_OK;
    if (d->graph) {
        VMLM_HIP_CHECK(hipStreamSynchronize(d->st));
        (void)hipGraphExecDestroy(d->graph);
        d->graph = nullptr;
    }
    d->prog = prog;
    d->fused = prog == PROG_FUSED;
    return VMLM_OK;
}

}  // namespace

extern "C" {

int vmlm_decoder_create(const vmlm_decoder_cfg *cfg, vmlm_decoder **out) {
    int rc = ensure_init();
    if (rc) return rc;
    VMLM_GUARD(cfg && out, "decoder: null argument");
    const vmlm_decoder_cfg &c = *cfg;
    VMLM_GUARD(c.head_dim == 64, "decoder: head_dim %u unsupported (64 only)", c.head_dim);
    VMLM_GUARD(c.n_heads * c.head_dim == c.hidden, "decoder: hidden != n_heads * head_dim");
    VMLM_GUARD(c.hidden % 128 == 0 && c.inter % 128 == 0,
               "decoder: hidden and inter must be multiples of 128");
    VMLM_GUARD(c.batch >= 1 && c.batch <= 16, "decoder: batch %u outside 1..16", c.batch);
    VMLM_GUARD(c.cap >= 2 && c.vocab >= 1 && c.n_layers >= 1, "decoder: empty shape");
    VMLM_GUARD(c.theta > 0.0f, "ROPE: theta must be > 0");
    vmlm_decoder *d = new vmlm_decoder();
    d->c = c;
    d->H = c.hidden;
    d->I = c.inter;
    d->NH = c.n_heads;
    d->V = c.vocab;
    d->B = c.batch;
    d->cap = c.cap;
    d->L = c.n_layers;
    d->w_layer = 4 * d->H * d->H + 3 * d->I * d->H;
    d->s_layer = 5 * d->H + 2 * d->I;
    d->rope_step = -2.0f / 64.0f * host_ln_f(c.theta);
    // k-slices of the K = hidden and K = inter projections (k-slice program)
    d->ks_h = ks_gemv_slices((int)d->H);
    d->ks_i = ks_gemv_slices((int)d->I);
    VMLM_GUARD(d->ks_h <= 16 && d->ks_i <= 16, "decoder: hidden %u / inter %u need over 16 k-slices",
               c.hidden, c.inter);
    d->seg = ks_gemv_window((int)d->H);  // 64 .. 384 columns
    d->seg_i = ks_gemv_window((int)d->I);
    d->prog = fused_ok(d) ? PROG_FUSED : fullk_ok(d) ? PROG_FULLK : PROG_KSLICE;
    d->fused = d->prog == PROG_FUSED;
    d->loaded.assign(d->L, false);
    auto cleanup = [&](int code) {
        vmlm_decoder_destroy(d);
        return code;
    };
    hipError_t e = hipStreamCreateWithFlags(&d->st, hipStreamNonBlocking);
    if (e != hipSuccess) return cleanup(hip_fail(e, "decoder stream"));
    d->hs = d->cap + 1;
    const size_t kvn = d->L * d->B * d->NH * d->hs * 64;
    if ((rc = dalloc(d, &d->wstage, d->w_layer)) || (rc = dalloc(d, &d->s, d->L * d->s_layer)) ||
        (rc = dalloc(d, &d->norms, d->L * 2 * d->H)) || (rc = dalloc(d, &d->embed, d->V * d->H)) ||
        (rc = dalloc(d, &d->lm_head, d->V * d->H)) || (rc = dalloc(d, &d->final_norm, d->H)) ||
        (rc = dalloc(d, &d->kc, kvn)) || (rc = dalloc(d, &d->vc, kvn)) ||
        (rc = dalloc(d, &d->wsw, d->L * d->w_layer)) ||
        (rc = dalloc(d, &d->x8, (size_t)Q8_T * d->B * d->H)) ||
        (rc = dalloc(d, &d->x8b, (size_t)Q8_T * d->H * 16)) ||
        (rc = dalloc(d, &d->x8s, d->H / d->seg * d->B)) ||
        (rc = dalloc(d, &d->x8ssp, d->H / d->seg * d->B)) ||
        (rc = dalloc(d, &d->act8, (size_t)Q8_T * d->B * d->I)) ||
        (rc = dalloc(d, &d->act8s, d->I / d->seg_i * d->B)) ||
        (rc = dalloc(d, &d->apart, d->NH * FK_APART * ATTN_PART)) ||
        (d->fused && (rc = dalloc(d, &d->ssp, d->H / 16 * d->B))) ||
        (rc = dalloc(d, &d->h, d->B * d->H)) || (rc = dalloc(d, &d->h2, d->B * d->H)) ||
        (rc = dalloc(d, &d->qkv, d->B * 3 * d->H)) || (rc = dalloc(d, &d->att, d->B * d->H)) ||
        (rc = dalloc(d, &d->act, d->B * d->I)) ||
        (rc = dalloc(d, &d->logits, d->B * d->V)) || (rc = dalloc(d, &d->t_x, 3 * d->B * d->H)) ||
        (rc = dalloc(d, &d->t_att, 3 * d->B * d->H)) ||
        (rc = dalloc(d, &d->t_act, 3 * d->B * d->I)) || (rc = dalloc(d, &d->tok, d->B)) ||
        (rc = dalloc(d, &d->tokens_out, d->cap * d->B)) || (rc = dalloc(d, &d->pos, 1)) ||
        (rc = dalloc(d, &d->step, 1)) || (rc = dalloc(d, &d->keys, d->B * KEY_SLOTS)) ||
        (rc = dalloc(d, &d->part, d->B * std::max({(size_t)d->ks_h * 3 * d->H,
                                                   (size_t)d->ks_h * 2 * d->I,
                                                   (size_t)d->ks_i * d->H}))))
        return cleanup(rc);
    if ((e = hipMemsetAsync(d->keys, 0, d->B * KEY_SLOTS * 8, d->st)) != hipSuccess ||
        (e = hipMemsetAsync(d->kc, 0, kvn * 4, d->st)) != hipSuccess ||
        (e = hipMemsetAsync(d->vc, 0, kvn * 4, d->st)) != hipSuccess ||
        (e = hipMemsetAsync(d->pos, 0, 4, d->st)) != hipSuccess ||
        (e = hipMemsetAsync(d->step, 0, 4, d->st)) != hipSuccess ||
        (e = hipMemsetAsync(d->x8b, 0, (size_t)Q8_T * d->H * 16, d->st)) != hipSuccess ||
        (e = hipStreamSynchronize(d->st)) != hipSuccess)
        return cleanup(hip_fail(e, "decoder init"));
    *out = d;
    return VMLM_OK;
}

int vmlm_decoder_destroy(vmlm_decoder *d) {
    if (!d) return VMLM_OK;
    if (d->st) (void)hipStreamSynchronize(d->st);
    if (d->graph) (void)hipGraphExecDestroy(d->graph);
    for (void *p : d->allocs) (void)hipFree(p);
    if (d->pf) (void)hipFree(d->pf);
    if (d->st) (void)hipStreamDestroy(d->st);
    delete d;
    return VMLM_OK;
}

int vmlm_decoder_load_layer(vmlm_decoder *d, uint32_t layer, const int8_t *wq, const float *sq,
                            const int8_t *wk, const float *sk, const int8_t *wv,
                            const float *sv, const int8_t *wo, const float *so,
                            const int8_t *wg, const float *sg, const int8_t *wu,
                            const float *su, const int8_t *wd, const float *sd,
                            const float *in_ln, const float *post_ln) {
    VMLM_GUARD(d && layer < d->L, "decoder: layer %u out of range", layer);
    const size_t H = d->H, I = d->I, l = layer;
    int8_t *W = d->wstage;  // stream-ordered: the previous layer's swizzles have read it
    float *S = d->s + l * d->s_layer;
    hipStream_t st = d->st;
    auto h2d = [&](void *dst, const void *src, size_t bytes) {
        return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
    };
    hipError_t e;
#define H2D(dst, src, bytes)                                         \
    if ((e = h2d(dst, src, bytes)) != hipSuccess) return hip_fail(e, "load_layer");
    H2D(W, wq, H * H);
    H2D(W + H * H, wk, H * H);
    H2D(W + 2 * H * H, wv, H * H);
    H2D(W + 3 * H * H, wo, H * H);
    int8_t *Wgu = W + 4 * H * H;
    // 16-row blocks: gate block b -> rows [32b, 32b+16), up block b -> [32b+16, 32b+32)
    if ((e = hipMemcpy2DAsync(Wgu, 32 * H, wg, 16 * H, 16 * H, I / 16, hipMemcpyHostToDevice,
                              st)) != hipSuccess ||
        (e = hipMemcpy2DAsync(Wgu + 16 * H, 32 * H, wu, 16 * H, 16 * H, I / 16,
                              hipMemcpyHostToDevice, st)) != hipSuccess)
        return hip_fail(e, "load_layer gate/up");
    H2D(Wgu + 2 * I * H, wd, H * I);
    {  // the copy in MFMA-operand order that every projection reads
        int rc;
        if ((rc = launch_swizzle_w(W, d->wsw + l * d->w_layer, (int)(3 * H), (int)H, st)) ||
            (rc = launch_swizzle_w(W + 3 * H * H, d->wsw + l * d->w_layer + 3 * H * H, (int)H,
                                   (int)H, st)) ||
            (rc = launch_swizzle_w(Wgu, d->wsw + l * d->w_layer + 4 * H * H, (int)(2 * I),
                                   (int)H, st)) ||
            (rc = launch_swizzle_w(Wgu + 2 * I * H, d->wsw + l * d->w_layer + 4 * H * H + 2 * I * H,
                                   (int)H, (int)I, st)))
            return rc;
    }
    H2D(S, sq, H * 4);
    H2D(S + H, sk, H * 4);
    H2D(S + 2 * H, sv, H * 4);
    H2D(S + 3 * H, so, H * 4);
    float *Sgu = S + 4 * H;
    if ((e = hipMemcpy2DAsync(Sgu, 32 * 4, sg, 16 * 4, 16 * 4, I / 16, hipMemcpyHostToDevice,
                              st)) != hipSuccess ||
        (e = hipMemcpy2DAsync(Sgu + 16, 32 * 4, su, 16 * 4, 16 * 4, I / 16,
                              hipMemcpyHostToDevice, st)) != hipSuccess)
        return hip_fail(e, "load_layer gate/up scales");
    H2D(Sgu + 2 * I, sd, H * 4);
    H2D(d->norms + l * 2 * H, in_ln, H * 4);
    H2D(d->norms + l * 2 * H + H, post_ln, H * 4);
#undef H2D
    VMLM_HIP_CHECK(hipStreamSynchronize(st));
    d->loaded[l] = true;
    return VMLM_OK;
}

int vmlm_decoder_load_globals(vmlm_decoder *d, const uint16_t *embed, const uint16_t *lm_head,
                              const float *final_norm) {
    VMLM_GUARD(d, "decoder: null");
    VMLM_HIP_CHECK(hipMemcpyAsync(d->embed, embed, d->V * d->H * 2, hipMemcpyHostToDevice, d->st));
    VMLM_HIP_CHECK(
        hipMemcpyAsync(d->lm_head, lm_head, d->V * d->H * 2, hipMemcpyHostToDevice, d->st));
    VMLM_HIP_CHECK(
        hipMemcpyAsync(d->final_norm, final_norm, d->H * 4, hipMemcpyHostToDevice, d->st));
    VMLM_HIP_CHECK(hipStreamSynchronize(d->st));
    d->loaded_globals = true;
    return VMLM_OK;
}

static int check_loaded(vmlm_decoder *d) {
    VMLM_GUARD(d, "decoder: null");
    VMLM_GUARD(d->loaded_globals, "decoder: embedding / LM head not loaded");
    for (size_t l = 0; l < d->L; ++l) VMLM_GUARD(d->loaded[l], "decoder: layer %zu not loaded", l);
    return VMLM_OK;
}

int vmlm_decoder_prefill(vmlm_decoder *d, const int32_t *tokens, uint32_t S,
                         int32_t *first_tokens, float *logits_last) {
    int rc = check_loaded(d);
    if (rc) return rc;
    VMLM_GUARD(S >= 1 && S < d->cap, "decoder: prompt length %u outside 1..cap-1", S);
    hipStream_t st = d->st;
    const size_t B = d->B, H = d->H, I = d->I, NH = d->NH, M = B * S;
    const int T = 3;
    // the prefill's buffers, carved from the session's workspace (256-byte
    // aligned parts); every projection input is int8 rows (a8, a8s)
    float *h, *h2, *qkv, *att, *o, *act, *a8s, *gwork = nullptr;
    int8_t *a8;
    int32_t *toks;
    char *kvw;
    float2 *rtab;  // RoPE (sin, cos) of positions 0 .. S-1 (one-launch attention)
    // k-slice work of the int8-row GEMMs whose grids would leave CUs idle
    // (gate/up runs as one slice: its epilogue forms SiLU(gate) * up)
    const size_t gw = std::max(std::max(gemm_i8_work_floats((int)M, (int)(3 * H), (int)H),
                                        gemm_i8_work_floats((int)M, (int)H, (int)H)),
                               gemm_i8_work_floats((int)M, (int)H, (int)I));
    const size_t parts[] = {M * H * 4, M * H * 4, M * 3 * H * 4, M * H * 4, M * H * 4, M * I * 4,
                            q8_rows_bytes(M, std::max(H, I)), M * 4, M * 4,
                            attention_prefill_work_bytes((int)S, (int)NH, (int)B), gw * 4,
                            S * 32 * sizeof(float2)};
    size_t need = 0;
    for (size_t b : parts) need += (b + 255) / 256 * 256;
    if (d->pf_bytes < need) {
        VMLM_HIP_CHECK(hipStreamSynchronize(st));
        if (d->pf) (void)hipFree(d->pf);
        d->pf = nullptr;
        d->pf_bytes = 0;
        hipError_t e = hipMalloc(&d->pf, need);
        if (e != hipSuccess) return hip_fail(e, "prefill workspace");
        d->pf_bytes = need;
    }
    {
        char *c = (char *)d->pf;
        int i = 0;
        auto carve = [&](auto **p) {
            *p = (std::remove_reference_t<decltype(*p)>)c;
            c += (parts[i++] + 255) / 256 * 256;
        };
        carve(&h), carve(&h2), carve(&qkv), carve(&att), carve(&o), carve(&act), carve(&a8);
        carve(&a8s), carve(&toks), carve(&kvw), carve(&gwork), carve(&rtab);
        if (!gw) gwork = nullptr;
    }
    auto run = [&]() -> int {
        VMLM_HIP_CHECK(hipMemcpyAsync(toks, tokens, M * 4, hipMemcpyHostToDevice, st));
        int r = launch_emb_bf16(h, H, d->embed, d->V, H, nullptr, toks, (int)M, st);
        if (r) return r;
        // k-sliced projections (grids that would leave CUs idle, small M) hand
        // their slices to the consumer, which sums them in order and applies
        // the column scale (no reduction launch): q/k/v to the attention's
        // prep pass, o and down (but the last) to the next rows_q8's residual
        // add
        const int ks_qkv = gemm_i8_kslices((int)M, (int)(3 * H), (int)H);
        const int ks_o = gemm_i8_kslices((int)M, (int)H, (int)H);
        const int ks_d = gemm_i8_kslices((int)M, (int)H, (int)I);
        // the rotation angles of the prompt positions, once for every layer
        const float2 *tab = nullptr;
        if (attention_prefill_one_launch((int)S, (int)NH, (int)B) && ks_qkv == 1) {
            if ((r = launch_rope_table(rtab, (int)S, 0.0f, d->rope_step, st))) return r;
            tab = rtab;
        }
        for (size_t l = 0; l < d->L; ++l) {
            // the input norm; from layer 1 on it first adds the previous
            // layer's down projection to its residual h2: h = h2 + down
            Slices down;
            if (l && ks_d > 1) down = Slices{gwork, ks_d, M * H, d->Sd(l - 1)};
            if ((r = l ? launch_rows_q8(h, H, d->InLn(l), d->c.eps, M, H, a8, a8s, st, h2, o, down)
                       : launch_rows_q8(h, H, d->InLn(l), d->c.eps, M, H, a8, a8s, st)))
                return r;
            GemmArgs g;
            g.W = d->Wqkv(l);
            g.w_blocked = true;
            g.scale = d->Sqkv(l);
            g.A8 = a8;
            g.a8s = a8s;
            g.work = gwork;
            g.work_floats = gw;
            g.lda = (int)H;
            g.M = (int)M;
            g.N = (int)(3 * H);
            g.K = (int)H;
            g.C = qkv;
            g.ldc = (int)(3 * H);
            g.keep_slices = ks_qkv > 1;
            if ((r = launch_gemm(g, st))) return r;
            g.keep_slices = false;
            // q and k stay unrotated: the attention's prep pass rotates them
            // and writes the rotated K and raw V rows to the cache (positions
            // 0..S-1)
            const float *qb = ks_qkv > 1 ? gwork : qkv;
            const Slices qs = ks_qkv > 1 ? Slices{gwork, ks_qkv, M * 3 * H, d->Sqkv(l)} : Slices{};
            if ((r = launch_attention_prefill(qb, qb + H, qb + 2 * H, att, (int)S, (int)NH,
                                              (int)(3 * H), (int)H, d->c.attn_scale, true, kvw,
                                              st, true, d->rope_step, 0.0f, (int)B, S * 3 * H,
                                              S * H, d->Kc(l), d->Vc(l), (int)d->hs, qs, tab)))
                return r;
            if ((r = launch_rows_q8(att, H, nullptr, 0.0f, M, H, a8, a8s, st))) return r;
            GemmArgs go = g;
            go.W = d->Wo(l);
            go.scale = d->So(l);
            go.N = (int)H;
            go.C = o;
            go.ldc = (int)H;
            go.keep_slices = ks_o > 1;
            if ((r = launch_gemm(go, st))) return r;
            // h2 = h + o, then the post-attention norm
            const Slices os = ks_o > 1 ? Slices{gwork, ks_o, M * H, d->So(l)} : Slices{};
            if ((r = launch_rows_q8(h2, H, d->PostLn(l), d->c.eps, M, H, a8, a8s, st, h, o, os)))
                return r;
            GemmArgs ggu = g;
            ggu.W = d->Wgu(l);
            ggu.scale = d->Sgu(l);
            ggu.N = (int)(2 * I);
            ggu.C = act;  // SiLU(gate) * up formed in the epilogue
            ggu.ldc = (int)I;
            ggu.silu_pairs = true;
            if ((r = launch_gemm(ggu, st))) return r;
            if ((r = launch_rows_q8(act, I, nullptr, 0.0f, M, I, a8, a8s, st))) return r;
            GemmArgs gd = g;
            gd.W = d->Wd(l);
            gd.scale = d->Sd(l);
            gd.lda = (int)I;
            gd.K = (int)I;
            gd.N = (int)H;
            gd.C = o;
            gd.ldc = (int)H;
            gd.keep_slices = ks_d > 1 && l + 1 < d->L;  // the last layer's is reduced into o
            if ((r = launch_gemm(gd, st))) return r;
        }
        // the last layer's residual add (the others are in the next input norm)
        if ((r = launch_ew(h, h2, o, M * H, VMLM_OP_EWADD, st))) return r;
        // last row of every sequence -> decode buffers, then the shared tail
        VMLM_HIP_CHECK(hipMemcpy2DAsync(d->h, H * 4, h + (S - 1) * H, S * H * 4, H * 4, B,
                                        hipMemcpyDeviceToDevice, st));
        if ((r = launch_rmsnorm(nullptr, d->h, d->final_norm, B, H, d->c.eps, d->t_x, T, (int)H,
                                st)))
            return r;
        if ((r = enqueue_head(d, false))) return r;
        d->reset_step = 0;
        d->reset_pos = (int32_t)S;
        VMLM_HIP_CHECK(hipMemcpyAsync(d->step, &d->reset_step, 4, hipMemcpyHostToDevice, st));
        VMLM_HIP_CHECK(hipMemcpyAsync(d->pos, &d->reset_pos, 4, hipMemcpyHostToDevice, st));
        if (first_tokens)
            VMLM_HIP_CHECK(hipMemcpyAsync(first_tokens, d->tok, B * 4, hipMemcpyDeviceToHost, st));
        if (logits_last)
            VMLM_HIP_CHECK(
                hipMemcpyAsync(logits_last, d->logits, B * d->V * 4, hipMemcpyDeviceToHost, st));
        return VMLM_OK;
    };
    rc = run();
    VMLM_HIP_CHECK(hipStreamSynchronize(st));
    if (rc) return rc;
    d->pos_host = S;
    d->step_host = 0;
    return vmlm_hip_check_guards();
}

int vmlm_decoder_decode(vmlm_decoder *d, uint32_t n_steps, int32_t *tokens_out,
                        float *logits_last) {
    int rc = check_loaded(d);
    if (rc) return rc;
    VMLM_GUARD(d->pos_host >= 1, "decoder: decode before prefill");
    VMLM_GUARD((size_t)d->pos_host + n_steps <= d->cap,
               "WRITECOL: decode would write position %zu beyond capacity %zu",
               (size_t)d->pos_host + n_steps - 1, d->cap);
    VMLM_GUARD((size_t)d->step_host + n_steps <= d->cap, "decoder: token log full");
    if (d->use_graph && (rc = ensure_graph(d))) return rc;
    for (uint32_t i = 0; i < n_steps; ++i) {
        if (d->use_graph) {
            VMLM_HIP_CHECK(hipGraphLaunch(d->graph, d->st));
        } else if ((rc = enqueue_any_step(d))) {
            return rc;
        }
    }
    const uint32_t first = d->step_host;
    if (tokens_out && n_steps)
        VMLM_HIP_CHECK(hipMemcpyAsync(tokens_out, d->tokens_out + (size_t)first * d->B,
                                      (size_t)n_steps * d->B * 4, hipMemcpyDeviceToHost, d->st));
    if (logits_last)
        VMLM_HIP_CHECK(hipMemcpyAsync(logits_last, d->logits, d->B * d->V * 4,
                                      hipMemcpyDeviceToHost, d->st));
    VMLM_HIP_CHECK(hipStreamSynchronize(d->st));
    d->pos_host += n_steps;
    d->step_host += n_steps;
    return vmlm_hip_check_guards();
}

int vmlm_decoder_position(const vmlm_decoder *d, uint32_t *pos) {
    VMLM_GUARD(d && pos, "decoder: null");
    *pos = d->pos_host;
    return VMLM_OK;
}

int vmlm_decoder_set_graph(vmlm_decoder *d, int enable) {
    VMLM_GUARD(d, "decoder: null");
    d->use_graph = enable != 0;
    return VMLM_OK;
}

void *vmlm_decoder_stream(vmlm_decoder *d) { return d ? (void *)d->st : nullptr; }

int vmlm_decoder_set_fused(vmlm_decoder *d, int enable) {
    VMLM_GUARD(d, "decoder: null");
    VMLM_GUARD(!enable || fused_ok(d), "decoder: the fused layer needs a batch of at most 5");
    return set_program(d, enable ? PROG_FUSED : PROG_KSLICE);
}

int vmlm_decoder_fused(const vmlm_decoder *d) { return d && d->fused ? 1 : 0; }

int vmlm_decoder_set_program(vmlm_decoder *d, int program) {
    VMLM_GUARD(d, "decoder: null");
    VMLM_GUARD(program >= PROG_KSLICE && program <= PROG_FULLK, "decoder: program %d", program);
    VMLM_GUARD(program != PROG_FUSED || fused_ok(d),
               "decoder: the fused layer needs a batch of at most 5");
    VMLM_GUARD(program != PROG_FULLK || fullk_ok(d),
               "decoder: the full-K program needs hidden 768, 1536 or 2304 and a batch of at "
               "most 16");
    return set_program(d, program);
}

int vmlm_decoder_program(const vmlm_decoder *d) { return d ? d->prog : -1; }

int vmlm_decoder_time_gemv(vmlm_decoder *d, int which, uint32_t iters, float *avg_us,
                           double *bytes_per_launch) {
    int rc = check_loaded(d);
    if (rc) return rc;
    VMLM_GUARD(which >= 0 && which <= 15 && iters >= 1, "time_gemv: which 0..15, iters >= 1");
    VMLM_GUARD(which <= 4 || which >= 8 || !d->fused,
               "time_gemv: 5..7 time a projection with its reduction (k-slice and full-K programs)");
    VMLM_GUARD(which < 14 || d->prog == PROG_FULLK,
               "time_gemv: 14, 15 time the q/k/v and gate/up projections of the full-K program "
               "at their other workgroup tilings");
    const int B = (int)d->B, H = (int)d->H, I = (int)d->I;
    // the launches of the decode step: the k-slice GEMVs, or the LM head (bf16)
    auto make_lm = [&]() {
        GemvArgs g;
        g.T = 3;
        g.M = B;
        g.lda = H;
        g.K = H;
        g.A = d->t_x;
        g.W = d->lm_head;
        g.w_int8 = false;
        g.N = (int)d->V;
        g.Y = d->logits;
        g.ldy = (int)d->V;
        g.tiles = 9;
        return g;
    };
    // 5, 6, 7: the o, gate/up or down projection and the kernel that reduces
    // its k-slice partials (residual RMSNorm into int8 rows, SiLU * up)
    // 8..11: a plain read of the q/k/v, o, gate/up or down weights of the
    // layer (stream_read_kernel), the single-launch floor of that shape
    const bool rd = which >= 8 && which <= 11;
    const int proj = which == 15 ? 2 : which >= 12 ? 0 : rd ? which - 8 : which >= 5 ? which - 4 : which;
    auto make = [&](size_t l) {
        switch (proj) {
        case 0: return step_gemv(d, d->Wqkv(l), d->t_x, 3 * H, H);
        case 1: return step_gemv(d, d->Wo(l), d->t_att, H, H);
        case 2: return step_gemv(d, d->Wgu(l), d->t_x, 2 * I, H);
        default: return step_gemv(d, d->Wd(l), d->t_act, H, I);
        }
    };
    // the fused program (batch <= 5) runs the full-K kernels with their row ops
    const bool fk = d->fused && which < 4;
    // the full-K program: q/k/v and gate/up (with SiLU * up) over the whole
    // K, down over f32 rows; 14: q/k/v at four tiles per workgroup, 15:
    // gate/up at one tile pair per workgroup
    const bool fq = d->prog == PROG_FULLK;
    auto fq_launch = [&](size_t l, int pr) {
        if (pr == 0 || pr == 2) {
            FqArgs f = fq_args(d, l, pr);
            if (which == 14) f.tw = 4;
            if (which == 15) f.tw = 2;
            return launch_fq_gemv(f, d->st);
        }
        return launch_ks_gemv(pr == 1 ? make(l) : fq_down(d, l), d->st);
    };
    auto read = [&](size_t l) {
        const KsArgs g = make(l);
        const size_t n16 = (size_t)g.N * g.K / 16;
        stream_read_kernel<<<(unsigned)((n16 + 2047) / 2048), 256, 0, d->st>>>(
            (const u32x4 *)g.W, n16, (uint32_t *)d->logits);
        VMLM_HIP_CHECK(hipGetLastError());
        return (int)VMLM_OK;
    };
    int8_t *x8 = fq ? d->x8b : d->x8;
    auto reduce = [&](size_t l) {
        if (which == 5)
            return launch_resid_q8(d->h, d->part, d->ks_h, H, d->So(l), d->h2, d->PostLn(l), B, H,
                                   d->seg, x8, d->x8s, d->x8ssp, d->st, fq);
        if (which == 6)  // (full-K: SiLU * up is in the projection's epilogue)
            return fq ? (int)VMLM_OK
                      : launch_silu_q8(d->part, d->ks_h, 2 * I, d->Sgu(l), B, I, d->seg_i,
                                       d->act8, d->act8s, d->st);
        return launch_resid_q8(d->h2, d->part, d->ks_i, H, d->Sd(l), d->h, d->InLn((l + 1) % d->L),
                               B, H, d->seg, x8, d->x8s, d->x8ssp, d->st, fq);
    };
    auto launch = [&](size_t l) {
        if (rd) return read(l);
        if (which == 13) {  // 13: an empty kernel (the per-launch fixed cost)
            empty_kernel<<<1, 64, 0, d->st>>>();
            VMLM_HIP_CHECK(hipGetLastError());
            return (int)VMLM_OK;
        }
        if (which == 12)  // 12: the decode attention of the layer
            return launch_attention_decode(attn_args(d, l), B, d->att, H, d->t_att, 3, H, d->st);
        if (which == 4) return launch_gemv(make_lm(), d->st);
        if (fk) return launch_fk_gemv(fk_args(d, l, which), d->st);
        int r = fq ? fq_launch(l, which == 14 ? 0 : which == 15 ? 2 : proj)
                   : launch_ks_gemv(make(l), d->st);
        return r || which < 5 || which >= 14 ? r : reduce(l);
    };
    // `iters` back-to-back launches captured into one HIP graph, as the
    // decode step runs; one event pair around a replay gives the mean launch
    // duration, launch gaps included. Successive launches walk the layers so
    // that no weight is re-read from cache.
    for (size_t l = 0; l < (which == 4 ? 1 : d->L); ++l)  // warm-up pass over every layer
        if ((rc = launch(l))) return rc;
    VMLM_HIP_CHECK(hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal));
    for (uint32_t i = 0; i < iters && !rc; ++i) rc = launch(which == 4 ? 0 : i % d->L);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(d->st, &g);
    if (rc || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return rc ? rc : hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    if ((e = hipEventCreate(&e0)) == hipSuccess && (e = hipEventCreate(&e1)) == hipSuccess &&
        (e = hipGraphLaunch(x, d->st)) == hipSuccess && (e = hipEventRecord(e0, d->st)) == hipSuccess &&
        (e = hipGraphLaunch(x, d->st)) == hipSuccess && (e = hipEventRecord(e1, d->st)) == hipSuccess &&
        (e = hipEventSynchronize(e1)) == hipSuccess)
        e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipGraphExecDestroy(x);
    if (e != hipSuccess) return hip_fail(e, "time_gemv replay");
    *avg_us = ms * 1000.0f / (float)iters;
    if (rd) {  // the weight bytes read
        const KsArgs k = make(0);
        *bytes_per_launch = (double)k.N * k.K;
        return VMLM_OK;
    }
    if (which == 13) {
        *bytes_per_launch = 0.0;
        return VMLM_OK;
    }
    if (which == 12) {  // K and V rows of the cached positions and the new row
        int pos = 0;
        VMLM_HIP_CHECK(hipMemcpy(&pos, d->pos, sizeof(int), hipMemcpyDeviceToHost));
        *bytes_per_launch = 512.0 * B * d->NH * (pos + 1);
        return VMLM_OK;
    }
    // algorithmic bytes of the projection: weights, row scales (int8), the
    // f32 activation in and the f32 result out (the partial sums and the
    // bf16 term planes are this implementation's, not the algorithm's)
    if (fk) {  // plus the residual rows that the o and down epilogues read
        const FkArgs f = fk_args(d, 0, which);
        const double nout = f.epi == FK_SILU ? f.N / 2.0 : (double)f.N;
        *bytes_per_launch = (double)f.N * f.K + 4.0 * f.N + 4.0 * B * f.K + 4.0 * B * nout +
                            (f.R ? 4.0 * B * f.N : 0.0);
        return VMLM_OK;
    }
    const bool i8 = which != 4;
    const double n = i8 ? make(0).N : make_lm().N, k = i8 ? make(0).K : make_lm().K;
    *bytes_per_launch = n * k * (i8 ? 1 : 2) + (i8 ? n * 4 : 0.0) + (double)B * k * 4 +
                        (double)B * n * 4;
    return VMLM_OK;
}

// B1 layer stack: x [T][d] -> transpose -> n_layers x (gather-dot, act) ->
// transpose back into y [T][d]. Connection arrays are device pointers.
int vmlm_b1_stack_forward(const vmlm_sparse_conn_w *layers, uint32_t n_layers, const float *x,
                          float *y, size_t n_tokens, uint16_t act, void *stream) {
    int rc = ensure_init();
    if (rc) return rc;
    VMLM_GUARD(layers && n_layers >= 1, "b1 stack: no layers");
    const size_t d = layers[0].n_neurons;
    for (uint32_t l = 0; l < n_layers; ++l) {
        const vmlm_sparse_conn_w &sc = layers[l];
        VMLM_GUARD(sc.n_neurons == d, "b1 stack: layer %u width %u != %zu", l, sc.n_neurons, d);
        VMLM_GUARD(sc.e == (size_t)sc.n_neurons * sc.k0,
                   "CONN_TRAIN: SparseConnW geometry inconsistent at layer %u", l);
        VMLM_GUARD(sc.k0 <= 1024, "B1: k0 exceeds the safe stack bound");
    }
    if (n_tokens == 0) return VMLM_OK;
    hipStream_t st = as_stream(stream);
    const int actk = act == 0xFFFF ? -1 : (int)act;
    std::vector<B1PlanJob> jobs(n_layers);
    std::vector<int> k0s(n_layers);
    for (uint32_t l = 0; l < n_layers; ++l) {
        k0s[l] = (int)layers[l].k0;
        jobs[l] = B1PlanJob{layers[l].w, layers[l].src_u32, nullptr, k0s[l]};
    }
    if (b1_stack_ok((int)d, k0s.data(), (int)n_layers)) {
        // one kernel for the whole stack (activations stay in LDS)
        void *plan = nullptr;
        VMLM_HIP_CHECK(
            hipMallocAsync(&plan, b1_stack_plan_bytes((int)d, k0s.data(), (int)n_layers), st));
        rc = launch_b1_stack(jobs.data(), (int)n_layers, (int)d, x, y, (int)n_tokens, actk, plan,
                             st);
        (void)hipFreeAsync(plan, st);
        return rc;
    }
    // layer by layer over the reference layout [d][t8], one lane per (neuron, token)
    const size_t t8 = (n_tokens + 63) / 64 * 64;
    float *a = nullptr, *b = nullptr;
    VMLM_HIP_CHECK(hipMallocAsync((void **)&a, d * t8 * 4, st));
    VMLM_HIP_CHECK(hipMallocAsync((void **)&b, d * t8 * 4, st));
    rc = launch_transpose_t8(x, n_tokens, d, a, t8, st);
    for (uint32_t l = 0; l < n_layers && !rc; ++l) {
        rc = launch_b1_forward(layers[l].w, layers[l].src_u32, (int)d, (int)layers[l].k0, a, t8,
                               (int)n_tokens, b, 0, actk, st);
        std::swap(a, b);
    }
    if (!rc) rc = launch_transpose_back(a, d, n_tokens, y, d, t8, st);
    (void)hipFreeAsync(a, st);
    (void)hipFreeAsync(b, st);
    return rc;
}


struct vmlm_b1_stack {
    void *plan = nullptr;
    std::vector<int> k0;
    size_t d = 0;
};

int vmlm_b1_stack_create(const vmlm_sparse_conn_w *layers, uint32_t n_layers, void *stream,
                         vmlm_b1_stack **out) {
    int rc = ensure_init();
    if (rc) return rc;
    VMLM_GUARD(out && layers && n_layers >= 1, "b1 stack: no layers");
    const size_t d = layers[0].n_neurons;
    std::vector<B1PlanJob> jobs(n_layers);
    std::vector<int> k0s(n_layers);
    for (uint32_t l = 0; l < n_layers; ++l) {
        const vmlm_sparse_conn_w &sc = layers[l];
        VMLM_GUARD(sc.n_neurons == d, "b1 stack: layer %u width %u != %zu", l, sc.n_neurons, d);
        VMLM_GUARD(sc.e == (size_t)sc.n_neurons * sc.k0,
                   "CONN_TRAIN: SparseConnW geometry inconsistent at layer %u", l);
        VMLM_GUARD(sc.k0 <= 1024, "B1: k0 exceeds the safe stack bound");
        k0s[l] = (int)sc.k0;
        jobs[l] = B1PlanJob{sc.w, sc.src_u32, nullptr, k0s[l]};
    }
    if (!b1_stack_ok((int)d, k0s.data(), (int)n_layers))
        return fail(VMLM_ERR_UNIMPL, "b1 stack plan: width %zu or k0 beyond the one-kernel stack",
                    d);
    hipStream_t st = as_stream(stream);
    vmlm_b1_stack *s = new vmlm_b1_stack();
    s->k0 = k0s;
    s->d = d;
    hipError_t e = hipMalloc(&s->plan, b1_stack_plan_bytes((int)d, k0s.data(), (int)n_layers));
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipMalloc (b1 stack plan)");
    }
    rc = launch_b1_stack_plan(jobs.data(), (int)n_layers, (int)d, s->plan, st);
    if (!rc) {
        e = hipStreamSynchronize(st);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    if (rc) {
        (void)hipFree(s->plan);
        delete s;
        return rc;
    }
    *out = s;
    return VMLM_OK;
}

int vmlm_b1_stack_run(vmlm_b1_stack *stack, const float *x, float *y, size_t n_tokens,
                      uint16_t act, void *stream) {
    VMLM_GUARD(stack, "b1 stack: null plan");
    VMLM_GUARD(n_tokens <= 0x7fffffff, "b1 stack: %zu tokens", n_tokens);
    return launch_b1_stack_run(stack->plan, stack->k0.data(), (int)stack->k0.size(),
                               (int)stack->d, x, y, (int)n_tokens, act == 0xFFFF ? -1 : (int)act,
                               as_stream(stream));
}

int vmlm_b1_stack_destroy(vmlm_b1_stack *stack) {
    if (!stack) return VMLM_OK;
    (void)hipFree(stack->plan);
    delete stack;
    return VMLM_OK;
}

}  // extern "C"

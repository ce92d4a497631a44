/*
 * vmlm_vm_oracle.c -- CPU restatement of the reference VM's loader and
 * interpreter (core/src/interp.rs), TEST INFRASTRUCTURE ONLY: the checker of
 * libvmlm_hip's device-resident executor (vmlm_vm_*). Only tests/ load it.
 *
 * Loading follows Vm::load_impl (core/src/interp.rs:108-236): the header,
 * TEXT, the const pool (copied, writable), zeroed activation / state /
 * gradient arenas, bind_slots (:351-396) and the load-time audit
 * audit_const_dtypes (:241-348). Execution follows Vm::run (:720-2370), arm
 * for arm, over the oracle's kernels (vmlm_oracle.c), with the reference's
 * exit codes as return values: 9 guard, 5 unimplemented op, 6 training op
 * without the train feature, 3 bad magic.
 *
 * Beyond the reference (marked "executor guard"): operand extents are
 * checked against the slots before reading or writing, where the reference
 * would read neighbouring memory, so that a malformed test program returns
 * 9 instead of faulting; and three opt-in flags give runtime operands that
 * the reference encodes at compile time (ROPE position, WRITECOL column,
 * SOFTMAX live width; bit 6 of `fl`, see sparrow_amd/vmb.py).
 */
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vmlm_oracle.h"

enum {
    OP_HALT = 0, OP_COPY = 2, OP_TRANSPOSE = 4, OP_CONCAT = 5, OP_SLICE = 6, OP_LAYERB = 7,
    OP_GEMM = 10, OP_BMM = 11, OP_OUTER = 12, OP_GEMV = 13, OP_EMB = 14,
    OP_EWADD = 20, OP_EWMUL = 21, OP_EWSUB = 22, OP_EWDIV = 23, OP_SCALE = 24, OP_ACT = 25,
    OP_EXP = 26, OP_LOG = 27, OP_CLAMP = 28, OP_NEG = 29, OP_LN = 30, OP_RMSNORM = 31,
    OP_SUM = 32, OP_MAX = 34, OP_SOFTMAX = 36, OP_MASK_MUL = 40, OP_TOPK_THRESH = 41,
    OP_TOPK_IDX = 42, OP_JMP = 46, OP_CMPLE = 47, OP_SAVE = 49, OP_LOAD = 50, OP_PRINT = 51,
    OP_SHAPE = 52, OP_BIAS = 53, OP_WRITECOL = 71, OP_EWMAX = 72, OP_GEMASK = 73,
    OP_LN_EPS = 85, OP_PUSH = 86, OP_POP = 87, OP_STACK_INIT = 88, OP_LOOP_CNT = 89,
    OP_ROPE = 90, OP_SIN = 91, OP_COS = 92, OP_TOPK_BY_STRENGTH = 93, OP_SPARSE_MATVEC = 94,
};
enum { DT_F32 = 0, DT_F16 = 1, DT_I8 = 2, DT_I32 = 3, DT_BF16 = 4 };
enum { SLOT_CONST = 0, SLOT_ACT = 1, SLOT_STATE = 2, SLOT_GRAD = 3, SLOT_PARAM = 4 };
#define FL_ACC 1u
#define FL_TRANS_B 2u
#define FL_CAUSAL 16u
#define FL_NNZ 64u
#define FL_SELGATE 128u
#define FL_RUNTIME 64u /* executor extension on ROPE / WRITECOL / SOFTMAX */
#define TOPK_MAX_L 2048

typedef struct {
    uint8_t op, fl;
    uint16_t dt;
    uint32_t dst, a, b;
} ins_t;

typedef struct {
    uint8_t *p; /* const: pool + off (layer base applied at access) */
    uint32_t rows, cols;
    uint8_t kind, dtype;
} slot_t;

struct vo_vm {
    uint8_t *img;
    size_t img_len;
    ins_t *text;
    size_t n_ins;
    uint8_t *cpool;
    size_t const_bytes;
    slot_t *slots;
    size_t n_slots;
    uint32_t *names;
    uint8_t *act, *state, *grad;
    size_t layer_base;
    float ln_eps;
    float *out;
    size_t n_out, cap_out;
    char msg[256];
};

static size_t dtype_size(uint8_t dt) {
    switch (dt) {
    case DT_F32: case DT_I32: return 4;
    case DT_BF16: case DT_F16: return 2;
    case DT_I8: return 1;
    default: return 0;
    }
}
static uint32_t u32_at(const uint8_t *p, size_t off) {
    uint32_t v;
    memcpy(&v, p + off, 4);
    return v;
}
static int fail(vo_vm *vm, int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(vm->msg, sizeof(vm->msg), fmt, ap);
    va_end(ap);
    return code;
}

/* --------------------------------------------------------------- loading */
static char g_load_err[256];
void vo_vm_last_load_error_set(const char *m) {
    strncpy(g_load_err, m, sizeof(g_load_err) - 1);
}
const char *vo_vm_last_load_error(void) { return g_load_err; }

void vo_vm_free(vo_vm *vm) {
    if (!vm) return;
    free(vm->img);
    free(vm->text);
    free(vm->slots);
    free(vm->names);
    free(vm->act);
    free(vm->state);
    free(vm->grad);
    free(vm->out);
    free(vm);
}

/* core/src/interp.rs:241-348 audit_const_dtypes: a non-f32 constant may be
 * only a GEMM's B operand (bf16 or i8) or a bf16 EMB table with an f32 dst. */
static int audit(vo_vm *vm) {
    for (size_t i = 0; i < vm->n_ins; ++i) {
        ins_t in = vm->text[i];
        if (in.op == OP_GEMM) {
            uint8_t bdt = in.b < vm->n_slots ? vm->slots[in.b].dtype : DT_F32;
            if (bdt == DT_BF16 || bdt == DT_I8) continue;
            if (bdt != DT_F32) return fail(vm, 9, "gemm B has no kernel for this dtype");
            continue;
        }
        if (in.op == OP_EMB && in.a < vm->n_slots) {
            if (vm->slots[in.a].dtype != DT_BF16) goto generic;
            if (in.dst < vm->n_slots && vm->slots[in.dst].dtype == DT_F32) continue;
        }
    generic:;
        int cd = 1, ca = 1, cb = 1;
        if (in.op == OP_SHAPE) cd = ca = cb = 0;
        else if (in.op == OP_LOOP_CNT) cd = 0, cb = 0;
        else if (in.op == OP_SLICE || in.op == OP_WRITECOL || in.op == OP_PUSH || in.op == OP_POP)
            cb = 0;
        uint32_t probe[3] = {cd ? in.dst : UINT32_MAX, ca ? in.a : UINT32_MAX,
                             cb ? in.b : UINT32_MAX};
        for (int k = 0; k < 3; ++k) {
            uint32_t s = probe[k];
            if (s >= vm->n_slots) continue;
            uint8_t dt = vm->slots[s].dtype;
            if (dt == DT_F32) continue;
            return fail(vm, 9, "op %u uses %s const at slot %u (only a GEMM may read a non-f32 operand)",
                        in.op, dt == DT_BF16 ? "bf16" : dt == DT_I8 ? "i8" : "non-f32", s);
        }
    }
    return 0;
}

/* core/src/interp.rs:108-236 load_impl + :351-396 bind_slots. */
int vo_vm_load(const uint8_t *image, size_t len, vo_vm **out) {
    *out = NULL;
    vo_vm *vm = calloc(1, sizeof(vo_vm));
    if (!vm) return 2;
    int rc = 0;
    if (len < 32 || u32_at(image, 0) != 0x4D4C4D56u) {
        rc = fail(vm, 3, "bad magic");
        goto bad;
    }
    vm->img = malloc(len);
    memcpy(vm->img, image, len);
    vm->img_len = len;
    size_t text_off = u32_at(image, 8), text_len = u32_at(image, 12);
    size_t const_off = u32_at(image, 16), meta_off = u32_at(image, 24);
    vm->const_bytes = u32_at(image, 20);
    if (text_off + text_len > len || const_off + vm->const_bytes > len || meta_off + 28 > len) {
        rc = fail(vm, 9, "image regions past its end");
        goto bad;
    }
    vm->n_ins = text_len / 16;
    vm->text = malloc((vm->n_ins + 1) * sizeof(ins_t));
    for (size_t i = 0; i < vm->n_ins; ++i) {
        const uint8_t *q = image + text_off + 16 * i;
        ins_t in;
        in.op = q[0];
        in.fl = q[1];
        memcpy(&in.dt, q + 2, 2);
        in.dst = u32_at(q, 4);
        in.a = u32_at(q, 8);
        in.b = u32_at(q, 12);
        vm->text[i] = in;
    }
    vm->cpool = vm->img + const_off;
    const uint8_t *meta = image + meta_off;
    size_t n_const = u32_at(meta, 0);
    vm->n_slots = u32_at(meta, 4);
    size_t slots_off = u32_at(meta, 8), act_b = u32_at(meta, 12), state_b = u32_at(meta, 16),
           grad_b = u32_at(meta, 20), names_off = u32_at(meta, 24);
    if (meta_off + names_off + 4 * vm->n_slots > len ||
        meta_off + 28 + 24 * n_const > len) {
        rc = fail(vm, 9, "META tables past the image end");
        goto bad;
    }
    vm->act = calloc(act_b + 64, 1);
    vm->state = calloc(state_b + 64, 1);
    vm->grad = calloc(grad_b + 64, 1);
    vm->ln_eps = 1e-5f;
    vm->slots = calloc(vm->n_slots + 1, sizeof(slot_t));
    vm->names = calloc(vm->n_slots + 1, 4);
    for (size_t i = 0; i < vm->n_slots; ++i) {
        const uint8_t *e = meta + slots_off + 16 * i;
        uint32_t kind = u32_at(e, 0), idx = u32_at(e, 4);
        slot_t s = {0};
        s.rows = u32_at(e, 8);
        s.cols = u32_at(e, 12);
        s.kind = (uint8_t)kind;
        s.dtype = DT_F32;
        vm->names[i] = u32_at(meta + names_off, 4 * i);
        size_t need = (size_t)s.rows * s.cols;
        if (kind == SLOT_CONST || kind == SLOT_PARAM) {
            if (idx >= n_const) {
                rc = fail(vm, 9, "slot %zu names const %u of %zu", i, idx, n_const);
                goto bad;
            }
            const uint8_t *ce = meta + 28 + 24 * (size_t)idx;
            uint32_t off = u32_at(ce, 0), clen = u32_at(ce, 4);
            s.dtype = ce[16];
            size_t esz = dtype_size(s.dtype);
            if (esz == 0) {
                rc = fail(vm, 9, "const has unknown dtype");
                goto bad;
            }
            /* executor guard: the slot's elements lie inside its constant */
            if (need * esz > clen || (size_t)off + clen > vm->const_bytes) {
                rc = fail(vm, 9, "slot %zu (%ux%u) exceeds its constant", i, s.rows, s.cols);
                goto bad;
            }
            s.p = vm->cpool + off;
        } else {
            size_t bytes = kind == SLOT_STATE ? state_b : kind == SLOT_GRAD ? grad_b : act_b;
            uint8_t *base = kind == SLOT_STATE ? vm->state : kind == SLOT_GRAD ? vm->grad : vm->act;
            if ((size_t)idx + need * 4 > bytes + 64) {
                rc = fail(vm, 9, "slot %zu (%ux%u) exceeds its arena", i, s.rows, s.cols);
                goto bad;
            }
            s.p = base + (idx / 4) * 4;
        }
        vm->slots[i] = s;
    }
    rc = audit(vm);
    if (rc) goto bad;
    *out = vm;
    return 0;
bad:
    /* keep the message readable through a failed load */
    {
        static char last[256];
        memcpy(last, vm->msg, sizeof(last));
        vo_vm_free(vm);
        vo_vm_last_load_error_set(last);
    }
    return rc;
}


/* --------------------------------------------------------------- access */
/* core/src/interp.rs:434-467 const_ptr(_based): constants move with the
 * layer base, bound-checked against the pool. */
static float *sp(vo_vm *vm, uint32_t i, int *rc) {
    if (i >= vm->n_slots) {
        *rc = fail(vm, 9, "slot %u does not exist", i);
        return NULL;
    }
    slot_t s = vm->slots[i];
    if (vm->layer_base == 0 || s.kind != SLOT_CONST) return (float *)s.p;
    size_t off = (size_t)(s.p - vm->cpool);
    size_t bytes = (size_t)s.rows * s.cols * dtype_size(s.dtype);
    if (off + vm->layer_base + bytes > vm->const_bytes) {
        *rc = fail(vm, 9, "layer base walks past the constant pool: off=%zu base=%zu bytes=%zu limit=%zu",
                   off, vm->layer_base, bytes, vm->const_bytes);
        return NULL;
    }
    return (float *)(vm->cpool + off + vm->layer_base);
}
#define SHAPE(i, r, c)                                  \
    size_t r = (i) < vm->n_slots ? vm->slots[i].rows : 0; \
    size_t c = (i) < vm->n_slots ? vm->slots[i].cols : 0
#define NEL(i) ((i) < vm->n_slots ? (size_t)vm->slots[i].rows * vm->slots[i].cols : 0)
#define DT(i) ((i) < vm->n_slots ? vm->slots[i].dtype : DT_F32)
#define P(name, i)                    \
    float *name = sp(vm, (i), &rc);   \
    if (rc) return rc
#define NEED(cond, ...)                              \
    do {                                             \
        if (!(cond)) return fail(vm, 9, __VA_ARGS__); \
    } while (0)

/* an f32 value held in a slot, used as a count or index: non-negative and
 * integral (the EMB rule, core/src/interp.rs:1351-1436) */
static int slot_index(vo_vm *vm, uint32_t s, size_t limit, size_t *val, const char *what) {
    int rc = 0;
    float *p = sp(vm, s, &rc);
    if (rc) return rc;
    float v = p[0];
    if (!(v >= 0.0f) || v >= (float)limit) return fail(vm, 9, "%s out of range", what);
    size_t u = (size_t)v;
    if ((float)u != v) return fail(vm, 9, "%s is not an integer", what);
    *val = u;
    return 0;
}

/* Rust's `f as usize`: saturating, NaN and negatives give 0 (the cast the
 * reference applies to f32-held offsets, ids and counts). */
static size_t as_usize(float f) {
    return f > 0.0f ? (f >= 1.8446744e19f ? (size_t)-1 : (size_t)f) : 0;
}

static void print_out(vo_vm *vm, const float *p, size_t n) {
    if (vm->n_out + n > vm->cap_out) {
        size_t cap = vm->cap_out ? vm->cap_out : 1024;
        while (cap < vm->n_out + n) cap *= 2;
        vm->out = realloc(vm->out, cap * sizeof(float));
        vm->cap_out = cap;
    }
    memcpy(vm->out + vm->n_out, p, n * sizeof(float));
    vm->n_out += n;
}

/* ops/src/kernels.rs:1462-1495 topk_thresh: the k-th largest by repeated
 * selection (strict `>` from -inf; values never above -inf are not taken). */
static float topk_thresh(const float *x, size_t n, size_t k) {
    char *used = calloc(n ? n : 1, 1);
    float best = -INFINITY;
    size_t found = 0;
    while (found < k && found < n) {
        size_t bi = (size_t)-1;
        float bv = -INFINITY;
        for (size_t i = 0; i < n; ++i)
            if (!used[i] && x[i] > bv) {
                bv = x[i];
                bi = i;
            }
        if (bi == (size_t)-1) break;
        used[bi] = 1;
        best = bv;
        ++found;
    }
    free(used);
    return best;
}

/* the selection of core/src/interp.rs:1745-1950 over one row of L values:
 * k rounds of "first untaken, replaced by a strictly greater untaken",
 * then the chosen indices ascending; returns how many were chosen. */
static size_t select_topk(const float *row, size_t L, size_t k, size_t *hit, char *taken) {
    for (size_t i = 0; i < L; ++i) taken[i] = 0;
    size_t nk = 0;
    for (size_t r = 0; r < k; ++r) {
        size_t best = 0;
        int found = 0;
        float bestv = 0.0f;
        for (size_t i = 0; i < L; ++i) {
            if (taken[i]) continue;
            float v = row[i];
            if (!found || v > bestv) {
                bestv = v;
                best = i;
                found = 1;
            }
        }
        if (!found) break;
        taken[best] = 1;
        hit[nk++] = best;
    }
    for (size_t i = 1; i < nk; ++i) {
        size_t v = hit[i], q = i;
        while (q > 0 && hit[q - 1] > v) {
            hit[q] = hit[q - 1];
            --q;
        }
        hit[q] = v;
    }
    return nk;
}

/* --------------------------------------------------------------- run */
static int exec(vo_vm *vm, ins_t in, size_t *ip);

int vo_vm_run(vo_vm *vm) {
    size_t ip = 0;
    vm->msg[0] = 0;
    while (ip < vm->n_ins) {
        ins_t in = vm->text[ip++];
        if (in.op == OP_HALT) break;
        int rc = exec(vm, in, &ip);
        if (rc) return rc;
    }
    return 0;
}

static int exec(vo_vm *vm, ins_t in, size_t *ip) {
    int rc = 0;
    const uint32_t d = in.dst, a = in.a, b = in.b;
    switch (in.op) {
    case OP_SHAPE: return 0;
    case OP_COPY: case OP_SAVE: case OP_LOAD: {
        NEED(NEL(d) >= NEL(a), "COPY: dst smaller than src"); /* executor guard */
        P(cd, d);
        P(ca, a);
        memmove(cd, ca, NEL(a) * 4);
        return 0;
    }
    case OP_GEMM: { /* core/src/interp.rs:734-813 */
        SHAPE(a, m, k);
        SHAPE(b, brows, bcols);
        int nt = (in.fl & FL_TRANS_B) == 0, acc = (in.fl & FL_ACC) != 0;
        uint8_t bt = DT(b);
        size_t n = nt ? brows : bcols;
        if (bt == DT_BF16 || bt == DT_I8) {
            NEED(nt, "%s NN gemm unimplemented", bt == DT_I8 ? "int8" : "bf16");
            NEED(!acc, "%s acc gemm unimplemented", bt == DT_I8 ? "int8" : "bf16");
        }
        if (bt == DT_I8) {
            NEED(in.dt < vm->n_slots && DT(in.dt) == DT_F32, "int8 gemm: scale slot must be f32");
            NEED(NEL(in.dt) >= brows, "int8 gemm: scale shorter than N rows");
        }
        NEED(NEL(d) >= m * n && brows * bcols >= n * k, "GEMM: operand extents"); /* executor guard */
        P(cc, d);
        P(ca, a);
        if (bt == DT_BF16) {
            P(cb, b);
            vo_gemm_nt_bf16(ca, (const uint16_t *)cb, cc, m, brows, k);
        } else if (bt == DT_I8) {
            P(cb, b);
            P(cs, in.dt);
            vo_gemm_nt_int8(ca, (const int8_t *)cb, cs, cc, m, brows, k);
        } else {
            NEED(bt == DT_F32, "gemm operand dtype unsupported");
            P(cb, b);
            if (nt) vo_gemm_nt(ca, cb, cc, m, brows, k, acc);
            else vo_gemm(ca, cb, cc, m, bcols, k, acc);
        }
        return 0;
    }
    case OP_GEMV: { /* :815-827 */
        SHAPE(a, m, k);
        NEED(NEL(b) >= k && NEL(d) >= m, "GEMV: operand extents");
        P(ca, a);
        P(cb, b);
        P(cc, d);
        for (size_t i = 0; i < m; ++i) {
            float s = 0.0f;
            for (size_t p = 0; p < k; ++p) s += ca[i * k + p] * cb[p];
            cc[i] = s;
        }
        return 0;
    }
    case OP_EWADD: case OP_EWMUL: case OP_EWSUB: case OP_EWDIV: { /* :829-883 */
        SHAPE(a, r, c);
        SHAPE(b, br, bc);
        NEED(NEL(d) >= r * c, "EW: dst smaller than a");
        P(ca, a);
        P(cb, b);
        P(cc, d);
        if (br == r && bc == c) {
            vo_ew_op(cc, ca, cb, r * c, in.op);
            return 0;
        }
        for (size_t i = 0; i < r; ++i)
            for (size_t j = 0; j < c; ++j) {
                float y;
                if (br == r && bc == 1) y = cb[i];
                else if (br == 1 && bc == c) y = cb[j];
                else if (br * bc == 1) y = cb[0];
                else return fail(vm, 8, "EW shape mismatch");
                float x = ca[i * c + j];
                cc[i * c + j] = in.op == OP_EWADD ? x + y : in.op == OP_EWMUL ? x * y
                              : in.op == OP_EWSUB ? x - y : x / y;
            }
        return 0;
    }
    case OP_ACT: { /* :885-892 */
        SHAPE(d, r, c);
        NEED(NEL(a) >= r * c, "ACT: src smaller than dst");
        P(cd, d);
        P(ca, a);
        memmove(cd, ca, r * c * 4);
        vo_act(cd, r * c, in.fl == 0 ? 0 : in.fl);
        return 0;
    }
    case OP_LN: { /* :894-905 */
        SHAPE(a, r, c);
        NEED(NEL(d) >= r * c && NEL(b) >= c && NEL(in.dt) >= c, "LN: operand extents");
        P(cd, d);
        P(ca, a);
        P(g, b);
        P(bias, in.dt);
        memmove(cd, ca, r * c * 4);
        vo_layernorm(cd, g, bias, r, c, vm->ln_eps);
        return 0;
    }
    case OP_LN_EPS: {
        P(cd, d);
        vm->ln_eps = cd[0];
        return 0;
    }
    case OP_RMSNORM: { /* :921-931 */
        SHAPE(a, r, c);
        NEED(NEL(d) >= r * c && NEL(b) >= c, "RMSNORM: operand extents");
        P(cd, d);
        P(ca, a);
        P(g, b);
        P(eps, in.dt);
        vo_rmsnorm(cd, ca, g, r, c, eps[0]);
        return 0;
    }
    case OP_PUSH: { /* :940-953 */
        SHAPE(a, sr, sc);
        SHAPE(d, str_, stc);
        NEED(sr * sc == stc, "PUSH: src elems != stack row width");
        NEED((size_t)b < str_, "PUSH: step past the stack");
        P(cs, a);
        P(cd, d);
        memmove(cd + (size_t)b * stc, cs, stc * 4);
        return 0;
    }
    case OP_POP: {
        SHAPE(d, dr, dc);
        SHAPE(a, str_, stc);
        NEED(dr * dc == stc, "POP: dst elems != stack row width");
        NEED((size_t)b < str_, "POP: step past the stack");
        P(cs, a);
        P(cd, d);
        memmove(cd, cs + (size_t)b * stc, stc * 4);
        return 0;
    }
    case OP_STACK_INIT: {
        P(ca, a);
        memset(ca, 0, NEL(a) * 4);
        return 0;
    }
    case OP_SOFTMAX: { /* :974-980; executor extension: live width from slot b */
        SHAPE(d, r, c);
        NEED(NEL(a) >= r * c, "SOFTMAX: src smaller than dst");
        P(cd, d);
        P(ca, a);
        memmove(cd, ca, r * c * 4);
        if (in.fl & FL_RUNTIME) {
            size_t live;
            if ((rc = slot_index(vm, b, c + 1, &live, "SOFTMAX: live width"))) return rc;
            for (size_t i = 0; i < r; ++i) {
                float *row = cd + i * c;
                float mx = -INFINITY;
                for (size_t j = 0; j < live; ++j)
                    if (row[j] > mx) mx = row[j];
                float sum = 0.0f;
                for (size_t j = 0; j < live; ++j) {
                    float e = vo_exp_f(row[j] - mx);
                    row[j] = e;
                    sum += e;
                }
                float inv = 1.0f / sum;
                for (size_t j = 0; j < live; ++j) row[j] *= inv;
                for (size_t j = live; j < c; ++j) row[j] = 0.0f;
            }
            return 0;
        }
        vo_softmax(cd, r, c, (in.fl & FL_CAUSAL) != 0);
        return 0;
    }
    case OP_OUTER: { /* :982-993 */
        SHAPE(a, vr, vc);
        SHAPE(b, kr, kc);
        size_t m = vr == 1 ? vc : vr, nn = kr == 1 ? kc : kr;
        NEED(NEL(d) >= m * nn, "OUTER: dst smaller than m x n");
        P(cs, d);
        P(cv, a);
        P(ck, b);
        vo_outer(cs, cv, ck, m, nn, 1.0f);
        return 0;
    }
    case OP_TOPK_THRESH: { /* :995-1004 */
        SHAPE(a, r, c);
        NEED(NEL(d) >= r, "TOPK_THRESH: dst shorter than rows");
        NEED(c <= 8192, "TOPK_THRESH: row wider than 8192");
        P(ca, a);
        P(cd, d);
        size_t k = in.fl < c ? in.fl : c;
        for (size_t i = 0; i < r; ++i) cd[i] = topk_thresh(ca + i * c, c, k);
        return 0;
    }
    case OP_LAYERB: { /* :1019-1043 */
        P(ca, a);
        float d0 = ca[0];
        if (d0 >= 0.0f) vm->layer_base += (size_t)d0;
        else {
            size_t back = (size_t)(-d0);
            vm->layer_base = back > vm->layer_base ? 0 : vm->layer_base - back;
        }
        return 0;
    }
    case OP_EWMAX: case OP_GEMASK: case OP_EXP: case OP_NEG: case OP_LOG: case OP_SIN:
    case OP_COS: case OP_CLAMP: { /* :1045-1065, 1133-1157, 1273-1318 */
        SHAPE(a, r, c);
        size_t n = r * c;
        NEED(NEL(d) >= n, "elementwise: dst smaller than src");
        if (in.op == OP_EWMAX) NEED(NEL(b) >= n, "EWMAX: b smaller than a");
        if (in.op == OP_CLAMP) NEED(NEL(b) >= 2, "CLAMP: bounds slot needs 2 values");
        P(ca, a);
        P(cd, d);
        float *cb = NULL;
        if (in.op == OP_EWMAX || in.op == OP_CLAMP) {
            cb = sp(vm, b, &rc);
            if (rc) return rc;
        }
        for (size_t i = 0; i < n; ++i) {
            float x = ca[i];
            switch (in.op) {
            case OP_EWMAX: { float y = cb[i]; cd[i] = x > y ? x : y; } break;
            case OP_GEMASK: cd[i] = x >= 0.0f ? 1.0f : 0.0f; break;
            case OP_EXP: cd[i] = vo_exp_f(x); break;
            case OP_NEG: cd[i] = -x; break;
            case OP_LOG: cd[i] = vo_ln_f(x); break;
            case OP_SIN: cd[i] = vo_sin_f(x); break;
            case OP_COS: cd[i] = vo_cos_f(x); break;
            default: { float lo = cb[0], hi = cb[1]; cd[i] = x < lo ? lo : x > hi ? hi : x; }
            }
        }
        return 0;
    }
    case OP_MASK_MUL: { /* :1067-1083 */
        SHAPE(d, r, c);
        SHAPE(b, brr, bcols);
        NEED(NEL(a) >= r * c &&
                 (r == 0 || (bcols == 1 ? NEL(b) >= r : NEL(b) >= (r - 1) * bcols + c)),
             "MASK_MUL: operand extents");
        (void)brr;
        P(cd, d);
        P(ca, a);
        P(cb, b);
        for (size_t i = 0; i < r; ++i)
            for (size_t j = 0; j < c; ++j)
                cd[i * c + j] = ca[i * c + j] * (bcols == 1 ? cb[i] : cb[i * bcols + j]);
        return 0;
    }
    case OP_JMP: *ip = d; return 0;
    case OP_CMPLE: {
        P(ca, a);
        P(cb, b);
        if (ca[0] <= cb[0]) *ip = d;
        return 0;
    }
    case OP_LOOP_CNT: { /* :1108-1131 */
        SHAPE(a, r, c);
        (void)c;
        NEED(r == 1, "LOOP_CNT: ctr must be [1,N]");
        NEED(d < *ip, "LOOP_CNT: target must be back");
        P(ca, a);
        float nv = ca[0] - 1.0f;
        ca[0] = nv;
        if (nv > 0.0f) *ip = d;
        return 0;
    }
    case OP_ROPE: { /* :1159-1223; executor extension: position from slot dt */
        SHAPE(a, r, c);
        NEED(c >= 2 && (c & 1) == 0, "ROPE: hd must be even >= 2");
        NEED(NEL(d) >= r * c, "ROPE: dst smaller than src");
        P(th, b);
        NEED(th[0] > 0.0f, "ROPE: theta must be > 0");
        size_t pos0 = in.dt;
        if (in.fl & FL_RUNTIME)
            if ((rc = slot_index(vm, in.dt, 1u << 24, &pos0, "ROPE: position"))) return rc;
        P(cd, d);
        P(ca, a);
        return vo_rope(cd, ca, r, c, th[0], (uint32_t)pos0) ? fail(vm, 9, "ROPE guard") : 0;
    }
    case OP_SCALE: { /* :1225-1235 */
        SHAPE(d, r, c);
        NEED(NEL(a) >= r * c, "SCALE: src smaller than dst");
        P(cd, d);
        P(ca, a);
        P(cb, b);
        float s = cb[0];
        memmove(cd, ca, r * c * 4);
        for (size_t i = 0; i < r * c; ++i) cd[i] *= s;
        return 0;
    }
    case OP_PRINT: {
        P(cd, d);
        print_out(vm, cd, NEL(d));
        return 0;
    }
    case OP_BIAS: { /* :1259-1269 */
        SHAPE(d, r, c);
        NEED(NEL(a) >= c, "BIAS: bias shorter than the row");
        P(cd, d);
        P(cb, a);
        vo_bias(cd, cb, r, c);
        return 0;
    }
    case OP_EMB: { /* :1351-1436 */
        SHAPE(a, r, c);
        NEED(NEL(d) >= c, "EMB: dst shorter than a row");
        size_t row;
        if ((rc = slot_index(vm, b, r, &row, "EMB: row index"))) return rc;
        P(cd, d);
        P(ca, a);
        if (DT(a) == DT_BF16) {
            const uint16_t *src = (const uint16_t *)ca + row * c;
            for (size_t i = 0; i < c; ++i) cd[i] = vo_bf16_to_f32(src[i]);
        } else {
            NEED(DT(a) == DT_F32, "EMB table dtype unsupported");
            for (size_t i = 0; i < c; ++i) cd[i] = ca[row * c + i];
        }
        return 0;
    }
    case OP_BMM: { /* :1440-1466 */
        SHAPE(a, abm, k);
        SHAPE(b, bk, nn);
        P(ca, a);
        P(cb, b);
        P(cc, d);
        if (bk == k) {
            NEED(NEL(d) >= abm * nn, "BMM: dst too small");
            vo_gemm(ca, cb, cc, abm, nn, k, 0);
            return 0;
        }
        NEED(k > 0 && bk % k == 0 && bk / k > 0 && abm % (bk / k) == 0, "BMM: batch shapes");
        size_t bs = bk / k, m = abm / bs;
        NEED(NEL(d) >= bs * m * nn, "BMM: dst too small");
        for (size_t bi = 0; bi < bs; ++bi)
            vo_gemm(ca + bi * m * k, cb + bi * k * nn, cc + bi * m * nn, m, nn, k, 0);
        return 0;
    }
    case OP_TRANSPOSE: { /* :1468-1484 */
        SHAPE(a, m, c);
        NEED(NEL(d) >= m * c, "TRANSPOSE: dst smaller than src");
        P(ca, a);
        P(cd, d);
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < c; ++j) cd[j * m + i] = ca[i * c + j];
        return 0;
    }
    case OP_SLICE: { /* :1486-1497 */
        SHAPE(d, dr, dc);
        SHAPE(a, sr, sc);
        size_t off = b;
        NEED(dr == 0 || dc == 0 || (dr - 1) * sc + off + dc <= sr * sc, "SLICE: reads past src");
        P(ca, a);
        P(cd, d);
        for (size_t i = 0; i < dr; ++i)
            for (size_t j = 0; j < dc; ++j) cd[i * dc + j] = ca[i * sc + off + j];
        return 0;
    }
    case OP_CONCAT: { /* :1499-1513 */
        SHAPE(a, r, ac);
        SHAPE(b, rb, bc);
        NEED(rb >= r && NEL(d) >= r * (ac + bc), "CONCAT: operand extents");
        P(pa, a);
        P(pb, b);
        P(pd, d);
        for (size_t i = 0; i < r; ++i) {
            for (size_t j = 0; j < ac; ++j) pd[i * (ac + bc) + j] = pa[i * ac + j];
            for (size_t j = 0; j < bc; ++j) pd[i * (ac + bc) + ac + j] = pb[i * bc + j];
        }
        return 0;
    }
    case OP_WRITECOL: { /* :1515-1533; executor extension: column from slot dt */
        SHAPE(d, dr, dc);
        SHAPE(a, sr, sc);
        size_t off = b;
        if (in.fl & FL_RUNTIME)
            if ((rc = slot_index(vm, in.dt, dc + 1, &off, "WRITECOL: column"))) return rc;
        NEED(off + sc <= dc, "WRITECOL: off + src.cols exceeds dst row width");
        NEED(sr >= dr, "WRITECOL: src has fewer rows than dst"); /* executor guard */
        P(ca, a);
        P(cd, d);
        for (size_t i = 0; i < dr; ++i)
            for (size_t j = 0; j < sc; ++j) cd[i * dc + off + j] = ca[i * sc + j];
        return 0;
    }
    case OP_SUM: { /* :1535-1546 */
        SHAPE(a, r, c);
        NEED(NEL(d) >= r, "SUM: dst shorter than rows");
        P(ca, a);
        P(cd, d);
        for (size_t i = 0; i < r; ++i) {
            float s = 0.0f;
            for (size_t j = 0; j < c; ++j) s += ca[i * c + j];
            cd[i] = s;
        }
        return 0;
    }
    case OP_MAX: { /* :1584-1621 */
        SHAPE(a, r, c);
        SHAPE(d, dr, dc);
        NEED(c != 0 && dr != 0 && dc != 0, "MAX: src or dst slot has width 0");
        NEED(dr == r && dc == 1, "MAX: dst must be [rows,1]");
        P(ca, a);
        P(cd, d);
        for (size_t i = 0; i < r; ++i) {
            const float *row = ca + i * c;
            float m = row[0];
            for (size_t j = 1; j < c; ++j)
                if (row[j] > m) m = row[j];
            cd[i] = m;
        }
        return 0;
    }
    case OP_TOPK_IDX: { /* :1649-1681 */
        SHAPE(a, r, c);
        SHAPE(d, dr, dc);
        NEED(r && c && dr && dc, "TOPK_IDX: src or dst slot has width 0");
        NEED(dr == 1 && dc == 1, "TOPK_IDX: dst must be [1,1]");
        P(ca, a);
        P(cd, d);
        return vo_topk_idx(ca, r, c, cd) ? fail(vm, 9, "TOPK_IDX guard") : 0;
    }
    case OP_TOPK_BY_STRENGTH: { /* :1743-1955 */
        SHAPE(a, sr, sc);
        SHAPE(d, dr, dc);
        NEED(sr && sc && dr && dc, "TOPK_BY_STRENGTH: src or dst slot has width 0");
        size_t k;
        int seg = (in.fl & FL_SELGATE) != 0;
        if (seg) {
            NEED(sc >= 1 && dc % 2 == 0, "TOPK_BY_STRENGTH: segmented dst must be [n,2k]");
            NEED(dr == sr, "TOPK_BY_STRENGTH: segmented dst rows != src rows");
        } else {
            NEED(dc == 2, "TOPK_BY_STRENGTH: dst must be [L,2]");
            NEED(dr >= sr * sc, "TOPK_BY_STRENGTH: dst needs L rows");
        }
        P(cs, a);
        P(ck, b);
        P(cd, d);
        float kf = ck[0];
        NEED(kf >= 0.0f, "TOPK_BY_STRENGTH: k is negative or NaN");
        k = as_usize(kf);
        size_t hit[TOPK_MAX_L];
        char taken[TOPK_MAX_L];
        if (seg) {
            size_t kseg = dc / 2;
            NEED(k <= sc, "TOPK_BY_STRENGTH: k > row width");
            NEED(k <= kseg, "TOPK_BY_STRENGTH: k > dst segment width");
            NEED(sc <= TOPK_MAX_L, "TOPK_BY_STRENGTH: row width exceeds the bitmap (2048)");
            for (size_t r = 0; r < sr; ++r) {
                const float *row = cs + r * sc;
                float *out = cd + r * dc;
                size_t nk = select_topk(row, sc, k, hit, taken);
                for (size_t i = 0; i < kseg; ++i) {
                    out[2 * i] = i < nk ? (float)hit[i] : 0.0f;
                    out[2 * i + 1] = i < nk ? row[hit[i]] : 0.0f;
                }
            }
            return 0;
        }
        size_t l = sr * sc;
        NEED(k <= l, "TOPK_BY_STRENGTH: k > L");
        NEED(l <= TOPK_MAX_L, "TOPK_BY_STRENGTH: L exceeds the selection bitmap (2048)");
        size_t nk = select_topk(cs, l, k, hit, taken);
        for (size_t i = 0; i < l; ++i) {
            cd[2 * i] = i < nk ? (float)hit[i] : 0.0f;
            cd[2 * i + 1] = i < nk ? cs[hit[i]] : 0.0f;
        }
        return 0;
    }
    case OP_SPARSE_MATVEC: { /* :2058-2346 */
        uint32_t wslot = in.fl & 0x3Fu, xslot = in.dt;
        int want_nnz = (in.fl & FL_NNZ) != 0, selgate = (in.fl & FL_SELGATE) != 0;
        SHAPE(a, orows, ocols);
        SHAPE(b, srows, scols);
        SHAPE(d, dr, dc);
        NEED(orows && ocols && srows && scols, "SPARSE_MATVEC: offsets or src slot has width 0");
        NEED(dr && dc, "SPARSE_MATVEC: dst slot has width 0");
        uint32_t selslot = selgate ? b + 1 : b;
        NEED(!selgate || selslot < vm->n_slots, "SPARSE_MATVEC: sel slot (src+1) does not exist");
        SHAPE(selslot, serows, secols);
        NEED(!selgate || (secols != 0 && secols % 2 == 0), "SPARSE_MATVEC: selgate needs an even sel width");
        NEED(ocols == 1 && scols == 1, "SPARSE_MATVEC: offsets and src must be column vectors");
        NEED(orows >= 2, "SPARSE_MATVEC: offsets must have n_neurons+1 entries");
        size_t n = orows - 1, nnz = srows;
        NEED(dc == 1 && dr >= n, "SPARSE_MATVEC: dst must be [n_neurons(,1)]");
        NEED(!want_nnz || dr >= n + 1, "SPARSE_MATVEC: nnz needs dst to be [n_neurons+1]");
        size_t nx = NEL(xslot);
        NEED(nx != 0, "SPARSE_MATVEC: x slot (dt) has width 0");
        NEED(NEL(wslot) != 0, "SPARSE_MATVEC: weight slot (fl) has width 0");
        NEED(NEL(wslot) >= nnz, "SPARSE_MATVEC: weight slot shorter than src"); /* executor guard */
        P(co, a);
        P(cs, b);
        P(cw, wslot);
        P(cx, xslot);
        P(cd, d);
        size_t done = 0;
        for (size_t j = 0; j < n; ++j) {
            size_t o0 = as_usize(co[j]), o1 = as_usize(co[j + 1]);
            NEED(o1 <= nnz && o0 <= o1, "SPARSE_MATVEC: offsets out of range j=%zu o0=%zu o1=%zu nnz=%zu",
                 j, o0, o1, nnz);
            if (o0 == o1) {
                cd[j] = 0.0f;
                continue;
            }
            float acc = 0.0f;
            if (selgate) {
                P(csel, selslot);
                size_t segw = secols / 2;
                NEED(segw && (j + 1) * segw * 2 <= serows * secols,
                     "SPARSE_MATVEC: sel table too small for n_neurons");
                int first = 1;
                for (size_t q = 0; q < segw; ++q) {
                    size_t rel = as_usize(csel[(j * segw + q) * 2]);
                    if (q > 0 && rel == 0) break;
                    size_t idx = o0 + rel;
                    NEED(idx >= o0 && idx < o1, "SPARSE_MATVEC: sel index outside its CSR row");
                    size_t sid = as_usize(cs[idx]);
                    NEED(sid < nx, "SPARSE_MATVEC: src_id out of range");
                    float term = cw[idx] * cx[sid];
                    acc = first ? term : acc + term;
                    first = 0;
                    ++done;
                }
                cd[j] = acc;
                continue;
            }
            for (size_t t = o0; t < o1; ++t) {
                size_t sid = as_usize(cs[t]);
                NEED(sid < nx, "SPARSE_MATVEC: src_id out of range");
                float term = cw[t] * cx[sid];
                acc = t == o0 ? term : acc + term;
                ++done;
            }
            cd[j] = acc;
        }
        if (want_nnz) cd[n] = (float)done;
        return 0;
    }
    case 60: case 61: case 62: case 63: case 64: case 65: case 66: case 67: case 68:
    case 69: case 70: case 80: case 81: case 82: case 83: case 84:
        return fail(vm, 6, "train feature disabled");
    default:
        return fail(vm, 5, "unimpl op %u", in.op);
    }
}

/* --------------------------------------------------------------- queries */
int vo_vm_find(const vo_vm *vm, uint32_t hash, uint32_t *slot) {
    for (size_t i = 0; i < vm->n_slots; ++i)
        if (vm->names[i] == hash) {
            *slot = (uint32_t)i;
            return 0;
        }
    return 7;
}
int vo_vm_slot(vo_vm *vm, uint32_t i, float **p, uint32_t *rows, uint32_t *cols,
               uint8_t *dtype) {
    int rc = 0;
    float *q = sp(vm, i, &rc);
    if (rc) return rc;
    *p = q;
    *rows = vm->slots[i].rows;
    *cols = vm->slots[i].cols;
    *dtype = vm->slots[i].dtype;
    return 0;
}
size_t vo_vm_output(const vo_vm *vm, float *dst, size_t cap) {
    size_t n = vm->n_out < cap ? vm->n_out : cap;
    if (dst && n) memcpy(dst, vm->out, n * sizeof(float));
    return vm->n_out;
}
const char *vo_vm_message(const vo_vm *vm) { return vm->msg; }

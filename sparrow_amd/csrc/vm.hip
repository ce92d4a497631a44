// vm.hip -- device-resident executor of .vmb programs: the reference VM's
// loader and interpreter (core/src/interp.rs) with every tensor in HBM.
//
// Load (Vm::load_impl, core/src/interp.rs:108-236): the image's TEXT and META
// are parsed on the host; the constant pool is uploaded to the device once
// (read-only there; a mapped weights region passed to vmlm_vm_load is shared
// by every VM loaded over the same host range); the activation, state and
// gradient arenas are allocated on the device, 64-byte aligned and zeroed;
// every slot is bound to a byte offset in its region (bind_slots :351-396);
// the load-time audit (audit_const_dtypes :241-348) runs over TEXT.
//
// Run (Vm::run :720-2370): the host walks TEXT and enqueues each opcode's
// kernels on the VM's stream with the slots' device addresses; constants
// are addressed through the layer base (const_ptr :434-467). Scalars that
// steer the host (LOOP_CNT / CMPLE / LAYERB operands, RMSNORM / LN eps, ROPE
// theta, SCALE factor) are read back from the device; values of constant
// slots are cached per device address since the pool never changes.
// Index guards that depend on device data (EMB rows, SPARSE_MATVEC offsets
// and sources, runtime columns and positions) set the library's device
// guard flag and skip the offending work; run() then returns 9.
//
// Status codes are the reference's exit codes: 9 guard, 5 unimplemented op,
// 6 training op (the engine's build without the train feature), 3 bad magic,
// 2 device failure. Beyond the reference, operand extents are checked
// against the slots before a kernel touches them (9 where the reference
// would read neighbouring memory), and bit 6 of `fl` gives three opcodes a
// runtime operand read from a slot (ROPE position from slot `dt`, WRITECOL
// column from slot `dt`, SOFTMAX live width from slot `b`).
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

namespace vmlm {

enum : uint8_t {
    VOP_HALT = 0, VOP_COPY = 2, VOP_TRANSPOSE = 4, VOP_CONCAT = 5, VOP_SLICE = 6,
    VOP_LAYERB = 7, VOP_GEMM = 10, VOP_BMM = 11, VOP_OUTER = 12, VOP_GEMV = 13, VOP_EMB = 14,
    VOP_EWADD = 20, VOP_EWMUL = 21, VOP_EWSUB = 22, VOP_EWDIV = 23, VOP_SCALE = 24,
    VOP_ACT = 25, VOP_EXP = 26, VOP_LOG = 27, VOP_CLAMP = 28, VOP_NEG = 29, VOP_LN = 30,
    VOP_RMSNORM = 31, VOP_SUM = 32, VOP_MAX = 34, VOP_SOFTMAX = 36, VOP_MASK_MUL = 40,
    VOP_TOPK_THRESH = 41, VOP_TOPK_IDX = 42, VOP_JMP = 46, VOP_CMPLE = 47, VOP_SAVE = 49,
    VOP_LOAD = 50, VOP_PRINT = 51, VOP_SHAPE = 52, VOP_BIAS = 53, VOP_WRITECOL = 71,
    VOP_EWMAX = 72, VOP_GEMASK = 73, VOP_LN_EPS = 85, VOP_PUSH = 86, VOP_POP = 87,
    VOP_STACK_INIT = 88, VOP_LOOP_CNT = 89, VOP_ROPE = 90, VOP_SIN = 91, VOP_COS = 92,
    VOP_TOPK_BY_STRENGTH = 93, VOP_SPARSE_MATVEC = 94,
};
enum : uint8_t { VDT_F32 = 0, VDT_F16 = 1, VDT_I8 = 2, VDT_I32 = 3, VDT_BF16 = 4 };
enum : uint32_t { VSLOT_CONST = 0, VSLOT_ACT = 1, VSLOT_STATE = 2, VSLOT_GRAD = 3,
                  VSLOT_PARAM = 4 };
constexpr uint8_t VFL_ACC = 1, VFL_TRANS_B = 2, VFL_CAUSAL = 16, VFL_NNZ = 64,
                  VFL_SELGATE = 128, VFL_RUNTIME = 64;
constexpr size_t VM_TOPK_MAX_L = 2048;

static size_t vdtype_size(uint8_t dt) {
    switch (dt) {
    case VDT_F32: case VDT_I32: return 4;
    case VDT_BF16: case VDT_F16: return 2;
    case VDT_I8: return 1;
    default: return 0;
    }
}

// ------------------------------------------------------------------ kernels
// An f32 value in device memory used as a count, column or position:
// non-negative, integral and below `limit` (the EMB rule); else the guard
// flag is set and -1 returned.
__device__ __forceinline__ long dev_index(const float *p, long limit, int *guard) {
    const float v = *p;
    bool bad = !(v >= 0.0f) || v >= (float)limit;
    long u = 0;
    if (!bad) {
        u = (long)v;
        bad = (float)u != v;
    }
    if (bad) {
        atomicOr(guard, 1);
        return -1;
    }
    return u;
}

// Device guard codes (bits of the VM's guard flag), reported by run() with
// the interpreter's message for the first in this order.
enum VmGuard : int { VG_INDEX = 1, VG_OFFSETS = 2, VG_SEL = 4, VG_SRC = 8 };

// Rust's `f as usize` (saturating: NaN and negatives give 0), the cast the
// reference applies to f32-held offsets and ids before checking them.
__device__ __forceinline__ size_t as_usize(float f) {
    return f > 0.0f ? (f >= 1.8446744e19f ? ~(size_t)0 : (size_t)f) : 0;
}

// EWADD/EWMUL/EWSUB/EWDIV with the broadcast forms of core/src/interp.rs:
// 829-883: b is [r,1] (mode 1), [1,c] (mode 2) or one value (mode 3).
__global__ __launch_bounds__(256) void vm_ew_bcast_kernel(float *d, const float *a,
                                                          const float *b, size_t r, size_t c,
                                                          int mode, int op) {
    const size_t n = r * c, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const float x = a[e];
        const float y = mode == 1 ? b[e / c] : mode == 2 ? b[e % c] : b[0];
        d[e] = op == VOP_EWADD ? x + y : op == VOP_EWMUL ? x * y : op == VOP_EWSUB ? x - y : x / y;
    }
}

// EXP / LOG / SIN / COS / NEG / GEMASK / CLAMP / EWMAX (:1045-1065,
// 1133-1157, 1273-1318): the reference's scalar functions, element by element.
__global__ __launch_bounds__(256) void vm_unary_kernel(float *d, const float *a, const float *b,
                                                       size_t n, int op) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const float x = a[e];
        float y;
        switch (op) {
        case VOP_EXP: y = exp_f(x); break;
        case VOP_LOG: y = ln_f(x); break;
        case VOP_SIN: { float s, c; sincos_f(x, &s, &c); y = s; } break;
        case VOP_COS: { float s, c; sincos_f(x, &s, &c); y = c; } break;
        case VOP_NEG: y = -x; break;
        case VOP_GEMASK: y = x >= 0.0f ? 1.0f : 0.0f; break;
        case VOP_CLAMP: { const float lo = b[0], hi = b[1]; y = x < lo ? lo : x > hi ? hi : x; } break;
        default: { const float z = b[e]; y = x > z ? x : z; }  // EWMAX
        }
        d[e] = y;
    }
}

// MASK_MUL (:1067-1083): d[i,j] = a[i,j] * (b[i] or b[i,j]).
__global__ __launch_bounds__(256) void vm_mask_mul_kernel(float *d, const float *a,
                                                          const float *b, size_t r, size_t c,
                                                          size_t bcols) {
    const size_t n = r * c, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const size_t i = e / c, j = e % c;
        d[e] = a[e] * (bcols == 1 ? b[i] : b[i * bcols + j]);
    }
}

// d[j * m + i] = a[i * c + j] (TRANSPOSE, :1468-1484).
__global__ __launch_bounds__(256) void vm_transpose_kernel(float *d, const float *a, size_t m,
                                                           size_t c) {
    const size_t n = m * c, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const size_t j = e / m, i = e % m;
        d[e] = a[i * c + j];
    }
}

// Row-strided copy: d[i * dld + doff + j] = s[i * sld + soff + j] for i < rows,
// j < cols (SLICE, WRITECOL, CONCAT halves, PUSH / POP). With `offp` the
// destination offset is read from the device (WRITECOL with a runtime column)
// and checked against `dlimit` columns.
__global__ __launch_bounds__(256) void vm_copy2d_kernel(float *d, size_t dld, size_t doff,
                                                        const float *s, size_t sld, size_t soff,
                                                        size_t rows, size_t cols,
                                                        const float *offp, size_t dlimit,
                                                        int *guard) {
    if (offp) {
        const long o = dev_index(offp, (long)dlimit + 1, guard);
        if (o < 0 || (size_t)o + cols > dlimit) {
            if (o >= 0) atomicOr(guard, 1);
            return;
        }
        doff = (size_t)o;
    }
    const size_t n = rows * cols, stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const size_t i = e / cols, j = e % cols;
        d[i * dld + doff + j] = s[i * sld + soff + j];
    }
}

// One thread per row, left to right: SUM (:1535-1546), MAX (:1584-1621:
// first element, then strict `>`) and GEMV (:815-827, s += a * b).
__global__ __launch_bounds__(256) void vm_rowwise_kernel(float *d, const float *a, const float *b,
                                                         size_t r, size_t c, int op) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < r; i += (size_t)gridDim.x * 256) {
        const float *row = a + i * c;
        float s;
        if (op == VOP_MAX) {
            s = row[0];
            for (size_t j = 1; j < c; ++j)
                if (row[j] > s) s = row[j];
        } else if (op == VOP_GEMV) {
            s = 0.0f;
            for (size_t j = 0; j < c; ++j) s += row[j] * b[j];
        } else {
            s = 0.0f;
            for (size_t j = 0; j < c; ++j) s += row[j];
        }
        d[i] = s;
    }
}

// SCALE (:1225-1235): d = a * s, s from the device.
__global__ __launch_bounds__(256) void vm_scale_kernel(float *d, const float *a, const float *sp,
                                                       size_t n) {
    const float s = *sp;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) d[e] = a[e] * s;
}

// EMB over an f32 table (:1423-1434); the bf16 table goes through
// emb_bf16_kernel.
__global__ void vm_emb_f32_kernel(float *d, const float *table, size_t rows, size_t cols,
                                  const float *rowf, int *guard) {
    const long row = dev_index(rowf, (long)rows, guard);
    if (row < 0) return;
    for (size_t i = threadIdx.x; i < cols; i += blockDim.x) d[i] = table[(size_t)row * cols + i];
}

// ---------------------------------------------------------------- fused blocks
// The decode loop of the reference's step-looped program repeats two
// opcode runs per head of every layer (tools/p14_gen_build.py:470-560): the
// cache append SLICE k, SLICE v, ROPE, TRANSPOSE x2, WRITECOL x2, and the
// attention SLICE q, ROPE, GEMM (scores), SCALE, SOFTMAX (live width), GEMM
// (context), WRITECOL. The loader recognises such runs over all heads and
// the executor runs each as one launch over the heads with the same results:
// the same rotation (rope_pair, the ROPE step), the same guards on the
// device position and live width, the softmax of vm_softmax_live_kernel
// (block max, exp_f, block sum, times 1 / sum), and the scratch slots left
// holding the last head's values as the opcode run leaves them. The score
// and context dot products are f32 sums in k order (the GEMM kernel's
// order differs; both are within the GEMM contract).
typedef __attribute__((address_space(1))) float gfloat;  // a float in global memory

struct VmKvAppend {
    const float *k, *v;          // [1, nh * hd] rows of k and v
    float *const *kc;            // [nh] caches [hd, cols] (K), then [nh] (V)
    const float *posp;
    float step;
    int hd, cols;
    float *kdh, *vdh, *kdrot, *kdT, *vdT;  // the last head's scratch
};

// One workgroup per head: rotates k at the device position, writes k and v
// into column `pos` of the head's caches.
__global__ __launch_bounds__(64) void vm_kv_append_kernel(VmKvAppend a, int nh, int *guard) {
    const int h = blockIdx.x, half = a.hd / 2;
    const long pos = dev_index(a.posp, 1L << 24, guard);  // ROPE's check
    const long col = dev_index(a.posp, (long)a.cols + 1, guard);  // WRITECOL's
    const bool wr = col >= 0 && col + 1 <= a.cols;
    if (col >= 0 && !wr) atomicOr(guard, 1);
    const float *kr = a.k + (size_t)h * a.hd, *vr = a.v + (size_t)h * a.hd;
    gfloat *kc = (gfloat *)a.kc[h], *vc = (gfloat *)a.kc[nh + h];  // global (from a device table)
    const bool last = h == nh - 1;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float x1 = kr[i], x2 = kr[i + half];
        if (last) {
            a.kdh[i] = x1;
            a.kdh[i + half] = x2;
        }
        if (pos < 0) continue;
        float y1, y2;
        rope_pair(x1, x2, (float)pos, i, a.step, &y1, &y2);
        if (last) {
            a.kdrot[i] = y1;
            a.kdrot[i + half] = y2;
            a.kdT[i] = y1;
            a.kdT[i + half] = y2;
        }
        if (wr) {
            kc[(size_t)i * a.cols + col] = y1;
            kc[(size_t)(i + half) * a.cols + col] = y2;
        }
    }
    for (int i = threadIdx.x; i < a.hd; i += blockDim.x) {
        const float x = vr[i];
        if (last) {
            a.vdh[i] = x;
            a.vdT[i] = x;
        }
        if (wr) vc[(size_t)i * a.cols + col] = x;
    }
}

struct VmHeadAttn {
    const float *q;              // [1, nh * hd]
    float *const *kc;            // [nh] K caches [hd, cols], then [nh] V caches
    const float *posp, *livep, *scalep;
    float step;
    int hd, cols;
    float *att;                  // [1, >= nh * hd]
    float *qdh, *qdrot, *scd, *ctxd;  // the last head's scratch
};
constexpr int VM_ATTN_MAX_COLS = 8192;

// One workgroup of 256 threads per head: q rotated into LDS, the scores of
// every cached column (sum over k in order) times the scale, the softmax of
// the first `live` columns (zeros past them), and the context over all
// columns, as the GEMM-SCALE-SOFTMAX-GEMM run computes them.
// FAST (hd = 64, at most 256 columns): every K and V value the thread uses
// is loaded before the query is rotated (none depends on it), so the
// workgroup waits for memory once instead of once per phase; the sums run in
// the same order, so the results are the same bits.
// APPEND (with FAST): the cache append of the same heads first (the append
// run just before the attention run, over the same caches): the workgroup
// writes its head's new K / V column as vm_kv_append_kernel does and uses
// the values it wrote in place of the ones it loaded from that column.
// NP > 1 (with FAST): NP workgroups per head, each forming the head's
// scores and softmax (the same bits in each) and the context rows of its
// part, 64 / NP of them; workgroup b takes head 8 (b / 32) + b % 8, part
// (b / 8) % 4, so a head's workgroups share an XCD (and its L2). Part 0
// writes the scratch slots and the appended column.
template <bool FAST, bool APPEND = false, int NP = 1>
__global__ __launch_bounds__(256) void vm_head_attn_kernel(VmHeadAttn a, int nh, int *guard,
                                                           VmKvAppend ap = {}) {
    extern __shared__ float sm[];     // q[hd], p[cols]
    __shared__ float red[4];
    __shared__ float knew[APPEND ? 64 : 1], vnew[APPEND ? 64 : 1];
    static_assert(NP == 1 || (FAST && NP == 4), "parts of the FAST form: 4");
    constexpr int VR = FAST ? 16 / NP : 1;  // V rows per wave
    float *qs = sm, *pr = sm + a.hd;
    const int bx = (int)blockIdx.x;
    const int h = NP > 1 ? ((bx >> 5) << 3) | (bx & 7) : bx, part = NP > 1 ? (bx >> 3) & 3 : 0;
    if (h >= nh) return;  // the grid's last group of 8 heads may be partial
    const int half = a.hd / 2, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int rbase = part * (64 / NP);     // this workgroup's first context row
    const bool p0 = part == 0;
    // the cache addresses come from a device table, so the compiler cannot
    // tell they are global: global pointers keep the loads global (flat
    // loads would make every counter wait drain the LDS traffic too)
    const gfloat *K = (const gfloat *)a.kc[h], *V = (const gfloat *)a.kc[nh + h];
    float kv[FAST ? 64 : 1], vv[VR][FAST ? 4 : 1];
    static_assert(FAST || !APPEND, "the append joins the FAST form");
    // APPEND: the position and the new k / v values are read before the
    // cache rows, so they arrive first
    long apos = -1, col = -1;
    float ax1 = 0.0f, ax2 = 0.0f, avx = 0.0f;
    if constexpr (APPEND) {
        apos = dev_index(ap.posp, 1L << 24, guard);
        col = dev_index(ap.posp, (long)ap.cols + 1, guard);
        if (tid < 32) {
            ax1 = ap.k[(size_t)h * 64 + tid];
            ax2 = ap.k[(size_t)h * 64 + tid + 32];
        } else if (tid >= 64 && tid < 128) {
            avx = ap.v[(size_t)h * 64 + tid - 64];
        }
    }
    if constexpr (FAST) {
        // column tid of every K row; columns lane + 64 i of V rows w + 4 j
#pragma unroll
        for (int k = 0; k < 64; ++k) kv[k] = tid < a.cols ? K[(size_t)k * a.cols + tid] : 0.0f;
#pragma unroll
        for (int j = 0; j < VR; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = lane + 64 * i;
                vv[j][i] = c < a.cols ? V[(size_t)(rbase + w + 4 * j) * a.cols + c] : 0.0f;
            }
    }
    if constexpr (APPEND) {
        // vm_kv_append_kernel's work for this head (hd = 64), the new column
        // also kept in LDS
        const bool wr = col >= 0 && col + 1 <= ap.cols;
        if (col >= 0 && !wr && tid == 0) atomicOr(guard, 1);
        const bool lastk = h == nh - 1 && p0;
        gfloat *kc = (gfloat *)ap.kc[h], *vc = (gfloat *)ap.kc[nh + h];
        if (tid < 32) {
            const float x1 = ax1, x2 = ax2;
            if (lastk) {
                ap.kdh[tid] = x1;
                ap.kdh[tid + 32] = x2;
            }
            if (apos >= 0) {
                float y1, y2;
                rope_pair(x1, x2, (float)apos, tid, ap.step, &y1, &y2);
                if (lastk) {
                    ap.kdrot[tid] = y1;
                    ap.kdrot[tid + 32] = y2;
                    ap.kdT[tid] = y1;
                    ap.kdT[tid + 32] = y2;
                }
                if (wr && p0) {
                    kc[(size_t)tid * ap.cols + col] = y1;
                    kc[(size_t)(tid + 32) * ap.cols + col] = y2;
                }
                knew[tid] = y1;
                knew[tid + 32] = y2;
            }
        } else if (tid >= 64 && tid < 128) {
            const int i = tid - 64;
            const float x = avx;
            if (lastk) {
                ap.vdh[i] = x;
                ap.vdT[i] = x;
            }
            if (apos >= 0 && wr && p0) vc[(size_t)i * ap.cols + col] = x;
            vnew[i] = x;
        }
        __syncthreads();
        if (apos >= 0 && wr) {  // the column as the append wrote it
            if (tid == col) {
#pragma unroll
                for (int k = 0; k < 64; ++k) kv[k] = knew[k];
            }
#pragma unroll
            for (int j = 0; j < VR; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (lane + 64 * i == col) vv[j][i] = vnew[rbase + w + 4 * j];
        }
    }
    const long pos = dev_index(a.posp, 1L << 24, guard);
    const long live = dev_index(a.livep, (long)a.cols + 1, guard);
    if (pos < 0 || live < 0) return;
    const bool last = h == nh - 1;
    const bool lastp0 = last && p0;  // the scratch slots, from part 0
    const float *qr = a.q + (size_t)h * a.hd;
    for (int i = tid; i < half; i += 256) {
        const float x1 = qr[i], x2 = qr[i + half];
        float y1, y2;
        rope_pair(x1, x2, (float)pos, i, a.step, &y1, &y2);
        qs[i] = y1;
        qs[i + half] = y2;
        if (lastp0) {
            a.qdh[i] = x1;
            a.qdh[i + half] = x2;
            a.qdrot[i] = y1;
            a.qdrot[i + half] = y2;
        }
    }
    __syncthreads();
    const float sc = *a.scalep;
    if constexpr (FAST) {
        if (tid < a.cols) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 64; ++k) s += qs[k] * kv[k];
            pr[tid] = s * sc;
        }
    } else {
        for (int c = tid; c < a.cols; c += 256) {
            float s = 0.0f;
            for (int k = 0; k < a.hd; ++k) s += qs[k] * K[(size_t)k * a.cols + c];
            pr[c] = s * sc;
        }
    }
    __syncthreads();
    const int lim = (int)live;
    float mx = -INFINITY;
    for (int i = tid; i < lim; i += 256) mx = fmaxf(mx, pr[i]);
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int i = tid; i < lim; i += 256) {
        const float e = exp_f(pr[i] - mx);
        pr[i] = e;
        s += e;
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / s;
    for (int i = tid; i < lim; i += 256) pr[i] *= inv;
    for (int i = lim + tid; i < a.cols; i += 256) pr[i] = 0.0f;
    __syncthreads();
    if (lastp0)
        for (int i = tid; i < a.cols; i += 256) a.scd[i] = pr[i];
    // context: wave w takes rows w, w + 4, ...; its lanes sum columns in
    // order per lane, then the wave sums its lanes
    auto store = [&](int r, float t) {
        t = wave_sum_dpp(t);
        if (lane == 0) {
            a.att[(size_t)h * a.hd + r] = t;
            if (last) a.ctxd[r] = t;
        }
    };
    if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < VR; ++j) {
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane + 64 * i < a.cols) t += pr[lane + 64 * i] * vv[j][i];
            store(rbase + w + 4 * j, t);
        }
    } else {
        for (int r = w; r < a.hd; r += 4) {
            const gfloat *vr = V + (size_t)r * a.cols;
            float t = 0.0f;
            for (int c = lane; c < a.cols; c += 64) t += pr[c] * vr[c];
            store(r, t);
        }
    }
}

// ROPE with the position read from the device (runtime position): the
// rotation of rope_kernel, positions pos + row.
__global__ void vm_rope_kernel(float *dst, const float *src, int rows, int hd, float step,
                               const float *posp, int *guard) {
    const long pos = dev_index(posp, 1L << 24, guard);
    if (pos < 0) return;
    const int half = hd / 2;
    const size_t n = (size_t)rows * half, stride = (size_t)gridDim.x * blockDim.x;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += stride) {
        const int row = (int)(idx / half), i = (int)(idx % half);
        const float *sr = src + (size_t)row * hd;
        float *dr = dst + (size_t)row * hd;
        float y1, y2;
        rope_pair(sr[i], sr[i + half], (float)pos + (float)row, i, step, &y1, &y2);
        dr[i] = y1;
        dr[i + half] = y2;
    }
}

// SOFTMAX with the live width read from the device: columns [0, live) as
// the softmax kernel (block max, exp_f, block sum, * 1/sum), the rest 0.
__global__ __launch_bounds__(256) void vm_softmax_live_kernel(float *p, int cols,
                                                              const float *livep, int *guard) {
    __shared__ float sh[4];
    const long live = dev_index(livep, (long)cols + 1, guard);
    if (live < 0) return;
    float *row = p + (size_t)blockIdx.x * cols;
    const int lim = (int)live;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < lim; i += 256) mx = fmaxf(mx, row[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    float s = 0.0f;
    for (int i = threadIdx.x; i < lim; i += 256) {
        const float e = exp_f(row[i] - mx);
        row[i] = e;
        s += e;
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    s = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < lim; i += 256) row[i] *= inv;
    for (int i = lim + threadIdx.x; i < cols; i += 256) row[i] = 0.0f;
}

// ops/src/kernels.rs:1462-1495 topk_thresh per row (one thread, the
// reference's repeated strict-`>` selection; `used` holds c flags per row).
__global__ __launch_bounds__(64) void vm_topk_thresh_kernel(float *d, const float *a, size_t r,
                                                            size_t c, size_t k,
                                                            unsigned char *used) {
    for (size_t i = (size_t)blockIdx.x * 64 + threadIdx.x; i < r; i += (size_t)gridDim.x * 64) {
        const float *x = a + i * c;
        unsigned char *u = used + i * c;
        for (size_t j = 0; j < c; ++j) u[j] = 0;
        float best = -__builtin_inff();
        size_t found = 0;
        while (found < k && found < c) {
            long bi = -1;
            float bv = -__builtin_inff();
            for (size_t j = 0; j < c; ++j)
                if (!u[j] && x[j] > bv) {
                    bv = x[j];
                    bi = (long)j;
                }
            if (bi < 0) break;
            u[bi] = 1;
            best = bv;
            ++found;
        }
        d[i] = best;
    }
}

// TOPK_BY_STRENGTH (:1743-1955) per row of L values (one thread each; the
// flat form is one row of sr * sc): k rounds of "the first untaken value,
// replaced by a strictly greater untaken one", then the chosen indices in
// ascending order with their values; `kseg` output pairs per row, the
// unused ones 0. k comes from the device and is checked there.
__global__ __launch_bounds__(64) void vm_topk_strength_kernel(float *d, size_t dld,
                                                              const float *s, size_t rows,
                                                              size_t L, const float *kp,
                                                              size_t kmax, size_t kseg,
                                                              unsigned char *taken, int *guard) {
    const float kf = *kp;
    const size_t k = as_usize(kf);
    if (!(kf >= 0.0f) || k > kmax) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(guard, 1);
        return;
    }
    for (size_t r = (size_t)blockIdx.x * 64 + threadIdx.x; r < rows; r += (size_t)gridDim.x * 64) {
        const float *row = s + r * L;
        unsigned char *t = taken + r * L;
        for (size_t i = 0; i < L; ++i) t[i] = 0;
        for (size_t q = 0; q < k; ++q) {
            long best = -1;
            float bv = 0.0f;
            for (size_t i = 0; i < L; ++i) {
                if (t[i]) continue;
                const float v = row[i];
                if (best < 0 || v > bv) {
                    bv = v;
                    best = (long)i;
                }
            }
            if (best < 0) break;
            t[best] = 1;
        }
        float *out = d + r * dld;
        size_t o = 0;
        for (size_t i = 0; i < L && o < kseg; ++i)
            if (t[i]) {
                out[2 * o] = (float)i;
                out[2 * o + 1] = row[i];
                ++o;
            }
        for (; o < kseg; ++o) out[2 * o] = out[2 * o + 1] = 0.0f;
    }
}

// SPARSE_MATVEC (:2058-2346), one thread per neuron j over its CSR row
// [off[j], off[j+1]) (or, with selgate, the row-relative survivors listed in
// sel[j]): first term assigned, then acc + w * x[src], in order. Offsets,
// survivors and source ids are checked here (guard flag, neuron skipped);
// each neuron's term count goes to cnt[j].
__global__ __launch_bounds__(64) void vm_sparse_matvec_kernel(
    float *d, const float *off, const float *src, const float *w, const float *x, size_t n,
    size_t nnz, size_t nx, const float *sel, size_t seg, unsigned *cnt, int *guard) {
    for (size_t j = (size_t)blockIdx.x * 64 + threadIdx.x; j < n; j += (size_t)gridDim.x * 64) {
        cnt[j] = 0;
        const size_t o0 = as_usize(off[j]), o1 = as_usize(off[j + 1]);
        if (o1 > nnz || o0 > o1) {
            atomicOr(guard, VG_OFFSETS);
            continue;
        }
        if (o0 == o1) {
            d[j] = 0.0f;
            continue;
        }
        float acc = 0.0f;
        unsigned done = 0;
        int bad = 0;
        if (sel) {
            for (size_t q = 0; q < seg; ++q) {
                const size_t rel = as_usize(sel[(j * seg + q) * 2]);
                if (q > 0 && rel == 0) break;
                const size_t idx = o0 + rel;
                if (idx < o0 || idx >= o1) {
                    bad = VG_SEL;
                    break;
                }
                const size_t sid = as_usize(src[idx]);
                if (sid >= nx) {
                    bad = VG_SRC;
                    break;
                }
                const float term = w[idx] * x[sid];
                acc = done == 0 ? term : acc + term;
                ++done;
            }
        } else {
            for (size_t t = o0; t < o1; ++t) {
                const size_t sid = as_usize(src[t]);
                if (sid >= nx) {
                    bad = VG_SRC;
                    break;
                }
                const float term = w[t] * x[sid];
                acc = t == o0 ? term : acc + term;
                ++done;
            }
        }
        if (bad) {
            atomicOr(guard, bad);
            continue;
        }
        d[j] = acc;
        cnt[j] = done;
    }
}

// The count of terms performed (FL_NNZ): d[0] = sum of cnt, one thread.
__global__ void vm_nnz_kernel(float *d, const unsigned *cnt, size_t n) {
    if (threadIdx.x != 0) return;
    size_t s = 0;
    for (size_t j = 0; j < n; ++j) s += cnt[j];
    d[0] = (float)s;
}

static unsigned vm_blocks(size_t n, unsigned per = 256) {
    size_t b = (n + per - 1) / per;
    return (unsigned)(b < 1 ? 1 : b > 65535 ? 65535 : b);
}

// ------------------------------------------------------------------ pools
// Constant pools on the device, shared by every VM loaded over the same
// mapped host range (vmlm_vm_load with `weights`); an image's own CONST
// region is uploaded privately.
// A swizzled copy (launch_swizzle_w) of an int8 constant: the layout the
// small-row GEMV and the int8-row GEMM read as whole 1 KiB MFMA blocks.
struct SwzConst {
    uint32_t rows, cols;
    int8_t *dev;
};
struct ConstPool {
    const void *host;  // null: private
    size_t len;
    char *dev;
    int refs;
    std::map<size_t, SwzConst> swz;  // by byte offset in the pool (int8 constants never change)
};
static std::mutex g_pool_mu;
static std::vector<ConstPool *> g_pools;
static size_t g_pool_uploads = 0;

static void pool_release(ConstPool *p) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(g_pool_mu);
    if (--p->refs > 0) return;
    for (size_t i = 0; i < g_pools.size(); ++i)
        if (g_pools[i] == p) g_pools.erase(g_pools.begin() + i);
    for (auto &kv : p->swz) (void)hipFree(kv.second.dev);
    (void)hipFree(p->dev);
    delete p;
}

}  // namespace vmlm

using namespace vmlm;

struct VmIns {
    uint8_t op, fl;
    uint16_t dt;
    uint32_t dst, a, b;
};
struct VmSlot {
    size_t off;  // byte offset in its region (constants: in the pool)
    uint32_t rows, cols;
    uint32_t kind;
    uint8_t dtype;
};

// A run of opcodes that the executor launches as one kernel (per-head decode
// runs: vm_kv_append_kernel, vm_head_attn_kernel; GEMMs of one input), or as
// one strided copy per stream (VF_COL_RUN: column-by-column cache writes).
enum VmFuseKind {
    VF_KV_APPEND = 1, VF_HEAD_ATTN = 2, VF_GEMMS = 3, VF_GATE_UP = 4, VF_COL_RUN = 5, VF_GEMM_ADD = 6,
    VF_KV_ATTN = 7  // a cache append run and the attention run after it
};
struct VmColStream {
    uint32_t c, x, y;   // the column slot, the slot sliced, the slot written
    uint32_t xo, yo;    // first column read from x, first column written to y
};
struct VmFused {
    int kind = 0;
    uint32_t start = 0;      // first instruction of the run
    uint32_t len = 0;        // instructions replaced
    uint32_t nh = 0, hd = 0, cols = 0;
    uint32_t k = 0, v = 0;   // KV_APPEND: the k and v rows; HEAD_ATTN: q in k
    uint32_t theta = 0, pos = 0, live = 0, scale = 0, att = 0;
    uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0;  // scratch slots, in opcode order
    float **tab = nullptr;   // device: the nh K cache addresses, then the nh V
    VmColStream col[2];      // VF_COL_RUN: nh streams of `cols` steps
    // VF_GEMMS / VF_GATE_UP after an RMSNORM of their input (start: the
    // RMSNORM): its source rows, gain, epsilon scalar and normalized rows
    bool norm = false;
    uint32_t nx = 0, ng = 0, ne = 0, ny = 0;
    std::vector<uint32_t> cslots;  // per-head runs: the cache slots in `tab`
    // VF_KV_ATTN: the attention run's q, live width, scale, output rows and
    // scratch slots (the append run's operands in the fields above)
    uint32_t aq = 0, alive = 0, ascale = 0, aatt = 0, a0 = 0, a1 = 0, a2 = 0, a3 = 0;
};

// The part of a LOOP_CNT body from its first instruction up to the first
// opcode that needs the host between steps (PRINT, the loop counter, jumps,
// LAYERB, LN_EPS): run eagerly on its first visit, captured into a HIP graph
// on the second and replayed from then on (see vmlm_vm_run).
enum VmSegState { VS_NEW = 0, VS_SEEN = 1, VS_GRAPH = 2, VS_EAGER = 3 };
struct VmSeg {
    uint32_t start = 0, end = 0;  // instructions [start, end)
    int state = VS_NEW;
    size_t base = 0;              // the layer base the graph was captured at
    hipGraphExec_t exec = nullptr;
};

struct vmlm_vm {
    std::vector<VmIns> text;
    std::vector<VmSlot> slots;
    std::vector<uint32_t> names;
    ConstPool *pool = nullptr;
    size_t const_bytes = 0;
    char *act = nullptr, *state = nullptr, *grad = nullptr;
    size_t act_b = 0, state_b = 0, grad_b = 0;
    hipStream_t st = nullptr;
    size_t layer_base = 0;
    float ln_eps = 1e-5f;
    std::vector<float> out;
    std::unordered_map<uintptr_t, float> kcache;  // values of constant scalars
    void *ws = nullptr;                            // executor workspace
    size_t ws_bytes = 0;
    unsigned long long *keys = nullptr;            // TOPK_IDX reduction keys
    int *guard = nullptr;  // this VM's device guard flag (index checks on device data)
    std::map<size_t, SwzConst> swz;  // the pool's swizzled int8 constants (owned by the pool)
    std::vector<VmFused> fused;      // opcode runs executed as one launch each
    std::vector<int32_t> fuse_at;    // per instruction: index into `fused`, or -1
    std::vector<VmSeg> segs;         // loop bodies replayed as HIP graphs
    std::vector<int32_t> seg_at;     // per instruction: index into `segs`, or -1
    bool graphs = true;              // vmlm_vm_set_graphs
};

static uint32_t rd32(const uint8_t *p, size_t off) {
    uint32_t v;
    std::memcpy(&v, p + off, 4);
    return v;
}

static void vm_free(vmlm_vm *vm) {
    if (!vm) return;
    if (vm->st) (void)hipStreamSynchronize(vm->st);
    pool_release(vm->pool);
    for (void *p : {(void *)vm->act, (void *)vm->state, (void *)vm->grad, vm->ws, (void *)vm->keys,
                    (void *)vm->guard})
        if (p) (void)hipFree(p);
    for (VmFused &f : vm->fused)
        if (f.tab) (void)hipFree(f.tab);
    for (VmSeg &g : vm->segs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (vm->st) (void)hipStreamDestroy(vm->st);
    delete vm;
}

// Drops every captured loop-body graph (they bake in device addresses and
// host-side values: the workspace, constant scalars, the LN epsilon); the
// bodies are captured again on their next visits.
static void vm_drop_graphs(vmlm_vm *vm) {
    for (VmSeg &g : vm->segs) {
        if (g.exec) {
            (void)hipStreamSynchronize(vm->st);
            (void)hipGraphExecDestroy(g.exec);
            g.exec = nullptr;
        }
        if (g.state == VS_GRAPH || g.state == VS_SEEN) g.state = VS_NEW;
    }
}

// core/src/interp.rs:241-348 audit_const_dtypes.
static int vm_audit(const vmlm_vm *vm) {
    const size_t ns = vm->slots.size();
    auto dt = [&](uint32_t s) { return s < ns ? vm->slots[s].dtype : (uint8_t)VDT_F32; };
    for (const VmIns &in : vm->text) {
        if (in.op == VOP_GEMM) {
            const uint8_t b = dt(in.b);
            if (b == VDT_BF16 || b == VDT_I8) continue;
            VMLM_GUARD(b == VDT_F32, "gemm B has no kernel for this dtype");
            continue;
        }
        if (in.op == VOP_EMB && dt(in.a) == VDT_BF16 && in.dst < ns && dt(in.dst) == VDT_F32)
            continue;
        bool cd = true, ca = true, cb = true;
        if (in.op == VOP_SHAPE) cd = ca = cb = false;
        else if (in.op == VOP_LOOP_CNT) cd = cb = false;
        else if (in.op == VOP_SLICE || in.op == VOP_WRITECOL || in.op == VOP_PUSH ||
                 in.op == VOP_POP)
            cb = false;
        const uint32_t probe[3] = {cd ? in.dst : UINT32_MAX, ca ? in.a : UINT32_MAX,
                                   cb ? in.b : UINT32_MAX};
        for (uint32_t s : probe) {
            if (s >= ns || dt(s) == VDT_F32) continue;
            const uint8_t d = dt(s);
            return fail(VMLM_ERR_GUARD,
                        "op %u uses %s const at slot %u (only a GEMM may read a non-f32 operand)",
                        in.op, d == VDT_BF16 ? "bf16" : d == VDT_I8 ? "i8" : "non-f32", s);
        }
    }
    return VMLM_OK;
}

static uint32_t written_slot(const VmIns &in);

// The loader's matcher for the decode loop's per-head runs (see
// VmKvAppend, VmHeadAttn): every head's run must be the same opcodes over
// the same scratch slots, with the row offsets of consecutive heads and a
// cache pair of its own; the shapes must make each opcode's static guard
// pass; the slots written must be f32 activation or state slots, distinct
// from each other and from the slots read; and no jump may land inside the
// run. Anything else runs opcode by opcode.
static int vm_detect_fusions(vmlm_vm *vm) {
    const std::vector<VmIns> &T = vm->text;
    const size_t n = T.size(), ns = vm->slots.size();
    vm->fuse_at.assign(n, -1);
    std::vector<char> target(n + 1, 0);
    for (const VmIns &in : T)
        if ((in.op == VOP_JMP || in.op == VOP_CMPLE || in.op == VOP_TOPK_THRESH ||
             in.op == VOP_LOOP_CNT) && in.dst <= n)
            target[in.dst] = 1;
    auto ok = [&](uint32_t i) { return i < ns; };
    auto rows = [&](uint32_t i) { return (size_t)vm->slots[i].rows; };
    auto cols = [&](uint32_t i) { return (size_t)vm->slots[i].cols; };
    auto f32 = [&](uint32_t i) { return ok(i) && vm->slots[i].dtype == VDT_F32; };
    auto data = [&](uint32_t i) {
        return f32(i) && (vm->slots[i].kind == VSLOT_ACT || vm->slots[i].kind == VSLOT_STATE);
    };
    auto same = [](const VmIns &x, uint8_t op, uint8_t fl, uint32_t d, uint32_t a, uint32_t b,
                   uint16_t dt) {
        return x.op == op && x.fl == fl && x.dst == d && x.a == a && x.b == b && x.dt == dt;
    };
    // written slots pairwise apart in memory and apart from every slot read
    // by the run (byte ranges in their regions: an image may place two slots
    // over the same arena bytes)
    auto overlap = [&](uint32_t a, uint32_t b) {
        if (a == b) return true;
        const VmSlot &x = vm->slots[a], &y = vm->slots[b];
        const bool cx = x.kind == VSLOT_CONST || x.kind == VSLOT_PARAM;
        const bool cy = y.kind == VSLOT_CONST || y.kind == VSLOT_PARAM;
        if (cx != cy || (!cx && x.kind != y.kind)) return false;
        const size_t xe = x.off + (size_t)x.rows * x.cols * vdtype_size(x.dtype);
        const size_t ye = y.off + (size_t)y.rows * y.cols * vdtype_size(y.dtype);
        return x.off < ye && y.off < xe;
    };
    auto disjoint = [&](const std::vector<uint32_t> &w, const std::vector<uint32_t> &r) {
        for (size_t a = 0; a < w.size(); ++a) {
            for (size_t b = a + 1; b < w.size(); ++b)
                if (overlap(w[a], w[b])) return false;
            for (uint32_t x : r)
                if (overlap(w[a], x)) return false;
        }
        return true;
    };
    constexpr uint8_t RT = VFL_RUNTIME;
    std::vector<float *> tab;
    for (size_t i = 0; i < n;) {
        const VmIns &h0 = T[i];
        VmFused f;
        std::vector<uint32_t> caches;
        const bool seven = i + 7 <= n;  // room for one head's run
        if (seven && h0.op == VOP_SLICE && h0.fl == 0 && h0.b == 0 && T[i + 1].op == VOP_SLICE &&
            T[i + 2].op == VOP_ROPE) {  // cache append
            const uint32_t kdh = h0.dst, kd = h0.a, vdh = T[i + 1].dst, vd = T[i + 1].a;
            const uint32_t kdrot = T[i + 2].dst, th = T[i + 2].b, pos = T[i + 2].dt;
            const uint32_t kdT = T[i + 3].dst, vdT = T[i + 4].dst;
            if (ok(kdh) && ok(vdh) && ok(kdrot) && ok(kdT) && ok(vdT)) {
                const size_t hd = cols(kdh);
                size_t j = 0;
                for (; i + 7 * (j + 1) <= n; ++j) {
                    const VmIns *g = &T[i + 7 * j];
                    const uint32_t off = (uint32_t)(j * hd);
                    if (!(same(g[0], VOP_SLICE, 0, kdh, kd, off, g[0].dt) &&
                          same(g[1], VOP_SLICE, 0, vdh, vd, off, g[1].dt) &&
                          same(g[2], VOP_ROPE, RT, kdrot, kdh, th, (uint16_t)pos) &&
                          same(g[3], VOP_TRANSPOSE, 0, kdT, kdrot, g[3].b, g[3].dt) &&
                          same(g[4], VOP_TRANSPOSE, 0, vdT, vdh, g[4].b, g[4].dt) &&
                          same(g[5], VOP_WRITECOL, RT, g[5].dst, kdT, 0, (uint16_t)pos) &&
                          same(g[6], VOP_WRITECOL, RT, g[6].dst, vdT, 0, (uint16_t)pos)))
                        break;
                    bool inside = false;
                    for (size_t t = 1; t <= 7; ++t) inside |= target[i + 7 * j + t] && t < 7;
                    if (j > 0) inside |= target[i + 7 * j];
                    if (inside) break;
                    caches.push_back(g[5].dst);
                    caches.push_back(g[6].dst);
                }
                const size_t nh = j;
                bool good = nh >= 2 && hd >= 2 && hd % 2 == 0 && hd <= 4096 && pos == T[i + 2].dt;
                good = good && data(kdh) && data(vdh) && data(kdrot) && data(kdT) && data(vdT) &&
                       f32(kd) && f32(vd) && f32(th) && f32(pos) && rows(kdh) == 1 &&
                       rows(vdh) == 1 && cols(vdh) == hd && rows(kdrot) == 1 &&
                       cols(kdrot) == hd && rows(kdT) == hd && cols(kdT) == 1 && rows(vdT) == hd &&
                       cols(vdT) == 1 && rows(kd) * cols(kd) >= nh * hd &&
                       rows(vd) * cols(vd) >= nh * hd;
                size_t cc = 0;
                for (size_t c = 0; good && c < caches.size(); ++c) {
                    const uint32_t x = caches[c];
                    good = data(x) && rows(x) == hd && cols(x) >= 1 && (c == 0 || cols(x) == cc);
                    cc = cols(x);
                }
                std::vector<uint32_t> w = {kdh, vdh, kdrot, kdT, vdT};
                w.insert(w.end(), caches.begin(), caches.end());
                good = good && disjoint(w, {kd, vd, th, pos});
                if (good) {
                    f.kind = VF_KV_APPEND;
                    f.len = (uint32_t)(7 * nh);
                    f.nh = (uint32_t)nh;
                    f.hd = (uint32_t)hd;
                    f.cols = (uint32_t)cc;
                    f.k = kd;
                    f.v = vd;
                    f.theta = th;
                    f.pos = pos;
                    f.s0 = kdh;
                    f.s1 = vdh;
                    f.s2 = kdrot;
                    f.s3 = kdT;
                    f.s4 = vdT;
                    // K caches (even entries), then V caches (odd)
                    std::vector<uint32_t> kc, vc;
                    for (size_t c = 0; c < caches.size(); c += 2) {
                        kc.push_back(caches[c]);
                        vc.push_back(caches[c + 1]);
                    }
                    caches = kc;
                    caches.insert(caches.end(), vc.begin(), vc.end());
                }
            }
        } else if (seven && h0.op == VOP_SLICE && h0.fl == 0 && h0.b == 0 && T[i + 1].op == VOP_ROPE &&
                   T[i + 2].op == VOP_GEMM) {  // attention per head
            const uint32_t qdh = h0.dst, qd = h0.a, qdrot = T[i + 1].dst, th = T[i + 1].b,
                           pos = T[i + 1].dt, scd = T[i + 2].dst, sc = T[i + 3].b,
                           live = T[i + 4].b, ctxd = T[i + 5].dst, att = T[i + 6].dst;
            if (ok(qdh) && ok(qdrot) && ok(scd) && ok(ctxd) && ok(att)) {
                const size_t hd = cols(qdh);
                size_t j = 0;
                std::vector<uint32_t> kc, vc;
                for (; i + 7 * (j + 1) <= n; ++j) {
                    const VmIns *g = &T[i + 7 * j];
                    const uint32_t off = (uint32_t)(j * hd);
                    if (!(same(g[0], VOP_SLICE, 0, qdh, qd, off, g[0].dt) &&
                          same(g[1], VOP_ROPE, RT, qdrot, qdh, th, (uint16_t)pos) &&
                          same(g[2], VOP_GEMM, VFL_TRANS_B, scd, qdrot, g[2].b, g[2].dt) &&
                          same(g[3], VOP_SCALE, 0, scd, scd, sc, g[3].dt) &&
                          same(g[4], VOP_SOFTMAX, RT, scd, scd, live, g[4].dt) &&
                          same(g[5], VOP_GEMM, 0, ctxd, scd, g[5].b, g[5].dt) &&
                          same(g[6], VOP_WRITECOL, 0, att, ctxd, off, g[6].dt)))
                        break;
                    bool inside = false;
                    for (size_t t = 1; t < 7; ++t) inside |= target[i + 7 * j + t];
                    if (j > 0) inside |= target[i + 7 * j];
                    if (inside) break;
                    kc.push_back(g[2].b);
                    vc.push_back(g[5].b);
                }
                const size_t nh = j, C = ok(scd) ? cols(scd) : 0;
                bool good = nh >= 2 && hd >= 2 && hd % 2 == 0 && hd <= 4096 && C >= 1 &&
                            C <= (size_t)VM_ATTN_MAX_COLS && data(qdh) && data(qdrot) &&
                            data(scd) && data(ctxd) && data(att) && f32(qd) && f32(th) &&
                            f32(pos) && f32(sc) && f32(live) && rows(qdh) == 1 &&
                            rows(qdrot) == 1 && cols(qdrot) == hd && rows(scd) == 1 &&
                            rows(ctxd) == 1 && cols(ctxd) == hd && rows(att) == 1 &&
                            cols(att) >= nh * hd && rows(qd) * cols(qd) >= nh * hd &&
                            rows(sc) * cols(sc) >= 1;
                for (size_t c = 0; good && c < nh; ++c)
                    good = f32(kc[c]) && rows(kc[c]) == hd && cols(kc[c]) == C && f32(vc[c]) &&
                           rows(vc[c]) == hd && cols(vc[c]) == C;
                std::vector<uint32_t> r = {qd, th, pos, sc, live};
                r.insert(r.end(), kc.begin(), kc.end());
                r.insert(r.end(), vc.begin(), vc.end());
                good = good && disjoint({qdh, qdrot, scd, ctxd, att}, r);
                if (good) {
                    f.kind = VF_HEAD_ATTN;
                    f.len = (uint32_t)(7 * nh);
                    f.nh = (uint32_t)nh;
                    f.hd = (uint32_t)hd;
                    f.cols = (uint32_t)C;
                    f.k = qd;
                    f.theta = th;
                    f.pos = pos;
                    f.live = live;
                    f.scale = sc;
                    f.att = att;
                    f.s0 = qdh;
                    f.s1 = qdrot;
                    f.s2 = scd;
                    f.s3 = ctxd;
                    caches = kc;
                    caches.insert(caches.end(), vc.begin(), vc.end());
                }
            }
        }
        // int8 GEMMs of one input at decode rows: two or three in a row (q/k/v),
        // or gate, up, ACT silu of gate, EWMUL by up (the run at `at`)
        auto q8_gemm = [&](const VmIns &x, uint32_t A) {
            if (!(x.op == VOP_GEMM && x.fl == 0 && x.a == A && ok(x.b) && ok(x.dst) && ok(x.dt)))
                return false;
            const VmSlot &B = vm->slots[x.b];
            const size_t m = rows(A), k = cols(A), nn = B.rows;
            return B.dtype == VDT_I8 && B.cols == k && nn >= 1 && f32(x.dt) &&
                   rows(x.dt) * cols(x.dt) >= nn && data(x.dst) &&
                   rows(x.dst) * cols(x.dst) >= m * nn;
        };
        auto match_gemms = [&](size_t at, VmFused &f) {
            const VmIns &h0 = T[at];
            const size_t i = at;
            if (!f.kind && h0.op == VOP_GEMM && h0.fl == 0 && f32(h0.a) && rows(h0.a) >= 1 &&
                rows(h0.a) <= (size_t)FX_ROWS && cols(h0.a) % 128 == 0 &&
                fx_run_blocks((int)cols(h0.a)) && q8_gemm(h0, h0.a)) {
                const uint32_t A = h0.a;
                const size_t M = rows(A);
                size_t j = 1;
                while (j < 3 && i + j < n && !target[i + j] && q8_gemm(T[i + j], A)) ++j;
                std::vector<uint32_t> dsts;
                for (size_t t = 0; t < j; ++t) dsts.push_back(T[i + t].dst);
                std::vector<uint32_t> reads = {A};
                for (size_t t = 0; t < j; ++t) {
                    reads.push_back(T[i + t].b);
                    reads.push_back(T[i + t].dt);
                }
                const VmIns *g = &T[i];
                const uint32_t gd = g[0].dst, ud = j >= 2 ? g[1].dst : 0;
                const size_t N = vm->slots[g[0].b].rows;
                const bool gate_up =
                    j >= 2 && i + 4 <= n && !target[i + 2] && !target[i + 3] &&
                    vm->slots[g[1].b].rows == N && g[2].op == VOP_ACT && g[2].fl == VMLM_ACT_SILU &&
                    g[2].a == gd && g[3].op == VOP_EWMUL && g[3].a == g[2].dst && g[3].b == ud &&
                    g[3].dst == g[2].dst && data(g[2].dst) && rows(g[2].dst) == M &&
                    cols(g[2].dst) == N && rows(gd) == M && cols(gd) == N && rows(ud) == M &&
                    cols(ud) == N;
                if (gate_up) {
                    std::vector<uint32_t> w = {gd, ud, g[2].dst};
                    std::vector<uint32_t> r2 = {A, g[0].b, g[0].dt, g[1].b, g[1].dt};
                    if (disjoint(w, r2)) {
                        f.kind = VF_GATE_UP;
                        f.len = 4;
                        f.nh = 2;
                        f.att = g[2].dst;  // act
                    }
                }
                if (!f.kind && j >= 2 && disjoint(dsts, reads)) {
                    f.kind = VF_GEMMS;
                    f.len = (uint32_t)j;
                    f.nh = (uint32_t)j;
                }
                // one GEMM, then the residual EWADD of its output (z = r + y, the
                // same shape, no broadcast): the GEMM's epilogue writes z too
                const VmIns &e = T[i + 1];
                if (!f.kind && j == 1 && i + 2 <= n && !target[i + 1] && e.op == VOP_EWADD &&
                    e.fl == 0 && ok(e.a) && ok(e.b) && ok(e.dst) && (e.a == gd) != (e.b == gd)) {
                    const uint32_t r = e.a == gd ? e.b : e.a, z = e.dst;
                    const bool shp = rows(gd) == M && cols(gd) == N && rows(e.a) == M &&
                                     cols(e.a) == N && rows(e.b) == M && cols(e.b) == N;
                    if (shp && data(z) && f32(r) && rows(z) * cols(z) >= M * N &&
                        disjoint({gd, z}, {A, g[0].b, g[0].dt, r})) {
                        f.kind = VF_GEMM_ADD;
                        f.len = 2;
                        f.nh = 1;
                        f.k = r;
                        f.att = z;
                    }
                }
            }
            return f.kind != 0;
        };
        // RMSNORM y <- x (gain g, epsilon e) of one row that feeds the GEMM
        // run after it (the decoder's input and post-attention norms at
        // decode): one launch that normalizes as the RMSNORM kernel does and
        // also writes y. The RMSNORM's extents hold statically; y has x's
        // shape, apart from x, g, e and the run's outputs.
        if (!f.kind && h0.op == VOP_RMSNORM && i + 2 <= n && !target[i + 1] && ok(h0.dst) &&
            ok(h0.a) && ok(h0.b) && ok(h0.dt)) {
            const uint32_t x = h0.a, y = h0.dst, gn = h0.b, e = h0.dt;
            VmFused fg;
            const bool good =
                match_gemms(i + 1, fg) && (fg.kind == VF_GEMMS || fg.kind == VF_GATE_UP) &&
                T[i + 1].a == y && data(y) && f32(x) && f32(gn) && f32(e) &&
                rows(e) * cols(e) >= 1 && rows(x) == 1 && rows(y) == 1 && cols(x) == cols(y) &&
                rows(gn) * cols(gn) >= cols(x) && fx_norm_ok((int)cols(x));
            std::vector<uint32_t> w = {y};  // each written slot once (ACT and EWMUL share one)
            for (uint32_t t = 0; good && t < fg.len; ++t) {
                const uint32_t ws_ = written_slot(T[i + 1 + t]);
                if (std::find(w.begin(), w.end(), ws_) == w.end()) w.push_back(ws_);
            }
            if (good && disjoint(w, {x, gn, e})) {
                f = fg;
                f.norm = true;
                f.len += 1;
                f.nx = x;
                f.ng = gn;
                f.ne = e;
                f.ny = y;
            }
        }
        if (!f.kind) match_gemms(i, f);
        // cache writes of a prompt, column by column (p12_build_minicpm.py:
        // 794-840): P steps of SLICE c <- x at column xo + p, then WRITECOL
        // y <- c at column yo + p, for one stream or two interleaved. The run
        // writes columns yo .. yo + P - 1 of y from xo .. xo + P - 1 of x and
        // leaves c holding column xo + P - 1, which two strided copies per
        // stream reproduce.
        auto col_pair = [&](size_t at) {
            return at + 2 <= n && T[at].op == VOP_SLICE && T[at].fl == 0 &&
                   T[at + 1].op == VOP_WRITECOL && T[at + 1].fl == 0 && T[at + 1].a == T[at].dst;
        };
        if (!f.kind && col_pair(i)) {
            const int Q = col_pair(i + 2) && T[i + 2].dst != h0.dst ? 2 : 1;
            size_t P = 0;
            for (;; ++P) {
                const size_t at = i + 2 * Q * P;
                bool okp = at + 2 * Q <= n;
                for (int q = 0; okp && q < Q; ++q) {
                    const VmIns &s0 = T[i + 2 * q], &w0 = T[i + 2 * q + 1];
                    const VmIns &sp = T[at + 2 * q], &wp = T[at + 2 * q + 1];
                    okp = col_pair(at + 2 * q) && sp.dst == s0.dst && sp.a == s0.a &&
                          (uint64_t)sp.b == (uint64_t)s0.b + P && wp.dst == w0.dst &&
                          (uint64_t)wp.b == (uint64_t)w0.b + P;
                }
                for (size_t t = 0; okp && t < (size_t)(2 * Q); ++t)
                    okp = (P == 0 && t == 0) || !target[at + t];  // no jump into the run
                if (!okp) break;
            }
            bool good = P >= 2;
            std::vector<uint32_t> w, r;
            for (int q = 0; good && q < Q; ++q) {
                const VmIns &s0 = T[i + 2 * q], &w0 = T[i + 2 * q + 1];
                const uint32_t c = s0.dst, x = s0.a, y = w0.dst;
                // the guards of SLICE and WRITECOL, at the run's last column
                good = ok(c) && ok(x) && ok(y) && data(c) && data(y) && f32(x) && cols(c) == 1 &&
                       rows(c) >= 1 && rows(c) >= rows(y) &&
                       (rows(c) - 1) * cols(x) + s0.b + P <= rows(x) * cols(x) &&
                       (size_t)w0.b + P <= cols(y);
                if (!good) break;
                f.col[q] = VmColStream{c, x, y, s0.b, w0.b};
                w.push_back(c);
                w.push_back(y);
                r.push_back(x);
            }
            if (good && disjoint(w, r)) {
                f.kind = VF_COL_RUN;
                f.len = (uint32_t)(2 * Q * P);
                f.nh = (uint32_t)Q;
                f.cols = (uint32_t)P;
            }
        }
        if (f.kind == VF_GEMMS || f.kind == VF_GATE_UP || f.kind == VF_COL_RUN ||
            f.kind == VF_GEMM_ADD) {  // no cache table
            f.start = (uint32_t)i;
            vm->fused.push_back(f);
            vm->fuse_at[i] = (int32_t)vm->fused.size() - 1;
            i += f.len;
            continue;
        }
        if (!f.kind) {
            ++i;
            continue;
        }
        f.start = (uint32_t)i;
        // the cache addresses (activation and state slots do not move)
        std::vector<float *> addr;
        for (uint32_t c : caches) {
            const VmSlot &sl = vm->slots[c];
            addr.push_back((float *)((sl.kind == VSLOT_STATE ? vm->state : vm->act) + sl.off));
        }
        f.cslots = caches;
        VMLM_HIP_CHECK(hipMalloc((void **)&f.tab, addr.size() * sizeof(float *)));
        vm->fused.push_back(f);  // freed with the VM from here on
        VMLM_HIP_CHECK(hipMemcpy(f.tab, addr.data(), addr.size() * sizeof(float *),
                                 hipMemcpyHostToDevice));
        vm->fuse_at[i] = (int32_t)vm->fused.size() - 1;
        i += f.len;
    }
    // A layer's cache append run and the attention run right after it, over
    // the same caches, position and theta (hd = 64, at most 256 columns): one
    // launch, each head's workgroup appending before it attends. The slots
    // either run writes stay apart from those the other reads (the caches
    // aside: the attention uses the column the append wrote).
    for (size_t r = 0; r + 1 < vm->fused.size(); ++r) {
        VmFused &a = vm->fused[r], &b = vm->fused[r + 1];
        if (a.kind != VF_KV_APPEND || b.kind != VF_HEAD_ATTN || b.start != a.start + a.len ||
            target[b.start] || a.nh != b.nh || a.hd != 64 || b.hd != 64 || a.cols != b.cols ||
            b.cols > 256 || a.pos != b.pos || a.theta != b.theta || a.cslots != b.cslots)
            continue;
        if (!disjoint({a.s0, a.s1, a.s2, a.s3, a.s4, b.s0, b.s1, b.s2, b.s3, b.att},
                      {a.k, a.v, a.theta, a.pos, b.k, b.scale, b.live}))
            continue;
        a.kind = VF_KV_ATTN;
        a.len += b.len;
        a.aq = b.k;
        a.alive = b.live;
        a.ascale = b.scale;
        a.aatt = b.att;
        a.a0 = b.s0;
        a.a1 = b.s1;
        a.a2 = b.s2;
        a.a3 = b.s3;
        vm->fuse_at[b.start] = -1;
        b.kind = 0;  // no longer run (its table is freed with the VM)
    }
    return VMLM_OK;
}

// The graph segments (VmSeg): for every LOOP_CNT, its body from the jump
// target up to the first opcode that needs the host between steps.
static void vm_detect_segments(vmlm_vm *vm) {
    const std::vector<VmIns> &T = vm->text;
    const size_t n = T.size();
    vm->seg_at.assign(n, -1);
    // opcodes that need the host between steps, and writes of a constant
    // slot (the host drops its cached constant scalars there)
    auto host_op = [&](const VmIns &in) {
        const uint8_t op = in.op;
        if (op == VOP_PRINT || op == VOP_LOOP_CNT || op == VOP_JMP || op == VOP_CMPLE ||
            op == VOP_TOPK_THRESH || op == VOP_LAYERB || op == VOP_LN_EPS || op == VOP_HALT)
            return true;
        const uint32_t w = written_slot(in);
        return w < vm->slots.size() &&
               (vm->slots[w].kind == VSLOT_CONST || vm->slots[w].kind == VSLOT_PARAM);
    };
    for (size_t i = 0; i < n; ++i) {
        if (T[i].op != VOP_LOOP_CNT || T[i].dst >= i || vm->seg_at[T[i].dst] >= 0) continue;
        VmSeg g;
        g.start = T[i].dst;
        g.end = g.start;
        while (g.end < i && !host_op(T[g.end])) ++g.end;
        if (g.end - g.start < 16) continue;  // too short to pay for a graph
        vm->seg_at[g.start] = (int32_t)vm->segs.size();
        vm->segs.push_back(g);
    }
}

extern "C" {

int vmlm_vm_load(const void *image, size_t len, const void *weights, size_t weights_len,
                 vmlm_vm **out) {
    VMLM_GUARD(out != nullptr && image != nullptr, "vm_load: null argument");
    *out = nullptr;
    int rc = ensure_init();
    if (rc) return rc;
    const uint8_t *img = (const uint8_t *)image;
    if (len < 32 || rd32(img, 0) != 0x4D4C4D56u) return fail(3, "bad magic");
    vmlm_vm *vm = new vmlm_vm();
    auto bad = [&](int code) {
        vm_free(vm);
        return code;
    };
    const size_t text_off = rd32(img, 8), text_len = rd32(img, 12), const_off = rd32(img, 16),
                 meta_off = rd32(img, 24);
    vm->const_bytes = rd32(img, 20);
    if (text_off + text_len > len || meta_off + 28 > len ||
        (!weights && const_off + vm->const_bytes > len) ||
        (weights && weights_len < vm->const_bytes))
        return bad(fail(VMLM_ERR_GUARD, "vm_load: image regions past its end"));
    vm->text.resize(text_len / 16);
    for (size_t i = 0; i < vm->text.size(); ++i) {
        const uint8_t *q = img + text_off + 16 * i;
        VmIns &in = vm->text[i];
        in.op = q[0];
        in.fl = q[1];
        std::memcpy(&in.dt, q + 2, 2);
        in.dst = rd32(q, 4);
        in.a = rd32(q, 8);
        in.b = rd32(q, 12);
    }
    const uint8_t *meta = img + meta_off;
    const size_t n_const = rd32(meta, 0), n_slot = rd32(meta, 4), slots_off = rd32(meta, 8),
                 names_off = rd32(meta, 24);
    vm->act_b = rd32(meta, 12);
    vm->state_b = rd32(meta, 16);
    vm->grad_b = rd32(meta, 20);
    if (meta_off + slots_off + 16 * n_slot > len || meta_off + names_off + 4 * n_slot > len ||
        meta_off + 28 + 24 * n_const > len)
        return bad(fail(VMLM_ERR_GUARD, "vm_load: META tables past the image end"));
    vm->slots.resize(n_slot);
    vm->names.resize(n_slot);
    for (size_t i = 0; i < n_slot; ++i) {
        const uint8_t *e = meta + slots_off + 16 * i;
        VmSlot &s = vm->slots[i];
        s.kind = rd32(e, 0);
        const uint32_t idx = rd32(e, 4);
        s.rows = rd32(e, 8);
        s.cols = rd32(e, 12);
        s.dtype = VDT_F32;
        vm->names[i] = rd32(meta + names_off, 4 * i);
        const size_t need = (size_t)s.rows * s.cols;
        if (s.kind == VSLOT_CONST || s.kind == VSLOT_PARAM) {
            if (idx >= n_const)
                return bad(fail(VMLM_ERR_GUARD, "slot %zu names const %u of %zu", i, idx, n_const));
            const uint8_t *ce = meta + 28 + 24 * (size_t)idx;
            const uint32_t off = rd32(ce, 0), clen = rd32(ce, 4);
            s.dtype = ce[16];
            const size_t esz = vdtype_size(s.dtype);
            if (esz == 0) return bad(fail(VMLM_ERR_GUARD, "const has unknown dtype"));
            if (need * esz > clen || (size_t)off + clen > vm->const_bytes)
                return bad(fail(VMLM_ERR_GUARD, "slot %zu (%ux%u) exceeds its constant", i,
                                s.rows, s.cols));
            s.off = off;
        } else {
            const size_t bytes = s.kind == VSLOT_STATE ? vm->state_b
                                 : s.kind == VSLOT_GRAD ? vm->grad_b : vm->act_b;
            if ((size_t)idx + need * 4 > bytes + 64)
                return bad(fail(VMLM_ERR_GUARD, "slot %zu (%ux%u) exceeds its arena", i, s.rows,
                                s.cols));
            s.off = idx / 4 * 4;
        }
    }
    if ((rc = vm_audit(vm))) return bad(rc);

    hipError_t e = hipStreamCreateWithFlags(&vm->st, hipStreamNonBlocking);
    if (e != hipSuccess) return bad(hip_fail(e, "vm stream"));
    // the constant pool: shared when the caller maps its weights, else private
    const void *host = weights ? weights : (const void *)(img + const_off);
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        if (weights)
            for (ConstPool *p : g_pools)
                if (p->host == weights && p->len == vm->const_bytes) {
                    ++p->refs;
                    vm->pool = p;
                    break;
                }
        if (!vm->pool) {
            ConstPool *p = new ConstPool{weights, vm->const_bytes, nullptr, 1};
            if ((e = hipMalloc(&p->dev, vm->const_bytes + 64)) != hipSuccess) {
                delete p;
                return bad(hip_fail(e, "const pool"));
            }
            if (vm->const_bytes &&
                (e = hipMemcpy(p->dev, host, vm->const_bytes, hipMemcpyHostToDevice)) != hipSuccess) {
                (void)hipFree(p->dev);
                delete p;
                return bad(hip_fail(e, "const pool upload"));
            }
            ++g_pool_uploads;
            if (weights) g_pools.push_back(p);
            vm->pool = p;
        }
    }
    for (auto [pp, bytes] : {std::pair<char **, size_t>{&vm->act, vm->act_b},
                             {&vm->state, vm->state_b}, {&vm->grad, vm->grad_b}}) {
        if ((e = hipMalloc((void **)pp, bytes + 64)) != hipSuccess) return bad(hip_fail(e, "arena"));
        if ((rc = launch_fill_zero(*pp, bytes + 64, vm->st))) return bad(rc);
    }
    if ((e = hipMalloc((void **)&vm->keys, ARGMAX_KEYS * sizeof(unsigned long long))) != hipSuccess) return bad(hip_fail(e, "vm keys"));
    if ((e = hipMalloc((void **)&vm->guard, 64)) != hipSuccess) return bad(hip_fail(e, "vm guard"));
    if ((rc = launch_fill_zero(vm->guard, 64, vm->st))) return bad(rc);
    if ((rc = vm_detect_fusions(vm))) return bad(rc);
    vm_detect_segments(vm);
    // every int8 constant (the audit admits them only as GEMM B) also in the
    // swizzled layout, made once per pool; a constant whose copy does not fit
    // in device memory stays row-major only
    std::map<size_t, SwzConst> made;
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        for (const VmSlot &s : vm->slots) {
            if (s.kind != VSLOT_CONST || s.dtype != VDT_I8 || !s.rows || s.rows % 16 ||
                s.cols % 64 || (((uintptr_t)vm->pool->dev + s.off) & 15) ||
                vm->pool->swz.count(s.off) || made.count(s.off))
                continue;
            int8_t *d = nullptr;
            if (hipMalloc((void **)&d, (size_t)s.rows * s.cols) != hipSuccess) {
                (void)hipGetLastError();
                continue;
            }
            if ((rc = launch_swizzle_w((const int8_t *)(vm->pool->dev + s.off), d, (int)s.rows,
                                       (int)s.cols, vm->st))) {
                (void)hipFree(d);
                for (auto &kv : made) (void)hipFree(kv.second.dev);
                return bad(rc);
            }
            made[s.off] = SwzConst{s.rows, s.cols, d};
        }
    }
    if ((e = hipStreamSynchronize(vm->st)) != hipSuccess) {
        for (auto &kv : made) (void)hipFree(kv.second.dev);
        return bad(hip_fail(e, "vm load"));
    }
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        for (auto &kv : made) vm->pool->swz.insert(kv);
        vm->swz = vm->pool->swz;
    }
    *out = vm;
    return VMLM_OK;
}

int vmlm_vm_destroy(vmlm_vm *vm) {
    vm_free(vm);
    return VMLM_OK;
}

int vmlm_vm_pool_uploads(size_t *n) {
    VMLM_GUARD(n, "null argument");
    std::lock_guard<std::mutex> lk(g_pool_mu);
    *n = g_pool_uploads;
    return VMLM_OK;
}

int vmlm_vm_swizzled_consts(const vmlm_vm *vm, size_t *n) {
    VMLM_GUARD(vm && n, "null argument");
    *n = vm->swz.size();
    return VMLM_OK;
}

int vmlm_vm_fused_runs(const vmlm_vm *vm, size_t *n) {
    VMLM_GUARD(vm && n, "null argument");
    size_t c = 0;
    for (const VmFused &f : vm->fused) c += f.kind != 0;
    *n = c;
    return VMLM_OK;
}

int vmlm_vm_fused_opcodes(const vmlm_vm *vm, size_t *n) {
    VMLM_GUARD(vm && n, "null argument");
    size_t c = 0;
    for (const VmFused &f : vm->fused) c += f.kind ? f.len : 0;
    *n = c;
    return VMLM_OK;
}

int vmlm_vm_set_graphs(vmlm_vm *vm, int on) {
    VMLM_GUARD(vm, "null vm");
    vm->graphs = on != 0;
    return VMLM_OK;
}

int vmlm_vm_graph_segments(const vmlm_vm *vm, size_t *n) {
    VMLM_GUARD(vm && n, "null argument");
    size_t c = 0;
    for (const VmSeg &g : vm->segs) c += g.state == VS_GRAPH;
    *n = c;
    return VMLM_OK;
}

void *vmlm_vm_stream(vmlm_vm *vm) { return vm ? (void *)vm->st : nullptr; }

}  // extern "C"

// ------------------------------------------------------------------ run
namespace {

struct Exec {
    vmlm_vm *vm;
    int *guard;
    bool capturing = false;  // inside a graph capture: nothing may read the device or allocate

    size_t nel(uint32_t s) const {
        return s < vm->slots.size() ? (size_t)vm->slots[s].rows * vm->slots[s].cols : 0;
    }
    uint32_t rows(uint32_t s) const { return s < vm->slots.size() ? vm->slots[s].rows : 0; }
    uint32_t cols(uint32_t s) const { return s < vm->slots.size() ? vm->slots[s].cols : 0; }
    uint8_t dt(uint32_t s) const {
        return s < vm->slots.size() ? vm->slots[s].dtype : (uint8_t)VDT_F32;
    }

    // core/src/interp.rs:434-467: a slot's device address, constants through
    // the layer base with its bound check.
    int ptr(uint32_t i, float **p) {
        VMLM_GUARD(i < vm->slots.size(), "slot %u does not exist", i);
        const VmSlot &s = vm->slots[i];
        char *base;
        size_t off = s.off;
        if (s.kind == VSLOT_CONST || s.kind == VSLOT_PARAM) {
            const size_t bytes = (size_t)s.rows * s.cols * vdtype_size(s.dtype);
            VMLM_GUARD(off + vm->layer_base + bytes <= vm->const_bytes,
                       "layer base walks past the constant pool: off=%zu base=%zu bytes=%zu limit=%zu",
                       off, vm->layer_base, bytes, vm->const_bytes);
            base = vm->pool->dev;
            off += vm->layer_base;
        } else {
            base = s.kind == VSLOT_STATE ? vm->state : s.kind == VSLOT_GRAD ? vm->grad : vm->act;
        }
        *p = (float *)(base + off);
        return VMLM_OK;
    }
    // element 0 of a slot on the host (constants cached by device address)
    int scalar(uint32_t i, float *v) {
        float *p;
        int rc = ptr(i, &p);
        if (rc) return rc;
        VMLM_GUARD(nel(i) >= 1 && dt(i) == VDT_F32, "slot %u holds no f32 value", i);
        const bool is_const = vm->slots[i].kind == VSLOT_CONST;
        if (is_const) {
            auto it = vm->kcache.find((uintptr_t)p);
            if (it != vm->kcache.end()) {
                *v = it->second;
                return VMLM_OK;
            }
        }
        VMLM_GUARD(!capturing, "graph capture: a device value read on the host");
        VMLM_HIP_CHECK(hipMemcpyAsync(v, p, 4, hipMemcpyDeviceToHost, vm->st));
        VMLM_HIP_CHECK(hipStreamSynchronize(vm->st));
        if (is_const) vm->kcache[(uintptr_t)p] = *v;
        return VMLM_OK;
    }
    int ws(size_t bytes, void **p) {
        if (bytes > vm->ws_bytes) {
            VMLM_GUARD(!capturing, "graph capture: workspace growth");
            vm_drop_graphs(vm);  // the old workspace is freed below
            VMLM_HIP_CHECK(hipStreamSynchronize(vm->st));
            if (vm->ws) VMLM_HIP_CHECK(hipFree(vm->ws));
            vm->ws = nullptr;
            vm->ws_bytes = 0;
            VMLM_HIP_CHECK(hipMalloc(&vm->ws, bytes));
            vm->ws_bytes = bytes;
        }
        *p = vm->ws;
        return VMLM_OK;
    }
    int copy(float *d, const float *s, size_t n) {
        if (n && d != s)
            VMLM_HIP_CHECK(hipMemcpyAsync(d, s, n * 4, hipMemcpyDeviceToDevice, vm->st));
        return VMLM_OK;
    }
    int copy2d(float *d, size_t dld, size_t doff, const float *s, size_t sld, size_t soff,
               size_t r, size_t c, const float *offp = nullptr, size_t dlimit = 0) {
        if (r * c == 0) return VMLM_OK;
        vm_copy2d_kernel<<<vm_blocks(r * c), 256, 0, vm->st>>>(d, dld, doff, s, sld, soff, r, c,
                                                               offp, dlimit, guard);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }

    int step(const VmIns &in, size_t *ip);
    int fused(const VmFused &f);
    int fused_gemms(const VmFused &f);
};

#define P_(name, slot)                 \
    float *name;                       \
    if ((rc = ptr((slot), &name))) return rc
#define NEED(cond, ...) VMLM_GUARD(cond, __VA_ARGS__)

int Exec::step(const VmIns &in, size_t *ip) {
    int rc = VMLM_OK;
    const uint32_t d = in.dst, a = in.a, b = in.b;
    hipStream_t st = vm->st;
    switch (in.op) {
    case VOP_SHAPE: return VMLM_OK;
    case VOP_COPY: case VOP_SAVE: case VOP_LOAD: {
        NEED(nel(d) >= nel(a), "COPY: dst smaller than src");
        P_(cd, d);
        P_(ca, a);
        return copy(cd, ca, nel(a));
    }
    case VOP_GEMM: {  // core/src/interp.rs:734-813
        const size_t m = rows(a), k = cols(a), brows = rows(b), bcols = cols(b);
        const bool nt = (in.fl & VFL_TRANS_B) == 0, acc = (in.fl & VFL_ACC) != 0;
        const uint8_t bt = dt(b);
        const size_t n = nt ? brows : bcols;
        if (bt == VDT_BF16 || bt == VDT_I8) {
            NEED(nt, "%s NN gemm unimplemented", bt == VDT_I8 ? "int8" : "bf16");
            NEED(!acc, "%s acc gemm unimplemented", bt == VDT_I8 ? "int8" : "bf16");
        }
        if (bt == VDT_I8) {
            NEED(in.dt < vm->slots.size() && dt(in.dt) == VDT_F32,
                 "int8 gemm: scale slot must be f32");
            NEED(nel(in.dt) >= brows, "int8 gemm: scale shorter than N rows");
        }
        NEED(nel(d) >= m * n && brows * bcols >= n * k, "GEMM: operand extents");
        P_(cc, d);
        P_(ca, a);
        P_(cb, b);
        if (bt == VDT_BF16)
            return vmlm_hip_gemm_nt_bf16(ca, (const uint16_t *)cb, cc, m, brows, k, st);
        if (bt == VDT_I8) {
            P_(cs, in.dt);
            // the swizzled copy made at load, when the read is one whole
            // constant of this shape (through the layer base too)
            const int8_t *wsw = nullptr;
            const auto it = vm->swz.find((size_t)((char *)cb - vm->pool->dev));
            if (it != vm->swz.end() && it->second.rows == brows && it->second.cols == bcols &&
                bcols == k)
                wsw = it->second.dev;
            return q8_gemm_vm(ca, (const int8_t *)cb, wsw, cs, cc, m, brows, k, st);
        }
        NEED(bt == VDT_F32, "gemm operand dtype unsupported");
        return nt ? vmlm_hip_gemm_nt(ca, cb, cc, m, brows, k, acc, st)
                  : vmlm_hip_gemm(ca, cb, cc, m, bcols, k, acc, st);
    }
    case VOP_GEMV: {
        const size_t m = rows(a), k = cols(a);
        NEED(nel(b) >= k && nel(d) >= m, "GEMV: operand extents");
        P_(ca, a);
        P_(cb, b);
        P_(cc, d);
        if (m == 0) return VMLM_OK;
        vm_rowwise_kernel<<<vm_blocks(m), 256, 0, st>>>(cc, ca, cb, m, k, VOP_GEMV);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_EWADD: case VOP_EWMUL: case VOP_EWSUB: case VOP_EWDIV: {
        const size_t r = rows(a), c = cols(a), br = rows(b), bc = cols(b);
        NEED(nel(d) >= r * c, "EW: dst smaller than a");
        P_(ca, a);
        P_(cb, b);
        P_(cc, d);
        if (br == r && bc == c) return launch_ew(cc, ca, cb, r * c, in.op, st);
        int mode = br == r && bc == 1 ? 1 : br == 1 && bc == c ? 2 : br * bc == 1 ? 3 : 0;
        if (!mode) return fail(8, "EW shape mismatch");
        if (r * c == 0) return VMLM_OK;
        vm_ew_bcast_kernel<<<vm_blocks(r * c), 256, 0, st>>>(cc, ca, cb, r, c, mode, in.op);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_ACT: {
        const size_t n = nel(d);
        NEED(nel(a) >= n, "ACT: src smaller than dst");
        P_(cd, d);
        P_(ca, a);
        if ((rc = copy(cd, ca, n))) return rc;
        return launch_act(cd, n, in.fl == 0 ? VMLM_ACT_RELU : in.fl, st);
    }
    case VOP_LN: {
        const size_t r = rows(a), c = cols(a);
        NEED(nel(d) >= r * c && nel(b) >= c && nel(in.dt) >= c, "LN: operand extents");
        P_(cd, d);
        P_(ca, a);
        P_(g, b);
        P_(bias, in.dt);
        if ((rc = copy(cd, ca, r * c))) return rc;
        return launch_layernorm(cd, g, bias, r, c, vm->ln_eps, st);
    }
    case VOP_LN_EPS: {
        const float old = vm->ln_eps;
        if ((rc = scalar(d, &vm->ln_eps))) return rc;
        if (vm->ln_eps != old) vm_drop_graphs(vm);  // LN opcodes baked the old value
        return VMLM_OK;
    }
    case VOP_RMSNORM: {
        const size_t r = rows(a), c = cols(a);
        NEED(nel(d) >= r * c && nel(b) >= c, "RMSNORM: operand extents");
        float eps;
        if ((rc = scalar(in.dt, &eps))) return rc;
        P_(cd, d);
        P_(ca, a);
        P_(g, b);
        return launch_rmsnorm(cd, ca, g, r, c, eps, nullptr, 0, 0, st);
    }
    case VOP_PUSH: case VOP_POP: {
        const uint32_t stk = in.op == VOP_PUSH ? d : a, one = in.op == VOP_PUSH ? a : d;
        const size_t w = cols(stk);
        NEED(nel(one) == w, in.op == VOP_PUSH ? "PUSH: src elems != stack row width"
                                              : "POP: dst elems != stack row width");
        NEED((size_t)b < rows(stk), "PUSH/POP: step past the stack");
        P_(cs, stk);
        P_(co, one);
        return in.op == VOP_PUSH ? copy(cs + (size_t)b * w, co, w) : copy(co, cs + (size_t)b * w, w);
    }
    case VOP_STACK_INIT: {
        P_(ca, a);
        return launch_fill_zero(ca, nel(a) * 4, st);
    }
    case VOP_SOFTMAX: {
        const size_t r = rows(d), c = cols(d);
        NEED(nel(a) >= r * c, "SOFTMAX: src smaller than dst");
        P_(cd, d);
        P_(ca, a);
        if ((rc = copy(cd, ca, r * c))) return rc;
        if (in.fl & VFL_RUNTIME) {
            P_(lp, b);
            if (r == 0 || c == 0) return VMLM_OK;
            vm_softmax_live_kernel<<<(unsigned)r, 256, 0, st>>>(cd, (int)c, lp, guard);
            VMLM_HIP_CHECK(hipGetLastError());
            return VMLM_OK;
        }
        return launch_softmax(cd, r, c, (in.fl & VFL_CAUSAL) != 0, st);
    }
    case VOP_OUTER: {
        const size_t m = rows(a) == 1 ? cols(a) : rows(a), nn = rows(b) == 1 ? cols(b) : rows(b);
        NEED(nel(d) >= m * nn, "OUTER: dst smaller than m x n");
        P_(cs, d);
        P_(cv, a);
        P_(ck, b);
        return launch_outer(cs, cv, ck, m, nn, 1.0f, st);
    }
    case VOP_TOPK_THRESH: {
        const size_t r = rows(a), c = cols(a);
        NEED(nel(d) >= r, "TOPK_THRESH: dst shorter than rows");
        NEED(c <= 8192, "TOPK_THRESH: row wider than 8192");
        P_(ca, a);
        P_(cd, d);
        void *used;
        if ((rc = ws(r * c + 1, &used))) return rc;
        if (r == 0) return VMLM_OK;
        vm_topk_thresh_kernel<<<vm_blocks(r, 64), 64, 0, st>>>(cd, ca, r, c, in.fl < c ? in.fl : c,
                                                                (unsigned char *)used);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_LAYERB: {
        float d0;
        if ((rc = scalar(a, &d0))) return rc;
        if (d0 >= 0.0f) {
            vm->layer_base += (size_t)d0;
        } else {
            const size_t back = (size_t)(-d0);
            vm->layer_base = back > vm->layer_base ? 0 : vm->layer_base - back;
        }
        return VMLM_OK;
    }
    case VOP_EWMAX: case VOP_GEMASK: case VOP_EXP: case VOP_NEG: case VOP_LOG: case VOP_SIN:
    case VOP_COS: case VOP_CLAMP: {
        const size_t n = nel(a);
        NEED(nel(d) >= n, "elementwise: dst smaller than src");
        if (in.op == VOP_EWMAX) NEED(nel(b) >= n, "EWMAX: b smaller than a");
        if (in.op == VOP_CLAMP) NEED(nel(b) >= 2, "CLAMP: bounds slot needs 2 values");
        P_(ca, a);
        P_(cd, d);
        float *cb = nullptr;
        if (in.op == VOP_EWMAX || in.op == VOP_CLAMP)
            if ((rc = ptr(b, &cb))) return rc;
        if (n == 0) return VMLM_OK;
        vm_unary_kernel<<<vm_blocks(n), 256, 0, st>>>(cd, ca, cb, n, in.op);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_MASK_MUL: {
        const size_t r = rows(d), c = cols(d), bc = cols(b);
        NEED(nel(a) >= r * c && (r == 0 || (bc == 1 ? nel(b) >= r : nel(b) >= (r - 1) * bc + c)),
             "MASK_MUL: operand extents");
        P_(cd, d);
        P_(ca, a);
        P_(cb, b);
        if (r * c == 0) return VMLM_OK;
        vm_mask_mul_kernel<<<vm_blocks(r * c), 256, 0, st>>>(cd, ca, cb, r, c, bc);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_JMP:
        *ip = d;
        return VMLM_OK;
    case VOP_CMPLE: {
        float x, y;
        if ((rc = scalar(a, &x)) || (rc = scalar(b, &y))) return rc;
        if (x <= y) *ip = d;
        return VMLM_OK;
    }
    case VOP_LOOP_CNT: {  // :1108-1131
        NEED(rows(a) == 1, "LOOP_CNT: ctr must be [1,N]");
        NEED(d < *ip, "LOOP_CNT: target must be back");
        float v;
        if ((rc = scalar(a, &v))) return rc;
        const float nv = v - 1.0f;
        P_(ca, a);
        VMLM_HIP_CHECK(hipMemcpyAsync(ca, &nv, 4, hipMemcpyHostToDevice, st));
        VMLM_HIP_CHECK(hipStreamSynchronize(st));  // `nv` lives on this frame
        if (nv > 0.0f) *ip = d;
        return VMLM_OK;
    }
    case VOP_ROPE: {  // :1159-1223
        const size_t r = rows(a), c = cols(a);
        NEED(c >= 2 && (c & 1) == 0, "ROPE: hd must be even >= 2");
        NEED(nel(d) >= r * c, "ROPE: dst smaller than src");
        float theta;
        if ((rc = scalar(b, &theta))) return rc;
        NEED(theta > 0.0f, "ROPE: theta must be > 0");
        P_(cd, d);
        P_(ca, a);
        if (in.fl & VFL_RUNTIME) {
            P_(pp, in.dt);
            if (r == 0) return VMLM_OK;
            const float step = -2.0f / (float)c * host_ln_f(theta);
            vm_rope_kernel<<<vm_blocks(r * c / 2), 256, 0, st>>>(cd, ca, (int)r, (int)c, step, pp,
                                                                 guard);
            VMLM_HIP_CHECK(hipGetLastError());
            return VMLM_OK;
        }
        return launch_rope(cd, ca, r, c, c, theta, (float)in.dt, 1, st);
    }
    case VOP_SCALE: {
        const size_t n = nel(d);
        NEED(nel(a) >= n && nel(b) >= 1, "SCALE: operand extents");
        P_(cd, d);
        P_(ca, a);
        P_(cb, b);
        if (n == 0) return VMLM_OK;
        vm_scale_kernel<<<vm_blocks(n), 256, 0, st>>>(cd, ca, cb, n);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_PRINT: {
        P_(cd, d);
        const size_t n = nel(d), o = vm->out.size();
        vm->out.resize(o + n);
        if (n) VMLM_HIP_CHECK(hipMemcpyAsync(vm->out.data() + o, cd, n * 4, hipMemcpyDeviceToHost, st));
        VMLM_HIP_CHECK(hipStreamSynchronize(st));
        return VMLM_OK;
    }
    case VOP_BIAS: {
        const size_t r = rows(d), c = cols(d);
        NEED(nel(a) >= c, "BIAS: bias shorter than the row");
        P_(cd, d);
        P_(cb, a);
        return launch_bias(cd, cb, r, c, st);
    }
    case VOP_EMB: {  // :1351-1436
        const size_t r = rows(a), c = cols(a);
        NEED(nel(d) >= c && nel(b) >= 1, "EMB: operand extents");
        P_(cd, d);
        P_(ca, a);
        P_(rowp, b);
        if (dt(a) == VDT_BF16)
            return launch_emb_bf16(cd, c, (const uint16_t *)ca, r, c, rowp, nullptr, 1, st, guard);
        NEED(dt(a) == VDT_F32, "EMB table dtype unsupported");
        vm_emb_f32_kernel<<<1, 256, 0, st>>>(cd, ca, r, c, rowp, guard);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_BMM: {  // :1440-1466
        const size_t abm = rows(a), k = cols(a), bk = rows(b), nn = cols(b);
        P_(ca, a);
        P_(cb, b);
        P_(cc, d);
        if (bk == k) {
            NEED(nel(d) >= abm * nn, "BMM: dst too small");
            return vmlm_hip_gemm(ca, cb, cc, abm, nn, k, false, st);
        }
        NEED(k > 0 && bk % k == 0 && bk / k > 0 && abm % (bk / k) == 0, "BMM: batch shapes");
        const size_t bs = bk / k, m = abm / bs;
        NEED(nel(d) >= bs * m * nn, "BMM: dst too small");
        for (size_t i = 0; i < bs; ++i)
            if ((rc = vmlm_hip_gemm(ca + i * m * k, cb + i * k * nn, cc + i * m * nn, m, nn, k,
                                    false, st)))
                return rc;
        return VMLM_OK;
    }
    case VOP_TRANSPOSE: {
        const size_t m = rows(a), c = cols(a);
        NEED(nel(d) >= m * c, "TRANSPOSE: dst smaller than src");
        P_(ca, a);
        P_(cd, d);
        if (m * c == 0) return VMLM_OK;
        vm_transpose_kernel<<<vm_blocks(m * c), 256, 0, st>>>(cd, ca, m, c);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_SLICE: {  // :1486-1497
        const size_t dr = rows(d), dc = cols(d), sc = cols(a);
        NEED(dr == 0 || dc == 0 || (dr - 1) * sc + b + dc <= nel(a), "SLICE: reads past src");
        P_(ca, a);
        P_(cd, d);
        return copy2d(cd, dc, 0, ca, sc, b, dr, dc);
    }
    case VOP_CONCAT: {
        const size_t r = rows(a), ac = cols(a), bc = cols(b);
        NEED(rows(b) >= r && nel(d) >= r * (ac + bc), "CONCAT: operand extents");
        P_(pa, a);
        P_(pb, b);
        P_(pd, d);
        if ((rc = copy2d(pd, ac + bc, 0, pa, ac, 0, r, ac))) return rc;
        return copy2d(pd, ac + bc, ac, pb, bc, 0, r, bc);
    }
    case VOP_WRITECOL: {  // :1515-1533
        const size_t dr = rows(d), dc = cols(d), sr = rows(a), sc = cols(a);
        NEED(sr >= dr, "WRITECOL: src has fewer rows than dst");
        P_(ca, a);
        P_(cd, d);
        if (in.fl & VFL_RUNTIME) {
            P_(cp, in.dt);
            return copy2d(cd, dc, 0, ca, sc, 0, dr, sc, cp, dc);
        }
        NEED((size_t)b + sc <= dc, "WRITECOL: off + src.cols exceeds dst row width");
        return copy2d(cd, dc, b, ca, sc, 0, dr, sc);
    }
    case VOP_SUM: case VOP_MAX: {
        const size_t r = rows(a), c = cols(a);
        if (in.op == VOP_MAX) {
            NEED(c != 0 && rows(d) != 0 && cols(d) != 0, "MAX: src or dst slot has width 0");
            NEED(rows(d) == r && cols(d) == 1, "MAX: dst must be [rows,1]");
        }
        NEED(nel(d) >= r, "SUM: dst shorter than rows");
        P_(ca, a);
        P_(cd, d);
        if (r == 0) return VMLM_OK;
        vm_rowwise_kernel<<<vm_blocks(r), 256, 0, st>>>(cd, ca, nullptr, r, c, in.op);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_TOPK_IDX: {  // :1649-1681
        NEED(rows(a) && cols(a) && rows(d) && cols(d), "TOPK_IDX: src or dst slot has width 0");
        NEED(rows(d) == 1 && cols(d) == 1, "TOPK_IDX: dst must be [1,1]");
        P_(ca, a);
        P_(cd, d);
        return launch_argmax(ca, cols(a), cd, nullptr, vm->keys, st);
    }
    case VOP_TOPK_BY_STRENGTH: {  // :1743-1955
        const size_t sr = rows(a), sc = cols(a), dr = rows(d), dc = cols(d);
        NEED(sr && sc && dr && dc, "TOPK_BY_STRENGTH: src or dst slot has width 0");
        const bool seg = (in.fl & VFL_SELGATE) != 0;
        size_t nrow, L, kmax, kseg;
        if (seg) {
            NEED(sc >= 1 && dc % 2 == 0, "TOPK_BY_STRENGTH: segmented dst must be [n,2k]");
            NEED(dr == sr, "TOPK_BY_STRENGTH: segmented dst rows != src rows");
            NEED(sc <= VM_TOPK_MAX_L, "TOPK_BY_STRENGTH: row width exceeds the bitmap (2048)");
            nrow = sr, L = sc, kseg = dc / 2, kmax = sc < kseg ? sc : kseg;
        } else {
            NEED(dc == 2, "TOPK_BY_STRENGTH: dst must be [L,2]");
            NEED(dr >= sr * sc, "TOPK_BY_STRENGTH: dst needs L rows");
            NEED(sr * sc <= VM_TOPK_MAX_L, "TOPK_BY_STRENGTH: L exceeds the selection bitmap (2048)");
            nrow = 1, L = sr * sc, kseg = L, kmax = L;
        }
        // k is checked on the host as well, so that its message is the reference's
        float kf;
        if ((rc = scalar(b, &kf))) return rc;
        NEED(kf >= 0.0f, "TOPK_BY_STRENGTH: k is negative or NaN");
        const size_t kk = kf >= 1.8446744e19f ? ~(size_t)0 : (size_t)kf;
        NEED(kk <= (seg ? sc : L), seg ? "TOPK_BY_STRENGTH: k > row width"
                                       : "TOPK_BY_STRENGTH: k > L");
        NEED(!seg || kk <= kseg, "TOPK_BY_STRENGTH: k > dst segment width");
        P_(cs, a);
        P_(ck, b);
        P_(cd, d);
        void *taken;
        if ((rc = ws(nrow * L, &taken))) return rc;
        vm_topk_strength_kernel<<<vm_blocks(nrow, 64), 64, 0, st>>>(
            cd, seg ? dc : 0, cs, nrow, L, ck, kmax, kseg, (unsigned char *)taken, guard);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    case VOP_SPARSE_MATVEC: {  // :2058-2346
        const uint32_t wslot = in.fl & 0x3Fu, xslot = in.dt;
        const bool want_nnz = (in.fl & VFL_NNZ) != 0, selgate = (in.fl & VFL_SELGATE) != 0;
        const size_t orows = rows(a), ocols = cols(a), srows = rows(b), scols = cols(b);
        const size_t dr = rows(d), dc = cols(d);
        NEED(orows && ocols && srows && scols, "SPARSE_MATVEC: offsets or src slot has width 0");
        NEED(dr && dc, "SPARSE_MATVEC: dst slot has width 0");
        const uint32_t selslot = selgate ? b + 1 : b;
        NEED(!selgate || selslot < vm->slots.size(), "SPARSE_MATVEC: sel slot (src+1) does not exist");
        const size_t secols = cols(selslot), serows = rows(selslot);
        NEED(!selgate || (secols != 0 && secols % 2 == 0),
             "SPARSE_MATVEC: selgate needs an even sel width");
        NEED(ocols == 1 && scols == 1, "SPARSE_MATVEC: offsets and src must be column vectors");
        NEED(orows >= 2, "SPARSE_MATVEC: offsets must have n_neurons+1 entries");
        const size_t n = orows - 1, nnz = srows;
        NEED(dc == 1 && dr >= n, "SPARSE_MATVEC: dst must be [n_neurons(,1)]");
        NEED(!want_nnz || dr >= n + 1, "SPARSE_MATVEC: nnz needs dst to be [n_neurons+1]");
        const size_t nx = nel(xslot);
        NEED(nx != 0, "SPARSE_MATVEC: x slot (dt) has width 0");
        NEED(nel(wslot) != 0, "SPARSE_MATVEC: weight slot (fl) has width 0");
        NEED(nel(wslot) >= nnz, "SPARSE_MATVEC: weight slot shorter than src");
        const size_t segw = secols / 2;
        NEED(!selgate || (segw && n * segw * 2 <= serows * secols),
             "SPARSE_MATVEC: sel table too small for n_neurons");
        P_(co, a);
        P_(cs, b);
        P_(cw, wslot);
        P_(cx, xslot);
        P_(cd, d);
        float *csel = nullptr;
        if (selgate && (rc = ptr(selslot, &csel))) return rc;
        void *cnt;
        if ((rc = ws(n * sizeof(unsigned), &cnt))) return rc;
        vm_sparse_matvec_kernel<<<vm_blocks(n, 64), 64, 0, st>>>(
            cd, co, cs, cw, cx, n, nnz, nx, csel, segw, (unsigned *)cnt, guard);
        VMLM_HIP_CHECK(hipGetLastError());
        if (want_nnz) {
            vm_nnz_kernel<<<1, 64, 0, st>>>(cd + n, (const unsigned *)cnt, n);
            VMLM_HIP_CHECK(hipGetLastError());
        }
        return VMLM_OK;
    }
    case 60: case 61: case 62: case 63: case 64: case 65: case 66: case 67: case 68:
    case 69: case 70: case 80: case 81: case 82: case 83: case 84:
        return fail(6, "train feature disabled");
    default:
        return fail(VMLM_ERR_UNIMPL, "unimpl op %u", in.op);
    }
}

}  // namespace

extern "C" {

// A run of int8 GEMMs over one input at decode rows in one launch
// (launch_fx_multi); each GEMM as OP_GEMM gives it, and with the gate/up
// pair the ACT silu and EWMUL after it; after an RMSNORM of the input, the
// normalized rows (written to the RMSNORM's output too) as its kernel gives
// them. The swizzled copies are looked up as OP_GEMM does (through the layer
// base); a run whose GEMMs are not all swizzled or all row-major, or a
// normalizing run over row-major weights, runs opcode by opcode.
int Exec::fused_gemms(const VmFused &f) {
    int rc = VMLM_OK;
    const VmIns *t0 = &vm->text[f.start];
    const VmIns *g = t0 + (f.norm ? 1 : 0);  // the GEMMs (after the RMSNORM)
    const uint32_t A = f.norm ? f.nx : g[0].a;  // the rows the kernel reads
    FxMultiArgs x;
    x.nseg = (int)f.nh;
    x.M = (int)rows(A);
    x.K = (int)cols(A);
    x.ldx = x.K;
    x.ldw = x.K;
    float *ca;
    if ((rc = ptr(A, &ca))) return rc;
    x.X = ca;
    int nsw = 0;
    for (int t = 0; t < x.nseg; ++t) {
        float *cb, *cs, *cc;
        if ((rc = ptr(g[t].b, &cb)) || (rc = ptr(g[t].dt, &cs)) || (rc = ptr(g[t].dst, &cc)))
            return rc;
        const size_t N = rows(g[t].b);
        const auto it = vm->swz.find((size_t)((char *)cb - vm->pool->dev));
        const bool sw = it != vm->swz.end() && it->second.rows == N && it->second.cols == cols(g[t].b);
        nsw += sw;
        x.seg[t].W = sw ? (const void *)it->second.dev : (const void *)cb;
        x.seg[t].scale = cs;
        x.seg[t].C = cc;
        x.seg[t].N = (int)N;
        x.seg[t].ldc = (int)N;
    }
    x.swizzled = nsw == x.nseg;
    if (f.kind == VF_GATE_UP) {
        float *act;
        if ((rc = ptr(f.att, &act))) return rc;
        x.act = act;
        x.ldact = x.seg[0].N;
    }
    if (f.kind == VF_GEMM_ADD) {
        float *r, *z;
        if ((rc = ptr(f.k, &r)) || (rc = ptr(f.att, &z))) return rc;
        x.radd = r;
        x.zadd = z;
    }
    bool aligned = ((uintptr_t)ca & 15) == 0;
    for (int t = 0; t < x.nseg; ++t) aligned = aligned && ((uintptr_t)x.seg[t].W & 15) == 0;
    if (f.norm) {  // the RMSNORM opcode's operands (its epsilon read as it reads it)
        float *gp, *yp;
        if ((rc = ptr(f.ng, &gp)) || (rc = ptr(f.ny, &yp)) || (rc = scalar(f.ne, &x.norm_eps)))
            return rc;
        x.norm_g = gp;
        x.norm_out = yp;
        aligned = aligned && ((uintptr_t)gp & 15) == 0 && ((uintptr_t)yp & 15) == 0;
    }
    // mixed layouts, operands OP_GEMM would not give this kernel, or a norm
    // over row-major weights: opcode by opcode
    if ((nsw != 0 && nsw != x.nseg) || !aligned || (f.norm && !x.swizzled)) {
        for (uint32_t t = 0; t < f.len; ++t) {
            size_t ip = f.start + t + 1;
            if ((rc = step(t0[t], &ip))) return rc;
        }
        return VMLM_OK;
    }
    return launch_fx_multi(x, vm->st);
}

// A run found by vm_detect_fusions, in one launch: the host-side guards of
// its opcodes (ROPE's theta), then the kernel with the device-side ones.
int Exec::fused(const VmFused &f) {
    int rc = VMLM_OK;
    if (f.kind == VF_GEMMS || f.kind == VF_GATE_UP || f.kind == VF_GEMM_ADD) return fused_gemms(f);
    if (f.kind == VF_COL_RUN) {
        for (uint32_t q = 0; q < f.nh; ++q) {
            const VmColStream &c = f.col[q];
            float *pc, *px, *py;
            if ((rc = ptr(c.c, &pc)) || (rc = ptr(c.x, &px)) || (rc = ptr(c.y, &py))) return rc;
            const size_t xc = cols(c.x);
            if ((rc = copy2d(py, cols(c.y), c.yo, px, xc, c.xo, rows(c.y), f.cols)) ||
                (rc = copy2d(pc, 1, 0, px, xc, (size_t)c.xo + f.cols - 1, rows(c.c), 1)))
                return rc;
        }
        return VMLM_OK;
    }
    float theta;
    if ((rc = scalar(f.theta, &theta))) return rc;
    VMLM_GUARD(theta > 0.0f, "ROPE: theta must be > 0");
    const float step = -2.0f / (float)f.hd * host_ln_f(theta);
    hipStream_t st = vm->st;
    VmKvAppend ap{};
    if (f.kind == VF_KV_APPEND || f.kind == VF_KV_ATTN) {
        float *k, *v, *pp, *s0, *s1, *s2, *s3, *s4;
        if ((rc = ptr(f.k, &k)) || (rc = ptr(f.v, &v)) || (rc = ptr(f.pos, &pp)) ||
            (rc = ptr(f.s0, &s0)) || (rc = ptr(f.s1, &s1)) || (rc = ptr(f.s2, &s2)) ||
            (rc = ptr(f.s3, &s3)) || (rc = ptr(f.s4, &s4)))
            return rc;
        ap.k = k;
        ap.v = v;
        ap.kc = f.tab;
        ap.posp = pp;
        ap.step = step;
        ap.hd = (int)f.hd;
        ap.cols = (int)f.cols;
        ap.kdh = s0;
        ap.vdh = s1;
        ap.kdrot = s2;
        ap.kdT = s3;
        ap.vdT = s4;
    }
    if (f.kind == VF_KV_APPEND) {
        vm_kv_append_kernel<<<f.nh, 64, 0, st>>>(ap, (int)f.nh, guard);
        VMLM_HIP_CHECK(hipGetLastError());
        return VMLM_OK;
    }
    const bool joined = f.kind == VF_KV_ATTN;
    VmHeadAttn a;
    float *q, *pp, *lp, *sp, *att, *s0, *s1, *s2, *s3;
    if ((rc = ptr(joined ? f.aq : f.k, &q)) || (rc = ptr(f.pos, &pp)) ||
        (rc = ptr(joined ? f.alive : f.live, &lp)) || (rc = ptr(joined ? f.ascale : f.scale, &sp)) ||
        (rc = ptr(joined ? f.aatt : f.att, &att)) || (rc = ptr(joined ? f.a0 : f.s0, &s0)) ||
        (rc = ptr(joined ? f.a1 : f.s1, &s1)) || (rc = ptr(joined ? f.a2 : f.s2, &s2)) ||
        (rc = ptr(joined ? f.a3 : f.s3, &s3)))
        return rc;
    a.q = q;
    a.kc = f.tab;
    a.posp = pp;
    a.livep = lp;
    a.scalep = sp;
    a.step = step;
    a.hd = (int)f.hd;
    a.cols = (int)f.cols;
    a.att = att;
    a.qdh = s0;
    a.qdrot = s1;
    a.scd = s2;
    a.ctxd = s3;
    // the FAST form over four workgroups per head (groups of 8 heads)
    const unsigned g4 = (f.nh + 7) / 8 * 32;
    if (joined)
        vm_head_attn_kernel<true, true, 4><<<g4, 256, (f.hd + f.cols) * sizeof(float), st>>>(
            a, (int)f.nh, guard, ap);
    else if (f.hd == 64 && f.cols <= 256)
        vm_head_attn_kernel<true, false, 4><<<g4, 256, (f.hd + f.cols) * sizeof(float), st>>>(
            a, (int)f.nh, guard);
    else
        vm_head_attn_kernel<false><<<f.nh, 256, (f.hd + f.cols) * sizeof(float), st>>>(a, (int)f.nh, guard);
    VMLM_HIP_CHECK(hipGetLastError());
    return VMLM_OK;
}

// The slot an instruction writes: `dst`, or `a` for LOOP_CNT (its counter)
// and STACK_INIT; UINT32_MAX for instructions that write no slot.
static uint32_t written_slot(const VmIns &in) {
    switch (in.op) {
    case VOP_SHAPE: case VOP_JMP: case VOP_CMPLE: case VOP_LAYERB: case VOP_PRINT:
    case VOP_HALT: case VOP_LN_EPS:
        return UINT32_MAX;
    case VOP_LOOP_CNT: case VOP_STACK_INIT:
        return in.a;
    default:
        return in.dst;
    }
}

// A program may write a constant slot (the interpreter's slot_mut does not
// distinguish kinds, core/src/interp.rs:477). In a private pool the write
// lands in this VM's own copy and the host's cache of constant scalars is
// dropped, so later CMPLE / LOOP_CNT / SCALE operands read the new value. A
// pool shared over mapped weights is read-only, as the interpreter's mapped
// pool is (cpool_readonly, :87, 2357-2362): such a write is refused with 9.
static int const_write_check(vmlm_vm *vm, const VmIns &in, size_t at) {
    const uint32_t w = written_slot(in);
    if (w >= vm->slots.size() || vm->slots[w].kind != VSLOT_CONST) return VMLM_OK;
    VMLM_GUARD(!vm->pool || !vm->pool->host,
               "weights are mapped read-only: instruction %zu (op %u) writes constant slot %u", at,
               (unsigned)in.op, w);
    vm->kcache.clear();
    vm_drop_graphs(vm);  // captured bodies may have baked the constant's old value
    return VMLM_OK;
}

// One instruction, or one fused run, at ip (advanced past it).
static int vm_exec_one(Exec &ex, size_t &ip, bool &halt) {
    vmlm_vm *vm = ex.vm;
    if (vm->fuse_at[ip] >= 0) {  // a matched run in one launch (no constant written)
        const VmFused &f = vm->fused[vm->fuse_at[ip]];
        const int rc = ex.fused(f);
        if (!rc) ip += f.len;
        return rc;
    }
    const VmIns in = vm->text[ip++];
    if (in.op == VOP_HALT) {
        halt = true;
        return VMLM_OK;
    }
    int rc = const_write_check(vm, in, ip - 1);
    return rc ? rc : ex.step(in, &ip);
}

// Captures segment g into a HIP graph and launches it once (this visit's
// work: capture itself runs nothing). Anything in the segment that would
// read the device on the host, allocate, or fail ends the capture; the
// caller then runs the segment opcode by opcode, which reports a real error
// where it occurs.
static int vm_capture(Exec &ex, VmSeg &g) {
    vmlm_vm *vm = ex.vm;
    if (hipStreamBeginCapture(vm->st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        (void)hipGetLastError();
        return VMLM_ERR_UNIMPL;
    }
    ex.capturing = true;
    size_t ip = g.start;
    bool halt = false;
    int rc = VMLM_OK;
    while (rc == VMLM_OK && ip < g.end && !halt) rc = vm_exec_one(ex, ip, halt);
    ex.capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(vm->st, &graph);
    hipGraphExec_t x = nullptr;
    if (rc == VMLM_OK && e == hipSuccess && graph && ip == g.end && !halt)
        e = hipGraphInstantiate(&x, graph, nullptr, nullptr, 0);
    else if (e == hipSuccess)
        e = hipErrorUnknown;
    if (graph) (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        if (x) (void)hipGraphExecDestroy(x);
        (void)hipGetLastError();
        return VMLM_ERR_UNIMPL;
    }
    g.exec = x;
    g.state = VS_GRAPH;
    g.base = vm->layer_base;
    VMLM_HIP_CHECK(hipGraphLaunch(x, vm->st));
    return VMLM_OK;
}

int vmlm_vm_run(vmlm_vm *vm) {
    VMLM_GUARD(vm, "vm_run: null vm");
    int rc = ensure_init();
    if (rc) return rc;
    // this VM's own guard flag: a guard raised by another VM or session on
    // another stream is neither lost nor reported here
    if ((rc = launch_fill_zero(vm->guard, sizeof(int), vm->st))) return rc;
    Exec ex{vm, vm->guard};
    size_t ip = 0;
    const size_t n = vm->text.size();
    bool halt = false;
    while (ip < n && !halt) {
        if (vm->graphs && vm->seg_at[ip] >= 0) {
            VmSeg &g = vm->segs[vm->seg_at[ip]];
            if (g.state == VS_GRAPH && g.base == vm->layer_base) {
                VMLM_HIP_CHECK(hipGraphLaunch(g.exec, vm->st));
                ip = g.end;
                continue;
            }
            if (g.state == VS_SEEN) {
                if (vm_capture(ex, g) == VMLM_OK) {  // captured and launched
                    ip = g.end;
                    continue;
                }
                g.state = VS_EAGER;  // opcode by opcode from now on
            } else if (g.state == VS_NEW) {
                g.state = VS_SEEN;  // the first visit runs eagerly (workspaces, scalars)
            }
        }
        if ((rc = vm_exec_one(ex, ip, halt))) {
            (void)hipStreamSynchronize(vm->st);
            return rc;
        }
    }
    int tripped = 0;
    VMLM_HIP_CHECK(hipMemcpyAsync(&tripped, vm->guard, sizeof(int), hipMemcpyDeviceToHost, vm->st));
    VMLM_HIP_CHECK(hipStreamSynchronize(vm->st));
    if (tripped & VG_OFFSETS)
        return fail(VMLM_ERR_GUARD, "SPARSE_MATVEC: offsets out of range (device check)");
    if (tripped & VG_SEL)
        return fail(VMLM_ERR_GUARD, "SPARSE_MATVEC: sel index outside its CSR row (device check)");
    if (tripped & VG_SRC)
        return fail(VMLM_ERR_GUARD, "SPARSE_MATVEC: src_id out of range (device check)");
    if (tripped)
        return fail(VMLM_ERR_GUARD,
                    "device guard tripped (code %d): row, position or column index out of range",
                    tripped);
    return VMLM_OK;
}

int vmlm_vm_find_slot(const vmlm_vm *vm, const char *name, uint32_t *slot) {
    VMLM_GUARD(vm && name && slot, "vm_find_slot: null argument");
    uint32_t h = 0x811C9DC5u;  // FNV-1a (core/src/format.rs hash32)
    for (const char *c = name; *c; ++c) h = (h ^ (uint8_t)*c) * 0x01000193u;
    for (size_t i = 0; i < vm->names.size(); ++i)
        if (vm->names[i] == h) {
            *slot = (uint32_t)i;
            return VMLM_OK;
        }
    return fail(7, "slot not found: %s", name);
}

int vmlm_vm_slot_info(vmlm_vm *vm, uint32_t slot, void **dptr, uint32_t *rows, uint32_t *cols,
                      uint8_t *dtype) {
    VMLM_GUARD(vm, "vm_slot_info: null vm");
    Exec ex{vm, vm->guard};
    float *p;
    int rc = ex.ptr(slot, &p);
    if (rc) return rc;
    if (dptr) *dptr = p;
    if (rows) *rows = vm->slots[slot].rows;
    if (cols) *cols = vm->slots[slot].cols;
    if (dtype) *dtype = vm->slots[slot].dtype;
    return VMLM_OK;
}

static int vm_xfer(vmlm_vm *vm, uint32_t slot, void *host, size_t count, bool write) {
    VMLM_GUARD(vm && (host || count == 0), "vm slot transfer: null argument");
    Exec ex{vm, vm->guard};
    float *p;
    int rc = ex.ptr(slot, &p);
    if (rc) return rc;
    VMLM_GUARD(vm->slots[slot].dtype == VDT_F32, "slot %u is not f32", slot);
    VMLM_GUARD(vm->slots[slot].kind != VSLOT_CONST || !write, "constant slot %u is read-only", slot);
    VMLM_GUARD(count <= ex.nel(slot), "slot %u holds %zu values, %zu requested", slot, ex.nel(slot),
               count);
    if (count)
        VMLM_HIP_CHECK(hipMemcpyAsync(write ? (void *)p : host, write ? host : (void *)p, count * 4,
                                      write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost, vm->st));
    VMLM_HIP_CHECK(hipStreamSynchronize(vm->st));
    return VMLM_OK;
}
int vmlm_vm_write_slot(vmlm_vm *vm, uint32_t slot, const float *host, size_t count) {
    return vm_xfer(vm, slot, (void *)host, count, true);
}
int vmlm_vm_read_slot(vmlm_vm *vm, uint32_t slot, float *host, size_t count) {
    return vm_xfer(vm, slot, host, count, false);
}

int vmlm_vm_output(vmlm_vm *vm, float *host, size_t cap, size_t *count) {
    VMLM_GUARD(vm && count, "vm_output: null argument");
    *count = vm->out.size();
    if (host && cap) std::memcpy(host, vm->out.data(), (cap < *count ? cap : *count) * 4);
    return VMLM_OK;
}
int vmlm_vm_clear_output(vmlm_vm *vm) {
    VMLM_GUARD(vm, "vm_clear_output: null vm");
    vm->out.clear();
    return VMLM_OK;
}

}  // extern "C"

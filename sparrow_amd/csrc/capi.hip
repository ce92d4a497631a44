// capi.hip -- the extern "C" boundary of libvmlm_hip.so (include/vmlm_hip.h).
//
// Layer 1 (vmlm_*): host pointers, exact vmlm-ops parameter lists; each call
// stages its operands in a per-stream device workspace, runs, copies back and
// synchronises (serialised by a mutex). Layer 2 (vmlm_hip_*): device pointers,
// asynchronous. Both validate like the reference interpreter's guards and
// return its exit codes instead of exiting.
#include <atomic>
#include <cstdarg>
#include <cstring>
#include <memory>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <utility>
#include <vector>

#include "internal.hpp"

namespace vmlm {

// ------------------------------------------------------------------ errors
static thread_local char g_err[1024] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(VMLM_ERR_DEVICE, "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
}

// ------------------------------------------------------------------ scratch
// Device memory of the allocation-free entry point
// (vmlm_hip_gemm_nt_int8_noalloc): one fixed array in the code object, held
// by every GPU the library is loaded on until the process ends. In host code
// `scratch` names a host-side stand-in, never a device address: init
// resolves the array's address on its device once (hipGetSymbolAddress) and
// only that pointer is passed to kernels.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
static void *g_scratch_ptr[MAX_DEVICES];  // device address of `scratch`, per device
static int g_scratch_status = VMLM_ERR_DEVICE;
static char g_scratch_err[256] = "scratch not set up";

// With `device` current: records the device address of `scratch`.
static void setup_scratch(int device) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        snprintf(g_scratch_err, sizeof(g_scratch_err), "hipGetSymbolAddress(scratch): %s",
                 hipGetErrorString(e));
        return;
    }
    if (device >= 0 && device < MAX_DEVICES) {
        g_scratch_ptr[device] = p;
        g_scratch_status = VMLM_OK;
    }
}

// ------------------------------------------------------------------ init
static std::once_flag g_once;
static int g_init_status = -1;
static std::atomic<bool> g_ready{false};
static hipStream_t g_stream = nullptr;
static int *g_guard = nullptr;
static std::mutex g_host_mutex;
static std::mutex g_event_mutex;
static std::vector<hipEvent_t> g_events;

static void do_init(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        g_init_status = fail(VMLM_ERR_DEVICE, "no HIP device available (%s)",
                             e == hipSuccess ? "count 0" : hipGetErrorString(e));
        return;
    }
    if ((e = hipSetDevice(device)) != hipSuccess) {
        g_init_status = hip_fail(e, "hipSetDevice");
        return;
    }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) {
        g_init_status = hip_fail(e, "hipGetDeviceProperties");
        return;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_status = fail(VMLM_ERR_DEVICE, "libvmlm_hip is built for gfx950, device is %s",
                             prop.gcnArchName);
        return;
    }
    if ((e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking)) != hipSuccess) {
        g_init_status = hip_fail(e, "hipStreamCreate");
        return;
    }
    if ((e = hipMalloc(&g_guard, sizeof(int))) != hipSuccess ||
        (e = hipMemset(g_guard, 0, sizeof(int))) != hipSuccess) {
        g_init_status = hip_fail(e, "guard flag");
        return;
    }
    setup_scratch(device);
    g_init_status = VMLM_OK;
    g_ready.store(true, std::memory_order_release);
}

int ensure_init() {
    std::call_once(g_once, do_init, 0);
    if (g_init_status != VMLM_OK) return fail(VMLM_ERR_DEVICE, "%s", g_err[0] ? g_err : "init failed");
    return VMLM_OK;
}
hipStream_t lib_stream() { return g_stream; }
int *guard_flag_ptr() { return g_guard; }

// ops/src/kernels.rs:240-255, host side
float host_ln_f(float x) {
    if (x <= 0.0f) return -88.0f;
    uint32_t bits;
    std::memcpy(&bits, &x, 4);
    int e = (int)((bits >> 23) & 0xffu) - 127;
    uint32_t mb = (bits & 0x007fffffu) | 0x3f800000u;
    float m;
    std::memcpy(&m, &mb, 4);
    if (m > 1.4142136f) {
        m *= 0.5f;
        e += 1;
    }
    float t = (m - 1.0f) / (m + 1.0f);
    float t2 = t * t;
    float p = 2.0f * t * (1.0f + t2 * (0.33333334f + t2 * (0.2f + t2 * 0.14285715f)));
    return p + (float)e * 0.69314718f;
}

// ------------------------------------------------------------------ staging
// Stream-ordered device buffers freed when the scope ends (after the stream
// work that uses them is enqueued).
// Temporaries of an entry point come from a per-stream arena of persistent
// device blocks, bump-allocated for the duration of the call and reused by
// the next call on the same stream (stream order keeps the uses apart); the
// arena's lock is held while the call enqueues its work. Requests above
// ARENA_BIG go to the stream-ordered allocator instead and are freed after.
constexpr size_t ARENA_BIG = (size_t)1 << 30;
struct Arena {
    std::recursive_mutex mu;  // an entry point may call another on the same stream
    std::vector<std::pair<char *, size_t>> blocks;
    size_t blk = 0, off = 0;
    int depth = 0;  // nested calls keep bumping; the outermost one resets
};
static std::mutex g_arena_map_mutex;
static std::unordered_map<hipStream_t, std::unique_ptr<Arena>> g_arenas;

static Arena &arena_for(hipStream_t st) {
    std::lock_guard<std::mutex> lk(g_arena_map_mutex);
    std::unique_ptr<Arena> &a = g_arenas[st];
    if (!a) a.reset(new Arena);
    return *a;
}

struct Stage {
    hipStream_t st;
    Arena &ar;
    std::unique_lock<std::recursive_mutex> lk;
    std::vector<void *> big;
    int status = VMLM_OK;
    explicit Stage(hipStream_t s) : st(s), ar(arena_for(s)), lk(ar.mu) {
        if (ar.depth++ == 0) {
            ar.blk = 0;
            ar.off = 0;
        }
    }
    ~Stage() {
        for (void *p : big) (void)hipFreeAsync(p, st);
        --ar.depth;
    }
    template <typename T>
    T *alloc(size_t count) {
        const size_t bytes = ((count ? count : 1) * sizeof(T) + 255) / 256 * 256;
        if (bytes > ARENA_BIG) {
            void *p = nullptr;
            hipError_t e = hipMallocAsync(&p, bytes, st);
            if (e != hipSuccess) {
                status = hip_fail(e, "hipMallocAsync");
                return nullptr;
            }
            big.push_back(p);
            return (T *)p;
        }
        while (ar.blk < ar.blocks.size()) {
            if (ar.off + bytes <= ar.blocks[ar.blk].second) {
                char *p = ar.blocks[ar.blk].first + ar.off;
                ar.off += bytes;
                return (T *)p;
            }
            ++ar.blk;
            ar.off = 0;
        }
        size_t sz = ar.blocks.empty() ? ((size_t)16 << 20) : ar.blocks.back().second * 2;
        if (sz < bytes) sz = bytes;
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess) {
            status = hip_fail(e, "hipMalloc (workspace)");
            return nullptr;
        }
        ar.blocks.emplace_back((char *)p, sz);
        ar.blk = ar.blocks.size() - 1;
        ar.off = bytes;
        return (T *)p;
    }
    template <typename T>
    T *upload(const T *host, size_t count) {
        T *d = alloc<T>(count);
        if (!d) return nullptr;
        if (count) {
            hipError_t e = hipMemcpyAsync(d, host, count * sizeof(T), hipMemcpyHostToDevice, st);
            if (e != hipSuccess) {
                status = hip_fail(e, "upload");
                return nullptr;
            }
        }
        return d;
    }
};

// Bump allocation inside the fixed scratch array: the workspace of the
// allocation-free entry point. A request past the end fails with status 9
// and nothing is launched.
struct ScratchBump {
    char *base;
    size_t cap;
    size_t off = 0;
    int status = VMLM_OK;
    template <typename T>
    T *alloc(size_t count) {
        if (status) return nullptr;
        const size_t bytes = (count * sizeof(T) + 255) / 256 * 256;
        if (off + bytes > cap) {
            status = fail(VMLM_ERR_GUARD,
                          "allocation-free call: this shape needs more than the %zu bytes of "
                          "scratch (%zu in use, %zu more requested)",
                          cap, off, bytes);
            return nullptr;
        }
        T *p = (T *)(base + off);
        off += bytes;
        return p;
    }
};

static int download(void *host, const void *dev, size_t bytes, hipStream_t st) {
    if (bytes) VMLM_HIP_CHECK(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, st));
    return VMLM_OK;
}

#define STAGE_OK(stg) \
    do {              \
        if ((stg).status) return (stg).status; \
    } while (0)

static inline size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// int8 / bf16 weight GEMM on device operands: C[m,n] = A[m,k] . W[n,k]^T (* scale).
// Pads K to a multiple of 128 when needed, then: int8 weights and m <= 16,
// the wide k-split GEMV; int8 weights, m > 16 and K unpadded, int8 rows and
// the int8 MFMA GEMM; otherwise A split into 3 bf16 terms and the GEMV kernel
// (m <= 16) or the tiled bf16 MFMA GEMM.
// Temporaries come from `stg`: the stream's arena (Stage) or the fixed
// scratch array of the allocation-free entry point (ScratchBump). Wsw, when
// given, is a swizzled copy of int8 W (launch_swizzle_w) that the caller
// keeps: the small-row launch and the int8-row GEMM read it instead of W.
template <class WS>
static int q_matmul(const float *a, const void *W, bool wi8, const float *scale, float *c,
                    size_t m, size_t n, size_t k, hipStream_t st, WS &stg,
                    const void *Wsw = nullptr) {
    if (m == 0 || n == 0) return VMLM_OK;
    const size_t esz = wi8 ? 1 : 2;
    const size_t Kp = round_up(k == 0 ? 1 : k, 128);  // one 128-byte GEMV chunk covers 128 k
    const void *Wd = W;
    if (Kp != k || ((uintptr_t)W & 15)) {
        // the padded weight copy is a device copy: refused up front while the
        // stream is being captured, so a capture never records it
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        VMLM_HIP_CHECK(hipStreamIsCapturing(st, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fail(VMLM_ERR_UNIMPL, "q8/bf16 GEMM with K %% 128 != 0 or unaligned weights "
                                         "stages a padded weight copy and cannot be captured");
        uint8_t *wp = stg.template alloc<uint8_t>(n * Kp * esz);
        STAGE_OK(stg);
        int rc0 = launch_fill_zero(wp, n * Kp * esz, st);
        if (rc0) return rc0;
        if (k) VMLM_HIP_CHECK(hipMemcpy2DAsync(wp, Kp * esz, W, k * esz, k * esz, n,
                                               hipMemcpyDeviceToDevice, st));
        Wd = wp;
    }
    const int T = 3;
    // int8 weights, up to FX_ROWS rows: one full-K launch whose waves split
    // their k-runs of the f32 rows into int8 terms themselves
    if (wi8 && m <= FX_ROWS && Wd == W && ((uintptr_t)a & 15) == 0 && k <= (size_t)1 << 30 &&
        fx_run_blocks((int)k)) {
        FxArgs x;
        x.W = Wsw ? Wsw : Wd;
        x.swizzled = Wsw != nullptr;
        x.ldw = (int)k;
        x.scale = scale;
        x.X = a;
        x.ldx = (int)k;
        x.C = c;
        x.ldc = (int)n;
        x.M = (int)m;
        x.N = (int)n;
        x.K = (int)k;
        return launch_fx_gemv(x, st);
    }
    // int8 weights, a few rows: the wide k-split GEMV splits the f32 rows
    // into terms while staging them, then the slices are reduced in order
    const size_t nch = Kp / 128;
    const int nc = nch % 2 == 0 ? 2 : nch % 3 == 0 ? 3 : 1;
    if (wi8 && m <= 16 && Wd == W && k % 4 == 0 && ((uintptr_t)a & 15) == 0 &&
        nch / nc <= 16) {
        const int ks = (int)(nch / nc);
        float *part = ks > 1 ? stg.template alloc<float>((size_t)ks * m * n) : nullptr;
        STAGE_OK(stg);
        GemvArgs g;
        g.W = Wd;
        g.w_int8 = true;
        g.scale = scale;
        g.X = a;
        g.ldx = (int)k;
        g.T = T;
        g.lda = (int)Kp;
        g.M = (int)m;
        g.N = (int)n;
        g.K = (int)Kp;
        g.tiles = 8;
        g.ksplit = ks;
        if (ks == 1) {
            g.Y = c;
            g.ldy = (int)n;
            return launch_gemv(g, st);
        }
        g.Y = part;
        g.ldy = (int)n;
        g.epi = EPI_PARTIAL;
        int rc = launch_gemv(g, st);
        if (rc) return rc;
        return launch_gemv_reduce(part, ks, (int)m, (int)n, scale, c, (int)n, st);
    }
    // int8 weights, many rows, unpadded K: the rows as int8 terms with a
    // per-row factor, then the int8 x int8 MFMA GEMM
    if (wi8 && m > 16 && Wd == W && Kp == k && k <= 8192 && ((uintptr_t)a & 15) == 0) {
        int8_t *a8 = stg.template alloc<int8_t>(q8_rows_bytes(m, k));
        float *a8s = stg.template alloc<float>(m);
        const size_t gw = gemm_i8_work_floats((int)m, (int)n, (int)k);
        float *gwork = gw ? stg.template alloc<float>(gw) : nullptr;
        // many rows: the weights swizzled into 1 KiB blocks first (one pass
        // over N x K bytes), so the GEMM's weight copies move whole blocks;
        // the allocation-free entry point keeps its scratch for the rows
        // (a swizzled copy the caller keeps is read as it is)
        const bool blk = Wsw || (std::is_same<WS, Stage>::value && m >= 256 && n % 16 == 0);
        int8_t *wsw = blk && !Wsw ? stg.template alloc<int8_t>(n * k) : nullptr;
        STAGE_OK(stg);
        int rc = launch_rows_q8(a, k, nullptr, 0.0f, m, k, a8, a8s, st);
        if (rc) return rc;
        if (wsw && (rc = launch_swizzle_w((const int8_t *)Wd, wsw, (int)n, (int)k, st))) return rc;
        GemmArgs g;
        g.W = Wsw ? Wsw : blk ? (const void *)wsw : Wd;
        g.w_blocked = blk;
        g.w_int8 = true;
        g.scale = scale;
        g.A8 = a8;
        g.a8s = a8s;
        g.work = gwork;
        g.work_floats = gw;
        g.lda = (int)k;
        g.M = (int)m;
        g.N = (int)n;
        g.K = (int)k;
        g.C = c;
        g.ldc = (int)n;
        rc = launch_gemm(g, st);
        if (rc) return rc;
        return launch_gemm_i8_nonfinite_rows(a, (int)k, (const int8_t *)Wd, (int)k, scale, a8s, c,
                                             (int)n, (int)m, (int)n, (int)k, st);
    }
    uint16_t *terms = stg.template alloc<uint16_t>((size_t)T * m * Kp);
    STAGE_OK(stg);
    int rc = launch_split_terms(a, k, (int)m, (int)k, T, terms, (int)Kp, st);
    if (rc) return rc;
    if (m > 16) {
        GemmArgs g;
        g.W = Wd;
        g.w_int8 = wi8;
        g.scale = scale;
        g.A = terms;
        g.T = T;
        g.lda = (int)Kp;
        g.M = (int)m;
        g.N = (int)n;
        g.K = (int)Kp;
        g.C = c;
        g.ldc = (int)n;
        return launch_gemm(g, st);
    }
    GemvArgs g;
    g.W = Wd;
    g.w_int8 = wi8;
    g.scale = scale;
    g.A = terms;
    g.T = T;
    g.lda = (int)Kp;
    g.M = (int)m;
    g.N = (int)n;
    g.K = (int)Kp;
    g.Y = c;
    g.ldy = (int)n;
    return launch_gemv(g, st);
}

// The int8 GEMM of the device VM, which keeps swizzled copies of its int8
// constants (wsw, or null where it has none).
int q8_gemm_vm(const float *a, const int8_t *q, const int8_t *wsw, const float *scale, float *c,
               size_t m, size_t n, size_t k, hipStream_t st) {
    VMLM_GUARD(scale != nullptr, "int8 gemm: scale slot must be f32 (null)");
    VMLM_GUARD(!wsw || n % 16 == 0, "int8 gemm: a swizzled copy needs N %% 16 == 0");
    Stage stg(st);
    return q_matmul(a, q, true, scale, c, m, n, k, st, stg, (const void *)wsw);
}
}  // namespace vmlm

using namespace vmlm;

#define INIT_OR_RETURN()              \
    do {                              \
        int _rc = ensure_init();      \
        if (_rc) return _rc;          \
    } while (0)

#define HOST_CALL_BEGIN()                                 \
    INIT_OR_RETURN();                                     \
    std::lock_guard<std::mutex> _lk(g_host_mutex);        \
    hipStream_t st = lib_stream()

#define FINISH(st_)                                       \
    do {                                                  \
        VMLM_HIP_CHECK(hipStreamSynchronize(st_));        \
        return vmlm_hip_check_guards();                   \
    } while (0)

extern "C" {

// ================================================================ library
int vmlm_hip_init(int device) {
    std::call_once(g_once, do_init, device);
    if (g_init_status != VMLM_OK) return fail(VMLM_ERR_DEVICE, "%s", g_err);
    return VMLM_OK;
}

const char *vmlm_hip_last_error(void) { return g_err; }
const char *vmlm_hip_version(void) { return "vmlm_hip 0.1 gfx950"; }

int vmlm_hip_sync(void) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipStreamSynchronize(lib_stream()));
    return VMLM_OK;
}

int vmlm_hip_malloc(void **dptr, size_t bytes) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipMalloc(dptr, bytes ? bytes : 1));
    return VMLM_OK;
}
int vmlm_hip_free(void *dptr) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipFree(dptr));
    return VMLM_OK;
}
int vmlm_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return VMLM_OK;
}
int vmlm_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipStreamSynchronize(lib_stream()));
    VMLM_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return VMLM_OK;
}
int vmlm_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, lib_stream()));
    VMLM_HIP_CHECK(hipStreamSynchronize(lib_stream()));
    return VMLM_OK;
}
int vmlm_hip_memset(void *dptr, int value, size_t bytes) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipMemset(dptr, value, bytes));
    return VMLM_OK;
}

int vmlm_hip_event_record(void *stream, int *event_id) {
    INIT_OR_RETURN();
    hipEvent_t ev;
    VMLM_HIP_CHECK(hipEventCreate(&ev));
    VMLM_HIP_CHECK(hipEventRecord(ev, as_stream(stream)));
    std::lock_guard<std::mutex> lk(g_event_mutex);
    g_events.push_back(ev);
    *event_id = (int)g_events.size() - 1;
    return VMLM_OK;
}
int vmlm_hip_event_elapsed_ms(int a, int b, float *ms) {
    INIT_OR_RETURN();
    std::lock_guard<std::mutex> lk(g_event_mutex);
    VMLM_GUARD(a >= 0 && b >= 0 && a < (int)g_events.size() && b < (int)g_events.size(),
               "event id out of range");
    VMLM_HIP_CHECK(hipEventSynchronize(g_events[b]));
    VMLM_HIP_CHECK(hipEventElapsedTime(ms, g_events[a], g_events[b]));
    return VMLM_OK;
}
int vmlm_hip_event_release_all(void) {
    INIT_OR_RETURN();
    std::lock_guard<std::mutex> lk(g_event_mutex);
    for (auto &e : g_events) (void)hipEventDestroy(e);
    g_events.clear();
    return VMLM_OK;
}

int vmlm_hip_capture_begin(void *stream) {
    INIT_OR_RETURN();
    VMLM_HIP_CHECK(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
    return VMLM_OK;
}

int vmlm_hip_capture_end(void *stream, void **graph) {
    INIT_OR_RETURN();
    VMLM_GUARD(graph, "capture_end: null graph");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    VMLM_HIP_CHECK(hipStreamEndCapture(as_stream(stream), &g));
    VMLM_GUARD(g, "capture_end: nothing captured");
    size_t n = 0;
    hipError_t e = hipGraphGetNodes(g, nullptr, &n);
    std::vector<hipGraphNode_t> nodes(n);
    if (e == hipSuccess && n) e = hipGraphGetNodes(g, nodes.data(), &n);
    int rc = e == hipSuccess ? VMLM_OK : hip_fail(e, "hipGraphGetNodes");
    for (size_t i = 0; rc == VMLM_OK && i < n; ++i) {
        hipGraphNodeType t;
        if ((e = hipGraphNodeGetType(nodes[i], &t)) != hipSuccess) rc = hip_fail(e, "node type");
        else if (t != hipGraphNodeTypeKernel)
            rc = fail(VMLM_ERR_UNIMPL, "capture_end: node %zu is not a kernel launch (type %d)",
                      i, (int)t);
    }
    hipGraphExec_t x = nullptr;
    if (rc == VMLM_OK && (e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0)) != hipSuccess)
        rc = hip_fail(e, "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc == VMLM_OK) *graph = (void *)x;
    return rc;
}

int vmlm_hip_graph_launch(void *graph, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(graph, "graph_launch: null graph");
    VMLM_HIP_CHECK(hipGraphLaunch((hipGraphExec_t)graph, as_stream(stream)));
    return VMLM_OK;
}

int vmlm_hip_graph_destroy(void *graph) {
    INIT_OR_RETURN();
    if (graph) VMLM_HIP_CHECK(hipGraphExecDestroy((hipGraphExec_t)graph));
    return VMLM_OK;
}

int vmlm_hip_check_guards(void) {
    INIT_OR_RETURN();
    int v = 0;
    VMLM_HIP_CHECK(hipMemcpy(&v, guard_flag_ptr(), sizeof(int), hipMemcpyDeviceToHost));
    if (v) {
        VMLM_HIP_CHECK(hipMemset(guard_flag_ptr(), 0, sizeof(int)));
        return fail(VMLM_ERR_GUARD, "device guard tripped (code %d): row/source index out of range",
                    v);
    }
    return VMLM_OK;
}

// ================================================================ layer 2
int vmlm_hip_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c,
                          size_t m, size_t n, size_t k, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(scale != nullptr, "int8 gemm: scale slot must be f32 (null)");
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    return q_matmul(a, q, true, scale, c, m, n, k, st, stg);
}
int vmlm_hip_gemm_nt_int8_noalloc(const float *a, const int8_t *q, const float *scale, float *c,
                                  size_t m, size_t n, size_t k, void *stream) {
    // never initialises the library itself (init allocates)
    if (!g_ready.load(std::memory_order_acquire))
        return fail(VMLM_ERR_DEVICE, "gemm_nt_int8_noalloc: call vmlm_hip_init first");
    if (g_scratch_status != VMLM_OK) return fail(g_scratch_status, "%s", g_scratch_err);
    VMLM_GUARD(scale != nullptr, "int8 gemm: scale slot must be f32 (null)");
    int dev = -1;
    VMLM_HIP_CHECK(hipGetDevice(&dev));
    VMLM_GUARD(dev >= 0 && dev < MAX_DEVICES && g_scratch_ptr[dev],
               "gemm_nt_int8_noalloc: no scratch set up on device %d", dev);
    ScratchBump ws{(char *)g_scratch_ptr[dev], NOALLOC_SCRATCH_BYTES};
    return q_matmul(a, q, true, scale, c, m, n, k, as_stream(stream), ws);
}
int vmlm_hip_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                          size_t k, void *stream) {
    INIT_OR_RETURN();
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    return q_matmul(a, b, false, nullptr, c, m, n, k, st, stg);
}
int vmlm_hip_gemm_nt_bf16bf16(const uint16_t *a, const uint16_t *b, float *c, size_t m,
                              size_t n, size_t k, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(k % 64 == 0 && ((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0,
               "bf16 x bf16 gemm: k %% 64 == 0 and 16-byte aligned operands required");
    if (m <= 16) {
        GemvArgs g;
        g.W = b;
        g.w_int8 = false;
        g.A = a;
        g.T = 1;
        g.lda = (int)k;
        g.M = (int)m;
        g.N = (int)n;
        g.K = (int)k;
        g.Y = c;
        g.ldy = (int)n;
        return launch_gemv(g, as_stream(stream));
    }
    GemmArgs g;
    g.W = b;
    g.w_int8 = false;
    g.A = a;
    g.T = 1;
    g.lda = (int)k;
    g.M = (int)m;
    g.N = (int)n;
    g.K = (int)k;
    g.C = c;
    g.ldc = (int)n;
    return launch_gemm(g, as_stream(stream));
}
static int dev_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                        bool acc, bool nt, hipStream_t st) {
    Stage stg(st);
    const size_t wf = gemm_f32_work_floats(m, n, k);
    float *work = wf ? stg.alloc<float>(wf) : nullptr;
    STAGE_OK(stg);
    return launch_gemm_f32(a, b, c, m, n, k, acc, nt, st, work);
}
int vmlm_hip_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                     bool acc, void *stream) {
    INIT_OR_RETURN();
    return dev_gemm_f32(a, b, c, m, n, k, acc, true, as_stream(stream));
}
int vmlm_hip_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                  bool acc, void *stream) {
    INIT_OR_RETURN();
    return dev_gemm_f32(a, b, c, m, n, k, acc, false, as_stream(stream));
}
int vmlm_hip_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                     float eps, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(cols > 0 || rows == 0, "RMSNORM: zero columns");
    return launch_rmsnorm(dst, src, g, rows, cols, eps, nullptr, 0, 0, as_stream(stream));
}
int vmlm_hip_softmax(float *p, size_t rows, size_t cols, bool causal, void *stream) {
    INIT_OR_RETURN();
    return launch_softmax(p, rows, cols, causal, as_stream(stream));
}
int vmlm_hip_act(float *dst, size_t n, uint16_t kind, void *stream) {
    INIT_OR_RETURN();
    return launch_act(dst, n, kind, as_stream(stream));
}
int vmlm_hip_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op,
                   void *stream) {
    INIT_OR_RETURN();
    return launch_ew(dst, x, y, n, op, as_stream(stream));
}
int vmlm_hip_scale(float *dst, const float *src, size_t n, float s, void *stream) {
    INIT_OR_RETURN();
    return launch_scale(dst, src, n, s, as_stream(stream));
}
int vmlm_hip_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
                  uint16_t pos0, void *stream) {
    INIT_OR_RETURN();
    return launch_rope(dst, src, rows, hd, hd, theta, (float)pos0, 1, as_stream(stream));
}
int vmlm_hip_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols,
                      const float *rowf, void *stream) {
    INIT_OR_RETURN();
    return launch_emb_bf16(dst, cols, table, rows, cols, rowf, nullptr, 1, as_stream(stream));
}
int vmlm_hip_topk_idx(const float *src, size_t rows, size_t cols, float *dst, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(rows > 0 && cols > 0, "TOPK_IDX: src or dst slot has width 0");
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    unsigned long long *keys = stg.alloc<unsigned long long>(ARGMAX_KEYS);
    STAGE_OK(stg);
    return launch_argmax(src, cols, dst, nullptr, keys, st);
}

static int check_conn(const vmlm_sparse_conn_w *sc) {
    VMLM_GUARD(sc != nullptr, "B1: null SparseConnW");
    VMLM_GUARD(sc->e == (size_t)sc->n_neurons * sc->k0,
               "CONN_TRAIN: SparseConnW geometry inconsistent: e=%zu but n_neurons*k0=%zu",
               sc->e, (size_t)sc->n_neurons * sc->k0);
    VMLM_GUARD(sc->k0 <= 1024, "B1: k0 exceeds the safe stack bound k0=%zu bound=1024", sc->k0);
    return VMLM_OK;
}

int vmlm_hip_b1_forward(const vmlm_sparse_conn_w *sc, const float *x, float *y,
                        size_t n_tokens, void *stream) {
    INIT_OR_RETURN();
    int rc = check_conn(sc);
    if (rc) return rc;
    // x, y: source-major [n][n_tokens] (n_tokens == 1: a plain vector)
    return launch_b1_forward(sc->w, sc->src_u32, (int)sc->n_neurons, (int)sc->k0, x, n_tokens,
                             (int)n_tokens, y, 1, -1, as_stream(stream));
}
// One T8 layer over the reference layout xt[n][t8]: through a plan (from the
// stream's workspace) when the shape allows it, else one lane per (neuron, token).
static int b1_t8_layer(const float *w, const uint32_t *src, int n, int k0, const float *xt,
                       size_t t8, size_t n_tokens, float *yt, Stage &stg, hipStream_t st) {
    if (n_tokens == 0 || n == 0) return VMLM_OK;
    if (b1_plan_ok(n, k0, n) && round_up(n_tokens, 16) <= t8) {
        B1PlanJobs jobs{};
        jobs.job[0] = B1PlanJob{w, src, stg.alloc<char>(b1_plan_bytes(n, k0)), k0};
        STAGE_OK(stg);
        int rc = launch_b1_plan(jobs, 1, n, n, st);
        if (rc) return rc;
        return launch_b1_t8_plan_layer(jobs.job[0].plan, n, k0, n, xt, 16, t8, (int)n_tokens, yt,
                                       16, t8, -1, st);
    }
    return launch_b1_forward(w, src, n, k0, xt, t8, (int)n_tokens, yt, 0, -1, st);
}

int vmlm_hip_b1_forward_t8(const vmlm_sparse_conn_w *sc, const float *xt, size_t t8,
                           size_t n_tokens, float *yt, void *stream) {
    INIT_OR_RETURN();
    int rc = check_conn(sc);
    if (rc) return rc;
    VMLM_GUARD(t8 >= n_tokens, "B1_T8: row stride t8 < n_tokens");
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    return b1_t8_layer(sc->w, sc->src_u32, (int)sc->n_neurons, (int)sc->k0, xt, t8, n_tokens, yt,
                       stg, st);
}
int vmlm_hip_b1_backward_fused(const vmlm_sparse_conn_w *sc, const float *dy, const float *x,
                               float *dw, float *dx, void *stream) {
    INIT_OR_RETURN();
    int rc = check_conn(sc);
    if (rc) return rc;
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    char *work = dx ? stg.alloc<char>(b1_rev_work_bytes(sc->e, sc->n_neurons)) : nullptr;
    STAGE_OK(stg);
    return launch_b1_backward(sc->w, nullptr, sc->src_u32, sc->n_neurons, sc->k0, dy, x, dw, dx,
                              work, st);
}
int vmlm_hip_b1_backward_t8(const float *w, const uint32_t *src_u32, const float *xt,
                            const float *dyt, size_t t8, size_t n, size_t k0, float *dxt,
                            float *dw, void *stream) {
    INIT_OR_RETURN();
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    char *work = stg.alloc<char>(b1_rev_work_bytes(n * k0, n));
    STAGE_OK(stg);
    return launch_b1_backward_t8(w, src_u32, xt, dyt, t8, n, k0, dxt, dw, work, st);
}
int vmlm_hip_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8,
                          void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(t8 >= t, "transpose_t8: t8 < t");
    return launch_transpose_t8(x, t, d, xt, t8, as_stream(stream));
}
int vmlm_hip_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out,
                               size_t os, size_t in_stride, void *stream) {
    INIT_OR_RETURN();
    return launch_transpose_back(a, rows, cols, out, os, in_stride, as_stream(stream));
}

int vmlm_hip_attention_prefill(const float *q, const float *k, const float *v, float *out,
                               size_t S, size_t n_heads, size_t head_dim, float theta,
                               uint16_t pos0, float scale, bool causal, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(head_dim == 64, "attention: head_dim %zu unsupported (64 only)", head_dim);
    VMLM_GUARD(theta > 0.0f, "ROPE: theta must be > 0");
    if (S == 0 || n_heads == 0) return VMLM_OK;
    hipStream_t st = as_stream(stream);
    Stage stg(st);
    const size_t W = n_heads * head_dim;
    char *work = stg.alloc<char>(attention_prefill_work_bytes((int)S, (int)n_heads, 1));
    STAGE_OK(stg);
    // K rotated as its bf16 terms are prepared, Q as the attention loads it
    return launch_attention_prefill(q, k, v, out, (int)S, (int)n_heads, (int)W, (int)W, scale,
                                    causal, work, st, true,
                                    -2.0f / (float)head_dim * host_ln_f(theta), (float)pos0);
}

int vmlm_hip_attention_decode(const float *q, const float *k_new, const float *v_new,
                              float *kcache, float *vcache, float *out, size_t n_heads,
                              size_t head_dim, size_t cap, size_t pos, float theta,
                              float scale, void *stream) {
    return vmlm_hip_attention_decode_split(q, k_new, v_new, kcache, vcache, out, n_heads,
                                           head_dim, cap, pos, theta, scale, -1, stream);
}

int vmlm_hip_attention_decode_split(const float *q, const float *k_new, const float *v_new,
                                    float *kcache, float *vcache, float *out, size_t n_heads,
                                    size_t head_dim, size_t cap, size_t pos, float theta,
                                    float scale, int split, void *stream) {
    INIT_OR_RETURN();
    VMLM_GUARD(split >= -1 && split <= 4096, "attention decode: split %d out of range", split);
    VMLM_GUARD(head_dim == 64, "attention: head_dim %zu unsupported (64 only)", head_dim);
    VMLM_GUARD(pos < cap, "WRITECOL: column %zu beyond cache capacity %zu", pos, cap);
    VMLM_GUARD(theta > 0.0f, "ROPE: theta must be > 0");
    hipStream_t st = as_stream(stream);
    DecodeArgs a;
    a.q = q;
    a.k_new = k_new;
    a.v_new = v_new;
    a.ldq = (int)(n_heads * head_dim);
    a.kc = kcache;
    a.vc = vcache;
    a.cap = (int)cap;
    a.H = (int)n_heads;
    a.posp = nullptr;
    a.pos = (int)pos;
    a.step = -2.0f / (float)head_dim * host_ln_f(theta);
    a.scale = scale;
    a.split = split;
    Stage stg(st);
    const size_t wf = attention_decode_work_floats(a, 1);
    float *work = wf ? stg.alloc<float>(wf) : nullptr;
    STAGE_OK(stg);
    return launch_attention_decode(a, 1, out, (int)(n_heads * head_dim), nullptr, 0, 0, st, work);
}

// ================================================================ layer 1
int vmlm_gemm_nt_int8(const float *a, const int8_t *q, const float *scale, float *c, size_t m,
                      size_t n, size_t k) {
    HOST_CALL_BEGIN();
    VMLM_GUARD(scale != nullptr, "int8 gemm: scale slot must be f32 (null)");
    if (m == 0 || n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *da = stg.upload(a, m * k);
        int8_t *dq = stg.upload(q, n * k);
        float *ds = stg.upload(scale, n);
        float *dc = stg.alloc<float>(m * n);
        STAGE_OK(stg);
        int rc = q_matmul(da, dq, true, ds, dc, m, n, k, st, stg);
        if (rc) return rc;
        rc = download(c, dc, m * n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_gemm_nt_bf16(const float *a, const uint16_t *b, float *c, size_t m, size_t n,
                      size_t k) {
    HOST_CALL_BEGIN();
    if (m == 0 || n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *da = stg.upload(a, m * k);
        uint16_t *db = stg.upload(b, n * k);
        float *dc = stg.alloc<float>(m * n);
        STAGE_OK(stg);
        int rc = q_matmul(da, db, false, nullptr, dc, m, n, k, st, stg);
        if (rc) return rc;
        rc = download(c, dc, m * n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

static int host_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                         bool acc, bool nt) {
    HOST_CALL_BEGIN();
    if (m == 0 || n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *da = stg.upload(a, m * k);
        float *db = stg.upload(b, n * k);
        float *dc = acc ? stg.upload((const float *)c, m * n) : stg.alloc<float>(m * n);
        const size_t wf = gemm_f32_work_floats(m, n, k);
        float *work = wf ? stg.alloc<float>(wf) : nullptr;
        STAGE_OK(stg);
        int rc = launch_gemm_f32(da, db, dc, m, n, k, acc, nt, st, work);
        if (rc) return rc;
        rc = download(c, dc, m * n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_gemm_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                 bool acc) {
    return host_gemm_f32(a, b, c, m, n, k, acc, true);
}
int vmlm_gemm(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
              bool acc) {
    return host_gemm_f32(a, b, c, m, n, k, acc, false);
}

int vmlm_jit_gemm_nt(const float *a, const float *b, float *c, uint64_t dims) {
    size_t m = dims & 0xFFFF, n = (dims >> 16) & 0xFFFF, k = (dims >> 32) & 0xFFFF;
    bool acc = ((dims >> 48) & 1) != 0;
    return vmlm_gemm_nt(a, b, c, m, n, k, acc);
}

int vmlm_rmsnorm(float *dst, const float *src, const float *g, size_t rows, size_t cols,
                 float eps) {
    HOST_CALL_BEGIN();
    if (rows == 0) return VMLM_OK;
    VMLM_GUARD(cols > 0, "RMSNORM: zero columns");
    {
        Stage stg(st);
        float *ds = stg.upload(src, rows * cols);
        float *dg = stg.upload(g, cols);
        float *dd = stg.alloc<float>(rows * cols);
        STAGE_OK(stg);
        int rc = launch_rmsnorm(dd, ds, dg, rows, cols, eps, nullptr, 0, 0, st);
        if (!rc) rc = download(dst, dd, rows * cols * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_softmax(float *p, size_t rows, size_t cols, bool causal) {
    HOST_CALL_BEGIN();
    if (rows == 0 || cols == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dp = stg.upload((const float *)p, rows * cols);
        STAGE_OK(stg);
        int rc = launch_softmax(dp, rows, cols, causal, st);
        if (!rc) rc = download(p, dp, rows * cols * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_act(float *dst, size_t n, uint16_t kind) {
    HOST_CALL_BEGIN();
    if (n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dd = stg.upload((const float *)dst, n);
        STAGE_OK(stg);
        int rc = launch_act(dd, n, kind, st);
        if (!rc) rc = download(dst, dd, n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_ew_op(float *dst, const float *x, const float *y, size_t n, uint8_t op) {
    HOST_CALL_BEGIN();
    if (n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dx = stg.upload(x, n), *dy = stg.upload(y, n), *dd = stg.alloc<float>(n);
        STAGE_OK(stg);
        int rc = launch_ew(dd, dx, dy, n, op, st);
        if (!rc) rc = download(dst, dd, n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_scale(float *dst, const float *src, size_t n, float s) {
    HOST_CALL_BEGIN();
    if (n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *ds = stg.upload(src, n), *dd = stg.alloc<float>(n);
        STAGE_OK(stg);
        int rc = launch_scale(dd, ds, n, s, st);
        if (!rc) rc = download(dst, dd, n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_rope(float *dst, const float *src, size_t rows, size_t hd, float theta,
              uint16_t pos0) {
    HOST_CALL_BEGIN();
    VMLM_GUARD(hd >= 2 && (hd & 1) == 0, "ROPE: hd must be even >= 2");
    VMLM_GUARD(theta > 0.0f, "ROPE: theta must be > 0");
    if (rows == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *ds = stg.upload(src, rows * hd), *dd = stg.alloc<float>(rows * hd);
        STAGE_OK(stg);
        int rc = launch_rope(dd, ds, rows, hd, hd, theta, (float)pos0, 1, st);
        if (!rc) rc = download(dst, dd, rows * hd * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

static int emb_guard(float rowf, size_t rows, size_t *row) {
    if (!(rowf >= 0.0f) || rowf >= (float)rows)
        return fail(VMLM_ERR_GUARD, "EMB: row index out of range row=%g table_rows=%zu",
                    (double)rowf, rows);
    size_t r = (size_t)rowf;
    if ((float)r != rowf)
        return fail(VMLM_ERR_GUARD, "EMB: row index is not an integer row=%g", (double)rowf);
    *row = r;
    return VMLM_OK;
}

int vmlm_emb_bf16(float *dst, const uint16_t *table, size_t rows, size_t cols, float rowf) {
    size_t row = 0;
    int rc = emb_guard(rowf, rows, &row);
    if (rc) return rc;
    HOST_CALL_BEGIN();
    {
        Stage stg(st);
        uint16_t *dt = stg.upload(table + row * cols, cols);
        float *dd = stg.alloc<float>(cols);
        int32_t zero = 0;
        int32_t *di = stg.upload(&zero, 1);
        STAGE_OK(stg);
        rc = launch_emb_bf16(dd, cols, dt, 1, cols, nullptr, di, 1, st);
        if (!rc) rc = download(dst, dd, cols * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_emb_f32(float *dst, const float *table, size_t rows, size_t cols, float rowf) {
    size_t row = 0;
    int rc = emb_guard(rowf, rows, &row);
    if (rc) return rc;
    std::memcpy(dst, table + row * cols, cols * sizeof(float));
    return VMLM_OK;
}

int vmlm_topk_idx(const float *src, size_t rows, size_t cols, float *dst) {
    VMLM_GUARD(rows > 0 && cols > 0, "TOPK_IDX: src or dst slot has width 0");
    HOST_CALL_BEGIN();
    {
        Stage stg(st);
        float *ds = stg.upload(src, cols), *dd = stg.alloc<float>(1);
        unsigned long long *keys = stg.alloc<unsigned long long>(ARGMAX_KEYS);
        STAGE_OK(stg);
        int rc = launch_argmax(ds, cols, dd, nullptr, keys, st);
        if (!rc) rc = download(dst, dd, sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

static int host_b1(const vmlm_sparse_conn_w *sc, const float *xt, size_t t8, size_t n_tokens,
                   float *yt, size_t *macs, int mode) {
    int rc = check_conn(sc);
    if (rc) return rc;
    const size_t n = sc->n_neurons, e = sc->e;
    for (size_t t = 0; t < e; ++t)
        VMLM_GUARD(sc->src_u32[t] < n, "B1: src_u32[%zu]=%u >= n_neurons=%zu", t, sc->src_u32[t],
                   n);
    HOST_CALL_BEGIN();
    {
        Stage stg(st);
        float *dw = stg.upload(sc->w, e);
        uint32_t *ds = stg.upload(sc->src_u32, e);
        float *dx = stg.upload(xt, n * t8);
        float *dy = stg.upload((const float *)yt, n * t8);
        STAGE_OK(stg);
        rc = mode == 0 ? b1_t8_layer(dw, ds, (int)n, (int)sc->k0, dx, t8, n_tokens, dy, stg, st)
                       : launch_b1_forward(dw, ds, (int)n, (int)sc->k0, dx, t8, (int)n_tokens, dy,
                                           mode, -1, st);
        if (!rc) rc = download(yt, dy, n * t8 * sizeof(float), st);
        if (rc) return rc;
    }
    if (macs) *macs = n * sc->k0;
    FINISH(st);
}

int vmlm_b1_forward(const vmlm_sparse_conn_w *sc, const float *x, float *y, size_t *macs) {
    return host_b1(sc, x, 1, 1, y, macs, 1);
}
int vmlm_b1_forward_t8(const vmlm_sparse_conn_w *sc, const float *xt, size_t t8,
                       size_t n_tokens, float *yt, size_t *macs) {
    VMLM_GUARD(t8 >= n_tokens, "B1_T8: row stride t8 < n_tokens");
    return host_b1(sc, xt, t8, n_tokens, yt, macs, 0);
}

// B1 backward on host buffers: `dw` and `dx` accumulate (+=) like the
// reference's; sources are checked against n_neurons (the square layer's
// source dimension) before anything runs.
static int host_b1_bwd(const vmlm_sparse_conn_w *sc, const float *dy, const float *x, float *dw,
                       float *dx, bool f32_ids) {
    int rc = check_conn(sc);
    if (rc) return rc;
    const size_t n = sc->n_neurons, e = sc->e;
    if (f32_ids) {
        VMLM_GUARD(sc->src != nullptr, "B1 backward: SparseConnW.src (f32 ids) is null");
        for (size_t t = 0; t < e; ++t) {
            const float f = sc->src[t];
            const size_t u = f > 0.0f ? (size_t)f : 0;
            VMLM_GUARD(u < n, "B1: src[%zu]=%g >= n_neurons=%zu", t, (double)f, n);
        }
    } else {
        for (size_t t = 0; t < e; ++t)
            VMLM_GUARD(sc->src_u32[t] < n, "B1: src_u32[%zu]=%u >= n_neurons=%zu", t,
                       sc->src_u32[t], n);
    }
    HOST_CALL_BEGIN();
    {
        Stage stg(st);
        float *dwt = stg.upload(sc->w, e);
        const float *dsf = f32_ids ? stg.upload((const float *)sc->src, e) : nullptr;
        const uint32_t *ds = f32_ids ? nullptr : stg.upload(sc->src_u32, e);
        float *ddy = stg.upload(dy, n);
        float *dxs = x ? stg.upload(x, n) : nullptr;
        float *ddw = dw ? stg.upload((const float *)dw, e) : nullptr;
        float *ddx = dx ? stg.upload((const float *)dx, n) : nullptr;
        char *work = dx ? stg.alloc<char>(b1_rev_work_bytes(e, n)) : nullptr;
        STAGE_OK(stg);
        rc = launch_b1_backward(dwt, dsf, ds, n, sc->k0, ddy, dxs, ddw, ddx, work, st);
        if (!rc && dw) rc = download(dw, ddw, e * sizeof(float), st);
        if (!rc && dx) rc = download(dx, ddx, n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_b1_backward(const vmlm_sparse_conn_w *sc, const float *dy, const float *x, float *dw,
                     size_t *macs) {
    int rc = host_b1_bwd(sc, dy, x, dw, nullptr, true);
    if (!rc && macs) *macs = sc->e;
    return rc;
}
int vmlm_b1_backward_dx(const vmlm_sparse_conn_w *sc, const float *dy, float *dx, size_t *accs) {
    int rc = host_b1_bwd(sc, dy, nullptr, nullptr, dx, false);
    if (!rc && accs) *accs = sc->e;
    return rc;
}
int vmlm_b1_backward_fused(const vmlm_sparse_conn_w *sc, const float *dy, const float *x,
                           float *dw, float *dx, size_t *conns) {
    int rc = host_b1_bwd(sc, dy, x, dw, dx, false);
    if (!rc && conns) *conns = sc->e;
    return rc;
}

int vmlm_b1_backward_t8(const float *w, const uint32_t *src_u32, const float *xt,
                        const float *dyt, size_t t8, size_t n, size_t k0, float *dxt,
                        float *dw) {
    VMLM_GUARD(t8 % 8 == 0, "B1_T8 backward: t8 = %zu is not a multiple of 8", t8);
    for (size_t t = 0; t < n * k0; ++t)
        VMLM_GUARD(src_u32[t] < n, "B1: src_u32[%zu]=%u >= n=%zu", t, src_u32[t], n);
    HOST_CALL_BEGIN();
    if (n == 0 || k0 == 0 || t8 == 0) return VMLM_OK;
    {
        Stage stg(st);
        const size_t e = n * k0;
        float *dwt = stg.upload(w, e);
        uint32_t *ds = stg.upload(src_u32, e);
        float *dxt_in = stg.upload(xt, n * t8);
        float *ddy = stg.upload(dyt, n * t8);
        float *ddx = stg.upload((const float *)dxt, n * t8);
        float *ddw = stg.upload((const float *)dw, e);
        char *work = stg.alloc<char>(b1_rev_work_bytes(e, n));
        STAGE_OK(stg);
        int rc = launch_b1_backward_t8(dwt, ds, dxt_in, ddy, t8, n, k0, ddx, ddw, work, st);
        if (!rc) rc = download(dxt, ddx, n * t8 * sizeof(float), st);
        if (!rc) rc = download(dw, ddw, e * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_transpose_t8(const float *x, size_t t, size_t d, float *xt, size_t t8) {
    VMLM_GUARD(t8 >= t, "transpose_t8: t8 < t");
    HOST_CALL_BEGIN();
    {
        Stage stg(st);
        float *dx = stg.upload(x, t * d), *dxt = stg.alloc<float>(d * t8);
        STAGE_OK(stg);
        int rc = launch_transpose_t8(dx, t, d, dxt, t8, st);
        if (!rc) rc = download(xt, dxt, d * t8 * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_transpose_t8_back(const float *a, size_t rows, size_t cols, float *out, size_t os,
                           size_t in_stride) {
    VMLM_GUARD(os >= rows && in_stride >= cols, "transpose_t8_back: stride too small");
    HOST_CALL_BEGIN();
    if (rows == 0 || cols == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *da = stg.upload(a, rows * in_stride);
        float *dout = stg.upload((const float *)out, cols * os);
        STAGE_OK(stg);
        int rc = launch_transpose_back(da, rows, cols, dout, os, in_stride, st);
        if (!rc) rc = download(out, dout, cols * os * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_attention_prefill(const float *q, const float *k, const float *v, float *out,
                           size_t S, size_t n_heads, size_t head_dim, float theta,
                           uint16_t pos0, float scale, bool causal) {
    HOST_CALL_BEGIN();
    const size_t n = S * n_heads * head_dim;
    if (n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dq = stg.upload(q, n), *dk = stg.upload(k, n), *dv = stg.upload(v, n);
        float *dout = stg.alloc<float>(n);
        STAGE_OK(stg);
        int rc = vmlm_hip_attention_prefill(dq, dk, dv, dout, S, n_heads, head_dim, theta,
                                            pos0, scale, causal, st);
        if (!rc) rc = download(out, dout, n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_attention_decode(const float *q, const float *k_new, const float *v_new,
                          float *kcache, float *vcache, float *out, size_t n_heads,
                          size_t head_dim, size_t cap, size_t pos, float theta, float scale) {
    return vmlm_attention_decode_split(q, k_new, v_new, kcache, vcache, out, n_heads, head_dim,
                                       cap, pos, theta, scale, -1);
}

int vmlm_attention_decode_split(const float *q, const float *k_new, const float *v_new,
                                float *kcache, float *vcache, float *out, size_t n_heads,
                                size_t head_dim, size_t cap, size_t pos, float theta, float scale,
                                int split) {
    HOST_CALL_BEGIN();
    const size_t w = n_heads * head_dim, cn = n_heads * cap * head_dim;
    {
        Stage stg(st);
        float *dq = stg.upload(q, w), *dk = stg.upload(k_new, w), *dv = stg.upload(v_new, w);
        float *dkc = stg.upload((const float *)kcache, cn);
        float *dvc = stg.upload((const float *)vcache, cn);
        float *dout = stg.alloc<float>(w);
        STAGE_OK(stg);
        int rc = vmlm_hip_attention_decode_split(dq, dk, dv, dkc, dvc, dout, n_heads, head_dim,
                                                 cap, pos, theta, scale, split, st);
        if (!rc) rc = download(out, dout, w * sizeof(float), st);
        if (!rc) rc = download(kcache, dkc, cn * sizeof(float), st);
        if (!rc) rc = download(vcache, dvc, cn * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

// ================================================================ jit helpers
int vmlm_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                   float eps) {
    HOST_CALL_BEGIN();
    if (rows == 0 || cols == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dx = stg.upload((const float *)x, rows * cols);
        float *dg = stg.upload(g, cols);
        float *db = stg.upload(b, cols);
        STAGE_OK(stg);
        int rc = launch_layernorm(dx, dg, db, rows, cols, eps, st);
        if (!rc) rc = download(x, dx, rows * cols * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc) {
    HOST_CALL_BEGIN();
    if (m == 0 || n == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *ds = stg.upload((const float *)s, m * n);
        float *dv = stg.upload(v, m);
        float *dk = stg.upload(k, n);
        STAGE_OK(stg);
        int rc = launch_outer(ds, dv, dk, m, n, sc, st);
        if (!rc) rc = download(s, ds, m * n * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_bias(float *d, const float *b, size_t rows, size_t cols) {
    HOST_CALL_BEGIN();
    if (rows == 0 || cols == 0) return VMLM_OK;
    {
        Stage stg(st);
        float *dd = stg.upload((const float *)d, rows * cols);
        float *db = stg.upload(b, cols);
        STAGE_OK(stg);
        int rc = launch_bias(dd, db, rows, cols, st);
        if (!rc) rc = download(d, dd, rows * cols * sizeof(float), st);
        if (rc) return rc;
    }
    FINISH(st);
}

int vmlm_jit_act(float *p, size_t n, uint64_t kind) { return vmlm_act(p, n, (uint16_t)kind); }
int vmlm_jit_ewadd(float *d, const float *x, const float *y, size_t n) {
    return vmlm_ew_op(d, x, y, n, VMLM_OP_EWADD);
}
int vmlm_jit_ewmul(float *d, const float *x, const float *y, size_t n) {
    return vmlm_ew_op(d, x, y, n, VMLM_OP_EWMUL);
}
int vmlm_jit_ewsub(float *d, const float *x, const float *y, size_t n) {
    return vmlm_ew_op(d, x, y, n, VMLM_OP_EWSUB);
}
int vmlm_jit_ewdiv(float *d, const float *x, const float *y, size_t n) {
    return vmlm_ew_op(d, x, y, n, VMLM_OP_EWDIV);
}
int vmlm_jit_bias(float *d, const float *b, size_t rows, size_t cols) {
    return vmlm_bias(d, b, rows, cols);
}
int vmlm_jit_ln(float *x, const float *g, const float *b, uint64_t dims, uint64_t pad) {
    (void)pad;
    return vmlm_layernorm(x, g, b, (size_t)(dims & 0xFFFFFFFFu), (size_t)(dims >> 32), 1e-5f);
}
int vmlm_jit_softmax(float *p, uint64_t dims, uint64_t causal) {
    return vmlm_softmax(p, (size_t)(dims & 0xFFFFFFFFu), (size_t)(dims >> 32), causal != 0);
}
int vmlm_jit_outer(float *s, const float *v, const float *k, uint64_t dims) {
    return vmlm_outer(s, v, k, (size_t)(dims & 0xFFFFFFFFu), (size_t)(dims >> 32), 1.0f);
}

int vmlm_hip_layernorm(float *x, const float *g, const float *b, size_t rows, size_t cols,
                       float eps, void *stream) {
    INIT_OR_RETURN();
    return launch_layernorm(x, g, b, rows, cols, eps, as_stream(stream));
}
int vmlm_hip_outer(float *s, const float *v, const float *k, size_t m, size_t n, float sc,
                   void *stream) {
    INIT_OR_RETURN();
    return launch_outer(s, v, k, m, n, sc, as_stream(stream));
}
int vmlm_hip_bias(float *d, const float *b, size_t rows, size_t cols, void *stream) {
    INIT_OR_RETURN();
    return launch_bias(d, b, rows, cols, as_stream(stream));
}

// ================================================================ Backend table
// Operands of the Backend functions: device (or managed) memory is used in
// place; anything else is host memory, staged through the call's workspace.
static bool device_ptr(const void *p) {
    hipPointerAttribute_t at{};
    if (!p || hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged;
}
static const float *bk_operand(Stage &stg, const float *p, size_t n) {
    return device_ptr(p) ? p : stg.upload(p, n);
}

// Runs a Backend reduction (0 dot, 1 sum, 2 max) and returns its value, or
// NaN with the message in vmlm_hip_last_error().
static float bk_scalar(int op, const float *a, const float *b, size_t n) {
    const float nan = __builtin_nanf("");
    if (ensure_init()) return nan;
    std::lock_guard<std::mutex> lk(g_host_mutex);
    hipStream_t st = lib_stream();
    float r = nan;
    {
        Stage stg(st);
        const float *da = bk_operand(stg, a, n);
        const float *db = op == 0 ? bk_operand(stg, b, n) : nullptr;
        float *out = stg.alloc<float>(1);
        float *part = op < 2 ? stg.alloc<float>(bk_reduce_work_floats()) : nullptr;
        char *work = op == 2 ? stg.alloc<char>(bk_max_work_bytes()) : nullptr;
        if (stg.status) return nan;
        int rc = op == 2 ? launch_bk_max(da, n, work, out, st)
                         : launch_bk_reduce(da, db, n, op == 0, part, out, st);
        if (rc) return nan;
        hipError_t e = hipMemcpyAsync(&r, out, sizeof(float), hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            hip_fail(e, "Backend reduction");
            return nan;
        }
    }
    return r;
}

// Runs a Backend elementwise op (0 axpy, 1 add, 2 scale_mul) into `y`.
static void bk_elementwise(int op, float *y, const float *x, float a, size_t n) {
    if (ensure_init() || n == 0) return;
    std::lock_guard<std::mutex> lk(g_host_mutex);
    hipStream_t st = lib_stream();
    Stage stg(st);
    const bool ydev = device_ptr(y);
    float *dy = ydev ? y : (op == 2 ? stg.alloc<float>(n) : stg.upload((const float *)y, n));
    const float *dx = bk_operand(stg, x, n);
    if (stg.status) return;
    int rc = op == 0 ? launch_bk_axpy(dy, dx, a, n, st)
             : op == 1 ? launch_bk_add(dy, dx, n, st)
                       : launch_bk_scale_mul(dy, dx, a, n, st);
    if (rc) return;
    hipError_t e = hipSuccess;
    if (!ydev) e = hipMemcpyAsync(y, dy, n * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) hip_fail(e, "Backend elementwise op");
}

float vmlm_backend_dot256(const float *a, const float *b, size_t n) {
    return bk_scalar(0, a, b, n);
}
void vmlm_backend_axpy256(float *y, const float *x, float a, size_t n) {
    bk_elementwise(0, y, x, a, n);
}
void vmlm_backend_add256(float *y, const float *x, size_t n) { bk_elementwise(1, y, x, 0.0f, n); }
float vmlm_backend_max256(const float *x, size_t n) { return bk_scalar(2, x, nullptr, n); }
float vmlm_backend_sum256(const float *x, size_t n) { return bk_scalar(1, x, nullptr, n); }
void vmlm_backend_scale_mul(float *dst, const float *src, float a, size_t n) {
    bk_elementwise(2, dst, src, a, n);
}

static const vmlm_backend_t g_backend = {
    "hip_gfx950",          vmlm_backend_dot256, vmlm_backend_axpy256, vmlm_backend_add256,
    vmlm_backend_max256,   vmlm_backend_sum256, vmlm_backend_scale_mul,
};
const vmlm_backend_t *vmlm_hip_backend(void) { return &g_backend; }

static const vmlm_hip_kernel_table_t g_kernels = {
    "hip_gfx950",      vmlm_gemm_nt_int8, vmlm_gemm_nt_bf16, vmlm_gemm_nt,
    vmlm_gemm,         vmlm_rmsnorm,      vmlm_softmax,      vmlm_act,
    vmlm_ew_op,        vmlm_b1_forward,   vmlm_b1_forward_t8,
};
const vmlm_hip_kernel_table_t *vmlm_hip_kernel_table(void) { return &g_kernels; }

}  // extern "C"

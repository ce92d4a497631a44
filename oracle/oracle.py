"""ctypes wrapper of the CPU oracle (oracle/_build/libvmlm_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. Nothing in sparrow_amd imports
it. Each wrapper documents the reference function it restates (the C source
cites file:line).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libvmlm_oracle.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if LIB_PATH.exists() and not force:
        return LIB_PATH
    flags = "-mavx2 -mfma"
    try:
        cpu = Path("/proc/cpuinfo").read_text()
        if " avx2" not in cpu or " fma" not in cpu:
            flags = ""
    except OSError:
        pass
    cmd = ["make", "-s"] + (["-B"] if force else []) + [f"ARCHFLAGS={flags}"]
    subprocess.run(cmd, cwd=HERE, check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    L = C.CDLL(str(LIB_PATH))
    sig = {
        "vo_set_threads": (None, [C.c_int]),
        "vo_get_threads": (C.c_int, []),
        "vo_round_f32": (C.c_float, [C.c_float]),
        "vo_exp_f": (C.c_float, [C.c_float]),
        "vo_ln_f": (C.c_float, [C.c_float]),
        "vo_sin_f": (C.c_float, [C.c_float]),
        "vo_cos_f": (C.c_float, [C.c_float]),
        "vo_floor_f": (C.c_float, [C.c_float]),
        "vo_tanh_f": (C.c_float, [C.c_float]),
        "vo_act_scalar": (C.c_float, [C.c_float, C.c_uint16]),
        "vo_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "vo_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "vo_map": (None, [C.c_int, _f32p, _f32p, _sz]),
        "vo_gemm_nt_int8": (None, [_f32p, _i8p, _f32p, _f32p, _sz, _sz, _sz]),
        "vo_gemm_nt_bf16": (None, [_f32p, _u16p, _f32p, _sz, _sz, _sz]),
        "vo_gemm_nt": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]),
        "vo_gemm": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]),
        "vo_rmsnorm": (None, [_f32p, _f32p, _f32p, _sz, _sz, C.c_float]),
        "vo_softmax": (None, [_f32p, _sz, _sz, C.c_int]),
        "vo_act": (None, [_f32p, _sz, C.c_uint16]),
        "vo_ew_op": (None, [_f32p, _f32p, _f32p, _sz, C.c_uint8]),
        "vo_scale": (None, [_f32p, _f32p, _sz, C.c_float]),
        "vo_rope": (C.c_int, [_f32p, _f32p, _sz, _sz, C.c_float, C.c_uint32]),
        "vo_emb_bf16": (C.c_int, [_f32p, _u16p, _sz, _sz, C.c_float]),
        "vo_emb_f32": (C.c_int, [_f32p, _f32p, _sz, _sz, C.c_float]),
        "vo_topk_idx": (C.c_int, [_f32p, _sz, _sz, _f32p]),
        "vo_neuron_seed": (C.c_uint32, [C.c_uint32, C.c_uint32]),
        "vo_neuron_rand": (C.c_uint32, [C.c_uint32, C.c_uint32]),
        "vo_neuron_conn_src": (C.c_uint32, [C.c_uint32] * 5),
        "vo_b1_dot_row_u32": (C.c_float, [_f32p, _u32p, _f32p, _sz]),
        "vo_b1_forward": (_sz, [_sz, _sz, _f32p, _u32p, _f32p, _f32p]),
        "vo_b1_forward_t8_scalar": (_sz, [_f32p, _u32p, _sz, _sz, _f32p, _sz, _sz, _f32p]),
        "vo_transpose_t8": (None, [_f32p, _sz, _sz, _f32p, _sz]),
        "vo_transpose_t8_back": (None, [_f32p, _sz, _sz, _f32p, _sz, _sz]),
        "vo_dot256": (C.c_float, [_f32p, _f32p, _sz]),
        "vo_axpy256": (None, [_f32p, _f32p, C.c_float, _sz]),
        "vo_add256": (None, [_f32p, _f32p, _sz]),
        "vo_max256": (C.c_float, [_f32p, _sz]),
        "vo_sum256": (C.c_float, [_f32p, _sz]),
        "vo_scale_mul": (None, [_f32p, _f32p, C.c_float, _sz]),
        "vo_layernorm": (None, [_f32p, _f32p, _f32p, _sz, _sz, C.c_float]),
        "vo_bias": (None, [_f32p, _f32p, _sz, _sz]),
        "vo_outer": (None, [_f32p, _f32p, _f32p, _sz, _sz, C.c_float]),
        "vo_b1_backward": (_sz, [_sz, _sz, _f32p, _f32p, _f32p, _f32p]),
        "vo_b1_backward_dx": (_sz, [_sz, _sz, _f32p, _u32p, _f32p, _f32p]),
        "vo_b1_backward_fused": (_sz, [_sz, _sz, _f32p, _u32p, _f32p, _f32p, _f32p, _f32p]),
        "vo_b1_backward_t8": (None, [_f32p, _u32p, _f32p, _f32p, _sz, _sz, _sz, _f32p, _f32p]),
        "vo_attention_prefill": (None, [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz,
                                        C.c_float, C.c_uint32, C.c_float, C.c_int]),
        "vo_attention_decode": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz,
                                       _sz, _sz, C.c_float, C.c_float]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    # decoder entry points take struct pointers
    L.vo_decoder_prefill.restype = C.c_int
    L.vo_decoder_prefill.argtypes = [C.c_void_p, _f32p, _f32p, _sz, _i32p, _sz,
                                     C.c_void_p, C.c_void_p]
    L.vo_decoder_step.restype = C.c_int
    L.vo_decoder_step.argtypes = [C.c_void_p, _f32p, _f32p, _sz, C.c_int32, _sz,
                                  C.c_void_p, C.c_void_p]
    L.vo_decoder_generate.restype = C.c_int
    L.vo_decoder_generate.argtypes = [C.c_void_p, _f32p, _f32p, _sz, _i32p, _sz, _sz,
                                      _i32p, C.c_void_p]
    # the VM
    L.vo_vm_load.restype = C.c_int
    L.vo_vm_load.argtypes = [C.c_char_p, _sz, C.POINTER(C.c_void_p)]
    L.vo_vm_run.restype = C.c_int
    L.vo_vm_run.argtypes = [C.c_void_p]
    L.vo_vm_free.restype = None
    L.vo_vm_free.argtypes = [C.c_void_p]
    L.vo_vm_find.restype = C.c_int
    L.vo_vm_find.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]
    L.vo_vm_slot.restype = C.c_int
    L.vo_vm_slot.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_void_p),
                             C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                             C.POINTER(C.c_uint8)]
    L.vo_vm_output.restype = _sz
    L.vo_vm_output.argtypes = [C.c_void_p, C.c_void_p, _sz]
    L.vo_vm_message.restype = C.c_char_p
    L.vo_vm_message.argtypes = [C.c_void_p]
    L.vo_vm_last_load_error.restype = C.c_char_p
    L.vo_vm_last_load_error.argtypes = []
    threads = int(os.environ.get("VMLM_ORACLE_THREADS", "0") or 0)
    if threads <= 0:
        threads = min(16, os.cpu_count() or 1)
    L.vo_set_threads(threads)
    _lib = L
    return L


def set_threads(n: int) -> None:
    lib().vo_set_threads(int(n))


def get_threads() -> int:
    return int(lib().vo_get_threads())


def _c(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


# ---------------------------------------------------------------- scalars
def exp_f(x: float) -> float:
    return lib().vo_exp_f(float(x))


def ln_f(x: float) -> float:
    return lib().vo_ln_f(float(x))


def sin_f(x: float) -> float:
    return lib().vo_sin_f(float(x))


def cos_f(x: float) -> float:
    return lib().vo_cos_f(float(x))


def floor_f(x: float) -> float:
    return lib().vo_floor_f(float(x))


def tanh_f(x: float) -> float:
    return lib().vo_tanh_f(float(x))


def round_f32(x: float) -> float:
    return lib().vo_round_f32(float(x))


MAP = {"exp": 0, "ln": 1, "sin": 2, "cos": 3, "tanh": 4, "floor": 5, "round": 6}


def vmap(name, x):
    """Elementwise scalar function over an array (name in MAP, or an int
    100+act_kind for act_scalar)."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    which = MAP[name] if isinstance(name, str) else int(name)
    lib().vo_map(which, x.reshape(-1), y.reshape(-1), x.size)
    return y


def act_scalar(x: float, kind: int) -> float:
    return lib().vo_act_scalar(float(x), int(kind))


def f32_to_bf16(a) -> np.ndarray:
    """tensor/src/dtype.rs:40-46 round-to-nearest-even, vectorised in numpy
    with the same integer formula."""
    u = _c(a, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- GEMMs
def gemm_nt_int8(a, q, scale):
    a, q, scale = _c(a, np.float32), _c(q, np.int8), _c(scale, np.float32)
    m, k = a.shape
    n = q.shape[0]
    c = np.empty((m, n), np.float32)
    lib().vo_gemm_nt_int8(a, q, scale, c, m, n, k)
    return c


def gemm_nt_bf16(a, b):
    a, b = _c(a, np.float32), _c(b, np.uint16)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.float32)
    lib().vo_gemm_nt_bf16(a, b, c, m, n, k)
    return c


def gemm_nt(a, b, c=None, acc=False):
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    lib().vo_gemm_nt(a, b, c, m, n, k, int(acc))
    return c


def gemm(a, b, c=None, acc=False):
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    lib().vo_gemm(a, b, c, m, n, k, int(acc))
    return c


# ---------------------------------------------------------------- row ops
def rmsnorm(x, g, eps):
    x, g = _c(x, np.float32), _c(g, np.float32)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().vo_rmsnorm(y, x, g, rows, cols, float(eps))
    return y


def softmax(p, causal=False):
    p = _c(p, np.float32).copy()
    rows, cols = p.shape
    lib().vo_softmax(p, rows, cols, int(causal))
    return p


# ---------------------------------------------------------------- B1 backward
def b1_backward(w, src, dy, x, dw=None):
    """ops/src/b1_pure.rs:642 (reads the f32 ids): dw += dy[i] * x[src]."""
    n, k0 = w.shape
    srcf = _c(src, np.float32)
    dw = np.zeros((n, k0), np.float32) if dw is None else _c(dw, np.float32).copy()
    lib().vo_b1_backward(n, k0, srcf, _c(dy, np.float32), _c(x, np.float32), dw)
    return dw


def b1_backward_dx(w, src, dy, dx):
    n, k0 = w.shape
    dx = _c(dx, np.float32).copy()
    lib().vo_b1_backward_dx(n, k0, _c(w, np.float32), _c(src, np.uint32), _c(dy, np.float32), dx)
    return dx


def b1_backward_fused(w, src, dy, x, dw, dx):
    n, k0 = w.shape
    dw, dx = _c(dw, np.float32).copy(), _c(dx, np.float32).copy()
    lib().vo_b1_backward_fused(n, k0, _c(w, np.float32), _c(src, np.uint32), _c(dy, np.float32),
                               _c(x, np.float32), dw, dx)
    return dw, dx


def b1_backward_t8(w, src, xt, dyt, dxt, dw):
    """ops/src/kernels.rs:3229: xt [d][t8], dyt [n][t8], dxt [d][t8], dw [n][k0]."""
    n, k0 = w.shape
    t8 = xt.shape[1]
    dxt, dw = _c(dxt, np.float32).copy(), _c(dw, np.float32).copy()
    lib().vo_b1_backward_t8(_c(w, np.float32), _c(src, np.uint32), _c(xt, np.float32),
                            _c(dyt, np.float32), t8, n, k0, dxt, dw)
    return dxt, dw


# ------------------------------------------------ Backend table, jit helpers
def dot256(a, b):
    a, b = _c(a, np.float32).ravel(), _c(b, np.float32).ravel()
    return np.float32(lib().vo_dot256(a, b, a.size))


def axpy256(y, x, a):
    y, x = _c(y, np.float32).ravel().copy(), _c(x, np.float32).ravel()
    lib().vo_axpy256(y, x, float(a), y.size)
    return y


def add256(y, x):
    y, x = _c(y, np.float32).ravel().copy(), _c(x, np.float32).ravel()
    lib().vo_add256(y, x, y.size)
    return y


def max256(x):
    x = _c(x, np.float32).ravel()
    return np.float32(lib().vo_max256(x, x.size))


def sum256(x):
    x = _c(x, np.float32).ravel()
    return np.float32(lib().vo_sum256(x, x.size))


def scale_mul(x, a):
    x = _c(x, np.float32).ravel()
    d = np.empty_like(x)
    lib().vo_scale_mul(d, x, float(a), x.size)
    return d


def layernorm(x, g, b, eps=1e-5):
    y = _c(x, np.float32).copy()
    rows, cols = y.shape
    lib().vo_layernorm(y, _c(g, np.float32), _c(b, np.float32), rows, cols, float(eps))
    return y


def bias(d, b):
    d = _c(d, np.float32).copy()
    rows, cols = d.shape
    lib().vo_bias(d, _c(b, np.float32), rows, cols)
    return d


def outer(s, v, k, sc=1.0):
    s = _c(s, np.float32).copy()
    m, n = s.shape
    lib().vo_outer(s, _c(v, np.float32), _c(k, np.float32), m, n, float(sc))
    return s


def act(x, kind):
    y = _c(x, np.float32).copy()
    lib().vo_act(y.reshape(-1), y.size, int(kind))
    return y


def ew_op(x, y, op):
    x, y = _c(x, np.float32), _c(y, np.float32)
    d = np.empty_like(x)
    lib().vo_ew_op(d.reshape(-1), x.reshape(-1), y.reshape(-1), x.size, int(op))
    return d


def scale(x, s):
    x = _c(x, np.float32)
    d = np.empty_like(x)
    lib().vo_scale(d.reshape(-1), x.reshape(-1), x.size, float(s))
    return d


def rope(x, theta, pos0):
    x = _c(x, np.float32)
    rows, hd = x.shape
    y = np.empty_like(x)
    st = lib().vo_rope(y, x, rows, hd, float(theta), int(pos0))
    if st:
        raise ValueError(f"ROPE guard failed (code {st})")
    return y


def emb_bf16(table, rowf):
    table = _c(table, np.uint16)
    rows, cols = table.shape
    y = np.empty(cols, np.float32)
    st = lib().vo_emb_bf16(y, table, rows, cols, float(rowf))
    return st, y


def topk_idx(x):
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    d = np.zeros(1, np.float32)
    st = lib().vo_topk_idx(x, x.shape[0], x.shape[1], d)
    return st, float(d[0])


# ---------------------------------------------------------------- B1
def neuron_seed(layer, i):
    return lib().vo_neuron_seed(layer, i)


def neuron_rand(seed, j):
    return lib().vo_neuron_rand(seed, j)


def neuron_conn_src(layer, i, j, n, k0):
    return lib().vo_neuron_conn_src(layer, i, j, n, k0)


def b1_forward(w, src, x):
    """ops/src/b1_pure.rs:151 b1_forward (AVX2 branch) for one token."""
    w, src, x = _c(w, np.float32), _c(src, np.uint32), _c(x, np.float32)
    n, k0 = w.shape
    y = np.empty(n, np.float32)
    lib().vo_b1_forward(n, k0, w, src, x, y)
    return y


def b1_forward_t8(w, src, xt, n_tokens):
    """ops/src/b1_pure.rs:271 b1_forward_t8 (bitwise scalar contract)."""
    w, src, xt = _c(w, np.float32), _c(src, np.uint32), _c(xt, np.float32)
    n, k0 = w.shape
    t8 = xt.shape[1]
    yt = np.zeros((n, t8), np.float32)
    lib().vo_b1_forward_t8_scalar(w, src, n, k0, xt, t8, n_tokens, yt)
    return yt


def transpose_t8(x, t8):
    x = _c(x, np.float32)
    t, d = x.shape
    xt = np.empty((d, t8), np.float32)
    lib().vo_transpose_t8(x, t, d, xt, t8)
    return xt


def transpose_t8_back(a, cols):
    a = _c(a, np.float32)
    rows, in_stride = a.shape
    out = np.empty((cols, rows), np.float32)
    lib().vo_transpose_t8_back(a, rows, cols, out, rows, in_stride)
    return out


# ---------------------------------------------------------------- attention
def attention_prefill(q, k, v, n_heads, theta=10000.0, pos0=0, scale=None, causal=True):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    S, W = q.shape
    hd = W // n_heads
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(hd)))
    out = np.empty_like(q)
    lib().vo_attention_prefill(q, k, v, out, S, n_heads, hd, float(theta), int(pos0),
                               float(scale), int(causal))
    return out


def attention_decode(q, k_new, v_new, kcache, vcache, pos, theta=10000.0, scale=None):
    """Caches [H, cap, hd] are updated in place at `pos`."""
    H, cap, hd = kcache.shape
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(hd)))
    out = np.empty(H * hd, np.float32)
    lib().vo_attention_decode(_c(q, np.float32).reshape(-1), _c(k_new, np.float32).reshape(-1),
                              _c(v_new, np.float32).reshape(-1), kcache, vcache, out, H, hd,
                              cap, int(pos), float(theta), float(scale))
    return out


# ---------------------------------------------------------------- decoder
class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("wq", "wk", "wv", "wo", "wg", "wu", "wd",
                 "sq", "sk", "sv", "so", "sg", "su", "sd", "in_ln", "post_ln")]


class _Model(C.Structure):
    _fields_ = [("n_layers", C.c_size_t), ("hidden", C.c_size_t), ("n_heads", C.c_size_t),
                ("head_dim", C.c_size_t), ("inter", C.c_size_t), ("vocab", C.c_size_t),
                ("eps", C.c_float), ("theta", C.c_float), ("attn_scale", C.c_float),
                ("layers", C.c_void_p), ("embed", C.c_void_p), ("lm_head", C.c_void_p),
                ("final_norm", C.c_void_p)]


class DecoderOracle:
    """CPU run of the MiniCPM-shaped program over host weight arrays.

    `weights` is the dict produced by sparrow_amd.decoder.make_weights (or any
    dict with the same keys); arrays are referenced, not copied.
    """

    def __init__(self, weights: dict, cfg: dict, cap: int):
        self.w = weights
        self.cfg = cfg
        self.cap = int(cap)
        nl = cfg["n_layers"]
        self._layers = (_Layer * nl)()
        for li in range(nl):
            L = weights["layers"][li]
            for name in _Layer._fields_:
                key = name[0]
                setattr(self._layers[li], key, L[key].ctypes.data)
        self._model = _Model(nl, cfg["hidden"], cfg["n_heads"], cfg["head_dim"], cfg["inter"],
                             cfg["vocab"], cfg["eps"], cfg["theta"], cfg["attn_scale"],
                             C.cast(self._layers, C.c_void_p), weights["embed"].ctypes.data,
                             weights["lm_head"].ctypes.data, weights["final_norm"].ctypes.data)
        shape = (nl, cfg["n_heads"], self.cap, cfg["head_dim"])
        self.kcache = np.zeros(shape, np.float32)
        self.vcache = np.zeros(shape, np.float32)

    def reset(self):
        self.kcache[...] = 0
        self.vcache[...] = 0

    def prefill(self, tokens):
        tokens = _c(tokens, np.int32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        hidden = np.empty(self.cfg["hidden"], np.float32)
        st = lib().vo_decoder_prefill(C.byref(self._model), self.kcache, self.vcache, self.cap,
                                      tokens, tokens.size, logits.ctypes.data,
                                      hidden.ctypes.data)
        if st:
            raise ValueError(f"oracle prefill failed ({st})")
        return logits, hidden

    def step(self, token, pos):
        logits = np.empty(self.cfg["vocab"], np.float32)
        hidden = np.empty(self.cfg["hidden"], np.float32)
        st = lib().vo_decoder_step(C.byref(self._model), self.kcache, self.vcache, self.cap,
                                   int(token), int(pos), logits.ctypes.data, hidden.ctypes.data)
        if st:
            raise ValueError(f"oracle step failed ({st})")
        return logits, hidden

    def generate(self, prompt, n_steps):
        prompt = _c(prompt, np.int32)
        toks = np.empty(n_steps + 1, np.int32)
        margins = np.empty(n_steps + 1, np.float32)
        st = lib().vo_decoder_generate(C.byref(self._model), self.kcache, self.vcache,
                                       self.cap, prompt, prompt.size, n_steps, toks,
                                       margins.ctypes.data)
        if st:
            raise ValueError(f"oracle generate failed ({st})")
        return toks, margins


# ---------------------------------------------------------------- the VM
class VmError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"exit {code}: {msg}")
        self.code, self.msg = code, msg


class OracleVm:
    """The reference VM restated on the CPU (vmlm_vm_oracle.c): load a .vmb
    image (core/src/interp.rs Vm::load), run it (Vm::run), read slots and
    the PRINT output. Failures raise VmError with the reference's exit code."""

    def __init__(self, image: bytes):
        self._h = None
        h = C.c_void_p()
        rc = lib().vo_vm_load(image, len(image), C.byref(h))
        if rc:
            raise VmError(rc, lib().vo_vm_last_load_error().decode())
        self._h = h

    def close(self):
        if self._h:
            lib().vo_vm_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def run(self):
        rc = lib().vo_vm_run(self._h)
        if rc:
            raise VmError(rc, lib().vo_vm_message(self._h).decode())

    def slot_index(self, name: str) -> int:
        from sparrow_amd.vmb import hash32
        i = C.c_uint32()
        if lib().vo_vm_find(self._h, hash32(name), C.byref(i)):
            raise KeyError(name)
        return i.value

    def read(self, name_or_index):
        i = name_or_index if isinstance(name_or_index, int) else self.slot_index(name_or_index)
        p, r, c, dt = C.c_void_p(), C.c_uint32(), C.c_uint32(), C.c_uint8()
        rc = lib().vo_vm_slot(self._h, i, C.byref(p), C.byref(r), C.byref(c), C.byref(dt))
        if rc:
            raise VmError(rc, lib().vo_vm_message(self._h).decode())
        if dt.value != 0:
            raise TypeError("only f32 slots are read back")
        buf = (C.c_float * (r.value * c.value)).from_address(p.value)
        return np.array(buf, np.float32).reshape(r.value, c.value)

    def write(self, name_or_index, values):
        i = name_or_index if isinstance(name_or_index, int) else self.slot_index(name_or_index)
        p, r, c, dt = C.c_void_p(), C.c_uint32(), C.c_uint32(), C.c_uint8()
        rc = lib().vo_vm_slot(self._h, i, C.byref(p), C.byref(r), C.byref(c), C.byref(dt))
        if rc or dt.value != 0:
            raise VmError(rc or 9, "slot not writable as f32")
        v = np.ascontiguousarray(values, np.float32).ravel()
        if v.size > r.value * c.value:
            raise ValueError("more values than the slot holds")
        C.memmove(p.value, v.ctypes.data, v.nbytes)

    def output(self):
        n = lib().vo_vm_output(self._h, None, 0)
        out = np.empty(n, np.float32)
        lib().vo_vm_output(self._h, out.ctypes.data, n)
        return out

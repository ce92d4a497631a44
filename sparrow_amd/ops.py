"""Host-array mirror of the vmlm-ops kernels, running on the MI355X.

Each function takes and returns numpy arrays with the reference function's
semantics and name (ops/src/kernels.rs, ops/src/b1_pure.rs, and the VM
opcode arms of core/src/interp.rs); the work runs in libvmlm_hip.so through
its host-pointer C ABI (layer 1 of include/vmlm_hip.h). Guard violations
raise VmlmError with code 9, as the reference interpreter exits with 9.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi, check, lib

ACT_RELU, ACT_GELU, ACT_SILU, ACT_SIGMOID, ACT_TANH, ACT_RELU2 = range(6)
OP_EWADD, OP_EWMUL, OP_EWSUB, OP_EWDIV = 20, 21, 22, 23


def _c(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


def _p(a):
    return a.ctypes.data


def gemm_nt_int8(a, q, scale):
    """ops/src/kernels.rs:1258 -- C = (A . Q^T) * scale[n]."""
    a, q, s = _c(a, np.float32), _c(q, np.int8), _c(scale, np.float32)
    m, k = a.shape
    n = q.shape[0]
    assert q.shape[1] == k and s.size >= n
    c = np.empty((m, n), np.float32)
    check(lib().vmlm_gemm_nt_int8(_p(a), _p(q), _p(s), _p(c), m, n, k))
    return c


def gemm_nt_bf16(a, b):
    """ops/src/kernels.rs:1202 -- C = A . B^T, B bf16 bits [n,k]."""
    a, b = _c(a, np.float32), _c(b, np.uint16)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.float32)
    check(lib().vmlm_gemm_nt_bf16(_p(a), _p(b), _p(c), m, n, k))
    return c


def gemm_nt(a, b, c=None, acc=False):
    """ops/src/kernels.rs:987 -- C (+)= A . B^T (f32)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    check(lib().vmlm_gemm_nt(_p(a), _p(b), _p(c), m, n, k, bool(acc)))
    return c


def gemm(a, b, c=None, acc=False):
    """ops/src/kernels.rs:407 -- C (+)= A . B (f32, NN)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    check(lib().vmlm_gemm(_p(a), _p(b), _p(c), m, n, k, bool(acc)))
    return c


def rmsnorm(x, g, eps):
    """ops/src/kernels.rs:1346."""
    x, g = _c(x, np.float32), _c(g, np.float32)
    rows, cols = x.shape
    y = np.empty_like(x)
    check(lib().vmlm_rmsnorm(_p(y), _p(x), _p(g), rows, cols, float(eps)))
    return y


def softmax(p, causal=False):
    """ops/src/kernels.rs:1389 (returns a new array)."""
    p = _c(p, np.float32).copy()
    rows, cols = p.shape
    check(lib().vmlm_softmax(_p(p), rows, cols, bool(causal)))
    return p


def act(x, kind):
    """ops/src/kernels.rs:1146 act_avx2 (returns a new array)."""
    y = _c(x, np.float32).copy()
    check(lib().vmlm_act(_p(y), y.size, int(kind)))
    return y


def ew_op(x, y, op):
    """ops/src/kernels.rs:1117."""
    x, y = _c(x, np.float32), _c(y, np.float32)
    d = np.empty_like(x)
    check(lib().vmlm_ew_op(_p(d), _p(x), _p(y), x.size, int(op)))
    return d


def scale(x, s):
    """core/src/interp.rs:1225 OP_SCALE."""
    x = _c(x, np.float32)
    d = np.empty_like(x)
    check(lib().vmlm_scale(_p(d), _p(x), x.size, float(s)))
    return d


def rope(x, theta, pos0):
    """core/src/interp.rs:1159 OP_ROPE over rows at positions pos0+row."""
    x = _c(x, np.float32)
    rows, hd = x.shape
    y = np.empty_like(x)
    check(lib().vmlm_rope(_p(y), _p(x), rows, hd, float(theta), int(pos0)))
    return y


def emb_bf16(table, rowf):
    """core/src/interp.rs:1351 OP_EMB over a bf16 table."""
    table = _c(table, np.uint16)
    rows, cols = table.shape
    y = np.empty(cols, np.float32)
    check(lib().vmlm_emb_bf16(_p(y), _p(table), rows, cols, float(rowf)))
    return y


def topk_idx(x):
    """core/src/interp.rs:1649 OP_TOPK_IDX: argmax of row 0 as a float."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    d = np.zeros(1, np.float32)
    check(lib().vmlm_topk_idx(_p(x), x.shape[0], x.shape[1], _p(d)))
    return float(d[0])


def _conn(w, src):
    """SparseConnW over host arrays: the u32 ids and their f32 copy (the
    struct's `src`, which b1_backward reads)."""
    w = _c(w, np.float32)
    src = _c(src, np.uint32)
    srcf = src.astype(np.float32)
    n, k0 = w.shape
    sc = _abi.SparseConnW(e=n * k0, k0=k0, layer=0, n_neurons=n, w=_p(w), src=_p(srcf),
                          src_u32=_p(src), act=None)
    return sc, (w, src, srcf)


def b1_forward(w, src, x):
    """ops/src/b1_pure.rs:151 -- one token: y[i] = sum_j w[i,j] x[src[i,j]]."""
    sc, keep = _conn(w, src)
    x = _c(x, np.float32)
    y = np.empty(sc.n_neurons, np.float32)
    macs = C.c_size_t(0)
    check(lib().vmlm_b1_forward(C.byref(sc), _p(x), _p(y), C.byref(macs)))
    return y, macs.value


def b1_forward_t8(w, src, xt, n_tokens, yt=None):
    """ops/src/b1_pure.rs:271 -- source-major tokens, bitwise scalar contract."""
    sc, keep = _conn(w, src)
    xt = _c(xt, np.float32)
    t8 = xt.shape[1]
    yt = np.zeros((sc.n_neurons, t8), np.float32) if yt is None else _c(yt, np.float32).copy()
    macs = C.c_size_t(0)
    check(lib().vmlm_b1_forward_t8(C.byref(sc), _p(xt), t8, int(n_tokens), _p(yt),
                                   C.byref(macs)))
    return yt, macs.value


def b1_backward(w, src, dy, x, dw=None):
    """ops/src/b1_pure.rs:642 -- dw += dy[i] * x[src] (over the f32 ids)."""
    sc, keep = _conn(w, src)
    dw = np.zeros(w.shape, np.float32) if dw is None else _c(dw, np.float32).copy()
    n = C.c_size_t(0)
    check(lib().vmlm_b1_backward(C.byref(sc), _p(_c(dy, np.float32)), _p(_c(x, np.float32)),
                                 _p(dw), C.byref(n)))
    return dw, n.value


def b1_backward_dx(w, src, dy, dx=None):
    """ops/src/b1_pure.rs:410 -- dx[src] += dy[i] * w, i and j ascending."""
    sc, keep = _conn(w, src)
    dx = np.zeros(sc.n_neurons, np.float32) if dx is None else _c(dx, np.float32).copy()
    n = C.c_size_t(0)
    check(lib().vmlm_b1_backward_dx(C.byref(sc), _p(_c(dy, np.float32)), _p(dx), C.byref(n)))
    return dx, n.value


def b1_backward_fused(w, src, dy, x, dw=None, dx=None):
    """ops/src/b1_pure.rs:466 -- dw and dx in one call."""
    sc, keep = _conn(w, src)
    dw = np.zeros(w.shape, np.float32) if dw is None else _c(dw, np.float32).copy()
    dx = np.zeros(sc.n_neurons, np.float32) if dx is None else _c(dx, np.float32).copy()
    n = C.c_size_t(0)
    check(lib().vmlm_b1_backward_fused(C.byref(sc), _p(_c(dy, np.float32)),
                                       _p(_c(x, np.float32)), _p(dw), _p(dx), C.byref(n)))
    return dw, dx, n.value


def b1_backward_t8(w, src, xt, dyt, dxt=None, dw=None):
    """ops/src/kernels.rs:3229 -- source-major [n][t8] activations."""
    w, src = _c(w, np.float32), _c(src, np.uint32)
    n, k0 = w.shape
    xt, dyt = _c(xt, np.float32), _c(dyt, np.float32)
    t8 = xt.shape[1]
    dxt = np.zeros((n, t8), np.float32) if dxt is None else _c(dxt, np.float32).copy()
    dw = np.zeros((n, k0), np.float32) if dw is None else _c(dw, np.float32).copy()
    check(lib().vmlm_b1_backward_t8(_p(w), _p(src), _p(xt), _p(dyt), t8, n, k0, _p(dxt), _p(dw)))
    return dxt, dw


def transpose_t8(x, t8):
    """ops/src/kernels.rs:1881."""
    x = _c(x, np.float32)
    t, d = x.shape
    xt = np.empty((d, t8), np.float32)
    check(lib().vmlm_transpose_t8(_p(x), t, d, _p(xt), t8))
    return xt


def transpose_t8_back(a, cols):
    """ops/src/kernels.rs:3307 with os = rows."""
    a = _c(a, np.float32)
    rows, in_stride = a.shape
    out = np.zeros((cols, rows), np.float32)
    check(lib().vmlm_transpose_t8_back(_p(a), rows, cols, _p(out), rows, in_stride))
    return out


def attention_prefill(q, k, v, n_heads, theta=10000.0, pos0=0, scale=None, causal=True):
    """tools/p12_build_minicpm.py:770-781 composition, fused."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    S, W = q.shape
    hd = W // n_heads
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(hd)))
    out = np.empty_like(q)
    check(lib().vmlm_attention_prefill(_p(q), _p(k), _p(v), _p(out), S, n_heads, hd,
                                       float(theta), int(pos0), float(scale), bool(causal)))
    return out


def attention_decode(q, k_new, v_new, kcache, vcache, pos, theta=10000.0, scale=None,
                     split=-1):
    """tools/p12_build_minicpm.py:941-967; caches [H, cap, hd] updated in place.
    `split`: 16-position sub-chunks per workgroup (0: one workgroup per head,
    -1: the library's choice); the result is the same bits for every split."""
    H, cap, hd = kcache.shape
    assert kcache.dtype == np.float32 and kcache.flags.c_contiguous
    assert vcache.dtype == np.float32 and vcache.flags.c_contiguous
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(hd)))
    q, k_new, v_new = (_c(t, np.float32).reshape(-1) for t in (q, k_new, v_new))
    out = np.empty(H * hd, np.float32)
    check(lib().vmlm_attention_decode_split(_p(q), _p(k_new), _p(v_new), _p(kcache),
                                            _p(vcache), _p(out), H, hd, cap, int(pos),
                                            float(theta), float(scale), int(split)))
    return out

"""B1 sparse connections (ops/src/conn.rs SparseConnW) and the layer stack.

`make_block_aligned` draws the benchmark's topology: each neuron keeps k0
sources made of k0/8 distinct 8-aligned blocks of 8 consecutive source ids
(the block-aligned layout of ops/src/kernels.rs:3389-3401), weights
N(0, 1/sqrt(k0)). `prng_sources` reproduces the reference's stateless PRNG
topology (core/src/conn_sparse.rs:157-214) for known-answer parity.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi, check, lib

M32 = 0xFFFFFFFF
GOLDEN = 0x9E3779B9


def _mix32(z):
    z = ((z ^ (z >> 16)) * 0x7FEB352D) & M32
    z = ((z ^ (z >> 15)) * 0x846CA68B) & M32
    return z ^ (z >> 16)


def prng_sources(layer: int, n: int, k0: int) -> np.ndarray:
    """neuron_conn_src(layer, i, j, n, k0) for all (i, j), vectorised (uint64
    arithmetic masked to 32 bits)."""
    i = np.arange(n, dtype=np.uint64)[:, None]
    j = np.arange(k0, dtype=np.uint64)[None, :]
    a = (GOLDEN * ((layer + 1) & M32)) & M32
    b = (0x85EBCA6B * ((i + 1) & M32)) & M32
    seed = _mix32(np.uint64(a) ^ b)
    jj = np.where(j == 0, np.uint64(M32), j)
    r = _mix32(seed ^ ((GOLDEN * ((jj + 1) & M32)) & M32))
    return (r % np.uint64(n)).astype(np.uint32)


def make_block_aligned(rng: np.random.Generator, n: int, k0: int):
    assert k0 % 8 == 0 and n % 8 == 0
    nb = n // 8
    blocks = np.stack([rng.choice(nb, size=k0 // 8, replace=False) for _ in range(n)])
    src = (blocks[:, :, None] * 8 + np.arange(8)[None, None, :]).reshape(n, k0)
    w = (rng.standard_normal((n, k0)) / np.sqrt(k0)).astype(np.float32)
    return w, src.astype(np.uint32)


class DeviceConn:
    """One layer's w / src_u32 resident in HBM, as a vmlm_sparse_conn_w."""

    def __init__(self, w: np.ndarray, src: np.ndarray, layer: int = 0):
        w = np.ascontiguousarray(w, np.float32)
        src = np.ascontiguousarray(src, np.uint32)
        n, k0 = w.shape
        if src.max(initial=0) >= n:
            raise ValueError("B1: source index >= n_neurons")
        L = lib()
        self._ptrs = []
        self.w_dev = self._upload(L, w)
        self.src_dev = self._upload(L, src)
        self.struct = _abi.SparseConnW(e=n * k0, k0=k0, layer=layer, n_neurons=n,
                                       w=self.w_dev, src=None, src_u32=self.src_dev, act=None)

    def _upload(self, L, a):
        p = C.c_void_p()
        check(L.vmlm_hip_malloc(C.byref(p), a.nbytes))
        check(L.vmlm_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes))
        self._ptrs.append(p)
        return p.value

    def free(self):
        for p in self._ptrs:
            lib().vmlm_hip_free(p)
        self._ptrs = []


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().vmlm_hip_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib().vmlm_hip_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def to_array(self, shape, dtype):
        out = np.empty(shape, dtype)
        check(lib().vmlm_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib().vmlm_hip_free(self.ptr)
            self.ptr = None


def stack_forward(layers: list[DeviceConn], x_dev: int, y_dev: int, n_tokens: int,
                  act: int = 4, stream=None) -> None:
    """y = act(gather-dot) through every layer (device pointers, async)."""
    arr = (_abi.SparseConnW * len(layers))(*[l.struct for l in layers])
    check(lib().vmlm_b1_stack_forward(arr, len(layers), x_dev, y_dev, int(n_tokens), int(act),
                                      stream))


class StackPlan:
    """A B1 stack with its connection plan built once (vmlm_b1_stack_create):
    run() is one kernel launch with no allocation. The plan holds the weights
    and indices as they were at creation."""

    def __init__(self, layers: list[DeviceConn], stream=None):
        arr = (_abi.SparseConnW * len(layers))(*[l.struct for l in layers])
        h = C.c_void_p()
        check(lib().vmlm_b1_stack_create(arr, len(layers), stream, C.byref(h)))
        self._h = h

    def run(self, x_dev: int, y_dev: int, n_tokens: int, act: int = 4, stream=None) -> None:
        check(lib().vmlm_b1_stack_run(self._h, x_dev, y_dev, int(n_tokens), int(act), stream))

    def close(self) -> None:
        if self._h:
            lib().vmlm_b1_stack_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

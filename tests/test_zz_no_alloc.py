"""The allocation-free int8 GEMM (vmlm_hip_gemm_nt_int8_noalloc), through the
C ABI, against the entry point it mirrors (vmlm_hip_gemm_nt_int8). Up to
M = 255 both run the same kernels. From M = 256 (N a multiple of 16) the
allocating call first swizzles the weights into 1 KiB blocks in its
workspace and runs the blocked int8-row GEMM, while the allocation-free call
keeps its scratch for the rows and runs the row-major form of the same GEMM
(its own tile shapes); both sum each term's int8 products exactly in int32
over the whole K (one k-slice at these grids) and combine them with the same
arithmetic, so the outputs are bitwise equal in every case. Both also stay
within 1e-4 x RMS of the CPU oracle. Two calls in a row share the scratch
array, the second with a smaller input, then the int8-row paths (M > 16,
M >= 256), then a shape whose temporaries exceed the scratch, which must
return 9 without touching the output."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def q8_case(rng, m, n, k):
    a = rng.standard_normal((m, k), dtype=np.float32)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)) / np.float32(127)
         + np.float32(1e-6)).astype(np.float32)
    return a, q, s


class Dev:
    def __init__(self, lib):
        self.lib, self.ptrs = lib, []

    def check(self, rc):
        assert rc == 0, self.lib.vmlm_hip_last_error().decode()

    def up(self, a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        self.check(self.lib.vmlm_hip_malloc(C.byref(p), a.nbytes))
        self.check(self.lib.vmlm_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes))
        self.ptrs.append(p)
        return p

    def down(self, p, shape):
        out = np.empty(shape, np.float32)
        self.check(self.lib.vmlm_hip_sync())
        self.check(self.lib.vmlm_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes))
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.vmlm_hip_free(p)


@pytest.fixture
def dev(hip):
    import sparrow_amd
    sparrow_amd.init(0)  # the allocation-free call never initialises the library
    d = Dev(hip)
    yield d
    d.free()


def run_both(dev, oracle, m, n, k, seed):
    rng = np.random.default_rng(seed)
    a, q, s = q8_case(rng, m, n, k)
    da, dq, ds = dev.up(a), dev.up(q), dev.up(s)
    dc0 = dev.up(np.full((m, n), np.nan, np.float32))
    dc1 = dev.up(np.full((m, n), np.nan, np.float32))
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, dc0, m, n, k, None))
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8_noalloc(da, dq, ds, dc1, m, n, k, None))
    want, got = dev.down(dc0, (m, n)), dev.down(dc1, (m, n))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k)
    ref = oracle.gemm_nt_int8(a, q, s)
    err = np.abs(got.astype(np.float64) - ref).max()
    assert err <= 1e-4 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))


def test_noalloc_matches_gemm_nt_int8(dev, oracle):
    run_both(dev, oracle, 16, 5760, 2304, 1)   # decode gate shape: 9 k-slices
    run_both(dev, oracle, 3, 1000, 1024, 2)    # smaller, right after
    run_both(dev, oracle, 40, 512, 2304, 3)    # int8 rows + ordered k-slices
    run_both(dev, oracle, 2, 70, 100, 4)       # K % 128 != 0: padded copy in scratch
    run_both(dev, oracle, 256, 512, 2304, 6)   # M >= 256: blocked (allocating) vs row-major
    run_both(dev, oracle, 300, 2304, 2304, 7)  # the same with ragged M


def test_noalloc_rejects_oversized(dev):
    m, n, k = 16, 122753, 2304                 # 9 slices x 16 x n x 4 B = 70 MB > 16 MiB
    rng = np.random.default_rng(5)
    a, q, s = q8_case(rng, m, n, k)
    da, dq, ds = dev.up(a), dev.up(q), dev.up(s)
    sentinel = np.full((m, n), 7.0, np.float32)
    dc = dev.up(sentinel)
    rc = dev.lib.vmlm_hip_gemm_nt_int8_noalloc(da, dq, ds, dc, m, n, k, None)
    assert rc == 9
    assert b"scratch" in dev.lib.vmlm_hip_last_error()
    assert np.array_equal(dev.down(dc, (m, n)), sentinel)

"""Prefill GEMM (M > 16) through the device-pointer API.

The kernel copies its tiles straight from global memory into a two-stage LDS
ring and writes C through an LDS-staged epilogue; these cases cover both tile
heights (64 rows, and 128 rows once the grid gives two workgroups per CU),
ragged M / N edges (the scalar store tail when rows are not 16-byte
multiples), short and long k-loops, and three-term (f32) activations with
int8 weights. The reference is float64 over the same bf16 / int8 operands:
every product is exact in f32, only the summation order differs, so the
bound is the 1e-4 x RMS contract of gemm_nt_bf16 / gemm_nt_int8
(ops/src/kernels.rs:1199-1287).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 1e-4


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def assert_close_rms(got, ref, tol=TOL):
    ref = np.asarray(ref, np.float64)
    err = float(np.abs(np.asarray(got, np.float64) - ref).max())
    rms = float(np.sqrt(np.mean(ref * ref)))
    assert err <= tol * max(rms, 1e-30), f"max|d|={err:.3e} rms={rms:.3e}"


class Device:
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

    def empty(self, nbytes):
        p = C.c_void_p()
        self.check(self.lib.vmlm_hip_malloc(C.byref(p), nbytes))
        self.ptrs.append(p)
        return p

    def down(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self.check(self.lib.vmlm_hip_sync())
        self.check(self.lib.vmlm_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes))
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.vmlm_hip_free(p)


@pytest.fixture
def dev(hip):
    d = Device(hip)
    yield d
    d.free()


@pytest.mark.parametrize("m,n,k", [(1024, 2048, 512),   # config 1
                                   (1, 2048, 512),      # config 1, M = 1 (GEMV path)
                                   (16, 2048, 512),     # GEMV path, 16 rows
                                   (5, 300, 192),       # GEMV path, ragged N
                                   (2048, 4096, 128),   # 128-row tiles
                                   (130, 201, 192),     # ragged, odd row stride
                                   (17, 128, 64)])      # one k-step, one spare row
def test_gemm_bf16_bf16(dev, m, n, k):
    rng = np.random.default_rng(m * 3 + n + k)
    a = bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    b = bf16_bits(rng.standard_normal((n, k), dtype=np.float32) / np.float32(np.sqrt(k)))
    da, db, dc = dev.up(a), dev.up(b), dev.empty(m * n * 4)
    dev.check(dev.lib.vmlm_hip_gemm_nt_bf16bf16(da, db, dc, m, n, k, None))
    got = dev.down(dc, (m, n), np.float32)
    ref = bf16_value(a).astype(np.float64) @ bf16_value(b).astype(np.float64).T
    assert_close_rms(got, ref)


@pytest.mark.parametrize("m,n,k", [(200, 2304, 5760),   # down projection, 90 k-steps
                                   (2048, 384, 256)])   # many row tiles
def test_gemm_int8_three_terms(dev, oracle, m, n, k):
    rng = np.random.default_rng(m + n * 5 + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, n)) / 127 + 1e-6).astype(np.float32)
    da, dq, ds, dc = dev.up(a), dev.up(q), dev.up(s), dev.empty(m * n * 4)
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, dc, m, n, k, None))
    got = dev.down(dc, (m, n), np.float32)
    ref = (a.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    assert_close_rms(got, ref)
    assert_close_rms(got, oracle.gemm_nt_int8(a, q, s))


def test_gemm_int8_row_split_paths_agree(dev):
    """Up to 256 rows are split into int8 terms by one launch (stats and terms
    per row), more rows by a stats launch and a blocked terms launch. Both
    form the same sums in the same order, so rows 0..255 of a 256-row and a
    257-row call give the same bits (N = 8192: neither call is k-sliced).
    Rows of mixed magnitude, a zero row and a NaN row are among them."""
    m, n, k = 257, 8192, 512
    rng = np.random.default_rng(257)
    a = rng.standard_normal((m, k), dtype=np.float32)
    a *= np.float32(10.0) ** rng.integers(-6, 7, size=(m, 1)).astype(np.float32)
    a[5] = 0.0
    a[17, 3] = np.nan
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, n)) / 127 + 1e-6).astype(np.float32)
    da, dq, ds = dev.up(a), dev.up(q), dev.up(s)
    c256, c257 = dev.empty(256 * n * 4), dev.empty(m * n * 4)
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, c256, 256, n, k, None))
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, c257, m, n, k, None))
    g256 = dev.down(c256, (256, n), np.float32)
    g257 = dev.down(c257, (m, n), np.float32)
    assert np.isnan(g256[17]).all() and (g256[5] == 0).all()
    np.testing.assert_array_equal(g256.view(np.uint32), g257[:256].view(np.uint32))
    ref = (a.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    ok = np.isfinite(ref).all(axis=1)
    for r in np.flatnonzero(ok)[:40]:
        assert_close_rms(g257[r], ref[r])


def test_gemm_int8_row_split_wave_path_agrees(dev):
    """From 2048 rows one launch splits every row with one wave (eight rows
    per workgroup, the row's maximum across the wave); below, the stats and
    terms launches do. Without a norm the split depends only on each row's
    maximum, so rows 0..2046 of a 2047-row and a 2048-row call give the same
    bits. Rows of mixed magnitude, a zero row and a NaN row are among them."""
    m, n, k = 2048, 8192, 512
    rng = np.random.default_rng(2048)
    a = rng.standard_normal((m, k), dtype=np.float32)
    a *= np.float32(10.0) ** rng.integers(-6, 7, size=(m, 1)).astype(np.float32)
    a[5] = 0.0
    a[1700, 3] = np.nan
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, n)) / 127 + 1e-6).astype(np.float32)
    da, dq, ds = dev.up(a), dev.up(q), dev.up(s)
    c_lo, c_hi = dev.empty((m - 1) * n * 4), dev.empty(m * n * 4)
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, c_lo, m - 1, n, k, None))
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, c_hi, m, n, k, None))
    g_lo = dev.down(c_lo, (m - 1, n), np.float32)
    g_hi = dev.down(c_hi, (m, n), np.float32)
    assert np.isnan(g_hi[1700]).all() and (g_hi[5] == 0).all()
    np.testing.assert_array_equal(g_lo.view(np.uint32), g_hi[:m - 1].view(np.uint32))
    ref = (a[:64].astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    for r in range(0, 64, 7):
        if r != 5:
            assert_close_rms(g_hi[r], ref[r])


@pytest.mark.parametrize("m,n", [(2048, 4096),    # 32 x 32 tiles of 64 x 128
                                 (2100, 4112)])   # ragged last tile row and column
def test_gemm_int8_many_tiles_exact(dev, m, n):
    """A large grid over blocked weights (M >= 256 swizzles the caller's
    weights; two LDS stages, four workgroups per CU). Integer activations
    give exact int8 terms and exact f32 sums, so the result is the float64
    product bit for bit; the ragged case clamps the copies of column tiles
    past the weights and stores only rows < M and columns < N. A NaN row goes
    through the f32 recomputation."""
    k = 256
    rng = np.random.default_rng(m + n)
    a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    a[m - 1, 7] = np.nan
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = np.ones(n, np.float32)
    da, dq, ds, dc = dev.up(a), dev.up(q), dev.up(s), dev.empty(m * n * 4)
    dev.check(dev.lib.vmlm_hip_gemm_nt_int8(da, dq, ds, dc, m, n, k, None))
    got = dev.down(dc, (m, n), np.float32)
    ref = a[:m - 1].astype(np.float64) @ q.astype(np.float64).T
    np.testing.assert_array_equal(got[:m - 1].astype(np.float64), ref)
    assert np.isnan(got[m - 1]).all()

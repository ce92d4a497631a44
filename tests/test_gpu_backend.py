"""GPU parity of the reference-layout Backend table (sys/src/lib.rs:29-38)
and the jit_* entry points (ops/src/kernels.rs:1017-1113) against the CPU
oracle, through the C ABI.

Bars: axpy256 / add256 / scale_mul / max256 (NaN and signed zeros included),
jit_act / jit_ew* / jit_bias / jit_outer bitwise; dot256 / sum256 within
1e-5 of sum|terms| (tree sums against the reference's 8-lane chains);
jit_ln within 1e-4 x RMS; jit_softmax to 1e-5 absolute with rows summing
to 1 (the bar of the softmax op). Backend functions are called with
host pointers and with device pointers."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def fp(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="module")
def table(hip):
    from sparrow_amd import _abi
    import sparrow_amd
    sparrow_amd.init(0)
    return C.cast(hip.vmlm_hip_backend(), C.POINTER(_abi.Backend)).contents


class Dev:
    def __init__(self, lib):
        self.lib, self.ptrs = lib, []

    def up(self, a):
        a = np.ascontiguousarray(a, np.float32)
        p = C.c_void_p()
        assert self.lib.vmlm_hip_malloc(C.byref(p), max(a.nbytes, 4)) == 0
        assert self.lib.vmlm_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0
        self.ptrs.append(p)
        return p

    def down(self, p, n):
        out = np.empty(n, np.float32)
        assert self.lib.vmlm_hip_sync() == 0
        assert self.lib.vmlm_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.vmlm_hip_free(p)


@pytest.fixture
def dev(hip):
    d = Dev(hip)
    yield d
    d.free()


def test_backend_layout(table):
    assert table.name == b"hip_gfx950"
    for f in ("dot256", "axpy256", "add256", "max256", "sum256", "scale_mul"):
        assert C.cast(getattr(table, f), C.c_void_p).value


@pytest.mark.parametrize("n", [0, 1, 7, 8, 33, 1000, 100003, 3000000])
def test_backend_dot_sum(table, dev, oracle, n):
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) + 0.5).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    t = a.astype(np.float64) * b
    for got in (table.dot256(fp(a), fp(b), n), table.dot256(dev.up(a), dev.up(b), n)):
        assert abs(got - t.sum()) <= 1e-5 * np.abs(t).sum() + 1e-30
        assert abs(got - oracle.dot256(a, b)) <= 1e-5 * np.abs(t).sum() + 1e-30
    for got in (table.sum256(fp(a), n), table.sum256(dev.up(a), n)):
        assert abs(got - a.astype(np.float64).sum()) <= 1e-5 * np.abs(a).sum() + 1e-30
    if n:
        ia = rng.integers(-50, 50, n).astype(np.float32)
        assert table.sum256(fp(ia), n) == oracle.sum256(ia)  # exact integer sums


@pytest.mark.parametrize("n", [0, 1, 5, 8, 9, 64, 1001, 65536 + 3, 2000000])
def test_backend_max_bitwise(table, dev, oracle, n):
    """NaNs at random places (the scan restarts after a NaN; a NaN that ends
    a lane survives it), signed zeros and infinities."""
    rng = np.random.default_rng(n + 1)
    cases = [rng.standard_normal(n).astype(np.float32)]
    x = rng.standard_normal(n).astype(np.float32)
    if n:
        x[rng.integers(0, n, max(1, n // 50))] = np.nan
        x[rng.integers(0, n, max(1, n // 50))] = 0.0
        x[rng.integers(0, n, max(1, n // 50))] = -0.0
    cases.append(x)
    cases.append(np.full(n, np.nan, np.float32))
    z = np.zeros(n, np.float32)
    z[::3] = -0.0
    cases.append(z)
    if n >= 16:
        y = np.full(n, -np.inf, np.float32)
        y[8 * (n // 8) - 1] = np.nan  # the last element of lane 7 of the 8-blocks
        cases.append(y)
    for c in cases:
        want = bits(np.float32(oracle.max256(c)))
        assert np.array_equal(bits(np.float32(table.max256(fp(c), n))), want)
        assert np.array_equal(bits(np.float32(table.max256(dev.up(c), n))), want)


@pytest.mark.parametrize("n", [1, 8, 45, 4099, 1000000])
def test_backend_elementwise_bitwise(table, dev, oracle, n):
    rng = np.random.default_rng(n + 2)
    y = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    a = np.float32(-0.731)
    y1 = y.copy()
    table.axpy256(fp(y1), fp(x), float(a), n)
    assert np.array_equal(bits(y1), bits(oracle.axpy256(y, x, a)))
    dy = dev.up(y)
    table.axpy256(dy, dev.up(x), float(a), n)
    assert np.array_equal(bits(dev.down(dy, n)), bits(oracle.axpy256(y, x, a)))
    y2 = y.copy()
    table.add256(fp(y2), fp(x), n)
    assert np.array_equal(bits(y2), bits(oracle.add256(y, x)))
    d = np.empty(n, np.float32)
    table.scale_mul(fp(d), fp(x), float(a), n)
    assert np.array_equal(bits(d), bits(oracle.scale_mul(x, a)))
    dd = dev.up(np.zeros(n, np.float32))
    table.scale_mul(dd, fp(x), float(a), n)  # device output, host input
    assert np.array_equal(bits(dev.down(dd, n)), bits(oracle.scale_mul(x, a)))


def test_backend_fma_control(table):
    """The fused 8-blocks and the two-rounding tail: a = x = 1 + 2^-12,
    y = -(1 + 2^-11) gives 2^-24 on the 8-block, 0 on the tail."""
    e = np.float32(1 + 2 ** -12)
    y = np.full(9, -(1 + 2 ** -11), np.float32)
    x = np.full(9, e, np.float32)
    table.axpy256(fp(y), fp(x), float(e), 9)
    assert np.all(y[:8] == np.float32(2 ** -24)) and y[8] == 0.0


def test_jit_elementwise_bitwise(hip, oracle):
    rng = np.random.default_rng(40)
    n = 4101
    x = rng.standard_normal(n).astype(np.float32)
    y = (rng.standard_normal(n) + 3).astype(np.float32)
    for kind in range(6):
        p = x.copy()
        assert hip.vmlm_jit_act(fp(p), n, kind) == 0
        assert np.array_equal(bits(p), bits(oracle.act(x, kind))), kind
    for name, op in (("ewadd", 20), ("ewmul", 21), ("ewsub", 22), ("ewdiv", 23)):
        d = np.empty(n, np.float32)
        assert getattr(hip, "vmlm_jit_" + name)(fp(d), fp(x), fp(y), n) == 0
        assert np.array_equal(bits(d), bits(oracle.ew_op(x, y, op))), name
    d = rng.standard_normal((37, 111)).astype(np.float32)
    b = rng.standard_normal(111).astype(np.float32)
    d1 = d.copy()
    assert hip.vmlm_jit_bias(fp(d1), fp(b), 37, 111) == 0
    assert np.array_equal(bits(d1), bits(oracle.bias(d, b)))


@pytest.mark.parametrize("m,n", [(1, 1), (3, 8), (17, 45), (256, 1000)])
def test_jit_outer_bitwise(hip, oracle, m, n):
    rng = np.random.default_rng(m * n)
    s = rng.standard_normal((m, n)).astype(np.float32)
    v = rng.standard_normal(m).astype(np.float32)
    k = rng.standard_normal(n).astype(np.float32)
    s1 = s.copy()
    assert hip.vmlm_jit_outer(fp(s1), fp(v), fp(k), m | (n << 32)) == 0
    assert np.array_equal(bits(s1), bits(oracle.outer(s, v, k, 1.0)))
    s2 = s.copy()
    assert hip.vmlm_outer(fp(s2), fp(v), fp(k), m, n, C.c_float(0.3)) == 0
    assert np.array_equal(bits(s2), bits(oracle.outer(s, v, k, 0.3)))


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 77), (64, 2304), (3, 9000)])
def test_jit_ln_softmax(hip, oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    y = x.copy()
    assert hip.vmlm_jit_ln(fp(y), fp(g), fp(b), rows | (cols << 32), 0) == 0
    ref = oracle.layernorm(x, g, b, 1e-5)
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert np.abs(y - ref).max() <= 1e-4 * rms
    if cols > 1:  # a constant row normalises to exactly b
        xc = np.full((1, cols), 2.5, np.float32)
        assert hip.vmlm_jit_ln(fp(xc), fp(g), fp(b), 1 | (cols << 32), 0) == 0
        assert np.array_equal(xc[0], b)
    for causal in (0, 1):
        p = x.copy()
        assert hip.vmlm_jit_softmax(fp(p), rows | (cols << 32), causal) == 0
        ref = oracle.softmax(x, bool(causal))
        # the softmax bar of test_gpu_ops.test_softmax_shapes: probabilities
        # (<= 1) to 1e-5 absolute, every row summing to 1
        assert np.abs(p - ref).max() <= 1e-5
        assert np.abs(p.astype(np.float64).sum(1) - 1).max() <= 1e-5


def test_jit_gemm_nt_dims(hip, oracle):
    rng = np.random.default_rng(41)
    m, n, k = 7, 33, 65
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    c = rng.standard_normal((m, n)).astype(np.float32)
    c1 = c.copy()
    assert hip.vmlm_jit_gemm_nt(fp(a), fp(b), fp(c1), m | (n << 16) | (k << 32) | (1 << 48)) == 0
    ref = oracle.gemm_nt(a, b, c, acc=True)
    assert np.abs(c1 - ref).max() <= 1e-4 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))


def test_device_variants(hip, dev, oracle):
    rng = np.random.default_rng(42)
    x = rng.standard_normal((9, 300)).astype(np.float32)
    g = rng.standard_normal(300).astype(np.float32)
    b = rng.standard_normal(300).astype(np.float32)
    dx = dev.up(x)
    assert hip.vmlm_hip_layernorm(dx, dev.up(g), dev.up(b), 9, 300, C.c_float(1e-5), None) == 0
    ref = oracle.layernorm(x, g, b, 1e-5)
    assert np.abs(dev.down(dx, x.size).reshape(x.shape) - ref).max() <= 1e-4 * np.abs(ref).max()
    dx = dev.up(x)
    assert hip.vmlm_hip_bias(dx, dev.up(g), 9, 300, None) == 0
    assert np.array_equal(bits(dev.down(dx, x.size)), bits(oracle.bias(x, g).ravel()))
    dx = dev.up(x)
    v = rng.standard_normal(9).astype(np.float32)
    assert hip.vmlm_hip_outer(dx, dev.up(v), dev.up(g), 9, 300, C.c_float(2.0), None) == 0
    assert np.array_equal(bits(dev.down(dx, x.size)), bits(oracle.outer(x, v, g, 2.0).ravel()))

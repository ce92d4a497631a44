"""GPU parity of the vmlm-ops kernels against the CPU oracle, through the
host-pointer C ABI (sparrow_amd.ops).

Bars: integer / index / elementwise work bit-exact;
f32-accumulated outputs within max|d| <= 1e-4 * RMS(reference)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rms(x):
    return float(np.sqrt(np.mean(np.asarray(x, np.float64) ** 2)))


def assert_close_rms(got, ref, tol=TOL):
    err = float(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)).max())
    assert err <= tol * max(rms(ref), 1e-30), f"max|d|={err:.3e} rms={rms(ref):.3e}"


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ops(hip):
    from sparrow_amd import ops
    return ops


def q8_case(rng, m, n, k):
    a = rng.standard_normal((m, k), dtype=np.float32)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)) / np.float32(127)
         + np.float32(1e-6)).astype(np.float32)
    return a, q, s


def test_q8_kat(ops):
    """tools/p13_q8_check.py:42-47 -> [[-1, -1]] exactly."""
    c = ops.gemm_nt_int8(np.float32([[1, 2, 3, 4]]), np.int8([[1, 0, -1, 0], [0, 2, 0, -2]]),
                         np.float32([0.5, 0.25]))
    assert np.array_equal(c, np.float32([[-1, -1]]))


@pytest.mark.parametrize("m,n,k", [(16, 2304, 2304), (1, 2304, 2304), (1, 5760, 2304),
                                   (4, 2304, 5760), (3, 17, 100), (40, 300, 256),
                                   (128, 512, 2304), (1, 2304, 5760), (2, 100, 2304),
                                   (4, 2304, 768), (1, 64, 128), (3, 48, 384), (2, 8192, 2304)])
def test_gemm_nt_int8(ops, oracle, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a, q, s = q8_case(rng, m, n, k)
    assert_close_rms(ops.gemm_nt_int8(a, q, s), oracle.gemm_nt_int8(a, q, s))


def test_gemm_nt_int8_rows_of_mixed_magnitude(ops, oracle):
    """M > 16 runs on int8 rows with one power-of-two factor per row: rows
    scaled from 1e-6 to 1e6 each stay within 1e-4 of their own RMS, and a
    zero row gives zeros."""
    rng = np.random.default_rng(17)
    a, q, s = q8_case(rng, 48, 320, 1024)
    a *= np.float32(10.0) ** rng.integers(-6, 7, size=(48, 1)).astype(np.float32)
    a[7] = 0.0
    got, ref = ops.gemm_nt_int8(a, q, s), oracle.gemm_nt_int8(a, q, s)
    assert not got[7].any()
    for i in range(48):
        if i != 7:
            assert_close_rms(got[i], ref[i])


@pytest.mark.parametrize("k", [512, 2304])
def test_gemm_nt_int8_exact_case_many_rows(ops, k):
    """Integer activations at M > 16 (int8 rows): each row's terms are exact
    and so is every int32 sum, so the result is exact. The grid is one
    64 x 128 tile; at K = 2304 (36 k-steps) it runs as 4 ordered k-slices
    (the rule needs N % 4 == 0 and at least 8 k-steps per slice), whose
    partial sums are exact too; at K = 512 it runs unsliced."""
    rng = np.random.default_rng(6)
    a = rng.integers(-3, 4, size=(40, k)).astype(np.float32)
    q = rng.integers(-127, 128, size=(128, k), dtype=np.int8)
    s = np.full(128, 1 / 64, np.float32)
    ref = (a.astype(np.float64) @ q.astype(np.float64).T) / 64
    assert np.array_equal(ops.gemm_nt_int8(a, q, s).astype(np.float64), ref)


def nonfinite_masks_equal(got, ref):
    for f in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(f(got), f(ref)), f.__name__


@pytest.mark.parametrize("m,k,path", [(40, 2304, "int8 rows"), (5, 2304, "k-split GEMV"),
                                      (24, 200, "bf16 terms"), (3, 100, "GEMV")])
def test_gemm_nt_int8_nonfinite(ops, oracle, m, k, path):
    """NaN and +-inf activations give the reference's pattern: a NaN row is
    all NaN; an infinite entry gives +-inf, or NaN where its weight is 0 or
    where +inf and -inf products meet (ops/src/kernels.rs:1256-1287 in f32).
    Rows without them stay within 1e-4 of their RMS. Covers the int8-row
    GEMM (M > 16, K % 128 == 0: rows with a NaN factor are recomputed in
    f32), the k-split GEMV (M <= 16) and the bf16-term paths."""
    rng = np.random.default_rng(m + k)
    n = 256
    a, q, s = q8_case(rng, m, n, k)
    a[1, 7] = np.nan
    a[2, 9] = np.inf
    a[2, 10] = np.inf
    q[:40, 9] = 0                      # inf * 0 -> NaN in those columns
    a[m - 1, 3] = -np.inf
    a[m - 2, 4] = np.inf               # +inf and -inf in one row
    a[m - 2, 5] = -np.inf
    q[40:80, 5] = -q[40:80, 4]         # columns where both products have one sign
    got, ref = ops.gemm_nt_int8(a, q, s), oracle.gemm_nt_int8(a, q, s)
    nonfinite_masks_equal(got, ref)
    assert np.isnan(got[1]).all()
    assert np.isposinf(got[2]).any() and np.isneginf(got[2]).any() and np.isnan(got[2, :40]).all()
    assert np.isfinite(got[m - 2]).sum() == 0
    clean = [i for i in range(m) if i not in (1, 2, m - 1, m - 2)]
    for i in clean:
        assert_close_rms(got[i], ref[i])


@pytest.mark.parametrize("m", [1, 4])
def test_gemm_nt_int8_nonfinite_few_rows(ops, oracle, m):
    """The one-launch form (M <= 4): a row holding NaN or +-inf gets the
    reference's f32 pattern (its products classified after the q8 sums come
    out NaN); the other rows are untouched."""
    rng = np.random.default_rng(90 + m)
    n, k = 256, 2304
    a, q, s = q8_case(rng, m, n, k)
    q[:40, 9] = 0                      # inf * 0 -> NaN in those columns
    q[40:80, 5] = -q[40:80, 4]
    a[0, 9] = -np.inf                  # -inf / +inf by the weight's sign, NaN at w = 0
    if m == 4:
        a[1, 7] = np.nan               # all NaN
        a[3, 4] = np.inf               # +inf and -inf in one row: NaN where the two
        a[3, 5] = -np.inf              # weights share a sign, +-inf elsewhere
    got, ref = ops.gemm_nt_int8(a, q, s), oracle.gemm_nt_int8(a, q, s)
    nonfinite_masks_equal(got, ref)
    assert np.isnan(got[0, :40]).all() and np.isinf(got[0, 40:]).all()
    assert np.isposinf(got[0]).any() and np.isneginf(got[0]).any()
    if m == 4:
        assert np.isnan(got[1]).all() and np.isfinite(got[3]).sum() == 0
        assert_close_rms(got[2], ref[2])


def test_gemm_nt_int8_exact_case_few_rows(ops):
    """Integer activations at M <= 4 (the one-launch form): the int8 terms,
    the int32 sums, the run factors and the wave-order sum are all exact."""
    rng = np.random.default_rng(8)
    for m, k in ((1, 2304), (3, 768), (4, 5760)):
        a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
        q = rng.integers(-127, 128, size=(64, k), dtype=np.int8)
        s = np.full(64, 1 / 64, np.float32)
        ref = (a.astype(np.float64) @ q.astype(np.float64).T) / 64
        assert np.array_equal(ops.gemm_nt_int8(a, q, s).astype(np.float64), ref), (m, k)


def test_gemm_nt_bf16_nonfinite(ops, oracle):
    """bf16 weights (term-split activations): the same non-finite pattern."""
    rng = np.random.default_rng(11)
    for m in (3, 20):
        a = rng.standard_normal((m, 256), dtype=np.float32)
        b = (rng.standard_normal((64, 256), dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
        b[:8, 6] = 0
        a[0, 6] = np.inf
        a[1, 2] = np.nan
        got, ref = ops.gemm_nt_bf16(a, b), oracle.gemm_nt_bf16(a, b)
        nonfinite_masks_equal(got, ref)
        for i in range(2, m):
            assert_close_rms(got[i], ref[i])


def test_gemm_nt_int8_exact_case(ops):
    """Integer activations and power-of-two scales: every term and partial
    sum is exact, so the result is exact."""
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 4, size=(5, 640)).astype(np.float32)
    q = rng.integers(-127, 128, size=(48, 640), dtype=np.int8)
    s = np.full(48, 1 / 64, np.float32)
    ref = (a.astype(np.float64) @ q.astype(np.float64).T) / 64
    assert np.array_equal(ops.gemm_nt_int8(a, q, s).astype(np.float64), ref)


@pytest.mark.parametrize("m,n,k", [(1, 5000, 2304), (16, 1000, 2304), (2, 33, 70),
                                   (64, 256, 512)])
def test_gemm_nt_bf16(ops, oracle, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = oracle.f32_to_bf16(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    assert_close_rms(ops.gemm_nt_bf16(a, b), oracle.gemm_nt_bf16(a, b))


@pytest.mark.parametrize("m,n,k", [(4, 8, 8), (1, 1, 64), (17, 23, 31), (512, 512, 64),
                                   (16, 16, 1), (64, 64, 64),
                                   # narrow outputs split over k (in-order slice sum)
                                   (512, 64, 512), (64, 64, 1024), (70, 33, 300)])
def test_gemm_nt_f32_and_nn(ops, oracle, m, n, k):
    rng = np.random.default_rng(m * n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((n, k), dtype=np.float32)
    c0 = rng.standard_normal((m, n), dtype=np.float32)
    assert_close_rms(ops.gemm_nt(a, b), oracle.gemm_nt(a, b))
    assert_close_rms(ops.gemm_nt(a, b, c0, acc=True), oracle.gemm_nt(a, b, c0, acc=True))
    bn = np.ascontiguousarray(b.T)
    assert_close_rms(ops.gemm(a, bn), oracle.gemm(a, bn))


def test_rmsnorm_softmax(ops, oracle):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, 2304), dtype=np.float32) * 3
    g = rng.uniform(0.5, 1.5, 2304).astype(np.float32)
    # the sum of squares is a tree sum instead of the reference's left-to-right
    # loop: ~sqrt(cols) * 2^-24 relative in the row scale
    assert_close_rms(ops.rmsnorm(x, g, 1e-5), oracle.rmsnorm(x, g, 1e-5), 1e-5)
    p = rng.standard_normal((37, 300), dtype=np.float32) * 4
    for causal in (False, True):
        got, ref = ops.softmax(p, causal), oracle.softmax(p, causal)
        assert np.abs(got - ref).max() <= 1e-6
        if causal:
            assert np.all(got[np.triu_indices(37, 1, 300)] == 0)


@pytest.mark.parametrize("rows,cols", [(600, 1024), (5, 2000), (3, 1)])
def test_softmax_shapes(ops, oracle, rows, cols):
    """Rows held by one wavefront (cols <= 1024) and the long-row path. The
    row sum is a tree sum against the reference's left-to-right loop; on a
    row of 1024 whose sum is ~1.014 the loop alone is 3.6e-6 from the exact
    sum (adding small terms to ~1 drops their low bits), so probabilities
    (<= 1) are held to 1e-5 absolute and every row to a sum of 1."""
    rng = np.random.default_rng(rows + cols)
    p = rng.standard_normal((rows, cols), dtype=np.float32) * 4
    for causal in (False, True):
        got, ref = ops.softmax(p, causal), oracle.softmax(p, causal)
        assert np.abs(got - ref).max() <= 1e-5
        assert np.abs(got.astype(np.float64).sum(1) - 1).max() <= 1e-5
        if causal:
            assert np.all(got[np.triu_indices(rows, 1, cols)] == 0)


@pytest.mark.parametrize("kind", range(6))
def test_act_bitwise(ops, oracle, kind):
    rng = np.random.default_rng(kind)
    x = (rng.standard_normal(1003, dtype=np.float32) * 6).astype(np.float32)
    x[:4] = [0.0, -0.0, 20.0, -20.0]
    assert np.array_equal(bits(ops.act(x, kind)), bits(oracle.act(x, kind)))


@pytest.mark.parametrize("op", [20, 21, 22, 23])
def test_ew_scale_bitwise(ops, oracle, op):
    rng = np.random.default_rng(op)
    x = rng.standard_normal(777, dtype=np.float32)
    y = rng.standard_normal(777, dtype=np.float32) + np.float32(0.1)
    assert np.array_equal(bits(ops.ew_op(x, y, op)), bits(oracle.ew_op(x, y, op)))
    assert np.array_equal(bits(ops.scale(x, 0.125)), bits(oracle.scale(x, 0.125)))


@pytest.mark.parametrize("offset", [0, 1, 3])
def test_elementwise_device_alignment(hip, oracle, offset):
    """Device-pointer element ops on buffers that start `offset` floats past a
    16-byte boundary: the aligned (four per thread) and scalar forms, and the
    ReLU body/tail split at n // 8 * 8, agree bitwise with the oracle."""
    import ctypes as C
    rng = np.random.default_rng(offset)
    n = 1029
    x = (rng.standard_normal(n, dtype=np.float32) * 6).astype(np.float32)
    x[:3] = [-0.0, np.nan, -3.0]
    x[-3:] = [-0.0, np.nan, -3.0]
    y = rng.standard_normal(n, dtype=np.float32) + np.float32(0.1)
    nb = (n + 8) * 4
    bufs = []
    for _ in range(3):
        p = C.c_void_p()
        assert hip.vmlm_hip_malloc(C.byref(p), nb) == 0
        bufs.append(p.value)
    dx, dy, dd = (b + 4 * offset for b in bufs)

    def up(dev, a):
        assert hip.vmlm_hip_memcpy_h2d(C.c_void_p(dev), a.ctypes.data, a.nbytes) == 0

    def down(dev):
        out = np.empty(n, np.float32)
        assert hip.vmlm_hip_sync() == 0
        assert hip.vmlm_hip_memcpy_d2h(out.ctypes.data, C.c_void_p(dev), out.nbytes) == 0
        return out

    try:
        up(dy, y)
        for kind in (0, 2, 4):
            up(dx, x)
            assert hip.vmlm_hip_act(C.c_void_p(dx), n, kind, None) == 0
            want = oracle.act(x, kind)
            got = down(dx)
            assert np.array_equal(np.isnan(got), np.isnan(want))
            ok = ~np.isnan(want)
            assert np.array_equal(bits(got[ok]), bits(want[ok])), kind
        up(dx, x)
        for op in (20, 21, 22, 23):
            assert hip.vmlm_hip_ew_op(C.c_void_p(dd), C.c_void_p(dx), C.c_void_p(dy), n, op,
                                      None) == 0
            got, want = down(dd), oracle.ew_op(x, y, op)
            ok = ~np.isnan(want)
            assert np.array_equal(bits(got[ok]), bits(want[ok])), op
        assert hip.vmlm_hip_scale(C.c_void_p(dd), C.c_void_p(dx), n, C.c_float(0.125), None) == 0
        got, want = down(dd), oracle.scale(x, 0.125)
        ok = ~np.isnan(want)
        assert np.array_equal(bits(got[ok]), bits(want[ok]))
    finally:
        for b in bufs:
            hip.vmlm_hip_free(C.c_void_p(b))


@pytest.mark.parametrize("pos0", [0, 1, 127, 1000, 65000])
def test_rope_bitwise(ops, oracle, pos0):
    rng = np.random.default_rng(pos0)
    x = rng.standard_normal((33, 64), dtype=np.float32)
    assert np.array_equal(bits(ops.rope(x, 10000.0, pos0)), bits(oracle.rope(x, 10000.0, pos0)))
    x = rng.standard_normal((5, 128), dtype=np.float32)
    assert np.array_equal(bits(ops.rope(x, 500000.0, pos0)),
                          bits(oracle.rope(x, 500000.0, pos0)))


def test_rope_guards(ops):
    from sparrow_amd import VmlmError
    with pytest.raises(VmlmError) as e:
        ops.rope(np.zeros((2, 63), np.float32), 10000.0, 0)
    assert e.value.code == 9


def test_emb_and_guards(ops, oracle):
    from sparrow_amd import VmlmError
    rng = np.random.default_rng(8)
    tab = oracle.f32_to_bf16(rng.standard_normal((50, 2304), dtype=np.float32))
    for r in (0, 17, 49):
        assert np.array_equal(bits(ops.emb_bf16(tab, float(r))),
                              bits(oracle.emb_bf16(tab, float(r))[1]))
    for bad in (-1.0, float("nan"), 50.0, 2.5):
        with pytest.raises(VmlmError) as e:
            ops.emb_bf16(tab, bad)
        assert e.value.code == 9


def test_topk_idx_bitexact(ops, oracle):
    rng = np.random.default_rng(9)
    for n in (1, 7, 122753):
        x = rng.standard_normal(n, dtype=np.float32)
        assert ops.topk_idx(x) == oracle.topk_idx(x)[1]
    x = np.zeros(5000, np.float32)
    x[[17, 300, 4999]] = 3.0  # ties: lowest index wins
    assert ops.topk_idx(x) == 17.0
    x = rng.standard_normal(1000, dtype=np.float32)
    x[0] = np.nan  # nothing compares > NaN: the scan keeps index 0
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 0.0


def test_topk_idx_edges(ops, oracle):
    """Cases the strict-`>` scan (core/src/interp.rs:1649-1681) fixes: -0.0
    and +0.0 tie (lowest index), NaN after index 0 is skipped, all-NaN gives
    0, -inf rows, and ties split across the workgroups of a long row."""
    x = np.array([-0.0, 0.0, -1.0], np.float32)
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 0.0
    x = np.array([-1.0, 0.0, -0.0], np.float32)
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 1.0
    x = np.array([1.0, np.nan, 2.0, np.nan], np.float32)
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 2.0
    x = np.full(4097, np.nan, np.float32)
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 0.0
    x = np.full(3000, -np.inf, np.float32)
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 0.0
    x = np.zeros(122753, np.float32)
    x[[120000, 5000, 70001]] = 7.5  # ties in different workgroups: lowest index
    assert ops.topk_idx(x) == oracle.topk_idx(x)[1] == 5000.0


@pytest.mark.parametrize("k0,n", [(1, 200), (1, 203), (2, 200), (2, 203), (2, 3), (4, 200),
                                  (4, 201), (8, 200), (20, 200), (32, 200), (37, 200)])
def test_b1_forward_bitwise(ops, oracle, k0, n):
    """b1_forward against the reference's packed rows (k0 in {1, 2, 4, 8},
    including k0 == 2, where rows 2r and 2r + 1 both get the pair's sum) and
    the 8-lane fold for the rows the packed path leaves (n not a multiple of
    the rows per 256-bit vector)."""
    rng = np.random.default_rng(k0 * 1000 + n)
    w = rng.standard_normal((n, k0), dtype=np.float32)
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    x = rng.standard_normal(n, dtype=np.float32)
    y, macs = ops.b1_forward(w, src, x)
    assert macs == n * k0
    assert np.array_equal(bits(y), bits(oracle.b1_forward(w, src, x)))


@pytest.mark.parametrize("k0,T,t8,n", [(32, 1024, 1024, 96), (20, 37, 40, 96), (1, 5, 8, 96),
                                       (0, 3, 8, 96), (33, 40, 48, 70),   # one lane per token
                                       (20, 37, 48, 100), (5, 16, 16, 33),  # planned, ragged
                                       (32, 200, 208, 1000), (1, 70, 80, 2032)])
def test_b1_forward_t8_bitwise(ops, oracle, k0, T, t8, n):
    """Planned layers (k0 <= 32, 16 | t8) and the one-lane-per-(neuron, token)
    kernel, bitwise against the t8 scalar contract."""
    rng = np.random.default_rng(k0 + T)
    w = rng.standard_normal((n, k0), dtype=np.float32)
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    x = rng.standard_normal((T, n), dtype=np.float32)
    xt = ops.transpose_t8(x, t8)
    assert np.array_equal(xt, oracle.transpose_t8(x, t8))
    yt, _ = ops.b1_forward_t8(w, src, xt, T)
    ref = oracle.b1_forward_t8(w, src, xt, T)
    assert np.array_equal(bits(yt[:, :T]), bits(ref[:, :T]))
    back = ops.transpose_t8_back(yt, T)
    assert np.array_equal(back, oracle.transpose_t8_back(yt, T))


def test_b1_t8_special_values(ops, oracle):
    """k0 = 5 pads each neuron's last group of four with three (zero row,
    weight -0.0) steps; the sums must keep signed zeros and infinities and
    produce NaN exactly where the contract does."""
    rng = np.random.default_rng(11)
    n, k0, T, t8 = 64, 5, 32, 32
    w = rng.standard_normal((n, k0), dtype=np.float32)
    w[:8] = -0.0                      # every product -0.0 (x > 0): sum -0.0
    w[8:16] = 0.0                     # +0.0 sums
    w[16:20, 2] = np.inf
    w[20:24, 0] = -np.inf
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    src[:16] = 0
    xt = rng.standard_normal((n, t8), dtype=np.float32)
    xt[0] = np.abs(xt[0]) + 0.5
    xt[1, ::3] = -0.0
    xt[2, ::5] = np.inf
    yt, _ = ops.b1_forward_t8(w, src, xt, T)
    ref = oracle.b1_forward_t8(w, src, xt, T)
    got, want = yt[:, :T], ref[:, :T]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))
    assert np.all(bits(got[:8]) == 0x80000000) and np.all(bits(got[8:16]) == 0)


def test_b1_guards(ops):
    from sparrow_amd import VmlmError
    w = np.ones((8, 4), np.float32)
    src = np.zeros((8, 4), np.uint32)
    src[3, 2] = 8  # out of range
    with pytest.raises(VmlmError) as e:
        ops.b1_forward(w, src, np.ones(8, np.float32))
    assert e.value.code == 9


@pytest.mark.parametrize("S,H", [(128, 4), (512, 36), (77, 2)])
def test_attention_prefill(ops, oracle, S, H):
    rng = np.random.default_rng(S + H)
    q, k, v = (rng.standard_normal((S, H * 64), dtype=np.float32) for _ in range(3))
    got = ops.attention_prefill(q, k, v, H)
    ref = oracle.attention_prefill(q, k, v, H)
    assert_close_rms(got, ref)
    assert np.array_equal(got[0], v[0]) or np.abs(got[0] - v[0]).max() <= 1e-6


def test_attention_prefill_one_launch_same_bits(ops, oracle):
    """Up to four 64-query blocks (S <= 256) over at least 256 workgroups
    (query blocks x heads) run as one launch from the f32 rows; longer
    prompts prepare bf16 term planes in a first launch. Causal rows see only
    earlier keys, so the first 256 output rows of a 300-token prompt (two
    launches) equal those of its 256-token prefix (one launch, 64 heads) bit
    for bit. Non-causal rows from the one launch match the oracle."""
    rng = np.random.default_rng(31)
    H = 64
    q, k, v = (rng.standard_normal((300, H * 64), dtype=np.float32) for _ in range(3))
    long_ = ops.attention_prefill(q, k, v, H, pos0=5)
    short = ops.attention_prefill(q[:256].copy(), k[:256].copy(), v[:256].copy(), H, pos0=5)
    assert np.array_equal(long_[:256].view(np.uint32), short.view(np.uint32))
    for S in (200, 256):
        got = ops.attention_prefill(q[:S].copy(), k[:S].copy(), v[:S].copy(), H, causal=False)
        ref = oracle.attention_prefill(q[:S], k[:S], v[:S], H, causal=False)
        assert_close_rms(got, ref)


@pytest.mark.parametrize("H,pos", [(36, 1023), (36, 700), (4, 511), (36, 300)])
def test_attention_decode_cfg2(ops, oracle, H, pos):
    """Config 2 decode: 1 query against a KV cache of length 1024 (pos 1023),
    and shorter caches: split over partitions of four 16-position
    sub-chunks merged in order (pos 1023, 700, 511: a partial last partition
    at 700), or one workgroup per head (pos 300: 19 sub-chunks, under the 32
    from which the library splits)."""
    rng = np.random.default_rng(2)
    hd, cap = 64, 1024
    kc = np.zeros((H, cap, hd), np.float32)
    vc = np.zeros((H, cap, hd), np.float32)
    kraw = rng.standard_normal((pos, H * hd), dtype=np.float32)
    for h in range(H):  # rotated keys at their positions 0..pos-1, raw values
        kc[h, :pos, :] = oracle.rope(kraw[:, h * hd:(h + 1) * hd], 10000.0, 0)
    vc[:, :pos, :] = rng.standard_normal((H, pos, hd), dtype=np.float32)
    q, kn, vn = (rng.standard_normal(H * hd, dtype=np.float32) for _ in range(3))
    kc2, vc2 = kc.copy(), vc.copy()
    got = ops.attention_decode(q, kn, vn, kc, vc, pos)
    ref = oracle.attention_decode(q, kn, vn, kc2, vc2, pos)
    assert_close_rms(got, ref)
    assert np.array_equal(bits(kc[:, pos]), bits(kc2[:, pos]))  # appended rotated k, bitwise
    assert np.array_equal(vc[:, pos], vc2[:, pos])


@pytest.mark.parametrize("pos", [1023, 700, 257, 100, 16, 15, 0])
def test_attention_decode_split_bitwise(ops, oracle, pos):
    """The cached positions split over workgroups of 1, 2, 3, 4, 8 or 64
    sub-chunks of 16 positions, or one workgroup per head: the same bits
    every time (the sub-chunk partials are merged in position order
    whichever workgroup computed them), within 1e-4 RMS of the oracle, and
    the appended row bitwise the oracle's. pos 0 attends the new row only;
    15 and 16 end a sub-chunk and start the next."""
    rng = np.random.default_rng(20 + pos)
    H, hd, cap = 8, 64, 1024
    kc = np.zeros((H, cap, hd), np.float32)
    vc = np.zeros((H, cap, hd), np.float32)
    kc[:, :pos, :] = rng.standard_normal((H, pos, hd), dtype=np.float32)
    vc[:, :pos, :] = rng.standard_normal((H, pos, hd), dtype=np.float32)
    q, kn, vn = (rng.standard_normal(H * hd, dtype=np.float32) for _ in range(3))
    kr, vr = kc.copy(), vc.copy()
    ref = oracle.attention_decode(q, kn, vn, kr, vr, pos)
    first = None
    for split in (0, -1, 1, 2, 3, 4, 8, 64):
        k2, v2 = kc.copy(), vc.copy()
        got = ops.attention_decode(q, kn, vn, k2, v2, pos, split=split)
        assert np.array_equal(bits(k2[:, pos]), bits(kr[:, pos])), split
        assert np.array_equal(v2[:, pos], vr[:, pos]), split
        assert np.array_equal(k2[:, :pos], kc[:, :pos]), split
        if first is None:
            first = got
            assert_close_rms(got, ref)
        else:
            assert np.array_equal(bits(got), bits(first)), split


def test_graph_capture_replay(hip, oracle):
    """Device-API ops captured into a HIP graph (vmlm_hip_capture_begin/end)
    and replayed three times, with eager work and synchronisations between
    the replays: every replay equals the eager result bitwise. gemm_nt with
    k = 0 clears C with a fill kernel, so it captures and replays like any
    other op; a call that would stage a device copy (int8 GEMM with K not a
    multiple of 128) returns 5 before it issues anything, and the capture
    stays valid."""
    import ctypes as C
    rng = np.random.default_rng(7)
    rows, cols = 37, 1024
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    g = (rng.standard_normal(cols, dtype=np.float32) * 0.5 + 1).astype(np.float32)
    nb = x.nbytes
    bufs = {}
    for name, size in (("x", nb), ("g", g.nbytes), ("y", nb), ("z", nb), ("w", nb)):
        p = C.c_void_p()
        assert hip.vmlm_hip_malloc(C.byref(p), size) == 0
        bufs[name] = p
    dx, dg, dy, dz, dw = (bufs[k] for k in ("x", "g", "y", "z", "w"))

    def down(dev):
        out = np.empty((rows, cols), np.float32)
        assert hip.vmlm_hip_sync() == 0
        assert hip.vmlm_hip_memcpy_d2h(out.ctypes.data, dev, out.nbytes) == 0
        return out

    def down_bytes(dev, n):
        out = np.empty(n, np.uint8)
        assert hip.vmlm_hip_sync() == 0
        assert hip.vmlm_hip_memcpy_d2h(out.ctypes.data, dev, n) == 0
        return out

    def seq():  # y = rmsnorm(x) * g; z = y + x
        return (hip.vmlm_hip_rmsnorm(dy, dx, dg, rows, cols, C.c_float(1e-5), None) or
                hip.vmlm_hip_ew_op(dz, dy, dx, rows * cols, 20, None))

    graph = C.c_void_p()
    try:
        assert hip.vmlm_hip_memcpy_h2d(dx, x.ctypes.data, nb) == 0
        assert hip.vmlm_hip_memcpy_h2d(dg, g.ctypes.data, g.nbytes) == 0
        assert seq() == 0
        want = down(dz)
        assert_close_rms(want, oracle.ew_op(oracle.rmsnorm(x, g, 1e-5), x, 20))
        assert hip.vmlm_hip_capture_begin(None) == 0
        assert seq() == 0
        assert hip.vmlm_hip_capture_end(None, C.byref(graph)) == 0 and graph.value
        for r in range(3):
            assert hip.vmlm_hip_memset(dz, 0xFF, nb) == 0  # garbage the result
            assert hip.vmlm_hip_memset(dy, 0xFF, nb) == 0
            assert hip.vmlm_hip_scale(dw, dx, rows * cols, C.c_float(0.5), None) == 0  # eager work
            assert hip.vmlm_hip_sync() == 0
            assert hip.vmlm_hip_graph_launch(graph, None) == 0
            assert np.array_equal(bits(down(dz)), bits(want)), r
        # k = 0 zero-fills C with a kernel, so it captures like any other op
        assert hip.vmlm_hip_memset(dw, 0xFF, 64) == 0
        assert hip.vmlm_hip_sync() == 0
        g0 = C.c_void_p()
        assert hip.vmlm_hip_capture_begin(None) == 0
        assert hip.vmlm_hip_gemm_nt(dx, dx, dw, 4, 4, 0, False, None) == 0
        assert hip.vmlm_hip_capture_end(None, C.byref(g0)) == 0 and g0.value
        try:
            for r in range(3):
                assert hip.vmlm_hip_memset(dw, 0xFF, 64) == 0
                assert hip.vmlm_hip_sync() == 0
                assert hip.vmlm_hip_graph_launch(g0, None) == 0
                assert hip.vmlm_hip_sync() == 0
                assert not down_bytes(dw, 64).any(), r
        finally:
            hip.vmlm_hip_graph_destroy(g0)
        # a call that would stage a device copy is refused before it issues
        # anything, and the capture stays empty and valid
        assert hip.vmlm_hip_capture_begin(None) == 0
        rc = hip.vmlm_hip_gemm_nt_int8(dx, dx, dx, dw, 2, 2, 100, None)
        empty = C.c_void_p()
        assert hip.vmlm_hip_capture_end(None, C.byref(empty)) == 0
        assert rc == 5
        if empty.value:
            hip.vmlm_hip_graph_destroy(empty)
        assert seq() == 0
        assert np.array_equal(bits(down(dz)), bits(want))
    finally:
        hip.vmlm_hip_graph_destroy(graph)
        for p in bufs.values():
            hip.vmlm_hip_free(p)
